// Depthwise KxK convolutions of the VisionHOPE block on channels-last maps, with
// the elementwise work around each convolution fused into its epilogue.
//
// Reference composition (models/block.py:63-107, models/layers.py:73-77):
//   cpe     x + dwconv3(x)                                   (block.py:102-103)
//   local   x + sigmoid(gate) * dwconv7(x)                   (block.py:63-66)
//   lepe    out + dwconv5(x_local)   (out: SRNL NHWC fp32)   (block.py:77-78),
//           accumulated in place (fp32) or written in the io dtype for proj_out
//   ffn     gelu(h + dwconv3(h))                             (layers.py:76-77)
// Each thread computes 8 consecutive channels of a row segment of pixels with fp32
// accumulation; taps are stored taps-major ([K*K][C], fp32) so one tap is two float4 loads.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "vh_common.h"

namespace vh {

enum DwEpilogue { DW_PLAIN = 0, DW_ADD_INPUT = 1, DW_GATE = 2, DW_ADD_GELU = 3, DW_ACCUM_F32 = 4, DW_ADD_F32_AUX = 5,
                  DW_ADD_GELU_SUMSQ = 6,     // 6: internal, DW_ADD_GELU + GRN partial sums (see below)
                  DW_ADD_INPUT_LN = 7 };     // 7: internal, DW_ADD_INPUT + the LayerNorm of the result

struct DwParams {
    const void* x;
    const float* taps;   // [K*K, C]
    const float* bias;   // [C] or null
    const void* aux;     // gate for DW_GATE (io dtype); fp32 addend for DW_ADD_F32_AUX
    void* out;           // io dtype, or fp32 for DW_ACCUM_F32
    int64_t B, H, W, C;
    float* partial;      // DW_ADD_GELU_SUMSQ: [B, blocks per image, C] sums of squares of out
    // DW_ADD_INPUT_LN: LayerNorm affine [C] fp32, eps, output [B, H, W, C] (io dtype) and
    // log2 of the lanes per pixel (C / 8, a power of two <= 32)
    const float* ln_w = nullptr;
    const float* ln_b = nullptr;
    float ln_eps = 0.f;
    void* out_norm = nullptr;
    int ln_lg = 0;
};

// Launch geometry: thread index -> (image, row, segment, channel group), with the
// divisions done by multiplication (all indices < 2^31, checked on the host).
struct DwGrid {
    uint32_t total;            // B * H * segs * G threads
    FastDiv G, segs, H;
};

// Eight consecutive channels at byte offset `off` of a buffer as raw 32-bit words; an
// offset past the buffer's range reads zeros (buffer addressing returns 0 out of range),
// so padding needs no branch and every load of a window can be in flight at once.
template <typename T>
struct Raw8 {
    static constexpr int N = sizeof(T) == 4 ? 2 : 1;   // 16-byte loads per 8 elements
    uint32_t w[4 * N];
};
template <typename T>
__device__ __forceinline__ Raw8<T> buffer_load8(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
    Raw8<T> r;
#pragma unroll
    for (int n = 0; n < Raw8<T>::N; ++n) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(off + 16 * n), 0, 0);
        r.w[4 * n] = v[0]; r.w[4 * n + 1] = v[1]; r.w[4 * n + 2] = v[2]; r.w[4 * n + 3] = v[3];
    }
    return r;
}
template <typename T>
__device__ __forceinline__ void decode8(const Raw8<T>& r, float (&v)[8]) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(r.w[j]);
    } else {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            v[2 * h] = to_f32(T{static_cast<uint16_t>(r.w[h] & 0xffffu)});
            v[2 * h + 1] = to_f32(T{static_cast<uint16_t>(r.w[h] >> 16)});
        }
    }
}

// Epilogue of one output pixel (8 channels at element offset `at`): the fused
// elementwise work of EPI on the accumulated window `acc` (bias included) and the
// input value `center` at the same position, then one store; DW_ADD_GELU_SUMSQ also
// adds the squares of the stored values to `sumsq`.
template <int EPI, typename T>
__device__ __forceinline__ void dw_store_pixel(const DwParams& p, int64_t at, float (&acc)[8],
                                               [[maybe_unused]] const float (&center)[8],
                                               [[maybe_unused]] float (&sumsq)[8],
                                               [[maybe_unused]] const float2* gq = nullptr) {
    if constexpr (EPI == DW_ACCUM_F32) {
        float* o = static_cast<float*>(p.out) + at;
        float prev[8];
        load8<float>(o, prev);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = prev[j] + acc[j];
        store8<float>(o, acc);
    } else {
        if constexpr (EPI == DW_ADD_F32_AUX) {
            float a[8];
            load8<float>(static_cast<const float*>(p.aux) + at, a);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = a[j] + acc[j];
        } else if constexpr (EPI == DW_GATE) {
            float gv[8];
            load8<T>(static_cast<const T*>(p.aux) + at, gv);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = center[j] + sigmoid_fast(gv[j]) * acc[j];
        } else if constexpr (EPI == DW_ADD_GELU || EPI == DW_ADD_GELU_SUMSQ) {
            // the interpolated GELU (gq: its table in LDS) for 2-byte outputs, else the
            // erfc form
            if (sizeof(T) == 2 && gq) {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = gelu_qi(center[j] + acc[j], gq);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = gelu_fast(center[j] + acc[j]);
            }
            if constexpr (EPI == DW_ADD_GELU_SUMSQ) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float r = to_f32(from_f32<T>(acc[j]));   // the stored value
                    sumsq[j] += r * r;
                }
            }
        } else if constexpr (EPI == DW_ADD_INPUT) {
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = center[j] + acc[j];
        }
        store8<T>(static_cast<T*>(p.out) + at, acc);
    }
}

// One thread per (image, row, segment of P pixels, 8 channels): each kernel row loads
// the P+K-1 input vectors of the segment once and reuses them for all K horizontal
// taps of the P outputs, so a K x K window costs (P+K-1)/P input loads per tap row
// instead of K.  Consecutive lanes take consecutive channel groups (coalesced), and
// consecutive blocks of one XCD take consecutive rows, so the rows above and below a
// block's own are read through the same L2.  The input is addressed as one buffer of
// `x_bytes` bytes (< 2^31): positions outside the image read zeros.
template <int K, int EPI, typename T, int P>
__global__ __launch_bounds__(256) void dwconv_nhwc_kernel(const DwParams p, const DwGrid g, const uint32_t x_bytes) {
    constexpr int R = K / 2, NI = P + K - 1;
    constexpr uint32_t OUTSIDE = 0x80000000u;
    // 256 threads per block, or whole channel groups (G * r threads) for the GRN sums
    const uint32_t idx = xcd_remap_any(blockIdx.x, gridDim.x) * blockDim.x + threadIdx.x;
    // GELU table of 2-byte outputs, copied to LDS by every thread before any returns
    [[maybe_unused]] const float2* gq = nullptr;
    if constexpr ((EPI == DW_ADD_GELU || EPI == DW_ADD_GELU_SUMSQ) && sizeof(T) == 2) {
        __shared__ float4 gq4[GELU_QI_N / 2];
        gelu_qi_fill(gq4, static_cast<int>(threadIdx.x), static_cast<int>(blockDim.x));
        __syncthreads();
        gq = reinterpret_cast<const float2*>(gq4);
    }
    if (idx >= g.total) return;
    const uint32_t t0 = fast_div(idx, g.G);
    const uint32_t cg = idx - t0 * g.G.d;
    const uint32_t t1 = fast_div(t0, g.segs);
    const uint32_t seg = t0 - t1 * g.segs.d;
    const uint32_t b = fast_div(t1, g.H);
    const int h = static_cast<int>(t1 - b * g.H.d);
    const int W = static_cast<int>(p.W), H = static_cast<int>(p.H), C = static_cast<int>(p.C);
    const int w0 = static_cast<int>(seg) * P;
    const int c = static_cast<int>(cg) * 8;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), 0, x_bytes, 0x00020000);
    // Byte offset of (row hh, column ww) of this image and channel group.
    const uint32_t row0 = static_cast<uint32_t>(b) * H;
    auto offset = [&](int hh, int ww) -> uint32_t {
        const bool ok = (static_cast<uint32_t>(hh) < static_cast<uint32_t>(H)) &
                        (static_cast<uint32_t>(ww) < static_cast<uint32_t>(W));
        const uint32_t off = (((row0 + hh) * static_cast<uint32_t>(W) + ww) * static_cast<uint32_t>(C) + c) * sizeof(T);
        return ok ? off : OUTSIDE;
    };

    float acc[P][8];
    {
        float b8[8];
        if (p.bias) load8<float>(p.bias + c, b8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float bj = p.bias ? b8[j] : 0.f;
#pragma unroll
            for (int px = 0; px < P; ++px) acc[px][j] = bj;
        }
    }
    [[maybe_unused]] float center[P][8];
    auto load_row = [&](int hh, Raw8<T> (&r)[NI]) {
#pragma unroll
        for (int i = 0; i < NI; ++i) r[i] = buffer_load8<T>(xr, offset(hh, w0 - R + i));
    };
    // Each input vector is decoded once and applied to every output of the segment
    // that it touches.
    auto compute_row = [&](int dy, const Raw8<T> (&r)[NI]) {
        float tp[K][8];
#pragma unroll
        for (int dx = 0; dx < K; ++dx) load8<float>(p.taps + (dy * K + dx) * C + c, tp[dx]);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            float v[8];
            decode8<T>(r[i], v);
            if constexpr (EPI == DW_ADD_INPUT || EPI == DW_GATE || EPI == DW_ADD_GELU || EPI == DW_ADD_GELU_SUMSQ ||
                          EPI == DW_ADD_INPUT_LN) {
                if (i >= R && i < R + P && dy == R) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) center[i - R][j] = v[j];
                }
            }
#pragma unroll
            for (int dx = 0; dx < K; ++dx) {
                const int px = i - dx;
                if (px >= 0 && px < P) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) acc[px][j] += v[j] * tp[dx][j];
                }
            }
        }
    };
    if constexpr (K == 3) {
        // Every load of the 3 x (P+2) window in flight at once.
        Raw8<T> raw[K][NI];
#pragma unroll
        for (int dy = 0; dy < K; ++dy) load_row(h + dy - R, raw[dy]);
#pragma unroll
        for (int dy = 0; dy < K; ++dy) compute_row(dy, raw[dy]);
    } else {
        // Larger windows: rows pipelined in two register sets (row dy+1 loads while
        // row dy computes), which keeps the register count within one wave's budget.
        Raw8<T> ra[NI], rb[NI];
        load_row(h - R, ra);
#pragma unroll 1
        for (int dy = 0; dy < K; dy += 2) {
            load_row(h + dy + 1 - R, rb);
            compute_row(dy, ra);
            if (dy + 1 == K) break;
            load_row(h + dy + 2 - R, ra);
            compute_row(dy + 1, rb);
        }
    }
    const int64_t pix0 = (static_cast<int64_t>(row0) + h) * W + w0;
    [[maybe_unused]] float sumsq[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if constexpr (EPI == DW_ADD_INPUT_LN) {
        // x + conv(x) as stored (rounded to T), then its LayerNorm over the pixel's C
        // channels: the C/8 lanes of one pixel segment are consecutive lanes (cg = lane
        // within the group), so the sums run as in layernorm_nhwc8_kernel with one group
        // of 8 channels per lane, and both outputs are the bits that the separate
        // kernels give.  A segment's lanes share w0, so the loop exit is uniform in a group.
        float lw[8], lb[8];
        load8<float>(p.ln_w + c, lw);
        load8<float>(p.ln_b + c, lb);
        const float inv_c = 1.f / static_cast<float>(C);   // exact for power-of-two C
#pragma unroll
        for (int px = 0; px < P; ++px) {
            if (w0 + px >= W) break;
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = center[px][j] + acc[px][j];
            if constexpr (std::is_same_v<T, bf16_t>) {
                // one conversion per pair, stored, then read back as the stored values
                uint32_t wv[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) wv[k] = pack_bf16x2(v[2 * k], v[2 * k + 1]);
                *reinterpret_cast<uint4*>(static_cast<T*>(p.out) + (pix0 + px) * C + c) =
                    make_uint4(wv[0], wv[1], wv[2], wv[3]);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[2 * k] = __uint_as_float(wv[k] << 16);
                    v[2 * k + 1] = __uint_as_float(wv[k] & 0xffff0000u);
                }
            } else {
                store8<T>(static_cast<T*>(p.out) + (pix0 + px) * C + c, v);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = to_f32(from_f32<T>(v[j]));
            }
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) sum += v[j];
            sum = ln_lane_sum(sum, p.ln_lg);
            const float mean = sum * inv_c;
            float sq = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[j] -= mean;
                sq += v[j] * v[j];
            }
            sq = ln_lane_sum(sq, p.ln_lg);
            const float rstd = __builtin_amdgcn_rsqf(sq * inv_c + p.ln_eps);
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = v[j] * rstd * lw[j] + lb[j];
            store8<T>(static_cast<T*>(p.out_norm) + (pix0 + px) * C + c, o);
        }
    } else {
#pragma unroll
        for (int px = 0; px < P; ++px) {
            if (w0 + px >= W) break;
            dw_store_pixel<EPI, T>(p, (pix0 + px) * C + c, acc[px], center[px], sumsq, gq);
        }
    }
    if constexpr (EPI == DW_ADD_GELU_SUMSQ) {
        // GRN partial sums: this block's threads cover whole channel groups of one image
        // (the host launches G * r threads, r pixel segments, and whole blocks per image),
        // blockDim / G threads per group; the first G threads add their group's rows in
        // order (deterministic).
        __shared__ float red[256 * 8];
#pragma unroll
        for (int j = 0; j < 8; ++j) red[threadIdx.x * 8 + j] = sumsq[j];
        __syncthreads();
        const int G = static_cast<int>(g.G.d);
        if (static_cast<int>(threadIdx.x) < G) {
            float tot[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int r = 0; r < static_cast<int>(blockDim.x) / G; ++r)
#pragma unroll
                for (int j = 0; j < 8; ++j) tot[j] += red[(r * G + threadIdx.x) * 8 + j];
            // Blocks of one image are consecutive logical blocks: partial [b][slab] is
            // row idx / blockDim of [B * blocks per image, C].
            float* dst = p.partial + static_cast<int64_t>(idx / blockDim.x) * C + 8 * threadIdx.x;
#pragma unroll
            for (int j = 0; j < 8; ++j) dst[j] = tot[j];
        }
    }
}

// LDS-tiled variant.  A block owns one image, a band of RB output rows and a slab of
// CS = 8 CG channels: it copies the band's input rows with their K/2-row halo (zeros
// outside the image, and K/2 zero columns either side) and the slab's taps into LDS
// once, then each thread computes P consecutive pixels x 8 channels of one output row
// from LDS.  Global memory sees each input vector of the band once (plus the halo)
// instead of once per tap row and segment, and every (pixel segment, channel group) of
// the map is a thread, which small maps need to fill the chip.  Per output the window
// is accumulated in the order of dwconv_nhwc_kernel (tap rows top to bottom, inputs
// left to right), so both kernels produce the same bits.
struct DwTile {
    int P;             // pixels per thread (7 or 8; 2 for 7x7 windows on maps up to 14 wide)
    int CG;            // 8-channel groups per block
    int segs;          // P-pixel segments per row
    int RB;            // output rows per band
    int bands;         // bands per image
    int slabs;         // channel slabs, C / (8 CG)
    int WP;            // tile row length in pixels: segs P + K - 1
    int TR;            // tile rows: RB + K - 1
    uint32_t x_bytes;  // LDS bytes of the input tile (at least the 8 KB reduction buffer)
    uint32_t lds_bytes;
    FastDiv wp_div, cg_div;
};

template <int K, int EPI, typename T, int P>
__global__ __launch_bounds__(256) void dwconv_tile_kernel(const DwParams p, const DwTile t) {
    constexpr int R = K / 2, NI = P + K - 1, VB = 8 * static_cast<int>(sizeof(T));
    extern __shared__ __align__(16) unsigned char dw_lds[];
    // GELU table of 2-byte outputs (visible after the staging barrier below)
    [[maybe_unused]] const float2* gq = nullptr;
    if constexpr ((EPI == DW_ADD_GELU || EPI == DW_ADD_GELU_SUMSQ) && sizeof(T) == 2) {
        __shared__ float4 gq4[GELU_QI_N / 2];
        gelu_qi_fill(gq4, static_cast<int>(threadIdx.x), 256);
        gq = reinterpret_cast<const float2*>(gq4);
    }
    const int CG = t.CG, CS = 8 * CG, H = static_cast<int>(p.H), W = static_cast<int>(p.W);
    const int64_t C = p.C;
    // Slabs of one (image, band) are adjacent blocks (they read the same input lines),
    // then the bands of one image (they share halo rows).
    const uint32_t l = xcd_remap_any(blockIdx.x, gridDim.x);
    const uint32_t slab = l % static_cast<uint32_t>(t.slabs), l1 = l / static_cast<uint32_t>(t.slabs);
    const int band = static_cast<int>(l1 % static_cast<uint32_t>(t.bands));
    const int64_t b = l1 / static_cast<uint32_t>(t.bands);
    const int h0 = band * t.RB;
    const int c0 = static_cast<int>(slab) * CS;
    const int tid = threadIdx.x;
    unsigned char* xs = dw_lds;
    float* tps = reinterpret_cast<float*>(dw_lds + t.x_bytes);

    // Stage the tile: vector e = (tile row, tile column, group) in that order, so the
    // LDS address is 16 e (or 32 e for FP32) and consecutive lanes copy consecutive
    // 16-byte pieces of one pixel's slab.
    const T* xb = static_cast<const T*>(p.x) + b * H * W * C + c0;
    const int nvec = t.TR * t.WP * CG;
    constexpr int NB = 4;
    for (int base = tid; base < nvec; base += 256 * NB) {
        Raw8<T> v[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int e = base + 256 * u;
            const uint32_t pix = fast_div(static_cast<uint32_t>(e), t.cg_div);
            const int g = e - static_cast<int>(pix) * CG;
            const uint32_t tr = fast_div(pix, t.wp_div);
            const int hh = h0 - R + static_cast<int>(tr), ww = static_cast<int>(pix - tr * t.WP) - R;
            const bool inside = e < nvec && static_cast<unsigned>(hh) < static_cast<unsigned>(H) &&
                                static_cast<unsigned>(ww) < static_cast<unsigned>(W);
#pragma unroll
            for (int n = 0; n < Raw8<T>::N; ++n) {
                uint4 q = make_uint4(0u, 0u, 0u, 0u);
                if (inside) q = *reinterpret_cast<const uint4*>(xb + (static_cast<int64_t>(hh) * W + ww) * C + 8 * g + 4 * n);
                v[u].w[4 * n] = q.x; v[u].w[4 * n + 1] = q.y; v[u].w[4 * n + 2] = q.z; v[u].w[4 * n + 3] = q.w;
            }
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int e = base + 256 * u;
            if (e < nvec) {
#pragma unroll
                for (int n = 0; n < Raw8<T>::N; ++n)
                    *reinterpret_cast<uint4*>(xs + e * VB + 16 * n) =
                        make_uint4(v[u].w[4 * n], v[u].w[4 * n + 1], v[u].w[4 * n + 2], v[u].w[4 * n + 3]);
            }
        }
    }
    for (int e = tid; e < K * K * 2 * CG; e += 256) {
        const int tap = e / (2 * CG), qd = e - tap * 2 * CG;
        *reinterpret_cast<float4*>(tps + tap * CS + 4 * qd) =
            *reinterpret_cast<const float4*>(p.taps + tap * C + c0 + 4 * qd);
    }
    __syncthreads();

    const int g = tid % CG, rs = tid / CG, s = rs % t.segs, r = rs / t.segs;
    const int h = h0 + r, w0 = s * P, c = c0 + 8 * g;
    [[maybe_unused]] float sumsq[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    auto vec_at = [&](int tr, int wc) {   // decoded input vector at tile (row, column)
        Raw8<T> raw;
        const unsigned char* src = xs + ((tr * t.WP + wc) * CG + g) * VB;
#pragma unroll
        for (int n = 0; n < Raw8<T>::N; ++n) {
            const uint4 q = *reinterpret_cast<const uint4*>(src + 16 * n);
            raw.w[4 * n] = q.x; raw.w[4 * n + 1] = q.y; raw.w[4 * n + 2] = q.z; raw.w[4 * n + 3] = q.w;
        }
        return raw;
    };
    if (r < t.RB && h < H) {
        float acc[P][8];
        {
            float b8[8];
            if (p.bias) load8<float>(p.bias + c, b8);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float bj = p.bias ? b8[j] : 0.f;
#pragma unroll
                for (int px = 0; px < P; ++px) acc[px][j] = bj;
            }
        }
        // Tap rows one at a time for 5x5 and 7x7 (unrolled, their taps and inputs would
        // take the whole register file).
        constexpr int DY_UNROLL = K == 3 ? K : 1;
#pragma unroll DY_UNROLL
        for (int dy = 0; dy < K; ++dy) {
            float tp[K][8];
#pragma unroll
            for (int dx = 0; dx < K; ++dx) {
                const float4 a = *reinterpret_cast<const float4*>(tps + (dy * K + dx) * CS + 8 * g);
                const float4 bq = *reinterpret_cast<const float4*>(tps + (dy * K + dx) * CS + 8 * g + 4);
                tp[dx][0] = a.x; tp[dx][1] = a.y; tp[dx][2] = a.z; tp[dx][3] = a.w;
                tp[dx][4] = bq.x; tp[dx][5] = bq.y; tp[dx][6] = bq.z; tp[dx][7] = bq.w;
            }
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                float v[8];
                decode8<T>(vec_at(r + dy, w0 + i), v);
#pragma unroll
                for (int dx = 0; dx < K; ++dx) {
                    const int px = i - dx;
                    if (px >= 0 && px < P) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[px][j] += v[j] * tp[dx][j];
                    }
                }
            }
        }
        const int64_t pix0 = (b * H + h) * W + w0;
#pragma unroll
        for (int px = 0; px < P; ++px) {
            if (w0 + px >= W) break;
            float center[8];
            if constexpr (EPI == DW_ADD_INPUT || EPI == DW_GATE || EPI == DW_ADD_GELU || EPI == DW_ADD_GELU_SUMSQ)
                decode8<T>(vec_at(r + R, w0 + px + R), center);
            dw_store_pixel<EPI, T>(p, (pix0 + px) * C + c, acc[px], center, sumsq, gq);
        }
    }
    if constexpr (EPI == DW_ADD_GELU_SUMSQ) {
        // GRN partial sums of this (image, band, slab): group g's threads in order; the
        // partial row of (image, band) is [b * bands + band][C].
        __syncthreads();
        float* red = reinterpret_cast<float*>(xs);
#pragma unroll
        for (int j = 0; j < 8; ++j) red[tid * 8 + j] = sumsq[j];
        __syncthreads();
        if (tid < CG) {
            float tot[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int k = 0; k < 256 / CG; ++k)
#pragma unroll
                for (int j = 0; j < 8; ++j) tot[j] += red[(k * CG + tid) * 8 + j];
            float* dst = p.partial + (b * t.bands + band) * C + c0 + 8 * tid;
#pragma unroll
            for (int j = 0; j < 8; ++j) dst[j] = tot[j];
        }
    }
}

namespace {

// Pixels per thread (register blocking along W) of dwconv_nhwc_kernel, measured on
// MI355X at the Tiny shapes (B=128; W = 56, 14 and 7): 8 pixels for 3x3, 4 for 5x5,
// 2 for 7x7 on wide maps and 8 on narrow ones.
inline int dw_default_pixels(int K, int64_t W) {
    // 3x3: 7 on widths that 7 divides and 8 does not (the Tiny 28, 14 and 7), so no
    // thread computes pixels past the row end; the segment count is unchanged there.
    if (K == 3) return (W % 8 != 0 && W % 7 == 0) ? 7 : 8;
    if (K == 5) return 4;
    return W >= 28 ? 2 : 8;
}

// Threads per block of the GRN partial-sum launch: G channel groups times the most
// pixel segments per block (at most 256 / G) that divide an image's rows x segments, so
// blocks hold whole channel groups and tile whole images.
inline int64_t dw_sumsq_block(int64_t G, int64_t rowsegs) {
    for (int64_t r = 256 / G; r > 1; --r)
        if (rowsegs % r == 0) return G * r;
    return G;
}

template <int K, typename T, int P>
void launch_dw_p(int epi, const DwParams& dp, hipStream_t s) {
    // The input of one launch is addressed as one buffer below 2^31 bytes: large batches
    // go in several launches of whole images.
    // The dw_launch_bytes override lowers the per-launch limit (tests use it to exercise
    // the split).
    int64_t limit = (int64_t(1) << 31) - 1;
    const Override forced_limit("dw_launch_bytes");
    if (forced_limit.set()) limit = std::min<int64_t>(limit, std::max<int64_t>(1, forced_limit.as_i64()));
    const int64_t image_elems = dp.H * dp.W * dp.C;
    const int64_t per_launch = std::max<int64_t>(1, limit / (image_elems * int64_t(sizeof(T))));
    const int64_t segs = (dp.W + P - 1) / P;
    // block size: 256 threads, or whole channel groups tiling whole images for the GRN sums
    const int64_t G = dp.C / 8;
    const uint32_t bd = epi == DW_ADD_GELU_SUMSQ && G <= 256 ? static_cast<uint32_t>(dw_sumsq_block(G, dp.H * segs)) : 256u;
    const size_t out_size = epi == DW_ACCUM_F32 ? sizeof(float) : sizeof(T);
    const size_t aux_size = epi == DW_ADD_F32_AUX ? sizeof(float) : sizeof(T);
    for (int64_t b0 = 0; b0 < dp.B; b0 += per_launch) {
        DwParams q = dp;
        q.B = std::min(per_launch, dp.B - b0);
        const int64_t skip = b0 * image_elems;
        q.x = static_cast<const char*>(dp.x) + skip * sizeof(T);
        q.out = static_cast<char*>(dp.out) + skip * out_size;
        if (dp.aux) q.aux = static_cast<const char*>(dp.aux) + skip * aux_size;
        if (dp.partial) q.partial = dp.partial + b0 * (dp.H * segs * (dp.C / 8) / bd) * dp.C;
        if (dp.out_norm) q.out_norm = static_cast<char*>(dp.out_norm) + skip * sizeof(T);
        DwGrid g;
        g.total = static_cast<uint32_t>(q.B * q.H * segs * (q.C / 8));
        g.G = make_fastdiv(static_cast<uint32_t>(q.C / 8));
        g.segs = make_fastdiv(static_cast<uint32_t>(segs));
        g.H = make_fastdiv(static_cast<uint32_t>(q.H));
        const uint32_t x_bytes = static_cast<uint32_t>(q.B * image_elems * int64_t(sizeof(T)));
        const dim3 grid((g.total + bd - 1) / bd);
        switch (epi) {
#define VH_DW(E)                                                                                         \
    case E: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, E, T, P>), grid, dim3(bd), 0, s, q, g, x_bytes); \
        break;
            VH_DW(DW_PLAIN) VH_DW(DW_ADD_INPUT) VH_DW(DW_GATE) VH_DW(DW_ADD_GELU) VH_DW(DW_ACCUM_F32)
            VH_DW(DW_ADD_F32_AUX) VH_DW(DW_ADD_GELU_SUMSQ)
#undef VH_DW
            case DW_ADD_INPUT_LN:
                if constexpr (K == 3)
                    hipLaunchKernelGGL((dwconv_nhwc_kernel<K, DW_ADD_INPUT_LN, T, P>), grid, dim3(256), 0, s, q, g, x_bytes);
                break;
        }
    }
}

inline int dw_pixels(int K, int64_t W) { return dw_default_pixels(K, W); }

// Blocks per image of the depthwise grid with the GRN partial-sum epilogue, or 0 when the
// channels do not form at most 256 groups of 8.
inline int64_t dw_blocks_per_image(int K, int64_t H, int64_t W, int64_t C) {
    const int64_t G = C / 8, segs = (W + dw_pixels(K, W) - 1) / dw_pixels(K, W);
    if (C % 8 != 0 || G > 256 || G < 1) return 0;
    return H * segs * G / dw_sumsq_block(G, H * segs);
}

// Plan of dwconv_tile_kernel for a map of `es`-byte elements (2-byte maps: bf16 and
// fp16), or false when it does not apply (FP32, a row's segments x channel groups above one block, a tile above 64 KB of LDS,
// more than 2^31 blocks); dwconv_nhwc_kernel covers those.  The slab width trades the
// halo re-read (K - 1 extra rows per band: wide bands want narrow slabs) against the
// bytes of one pixel a load covers contiguously (64 bf16 channels fill a 128-byte
// line): the lowest (RB + K - 1) / RB x sqrt(128 / min(128, slab bytes)) wins, the
// wider slab on ties.  The dw_tile override "0" turns the variant off and "2" uses it
// wherever it applies (tests compare the kernels); dw_tile_cs=<channels> forces a slab
// width and dw_tile_p=<pixels> the pixels per thread (measurements).
inline bool dw_tile_plan(int K, int64_t B, int64_t H, int64_t W, int64_t C, int es, DwTile& t) {
    const Override mode("dw_tile");
    if (mode.set() && mode.value[0] == '0') return false;
    const bool everywhere = mode.set() && mode.value[0] == '2';
    const Override forced_cs("dw_tile_cs");
    const int force = forced_cs.set() ? forced_cs.as_int() : 0;
    if (es != 2 || B <= 0 || H <= 0 || W <= 0 || C % 8 != 0) return false;
    // Measured on MI355X at the Tiny shapes (B = 128, bf16): faster than the per-thread
    // window kernel for 7x7 at every map size (56x56: 37 vs 64 us, 28x28: 20 vs 37 us)
    // and for 5x5 from 28x28 up; slower for 3x3, whose staging is not overlapped with
    // computation (memory-bound there), and for 5x5 on 14x14 and 7x7 maps.
    if (!everywhere && (K == 3 || (K == 5 && W < 28))) return false;
    int P = (W % 7 == 0) ? 7 : 8;
    if (K == 7 && W <= 14) P = 2;   // small maps: 3.5x the threads for (P + 6) / P input reads
    const Override forced_p("dw_tile_p");
    if (forced_p.set()) {
        const int v = forced_p.as_int();
        if (v == 2 || (v == 7 && W % 7 == 0) || v == 8) P = v;
    }
    if (P == 2 && K != 7) P = (W % 7 == 0) ? 7 : 8;
    const int64_t segs = (W + P - 1) / P;
    bool found = false;
    double best = 0.0;
    for (int cs : {64, 32, 16, 8}) {
        if (C % cs != 0 || (force && cs != force)) continue;
        const int64_t cg = cs / 8;
        if (segs * cg > 256) continue;
        const int64_t rb = std::min<int64_t>(H, 256 / (segs * cg));
        const int64_t wp = segs * P + K - 1, tr = rb + K - 1;
        const int64_t xb = std::max<int64_t>(tr * wp * cs * es, 256 * 8 * 4);
        const int64_t lds = xb + int64_t(K) * K * cs * 4;
        if (lds > 64 * 1024) continue;
        const double score = double(tr) / double(rb) * std::sqrt(128.0 / std::min<int64_t>(128, cs * es));
        if (found && score >= best - 1e-9) continue;
        found = true;
        best = score;
        t.P = P; t.CG = static_cast<int>(cg); t.segs = static_cast<int>(segs); t.RB = static_cast<int>(rb);
        t.WP = static_cast<int>(wp); t.TR = static_cast<int>(tr);
        t.x_bytes = static_cast<uint32_t>(xb); t.lds_bytes = static_cast<uint32_t>(lds);
    }
    if (!found) return false;
    t.bands = static_cast<int>((H + t.RB - 1) / t.RB);
    t.slabs = static_cast<int>(C / (8 * t.CG));
    if (B * t.bands * t.slabs >= (int64_t(1) << 31)) return false;
    t.wp_div = make_fastdiv(static_cast<uint32_t>(t.WP));
    t.cg_div = make_fastdiv(static_cast<uint32_t>(t.CG));
    return true;
}

template <int K, typename T, int P>
void launch_dw_tile(int epi, const DwParams& dp, const DwTile& t, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(dp.B * t.bands * t.slabs));
    switch (epi) {
#define VH_DWT(E)                                                                                           \
    case E: hipLaunchKernelGGL((dwconv_tile_kernel<K, E, T, P>), grid, dim3(256), t.lds_bytes, s, dp, t); \
        break;
        VH_DWT(DW_PLAIN) VH_DWT(DW_ADD_INPUT) VH_DWT(DW_GATE) VH_DWT(DW_ADD_GELU) VH_DWT(DW_ACCUM_F32)
        VH_DWT(DW_ADD_F32_AUX) VH_DWT(DW_ADD_GELU_SUMSQ)
#undef VH_DWT
    }
}

// Rows of GRN partial sums per image that the launch for this map writes (the bands of
// the tiled kernel, else the blocks of dwconv_nhwc_kernel), 0 when neither covers it.
inline int64_t dw_partial_rows(int K, int64_t B, int64_t H, int64_t W, int64_t C, int es) {
    DwTile t;
    if (dw_tile_plan(K, B, H, W, C, es, t)) return t.bands;
    return dw_blocks_per_image(K, H, W, C);
}

template <int K, typename T>
void launch_dw(int epi, const DwParams& dp, hipStream_t s) {
    if constexpr (sizeof(T) == 2) {
        DwTile t;
        if (epi != DW_ADD_INPUT_LN && dw_tile_plan(K, dp.B, dp.H, dp.W, dp.C, 2, t)) {
            if (t.P == 7) launch_dw_tile<K, T, 7>(epi, dp, t, s);
            else if constexpr (K == 7) {
                if (t.P == 2) launch_dw_tile<K, T, 2>(epi, dp, t, s);
                else launch_dw_tile<K, T, 8>(epi, dp, t, s);
            } else launch_dw_tile<K, T, 8>(epi, dp, t, s);
            return;
        }
    }
    if constexpr (K == 3) {
        if (dw_pixels(K, dp.W) == 7) launch_dw_p<K, T, 7>(epi, dp, s);
        else launch_dw_p<K, T, 8>(epi, dp, s);
    }
    else if constexpr (K == 5) launch_dw_p<K, T, 4>(epi, dp, s);
    else if (dw_pixels(K, dp.W) == 2) launch_dw_p<K, T, 2>(epi, dp, s);
    else launch_dw_p<K, T, 8>(epi, dp, s);
}

}  // namespace
}  // namespace vh

using namespace vh;

extern "C" int vh_dwconv2d_nhwc_forward(const void* x, int32_t io_dtype, const float* taps,
                                        const float* bias, int32_t ksize, int32_t epilogue,
                                        const void* aux, void* out, int64_t B, int64_t H,
                                        int64_t W, int64_t C, void* stream) {
    VH_REQUIRE(x && taps && out, VH_ERR_ARG, "depthwise conv pointers must not be null");
    VH_REQUIRE(B > 0 && H > 0 && W > 0 && C > 0, VH_ERR_SHAPE, "depthwise conv expects nonempty NHWC input");
    VH_REQUIRE(C % 8 == 0, VH_ERR_SHAPE, "depthwise conv needs C %% 8 == 0, got %lld", (long long)C);
    VH_REQUIRE(ksize == 3 || ksize == 5 || ksize == 7, VH_ERR_ARG, "kernel size must be 3, 5 or 7, got %d", ksize);
    VH_REQUIRE(epilogue >= DW_PLAIN && epilogue <= DW_ADD_F32_AUX, VH_ERR_ARG, "unknown epilogue %d", epilogue);
    VH_REQUIRE((epilogue != DW_GATE && epilogue != DW_ADD_F32_AUX) || aux != nullptr, VH_ERR_ARG,
               "epilogue %d needs the aux tensor", epilogue);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(taps) | reinterpret_cast<uintptr_t>(bias) |
                            reinterpret_cast<uintptr_t>(aux);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "depthwise conv tensors must be 16-byte aligned");
    VH_REQUIRE(H * W * C * dtype_bytes(io_dtype) < (int64_t(1) << 31), VH_ERR_SHAPE,
               "depthwise conv image too large (one image must be below 2 GiB)");
    DwParams dp{x, taps, bias, aux, out, B, H, W, C, nullptr};
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto go = [&](auto tv) {
        using T = decltype(tv);
        if (ksize == 3) launch_dw<3, T>(epilogue, dp, s);
        else if (ksize == 5) launch_dw<5, T>(epilogue, dp, s);
        else launch_dw<7, T>(epilogue, dp, s);
    };
    switch (io_dtype) {
        case VH_DTYPE_F32: go(float{}); break;
        case VH_DTYPE_BF16: go(bf16_t{}); break;
        default: go(f16_t{}); break;
    }
    return check_launch("dwconv_nhwc_kernel");
}

extern "C" int vh_dwconv2d_add_layernorm2d_forward(const void* x, int32_t io_dtype, const float* taps,
                                                  const float* bias, int32_t ksize, const float* ln_weight,
                                                  const float* ln_bias, float eps, void* out, void* out_norm,
                                                  int64_t B, int64_t H, int64_t W, int64_t C, void* stream) {
    VH_REQUIRE(x && taps && out && out_norm && ln_weight && ln_bias, VH_ERR_ARG,
               "depthwise conv + LayerNorm pointers must not be null");
    VH_REQUIRE(B > 0 && H > 0 && W > 0 && C > 0, VH_ERR_SHAPE, "depthwise conv + LayerNorm expects nonempty NHWC input");
    VH_REQUIRE(ksize == 3, VH_ERR_ARG, "depthwise conv + LayerNorm takes kernel size 3, got %d", ksize);
    const int64_t ng = C / 8;
    VH_REQUIRE(C % 8 == 0 && ng <= 32 && (ng & (ng - 1)) == 0, VH_ERR_SHAPE,
               "depthwise conv + LayerNorm needs C = 8 * 2^k <= 256, got %lld", (long long)C);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    VH_REQUIRE(eps > 0.f, VH_ERR_ARG, "LayerNorm eps must be positive");
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(out_norm) | reinterpret_cast<uintptr_t>(taps) |
                            reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(ln_weight) |
                            reinterpret_cast<uintptr_t>(ln_bias);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "depthwise conv + LayerNorm tensors must be 16-byte aligned");
    VH_REQUIRE(H * W * C * dtype_bytes(io_dtype) < (int64_t(1) << 31), VH_ERR_SHAPE,
               "depthwise conv image too large (one image must be below 2 GiB)");
    DwParams dp{x, taps, bias, nullptr, out, B, H, W, C, nullptr};
    dp.ln_w = ln_weight;
    dp.ln_b = ln_bias;
    dp.ln_eps = eps;
    dp.out_norm = out_norm;
    int lg = 0;
    while ((int64_t(1) << lg) < ng) ++lg;
    dp.ln_lg = lg;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (io_dtype) {
        case VH_DTYPE_F32: launch_dw<3, float>(DW_ADD_INPUT_LN, dp, s); break;
        case VH_DTYPE_BF16: launch_dw<3, bf16_t>(DW_ADD_INPUT_LN, dp, s); break;
        default: launch_dw<3, f16_t>(DW_ADD_INPUT_LN, dp, s); break;
    }
    return check_launch("dwconv_nhwc_kernel (add + LayerNorm)");
}

extern "C" size_t vh_dwconv2d_gelu_grn_workspace_bytes(int64_t B, int64_t H, int64_t W, int64_t C, int32_t ksize) {
    if (B <= 0 || H <= 0 || W <= 0 || (ksize != 3 && ksize != 5 && ksize != 7)) return 0;
    // One size for every io dtype: the larger of the 2- and 4-byte launches' needs, 0
    // unless both are covered.
    const int64_t rows2 = dw_partial_rows(ksize, B, H, W, C, 2), rows4 = dw_partial_rows(ksize, B, H, W, C, 4);
    if (rows2 == 0 || rows4 == 0) return 0;
    return static_cast<size_t>(B * std::max(rows2, rows4) * C) * sizeof(float);
}

extern "C" int vh_dwconv2d_gelu_grn_forward(const void* x, int32_t io_dtype, const float* taps, const float* bias,
                                            int32_t ksize, const float* gamma, float eps, void* out, float* gx,
                                            float* inv_den, float* scale, int64_t B, int64_t H, int64_t W,
                                            int64_t C, void* workspace, size_t workspace_bytes, void* stream) {
    VH_REQUIRE(x && taps && out && gamma && gx && inv_den && scale, VH_ERR_ARG,
               "depthwise conv + GRN statistics pointers must not be null");
    VH_REQUIRE(B > 0 && H > 0 && W > 0 && C > 0 && B <= 65535, VH_ERR_SHAPE,
               "depthwise conv + GRN statistics expects nonempty NHWC input and B <= 65535");
    VH_REQUIRE(ksize == 3 || ksize == 5 || ksize == 7, VH_ERR_ARG, "kernel size must be 3, 5 or 7, got %d", ksize);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    const int64_t rows = dw_partial_rows(ksize, B, H, W, C, dtype_bytes(io_dtype));
    VH_REQUIRE(rows > 0 && vh_dwconv2d_gelu_grn_workspace_bytes(B, H, W, C, ksize) > 0, VH_ERR_SHAPE,
               "GRN partial sums do not cover this map (C %% 8, or a row too wide for one block)");
    VH_REQUIRE(H * W * C * dtype_bytes(io_dtype) < (int64_t(1) << 31), VH_ERR_SHAPE,
               "depthwise conv image too large (one image must be below 2 GiB)");
    const size_t need = vh_dwconv2d_gelu_grn_workspace_bytes(B, H, W, C, ksize);
    VH_REQUIRE(workspace && workspace_bytes >= need, VH_ERR_WORKSPACE,
               "depthwise conv + GRN statistics workspace needs %zu bytes, got %zu", need,
               workspace ? workspace_bytes : (size_t)0);
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(taps) | reinterpret_cast<uintptr_t>(bias);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "depthwise conv tensors must be 16-byte aligned");
    DwParams dp{x, taps, bias, nullptr, out, B, H, W, C, static_cast<float*>(workspace)};
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto go = [&](auto tv) {
        using T = decltype(tv);
        if (ksize == 3) launch_dw<3, T>(DW_ADD_GELU_SUMSQ, dp, s);
        else if (ksize == 5) launch_dw<5, T>(DW_ADD_GELU_SUMSQ, dp, s);
        else launch_dw<7, T>(DW_ADD_GELU_SUMSQ, dp, s);
    };
    switch (io_dtype) {
        case VH_DTYPE_F32: go(float{}); break;
        case VH_DTYPE_BF16: go(bf16_t{}); break;
        default: go(f16_t{}); break;
    }
    int rc = check_launch("dwconv_nhwc_kernel (GRN partial sums)");
    if (rc) return rc;
    return launch_grn_finalize(static_cast<const float*>(workspace), gx, inv_den, B, C, rows, eps, gamma, scale, s);
}
