// Memory-bound tail of the SRNL operator for gfx950: direction fusion, GRN,
// LayerNorm over channels, query normalisation and the residual add.
//
// All kernels read activations in their storage order with consecutive lanes
// on consecutive addresses, reduce with wave64 butterflies (__shfl_xor) and
// write fp32 results once.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "vh_common.h"

namespace vh {

// ---------------------------------------------------------------------------
// Direction fusion (utils/csrc/direction_fusion.cu:11-65):
//   out[b, c, h, w] = sum_r scale[r, c] * (y_r[t_r] + skip_r[c] * x_r[t_r])
// with y, x in the serialized layout [B, 4, heads, L, D].  One thread per
// output element in output storage order (coalesced writes); the four reads
// of a pixel hit D-element rows that neighbouring threads share in cache.
// ---------------------------------------------------------------------------
struct FusionParams {
    const void* y;
    const void* x;
    const float* skip;
    int skip_per_dir;
    const float* scale;
    float* out;
    int64_t B, heads, H, W;
    int channels_last;
};

template <int D, typename T>
__global__ __launch_bounds__(256) void direction_fusion_kernel(const FusionParams p) {
    const int64_t C = p.heads * D;
    const int64_t L = p.H * p.W;
    const int64_t total = p.B * C * L;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    int64_t b, c, h, w;
    if (p.channels_last) {
        c = idx % C;
        w = (idx / C) % p.W;
        h = (idx / (C * p.W)) % p.H;
        b = idx / (C * L);
    } else {
        w = idx % p.W;
        h = (idx / p.W) % p.H;
        c = (idx / L) % C;
        b = idx / (C * L);
    }
    const int64_t head = c / D;
    const int64_t i = c % D;
    const T* y = static_cast<const T*>(p.y);
    const T* x = static_cast<const T*>(p.x);
    const int64_t base = (b * 4 * p.heads + head) * L * D + i;
    const int64_t stride_dir = p.heads * L * D;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t at = base + r * stride_dir + pixel_to_scan(r, h, w, p.H, p.W) * D;
        const float ds = p.skip[(p.skip_per_dir ? r * C : 0) + c];
        v[r] = to_f32(y[at]) + ds * to_f32(x[at]);
    }
    float out = p.scale[c] * v[0];
    out += p.scale[C + c] * v[1];
    out += p.scale[2 * C + c] * v[2];
    out += p.scale[3 * C + c] * v[3];
    p.out[idx] = out;
}

// Channels-last output, D >= 8: one thread per (image, pixel, 8-channel group), 16-byte
// reads of y and x per direction, one 32-byte write.  Same summation order.
template <int D, typename T>
__global__ __launch_bounds__(256) void direction_fusion8_kernel(const FusionParams p, const float inv_w,
                                                               const float inv_g) {
    constexpr int GD = D / 8;  // channel groups per head
    const int G = static_cast<int>(p.heads) * GD;
    const int L = static_cast<int>(p.H * p.W);
    const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= static_cast<uint32_t>(L * G)) return;
    const int64_t b = blockIdx.y;
    uint32_t pix, cg, h, w;
    divmod24(idx, static_cast<uint32_t>(G), inv_g, pix, cg);
    divmod24(pix, static_cast<uint32_t>(p.W), inv_w, h, w);
    const int head = static_cast<int>(cg) / GD, i0 = (static_cast<int>(cg) % GD) * 8;
    const int C = G * 8, c0 = static_cast<int>(cg) * 8;
    const T* y = static_cast<const T*>(p.y);
    const T* x = static_cast<const T*>(p.x);
    const int64_t base = (b * 4 * p.heads + head) * static_cast<int64_t>(L) * D + i0;
    const int64_t stride_dir = p.heads * static_cast<int64_t>(L) * D;
    float out[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t at = base + r * stride_dir + pixel_to_scan(r, h, w, p.H, p.W) * D;
        float yv[8], xv[8];
        load8<T>(y + at, yv);
        load8<T>(x + at, xv);
        const float* sk = p.skip + (p.skip_per_dir ? r * C : 0) + c0;
        const float* sc = p.scale + r * C + c0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = yv[j] + sk[j] * xv[j];
            out[j] = r == 0 ? sc[j] * v : out[j] + sc[j] * v;
        }
    }
    const float z[8] = {out[0], out[1], out[2], out[3], out[4], out[5], out[6], out[7]};
    store8<float>(p.out + (b * L + pix) * static_cast<int64_t>(C) + c0, z);
}

// Channels-last output, D >= 8, tiled: one workgroup per (image, TH x TW pixel tile,
// chunk of at most 96 channels), the chunks of a tile in consecutive workgroups; the launch
// uses 4 x 4 tiles (measured best against 8 x 8, 4 x 8, 8 x 4, 2 x 8, 8 x 2 and 16 x 16 at
// 56x56x96 and 28x28x192).  Thread k owns item k = (head,
// pixel, 8-channel group), group fastest; the workgroup has exactly as many threads as
// items, rounded up to whole waves (192 for 96 channels).  The row scans (directions 0,
// 1) are read at the item's pixel in row-major order within the tile and the column scans
// (2, 3) at its pixel in column-major order, so consecutive lanes read consecutive tokens
// of one head (runs of TW or TH tokens) in both cases.  All eight 16-byte loads of a
// thread are issued before any arithmetic; the row-scan sums go to LDS (at most 16 x 96
// floats), the column-scan terms are added at the transposed pixel after a barrier, and
// the tile is written as channels-last pixel rows.  Summation order ((c0 + c1) + c2) + c3
// as above.
template <int D, typename T>
__global__ __launch_bounds__(256) void direction_fusion_tile_kernel(const FusionParams p, const uint32_t tiles_w,
                                                                    const int th_log2, const int tw_log2,
                                                                    const int heads_per_block, const float inv_g,
                                                                    const uint32_t chunks_x) {
    constexpr int GD = D / 8;
    extern __shared__ float acc[];   // [TH * TW pixels, row-major][heads_per_block * D]
    const int C = static_cast<int>(p.heads) * D;
    // chunks_x > 1: the channel chunks of one tile are consecutive workgroups
    const uint32_t chunk = chunks_x > 1 ? blockIdx.x % chunks_x : blockIdx.z;
    const uint32_t tile = chunks_x > 1 ? blockIdx.x / chunks_x : blockIdx.x;
    const int head0 = static_cast<int>(chunk) * heads_per_block;
    const int nh = min(heads_per_block, static_cast<int>(p.heads) - head0);
    const int CB = nh * D, G = nh * GD;
    const int TH = 1 << th_log2, TW = 1 << tw_log2, npx = TH * TW;
    const int64_t L = p.H * p.W;
    const int64_t b = blockIdx.y;
    const int th0 = static_cast<int>(tile / tiles_w) * TH, tw0 = static_cast<int>(tile % tiles_w) * TW;
    const T* y = static_cast<const T*>(p.y);
    const T* x = static_cast<const T*>(p.x);
    const int64_t stride_dir = p.heads * L * D;
    const int items = npx * G;
    const int k = static_cast<int>(threadIdx.x);
    const int gi = k % GD, kk = k / GD, q = kk & (npx - 1), hl = kk >> (th_log2 + tw_log2);
    const int head = head0 + hl;
    const int c0 = head * D + gi * 8;
    const int64_t base = (b * 4 * p.heads + head) * L * D + gi * 8;
    // the item's pixel in the row phase (directions 0, 1) and in the column phase (2, 3)
    const int ph[2] = {q >> tw_log2, q & (TH - 1)};
    const int pw[2] = {q & (TW - 1), q >> th_log2};
    bool live[2];
    Pack8<T> ry[4], rx[4];
    auto fetch = [&](int phase) {
        const int64_t h = th0 + ph[phase], w = tw0 + pw[phase];
        live[phase] = k < items && h < p.H && w < p.W;
        if (live[phase]) {
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const int r = 2 * phase + rr;
                const int64_t at = base + r * stride_dir + pixel_to_scan(r, h, w, p.H, p.W) * D;
                ry[r] = load_pack8<T>(y + at);
                rx[r] = load_pack8<T>(x + at);
            }
        }
    };
    fetch(0);
    fetch(1);
    // Per-channel skip and scale of all four directions, loaded behind the data so their
    // latency is not paid after the phase barrier.
    float sk[4][8], sc[4][8];
    if (k < items) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            load8<float>(p.skip + (p.skip_per_dir ? r * C : 0) + c0, sk[r]);
            load8<float>(p.scale + r * C + c0, sc[r]);
        }
    }
#pragma unroll
    for (int phase = 0; phase < 2; ++phase) {
        if (live[phase]) {
            float* a = acc + (ph[phase] * TW + pw[phase]) * CB + hl * D + gi * 8;
            float out[8];
            if (phase == 1) {
#pragma unroll
                for (int j = 0; j < 8; ++j) out[j] = a[j];
            }
#pragma unroll
            for (int rr = 0; rr < 2; ++rr) {
                const int r = 2 * phase + rr;
                float yv[8], xv[8];
                pack8_to_f32<T>(ry[r], yv);
                pack8_to_f32<T>(rx[r], xv);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float v = yv[j] + sk[r][j] * xv[j];
                    out[j] = r == 0 ? sc[r][j] * v : out[j] + sc[r][j] * v;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) a[j] = out[j];
        }
        __syncthreads();
    }
    // the last chunk of heads may hold fewer than heads_per_block heads (inv_g is 1 / G of a full chunk)
    const float inv_gc = nh == heads_per_block ? inv_g : 1.0f / static_cast<float>(G);
    for (uint32_t i = threadIdx.x; i < static_cast<uint32_t>(items); i += blockDim.x) {
        uint32_t px, cg;
        divmod24(i, static_cast<uint32_t>(G), inv_gc, px, cg);
        const int64_t h = th0 + (px >> tw_log2), w = tw0 + (px & static_cast<uint32_t>(TW - 1));
        if (h >= p.H || w >= p.W) continue;
        const float* a = acc + px * CB + cg * 8;
        const float z[8] = {a[0], a[1], a[2], a[3], a[4], a[5], a[6], a[7]};
        store8<float>(p.out + (b * L + h * p.W + w) * static_cast<int64_t>(C) + head0 * D + cg * 8, z);
    }
}

// ---------------------------------------------------------------------------
// GRN (utils/grn.py:26-38, utils/csrc/grn_cuda.cu:46-124) on channels-last x.
//   pass 1  partial[b, slab, c] = sum over the slab's pixels of x^2
//   pass 2  gx[b, c] = sqrt(sum_slab partial), inv_den[b] = 1 / (mean_c gx + eps)
//   pass 3  y = x * (1 + gamma_c * gx * inv_den) + beta_c
// ---------------------------------------------------------------------------
constexpr int kGrnRowsPerSlab = 64;

template <typename T>
__global__ __launch_bounds__(256) void grn_partial_kernel(const T* __restrict__ x,
                                                         float* __restrict__ partial, int64_t C,
                                                         int64_t S, int64_t nslab) {
    extern __shared__ float red[];
    const int64_t b = blockIdx.y;
    const int64_t slab = blockIdx.x;
    const int64_t s0 = slab * kGrnRowsPerSlab;
    const int64_t s1 = std::min<int64_t>(S, s0 + kGrnRowsPerSlab);
    const int ct = static_cast<int>(std::min<int64_t>(C, 256));
    const int rp = 256 / ct;                       // row phases
    const int tc = threadIdx.x % ct, tr = threadIdx.x / ct;
    const T* xb = x + b * S * C;
    for (int64_t c = tc; c < C; c += ct) {
        float acc = 0.f;
        if (tr < rp) {
            for (int64_t s = s0 + tr; s < s1; s += rp) {
                const float v = to_f32(xb[s * C + c]);
                acc += v * v;
            }
            red[tr * C + c] = acc;
        }
    }
    __syncthreads();
    for (int64_t c = threadIdx.x; c < C; c += 256) {
        float acc = 0.f;
        for (int q = 0; q < rp; ++q) acc += red[q * C + c];
        partial[(b * nslab + slab) * C + c] = acc;
    }
}

// One block of 1024 threads per image.  With C < 1024 the threads split the slabs
// into SG = 1024 / C groups (thread t: channel t % C, slabs t / C, t / C + SG, ...),
// so many partial sums are in flight at once; the groups are then added in a fixed
// order (deterministic).
constexpr int kGrnFinalizeThreads = 1024;

__global__ __launch_bounds__(kGrnFinalizeThreads) void grn_finalize_kernel(const float* __restrict__ partial,
                                                                           float* __restrict__ gx,
                                                                           float* __restrict__ inv_den, int64_t C,
                                                                           int64_t nslab, float eps,
                                                                           const float* __restrict__ gamma = nullptr,
                                                                           float* __restrict__ scale = nullptr) {
    constexpr int NT = kGrnFinalizeThreads;
    __shared__ float wsum[NT / 64];
    __shared__ float red[NT];
    __shared__ float inv_sh;
    const int64_t b = blockIdx.x;
    const int t = threadIdx.x;
    float local = 0.f;
    if (C < NT) {
        const int SG = static_cast<int>(NT / C);
        const int sg = static_cast<int>(t / C);
        const int64_t c = t % C;
        float a0 = 0.f, a1 = 0.f;
        if (sg < SG) {
            const float* pc = partial + b * nslab * C + c;
            int64_t s = sg;
            // Eight loads in flight, added in the order of the loop below.
            for (; s + 7 * SG < nslab; s += 8 * SG) {
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = pc[(s + j * SG) * C];
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    a0 += v[j];
                    a1 += v[j + 1];
                }
            }
            for (; s + SG < nslab; s += 2 * SG) {
                a0 += pc[s * C];
                a1 += pc[(s + SG) * C];
            }
            if (s < nslab) a0 += pc[s * C];
        }
        red[t] = a0 + a1;
        __syncthreads();
        if (sg == 0) {
            float acc = 0.f;
            for (int q = 0; q < SG; ++q) acc += red[q * C + c];
            const float g = sqrtf(acc);
            gx[b * C + c] = g;
            local = g;
        }
    } else {
        for (int64_t c = t; c < C; c += NT) {
            // Four independent partial sums (a0 takes slabs 0, 4, 8, ...).
            const float* pc = partial + b * nslab * C + c;
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            // Slab s goes to a(s % 4) below the last multiple of 4 and to a0 after it; the
            // slabs are loaded sixteen at a time, all in flight, and added in that order.
            const int64_t full = nslab & ~int64_t(3);
            for (int64_t s = 0; s < nslab; s += 16) {
                float v[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) v[j] = s + j < nslab ? pc[(s + j) * C] : 0.f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int64_t g = s + j;
                    if (g < full) {
                        if (j % 4 == 0) a0 += v[j];
                        else if (j % 4 == 1) a1 += v[j];
                        else if (j % 4 == 2) a2 += v[j];
                        else a3 += v[j];
                    } else if (g < nslab) {
                        a0 += v[j];
                    }
                }
            }
            const float acc = (a0 + a1) + (a2 + a3);
            const float g = sqrtf(acc);
            gx[b * C + c] = g;
            local += g;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off);
    if ((t & 63) == 0) wsum[t >> 6] = local;
    __syncthreads();
    if (t == 0) {
        float total = 0.f;
        for (int w = 0; w < NT / 64; ++w) total += wsum[w];
        const float inv = 1.f / (total / static_cast<float>(C) + eps);
        inv_den[b] = inv;
        inv_sh = inv;
    }
    if (scale) {
        // The per-(image, channel) factor 1 + gamma nx of the apply step, for consumers
        // that apply GRN as they load its input (same fp32 operations as grn_apply8).
        __syncthreads();
        const float inv = inv_sh;
        for (int64_t c = t; c < C; c += NT) {
            const float nx = gx[b * C + c] * inv;
            scale[b * C + c] = 1.f + gamma[c] * nx;
        }
    }
}

template <typename T, typename TO>
__global__ __launch_bounds__(256) void grn_apply_kernel(const T* __restrict__ x,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta,
                                                       const float* __restrict__ gx,
                                                       const float* __restrict__ inv_den,
                                                       TO* __restrict__ y, int64_t C, int64_t S,
                                                       int64_t total) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += stride) {
        const int64_t c = idx % C;
        const int64_t b = idx / (S * C);
        const float nx = gx[b * C + c] * inv_den[b];
        y[idx] = from_f32<TO>(to_f32(x[idx]) * (1.f + gamma[c] * nx) + beta[c]);
    }
}

// Vectorised GRN for C % 8 == 0, C <= 2048 and 16-byte aligned tensors: each thread
// owns 8 consecutive channels of a pixel (one 16-byte load of bf16/fp16), a block is
// G = C/8 channel groups x R = 256/G pixel rows, so every thread keeps the same channels
// for the whole block and no index arithmetic runs per element.
template <typename T>
__global__ __launch_bounds__(256) void grn_partial8_kernel(const T* __restrict__ x, float* __restrict__ partial,
                                                          int C, int S, int rows_per_slab, int nslab) {
    extern __shared__ float red[];  // [R][C]
    const int G = C / 8, R = static_cast<int>(blockDim.x) / G;
    const int g = static_cast<int>(threadIdx.x) % G, rr = static_cast<int>(threadIdx.x) / G;
    const int b = blockIdx.y, slab = blockIdx.x;
    const int s0 = slab * rows_per_slab, s1 = min(S, s0 + rows_per_slab);
    const T* xb = x + static_cast<int64_t>(b) * S * C + g * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = s0 + rr; s < s1; s += R) {
        float v[8];
        load8<T>(xb + static_cast<int64_t>(s) * C, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += v[j] * v[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) red[rr * C + g * 8 + j] = acc[j];
    __syncthreads();
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        float t = 0.f;
        for (int q = 0; q < R; ++q) t += red[q * C + c];
        partial[(static_cast<int64_t>(b) * nslab + slab) * C + c] = t;
    }
}

// Wide maps (C / 8 > 256 channel groups, e.g. 2560 FFN channels): thread t takes channel
// groups t, t + 256, ... of every row of the slab (partial sums) or of the workgroup's rows
// (apply, from the gx and inv_den that grn_finalize_kernel wrote).
template <typename T>
__global__ __launch_bounds__(256) void grn_partial8_wide_kernel(const T* __restrict__ x, float* __restrict__ partial,
                                                               int C, int S, int rows_per_slab, int nslab) {
    const int G = C / 8, b = blockIdx.y, slab = blockIdx.x;
    const int s0 = slab * rows_per_slab, s1 = min(S, s0 + rows_per_slab);
    for (int g = threadIdx.x; g < G; g += 256) {
        const T* xb = x + static_cast<int64_t>(b) * S * C + g * 8;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int s = s0; s < s1; ++s) {
            float v[8];
            load8<T>(xb + static_cast<int64_t>(s) * C, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += v[j] * v[j];
        }
        store8<float>(partial + (static_cast<int64_t>(b) * nslab + slab) * C + g * 8, acc);
    }
}

// gx[b, c] = sqrt(sum over the slabs): a workgroup takes 64 channels of one image and 4
// threads per channel, thread j summing slabs j, j + 4, ... (two accumulators), and the four
// partial sums meet in LDS in a fixed order (deterministic).  Grid: channel blocks x images.
__global__ __launch_bounds__(256) void grn_gx_kernel(const float* __restrict__ partial, float* __restrict__ gx, int C,
                                                    int nslab) {
    __shared__ float part[4][64];
    const int cl = threadIdx.x & 63, j = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl, b = blockIdx.y;
    float a0 = 0.f, a1 = 0.f;
    if (c < C) {
        const float* pc = partial + static_cast<int64_t>(b) * nslab * C + c;
        int s = j;
        for (; s + 4 < nslab; s += 8) {
            a0 += pc[static_cast<int64_t>(s) * C];
            a1 += pc[static_cast<int64_t>(s + 4) * C];
        }
        if (s < nslab) a0 += pc[static_cast<int64_t>(s) * C];
    }
    part[j][cl] = a0 + a1;
    __syncthreads();
    if (j == 0 && c < C)
        gx[static_cast<int64_t>(b) * C + c] = sqrtf((part[0][cl] + part[1][cl]) + (part[2][cl] + part[3][cl]));
}

// The statistics of grn_finalize_kernel for few images with many slabs (B = 8 at 512^2:
// 256 slabs per image), where one workgroup per image leaves most CUs idle and waits on
// its loads.  Step 1, gx: a workgroup takes 64 channels of one image, thread j of a channel
// sums slabs j, j + 4, ... into eight accumulators (eight loads in flight), and the four
// sums meet in LDS in a fixed order.  Grid: channel blocks x images.
__global__ __launch_bounds__(256) void grn_gx8_kernel(const float* __restrict__ partial, float* __restrict__ gx, int C,
                                                     int nslab) {
    __shared__ float part[4][64];
    const int cl = threadIdx.x & 63, j = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl, b = blockIdx.y;
    float a = 0.f;
    if (c < C) {
        const float* pc = partial + static_cast<int64_t>(b) * nslab * C + c;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        int s = j;
        for (; s + 28 < nslab; s += 32) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = pc[static_cast<int64_t>(s + 4 * u) * C];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc[u] += v[u];
        }
        for (; s < nslab; s += 4) acc[0] += pc[static_cast<int64_t>(s) * C];
        a = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    }
    part[j][cl] = a;
    __syncthreads();
    if (j == 0 && c < C)
        gx[static_cast<int64_t>(b) * C + c] = sqrtf((part[0][cl] + part[1][cl]) + (part[2][cl] + part[3][cl]));
}

// Step 2: inv_den[b] = 1 / (mean_c gx[b, c] + eps) and, when asked, the apply factor
// scale[b, c] = 1 + gamma[c] gx[b, c] inv_den[b] (the fp32 operations of grn_finalize_kernel).
// One workgroup per image.
__global__ __launch_bounds__(256) void grn_image_scale_kernel(const float* __restrict__ gx, float* __restrict__ inv_den,
                                                             int64_t C, float eps, const float* __restrict__ gamma,
                                                             float* __restrict__ scale) {
    __shared__ float wsum[4];
    __shared__ float inv_sh;
    const int64_t b = blockIdx.x;
    const int t = threadIdx.x;
    float local = 0.f;
    for (int64_t c = t; c < C; c += 256) local += gx[b * C + c];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off);
    if ((t & 63) == 0) wsum[t >> 6] = local;
    __syncthreads();
    if (t == 0) {
        const float total = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
        const float inv = 1.f / (total / static_cast<float>(C) + eps);
        inv_den[b] = inv;
        inv_sh = inv;
    }
    if (scale) {
        __syncthreads();
        const float inv = inv_sh;
        for (int64_t c = t; c < C; c += 256) scale[b * C + c] = 1.f + gamma[c] * (gx[b * C + c] * inv);
    }
}

// Apply for wide maps: every workgroup of image b forms inv_den from gx (fixed order, so all
// workgroups agree bit for bit) and workgroup 0 stores it.
template <typename T, typename TO>
__global__ __launch_bounds__(256) void grn_apply8_wide_kernel(const T* __restrict__ x, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             const float* __restrict__ gx,
                                                             float* __restrict__ inv_den, TO* __restrict__ y,
                                                             int C, int S, int rows_per_block, float eps) {
    const int G = C / 8, b = blockIdx.y;
    const int s0 = blockIdx.x * rows_per_block, s1 = min(S, s0 + rows_per_block);
    __shared__ float wsum[4];
    float local = 0.f;
    for (int c = threadIdx.x; c < C; c += 256) local += gx[static_cast<int64_t>(b) * C + c];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = local;
    __syncthreads();
    const float inv = 1.f / ((((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]) / static_cast<float>(C) + eps);
    if (blockIdx.x == 0 && threadIdx.x == 0) inv_den[b] = inv;
    for (int g = threadIdx.x; g < G; g += 256) {
        float sc[8], bt[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = g * 8 + j;
            sc[j] = 1.f + gamma[c] * (gx[static_cast<int64_t>(b) * C + c] * inv);
            bt[j] = beta[c];
        }
        const int64_t base = static_cast<int64_t>(b) * S * C + g * 8;
        for (int s = s0; s < s1; ++s) {
            float v[8];
            load8<T>(x + base + static_cast<int64_t>(s) * C, v);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = v[j] * sc[j] + bt[j];
            store8<TO>(y + base + static_cast<int64_t>(s) * C, v);
        }
    }
}

// GRN apply (y = x scale_c + beta_c, 8 channels per thread, 16-byte loads) with the
// statistics pass folded in: every workgroup of image b first
// reduces the per-slab partial sums of all C channels (fixed order, so every workgroup of
// the image gets bit-identical gx and inv_den) and workgroup 0 of the image stores them.
// This saves the separate statistics launch between the two streaming passes; it is used
// while the partial sums of one image are small (FOLD).  Without FOLD the workgroup reads
// gx that grn_gx_kernel wrote and forms inv_den from it the same way.
// 256 threads; thread t streams channel group t % G of rows t / G (t / G < 256 / G).
template <typename T, typename TO, bool FOLD>
__global__ __launch_bounds__(256) void grn_stats_apply8_kernel(const T* __restrict__ x, const float* __restrict__ partial,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ beta, float* __restrict__ gx,
                                                               float* __restrict__ inv_den, TO* __restrict__ y, int C,
                                                               int S, int nslab, int rows_per_block, float eps) {
    extern __shared__ float gsh[];   // [C]
    __shared__ float wsum[4];
    const int t = static_cast<int>(threadIdx.x);
    const int b = blockIdx.y;
    float local = 0.f;
    if constexpr (!FOLD) {
        for (int c = t; c < C; c += 256) {
            const float g = gx[static_cast<int64_t>(b) * C + c];
            gsh[c] = g;
            local += g;
        }
    }
    for (int c = t; FOLD && c < C; c += 256) {
        const float* pc = partial + static_cast<int64_t>(b) * nslab * C + c;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        int s = 0;
        for (; s + 4 <= nslab; s += 4) {
            a0 += pc[s * C];
            a1 += pc[(s + 1) * C];
            a2 += pc[(s + 2) * C];
            a3 += pc[(s + 3) * C];
        }
        for (; s < nslab; ++s) a0 += pc[s * C];
        const float g = sqrtf((a0 + a1) + (a2 + a3));
        gsh[c] = g;
        local += g;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off);
    if ((t & 63) == 0) wsum[t >> 6] = local;
    __syncthreads();
    const float inv = 1.f / ((((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]) / static_cast<float>(C) + eps);
    if (blockIdx.x == 0) {
        if (FOLD)
            for (int c = t; c < C; c += 256) gx[static_cast<int64_t>(b) * C + c] = gsh[c];
        if (t == 0) inv_den[b] = inv;
    }
    const int G = C / 8, R = 256 / G;
    const int g = t % G, rr = t / G;
    if (rr >= R) return;
    float sc[8], bt[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = g * 8 + j;
        sc[j] = 1.f + gamma[c] * (gsh[c] * inv);
        bt[j] = beta[c];
    }
    const int s0 = blockIdx.x * rows_per_block, s1 = min(S, s0 + rows_per_block);
    const int64_t base = static_cast<int64_t>(b) * S * C + g * 8;
    for (int s = s0 + rr; s < s1; s += R) {
        float v[8];
        load8<T>(x + base + static_cast<int64_t>(s) * C, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = v[j] * sc[j] + bt[j];
        store8<TO>(y + base + static_cast<int64_t>(s) * C, v);
    }
}

// One-pass GRN: x is read from HBM once and held in registers between the statistics and
// the apply step.  An image of S rows is split into `pieces` pieces of R x V rows (R = rows
// per pass of the workgroup, V = rows per thread), workgroup i taking piece i % pieces of
// image i / pieces; the pieces of one image publish their per-channel sums of squares to
// the workspace, count themselves on the image's counter, wait until all pieces of the
// image have counted, then every piece reduces the same partial sums in the same order
// (bit-identical gx and inv_den; piece 0 stores them) and applies y = x scale_c + beta_c
// to the rows it holds.
//
// Forward progress: each XCD dispatches its workgroups in increasing index order, so every
// workgroup below the lowest index not yet dispatched (m) is resident or finished.  Images
// whose pieces all lie below m complete; only the one image holding m can wait on a
// workgroup that has not started, and it holds fewer than pieces <= kGrnMaxPieces slots of
// an XCD (each holds hundreds of workgroups), so the others keep finishing and m is
// dispatched.  That dispatch order is observed behaviour of the hardware, not a documented
// guarantee, so nothing rests on it for correctness: the wait is bounded (spin_limit
// sleeps, kGrnSpinLimit unless overridden), and a piece that gives up computes its image's
// statistics itself from x (all S rows, read again) instead of from the other pieces'
// partial sums.  Its output is then correct to FP32 rounding of a different summation
// order, and it adds one to the fallback word of its image's line, which the host reads
// with vh_grn_workspace_fallbacks.  No counter is shared by all workgroups (one shared word
// costs a serialised atomic per workgroup).
//
// Synchronisation words: a fixed header of kGrnSyncImages 128-byte lines at the start of the
// workspace (the partial sums of every GRN path start after it, so no path ever writes
// into it), one line per image of a launch: word 0 counts the pieces that published, word
// 16 the pieces done.  They must be zero when the launch starts; the last piece of each
// image resets both, so the launch leaves them zero.  Word 8 counts fallbacks and is never
// reset by a kernel.  A launch covers at most kGrnSyncImages images; larger batches take
// several launches.
constexpr int kGrnVec = 8;                  // rows per thread held in registers (or 2 kGrnVec)
constexpr int kGrnMaxPieces = 64;
constexpr uint32_t kGrnSpinLimit = 1u << 20;
constexpr int kGrnSyncWords = 32;           // per image
constexpr int kGrnFallbackWord = 8;         // within an image's line
constexpr int kGrnSyncImages = 256;

template <typename T, typename TO, int V>
__global__ __launch_bounds__(256) void grn_onepass8_kernel(const T* __restrict__ x, const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float* __restrict__ gx,
                                                          float* __restrict__ inv_den, TO* __restrict__ y,
                                                          uint32_t* __restrict__ sync, float* __restrict__ partial,
                                                          int C, int S, int pieces, int b0, float eps, int piece_rows,
                                                          uint32_t spin_limit) {
    extern __shared__ __align__(16) float red[];   // [R][C] partial sums, then [C] gx; FP32 staging
    __shared__ uint32_t word;
    __shared__ float wsum[4];
    const int t = static_cast<int>(threadIdx.x);
    const int nt = static_cast<int>(blockDim.x);
    const int G = C / 8, R = 256 / G;
    const int bl = static_cast<int>(blockIdx.x / static_cast<uint32_t>(pieces));   // image within the launch
    const int b = b0 + bl;
    const int piece = static_cast<int>(blockIdx.x % static_cast<uint32_t>(pieces));
    uint32_t* const counted = sync + bl * kGrnSyncWords;
    uint32_t* const done = counted + kGrnSyncWords / 2;
    const int g = t % G, rr = t / G;
    const bool lane_rows = rr < R;
    const int s0 = piece * piece_rows, s1 = min(S, s0 + piece_rows);   // piece_rows <= R * V
    const T* xb = x + static_cast<int64_t>(b) * S * C + g * 8;
    Pack8<T> raw[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int s = s0 + rr + v * R;
        if (lane_rows && s < s1) raw[v] = load_pack8<T>(xb + static_cast<int64_t>(s) * C);
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < V; ++v) {
        if (lane_rows && s0 + rr + v * R < s1) {
            float f[8];
            pack8_to_f32<T>(raw[v], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += f[j] * f[j];
        }
    }
    if (lane_rows) {
#pragma unroll
        for (int j = 0; j < 8; ++j) red[rr * C + g * 8 + j] = acc[j];
    }
    __syncthreads();
    // The partial sums travel as agent-scope atomic stores and loads (sc1), each coherent
    // across the XCDs' L2 caches on its own, so no L2 write-back or invalidation is needed
    // (a release fence would write back every dirty line of y in the L2, an acquire would
    // invalidate it, once per piece).  Ordering: an agent-scope store's completion (vmcnt)
    // means it is visible at agent scope -- the same wait the compiler's own release
    // sequence relies on for prior atomic stores -- so every thread waits for its stores
    // before the barrier and thread 0 counts after it; the loads of the other pieces' sums
    // are issued after thread 0 has seen the full count.
    float* const mine = partial + (static_cast<int64_t>(b) * pieces + piece) * C;
    for (int c = t; c < C; c += nt) {
        float sum = 0.f;
        for (int q = 0; q < R; ++q) sum += red[q * C + c];
        __hip_atomic_store(&mine[c], sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0) {
        __hip_atomic_fetch_add(counted, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t spins = 0;
        while (__hip_atomic_load(counted, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
                   static_cast<uint32_t>(pieces) &&
               spins < spin_limit) {
            __builtin_amdgcn_s_sleep(2);
            ++spins;
        }
        word = spins < spin_limit;
        if (spins >= spin_limit) atomicAdd(counted + kGrnFallbackWord, 1u);
    }
    __syncthreads();
    const bool complete = word != 0;   // uniform over the workgroup
    if (!complete) {
        // Fallback: this piece's own sums of squares over every row of the image, into the
        // [R][C] LDS rows (its own piece's sums there are superseded).
        float a8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (lane_rows) {
            for (int s = rr; s < S; s += R) {
                float f[8];
                pack8_to_f32<T>(load_pack8<T>(xb + static_cast<int64_t>(s) * C), f);
#pragma unroll
                for (int j = 0; j < 8; ++j) a8[j] += f[j] * f[j];
            }
        }
        __syncthreads();
        if (lane_rows) {
#pragma unroll
            for (int j = 0; j < 8; ++j) red[rr * C + g * 8 + j] = a8[j];
        }
        __syncthreads();
    }
    float* const gsh = red;   // the [R][C] sums are no longer needed once read
    float local = 0.f;
    float* const img = partial + static_cast<int64_t>(b) * pieces * C;
    for (int c = t; c < C; c += nt) {
        float gv;
        if (complete) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
            int p = 0;
            auto at = [&](int pc) { return __hip_atomic_load(&img[pc * C + c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
            for (; p + 4 <= pieces; p += 4) {
                a0 += at(p);
                a1 += at(p + 1);
                a2 += at(p + 2);
                a3 += at(p + 3);
            }
            for (; p < pieces; ++p) a0 += at(p);
            gv = sqrtf((a0 + a1) + (a2 + a3));
        } else {
            // column c of the [R][C] rows is read and written by this thread only
            float sum = 0.f;
            for (int q = 0; q < R; ++q) sum += red[q * C + c];
            gv = sqrtf(sum);
        }
        gsh[c] = gv;
        local += gv;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off);
    if ((t & 63) == 0) wsum[t >> 6] = local;
    __syncthreads();
    float total_g = wsum[0];
    for (int w = 1; w < (nt + 63) / 64; ++w) total_g += wsum[w];
    const float inv = 1.f / (total_g / static_cast<float>(C) + eps);
    if (piece == 0) {
        for (int c = t; c < C; c += nt) gx[static_cast<int64_t>(b) * C + c] = gsh[c];
        if (t == 0) inv_den[b] = inv;
    }
    if constexpr (sizeof(TO) == 4) {
        // FP32 output: thread t = rr * G + g writes bytes [32 t, 32 t + 32) of the R * C
        // outputs of step v, so a wave's outputs are one contiguous 2 KB range.  They go
        // through the wave's own 2 KB of LDS and out in two stores whose 64 lanes write
        // consecutive 16-byte chunks (one contiguous 1 KB run per instruction); the
        // exchange stays inside the wave.
        float sc[8], bt[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = lane_rows ? g * 8 + j : j;
            sc[j] = 1.f + gamma[c] * (gsh[c] * inv);
            bt[j] = beta[c];
        }
        float4* const wst = reinterpret_cast<float4*>(red + ((R * C + 3) & ~3)) + (t >> 6) * 128;
        const int wl = t & 63;
        char* const yb = reinterpret_cast<char*>(y + static_cast<int64_t>(b) * S * C);
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int sv = s0 + v * R;
            if (sv >= s1) break;
            float f[8];
            pack8_to_f32<T>(raw[v], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = f[j] * sc[j] + bt[j];
            wst[2 * wl] = make_float4(f[0], f[1], f[2], f[3]);
            wst[2 * wl + 1] = make_float4(f[4], f[5], f[6], f[7]);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int64_t nbytes = static_cast<int64_t>(min(R, s1 - sv)) * C * 4;
            const int64_t o0 = static_cast<int64_t>(t >> 6) * 2048 + 16 * wl;
            const float4 c0 = wst[wl], c1 = wst[64 + wl];
            if (o0 < nbytes) *reinterpret_cast<float4*>(yb + static_cast<int64_t>(sv) * C * 4 + o0) = c0;
            if (o0 + 1024 < nbytes) *reinterpret_cast<float4*>(yb + static_cast<int64_t>(sv) * C * 4 + o0 + 1024) = c1;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    } else if (lane_rows) {
        float sc[8], bt[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = g * 8 + j;
            sc[j] = 1.f + gamma[c] * (gsh[c] * inv);
            bt[j] = beta[c];
        }
        TO* yb = y + static_cast<int64_t>(b) * S * C + g * 8;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            const int s = s0 + rr + v * R;
            if (s < s1) {
                float f[8];
                pack8_to_f32<T>(raw[v], f);
#pragma unroll
                for (int j = 0; j < 8; ++j) f[j] = f[j] * sc[j] + bt[j];
                store8<TO>(yb + static_cast<int64_t>(s) * C, f);
            }
        }
    }
    if (t == 0) {
        // every piece of image b has passed its wait once done reaches pieces
        if (atomicAdd(done, 1u) == static_cast<uint32_t>(pieces) - 1) {
            __hip_atomic_store(counted, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// LayerNorm over C per pixel (models/layers.py:25-35; Triton arithmetic of
// utils/layer_norm_cuda.py:44-57): mean, biased centred variance,
// y = (x - mean) * rstd * w + b.
// Channels-last: TPR lanes per pixel row, values kept in registers.
// ---------------------------------------------------------------------------
template <typename T, typename TO, int TPR, int MAXV>
__global__ __launch_bounds__(256) void layernorm_nhwc_kernel(const T* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ bias,
                                                            TO* __restrict__ y,
                                                            float* __restrict__ mean_out,
                                                            float* __restrict__ rstd_out,
                                                            int64_t rows, int C, float eps) {
    constexpr int RPB = 256 / TPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR;
    const int lane = threadIdx.x % TPR;
    const bool active = row < rows;
    const T* xr = x + (active ? row : 0) * C;
    float v[MAXV];
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
        const int c = lane + k * TPR;
        v[k] = (active && c < C) ? to_f32(xr[c]) : 0.f;
        sum += v[k];
    }
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    const float mean = sum / static_cast<float>(C);
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
        const int c = lane + k * TPR;
        const float d = (c < C) ? v[k] - mean : 0.f;
        v[k] = d;
        sq += d * d;
    }
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
    const float rstd = 1.f / sqrtf(sq / static_cast<float>(C) + eps);
    if (!active) return;
    TO* yr = y + row * C;
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
        const int c = lane + k * TPR;
        if (c < C) yr[c] = from_f32<TO>(v[k] * rstd * w[c] + bias[c]);
    }
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = rstd;
    }
}

// Channels-last, C % 8 == 0: LPR = 2^lpr_log2 lanes per pixel row, each lane GP groups
// of 8 channels (group k*LPR + lane), 16-byte loads and stores.
// ADD: the normalised row is x + r rounded to T (a residual add), which is also stored
// to x_sum, so the sum is read once instead of being written by one kernel and read by
// the next.
// STAGE: the workgroup's output rows (one contiguous range of rows * C values) are
// assembled in LDS and stored in 16-byte chunks by consecutive lanes, so every store
// instruction of a wave writes one contiguous 1 KB run (a lane's own 8 outputs would
// leave 16-byte gaps in each instruction's footprint).  Dynamic LDS of
// (256 / LPR) * C * sizeof(TO) bytes.  The row sums run on the VALU (ln_lane_sum: DPP
// and row-swap permutes, no LDS round trips).
template <typename T, typename TO, int GP, bool ADD = false, bool STAGE = false>
__global__ __launch_bounds__(256) void layernorm_nhwc8_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                             const float* __restrict__ bias, TO* __restrict__ y,
                                                             float* __restrict__ mean_out,
                                                             float* __restrict__ rstd_out, int64_t rows, int C,
                                                             int lpr_log2, float eps, const T* __restrict__ r = nullptr,
                                                             T* __restrict__ x_sum = nullptr) {
    const int LPR = 1 << lpr_log2;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 >> lpr_log2) + (threadIdx.x >> lpr_log2);
    const int lane = threadIdx.x & (LPR - 1);
    const bool active = row < rows;
    const T* xr = x + (active ? row : 0) * C;
    // The affine parameters of this lane's channels are loaded first, so their latency
    // overlaps the row's loads and reductions.
    float wv[GP][8], bv[GP][8];
#pragma unroll
    for (int k = 0; k < GP; ++k) {
        load8<float>(w + (k * LPR + lane) * 8, wv[k]);
        load8<float>(bias + (k * LPR + lane) * 8, bv[k]);
    }
    float v[GP][8];
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < GP; ++k) {
        load8<T>(xr + (k * LPR + lane) * 8, v[k]);
        if constexpr (ADD) {
            float rv[8];
            load8<T>(r + (active ? row : 0) * C + (k * LPR + lane) * 8, rv);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[k][j] = to_f32(from_f32<T>(v[k][j] + rv[j]));
            if (active) store8<T>(x_sum + row * C + (k * LPR + lane) * 8, v[k]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) sum += v[k][j];
    }
    sum = ln_lane_sum(sum, lpr_log2);
    const float inv_c = 1.f / static_cast<float>(C);   // exact for power-of-two C
    const float mean = sum * inv_c;
    float sq = 0.f;
#pragma unroll
    for (int k = 0; k < GP; ++k)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[k][j] -= mean;
            sq += v[k][j] * v[k][j];
        }
    sq = ln_lane_sum(sq, lpr_log2);
    const float rstd = __builtin_amdgcn_rsqf(sq * inv_c + eps);   // hardware reciprocal square root
    if constexpr (STAGE) {
        extern __shared__ __align__(16) unsigned char ln_stage[];
        TO* st = reinterpret_cast<TO*>(ln_stage) + (threadIdx.x >> lpr_log2) * C;
#pragma unroll
        for (int k = 0; k < GP; ++k) {
            const int c = (k * LPR + lane) * 8;
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = v[k][j] * rstd * wv[k][j] + bv[k][j];
            store8<TO>(st + c, o);
        }
        __syncthreads();
        const int64_t row0 = static_cast<int64_t>(blockIdx.x) * (256 >> lpr_log2);
        const int64_t nr = min(static_cast<int64_t>(256 >> lpr_log2), rows - row0);
        const int n16 = static_cast<int>(nr * C * static_cast<int64_t>(sizeof(TO)) / 16);
        const uint4* src = reinterpret_cast<const uint4*>(ln_stage);
        uint4* dst = reinterpret_cast<uint4*>(y + row0 * C);
        for (int m = threadIdx.x; m < n16; m += 256) dst[m] = src[m];
        if (!active) return;
    } else {
        if (!active) return;
#pragma unroll
        for (int k = 0; k < GP; ++k) {
            const int c = (k * LPR + lane) * 8;
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = v[k][j] * rstd * wv[k][j] + bv[k][j];
            store8<TO>(y + row * C + c, o);
        }
    }
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = rstd;
    }
}

// NCHW storage: one thread per pixel, channel loop (coalesced over pixels).
template <typename T, typename TO>
__global__ __launch_bounds__(256) void layernorm_nchw_kernel(const T* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ bias,
                                                            TO* __restrict__ y,
                                                            float* __restrict__ mean_out,
                                                            float* __restrict__ rstd_out,
                                                            int64_t B, int64_t C, int64_t S,
                                                            float eps) {
    const int64_t pix = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (pix >= B * S) return;
    const int64_t b = pix / S, s = pix % S;
    const T* xb = x + b * C * S + s;
    float sum = 0.f;
    for (int64_t c = 0; c < C; ++c) sum += to_f32(xb[c * S]);
    const float mean = sum / static_cast<float>(C);
    float sq = 0.f;
    for (int64_t c = 0; c < C; ++c) {
        const float d = to_f32(xb[c * S]) - mean;
        sq += d * d;
    }
    const float rstd = 1.f / sqrtf(sq / static_cast<float>(C) + eps);
    TO* yb = y + b * C * S + s;
    for (int64_t c = 0; c < C; ++c) yb[c * S] = from_f32<TO>((to_f32(xb[c * S]) - mean) * rstd * w[c] + bias[c]);
    if (mean_out) mean_out[pix] = mean;
    if (rstd_out) rstd_out[pix] = rstd;
}

// ---------------------------------------------------------------------------
// Query normalisation + relayout (utils/csrc/query_normalization.cu:135-177):
// [B, R, N, heads*D] -> [B, R, heads, N, D] fp32, inv_norm [B, R, heads, N].
// ---------------------------------------------------------------------------
template <int D, typename T>
__global__ __launch_bounds__(256) void qnorm_kernel(const T* __restrict__ q, float* __restrict__ out,
                                                   float* __restrict__ inv_norm, int64_t B,
                                                   int64_t R, int64_t N, int64_t heads) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t total = B * R * N * heads;
    if (idx >= total) return;
    const int64_t head = idx % heads;
    const int64_t t = (idx / heads) % N;
    const int64_t br = idx / (heads * N);
    const T* src = q + (br * N + t) * heads * D + head * D;
    float v[D];
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
        v[j] = to_f32(src[j]);
        sq += v[j] * v[j];
    }
    const float inv = 1.f / fmaxf(sqrtf(sq), 1e-12f);
    float* dst = out + ((br * heads + head) * N + t) * D;
#pragma unroll
    for (int j = 0; j < D; ++j) dst[j] = v[j] * inv;
    inv_norm[(br * heads + head) * N + t] = inv;
}

// ---------------------------------------------------------------------------
// Residual add (utils/residual.py:31-52): out = residual + branch * gamma_c * mask_b.
// ---------------------------------------------------------------------------
template <typename TR, typename TB>
__global__ __launch_bounds__(256) void residual_kernel(const TR* __restrict__ res,
                                                      const TB* __restrict__ br,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ mask,
                                                      float* __restrict__ out, int64_t total,
                                                      int64_t channels, int64_t spatial) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += stride) {
        const int64_t c = idx % channels;
        const int64_t b = idx / (channels * spatial);
        out[idx] = to_f32(res[idx]) + to_f32(br[idx]) * gamma[c] * mask[b];
    }
}

namespace {

template <typename F>
int dispatch_d(int d, F&& f) {
    switch (d) {
        case 4: f(std::integral_constant<int, 4>{}); return VH_OK;
        case 8: f(std::integral_constant<int, 8>{}); return VH_OK;
        case 16: f(std::integral_constant<int, 16>{}); return VH_OK;
        case 32: f(std::integral_constant<int, 32>{}); return VH_OK;
        case 64: f(std::integral_constant<int, 64>{}); return VH_OK;
    }
    return set_error(VH_ERR_HEAD_DIM, "head_dim must be one of 4, 8, 16, 32, 64; got %d", d);
}

template <typename F>
int dispatch_t(int t, F&& f) {
    switch (t) {
        case VH_DTYPE_F32: f(float{}); return VH_OK;
        case VH_DTYPE_BF16: f(bf16_t{}); return VH_OK;
        case VH_DTYPE_F16: f(f16_t{}); return VH_OK;
    }
    return set_error(VH_ERR_DTYPE, "unsupported dtype code %d", t);
}

unsigned grid_for(int64_t total, int64_t cap) {
    return static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((total + 255) / 256, cap)));
}

// Vectorised channels-last LayerNorm when C % 8 == 0 and every tensor is 16-byte aligned:
// LPR = largest power of two (<= 32) dividing C/8, GP = C/8/LPR groups per lane.
template <typename T, typename TO>
bool launch_ln_nhwc8(const void* x, const float* w, const float* b, void* yv, float* mean, float* rstd,
                     int64_t rows, int C, float eps, hipStream_t s) {
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                            reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(yv);
    if (C % 8 != 0 || align % 16 != 0) return false;
    const int ng = C / 8;
    int lg = 0;
    while (lg < 5 && ng % (2 << lg) == 0) ++lg;
    const int gp = ng >> lg;
    const unsigned blocks = static_cast<unsigned>((rows + (256 >> lg) - 1) / (256 >> lg));
    const T* xp = static_cast<const T*>(x);
    TO* y = static_cast<TO*>(yv);
    // Staged stores while the workgroup's rows fit in 32 KB of LDS (GP <= 4 for FP32 out).
    const size_t stage = static_cast<size_t>(256 >> lg) * C * sizeof(TO);
    const Override staged("ln_stage");
    if (stage <= 32768 && !(staged.set() && staged.value[0] == '0')) {
        switch (gp) {
#define VH_LN8S(G)                                                                                              \
    case G:                                                                                                     \
        hipLaunchKernelGGL((layernorm_nhwc8_kernel<T, TO, G, false, true>), dim3(blocks), dim3(256), stage, s, xp, \
                           w, b, y, mean, rstd, rows, C, lg, eps);                                              \
        return true;
            VH_LN8S(1) VH_LN8S(2) VH_LN8S(3) VH_LN8S(4)
#undef VH_LN8S
        }
    }
    switch (gp) {
#define VH_LN8(G)                                                                                        \
    case G:                                                                                              \
        hipLaunchKernelGGL((layernorm_nhwc8_kernel<T, TO, G>), dim3(blocks), dim3(256), 0, s, xp, w, b, y, \
                           mean, rstd, rows, C, lg, eps);                                                \
        return true;
        VH_LN8(1) VH_LN8(2) VH_LN8(3) VH_LN8(4) VH_LN8(5) VH_LN8(6) VH_LN8(7) VH_LN8(8)
#undef VH_LN8
    }
    return false;
}

template <typename T, typename TO>
bool launch_add_ln_nhwc8(const void* x, const void* r, const float* w, const float* b, void* x_sum, void* yv,
                         int64_t rows, int C, float eps, hipStream_t s) {
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(r) |
                            reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(b) |
                            reinterpret_cast<uintptr_t>(x_sum) | reinterpret_cast<uintptr_t>(yv);
    if (C % 8 != 0 || align % 16 != 0) return false;
    const int ng = C / 8;
    int lg = 0;
    while (lg < 5 && ng % (2 << lg) == 0) ++lg;
    const int gp = ng >> lg;
    const unsigned blocks = static_cast<unsigned>((rows + (256 >> lg) - 1) / (256 >> lg));
    const T* xp = static_cast<const T*>(x);
    const T* rp = static_cast<const T*>(r);
    T* sp = static_cast<T*>(x_sum);
    TO* y = static_cast<TO*>(yv);
    switch (gp) {
#define VH_ALN8(G)                                                                                      \
    case G:                                                                                             \
        hipLaunchKernelGGL((layernorm_nhwc8_kernel<T, TO, G, true>), dim3(blocks), dim3(256), 0, s, xp, w, \
                           b, y, nullptr, nullptr, rows, C, lg, eps, rp, sp);                           \
        return true;
        VH_ALN8(1) VH_ALN8(2) VH_ALN8(3) VH_ALN8(4) VH_ALN8(5) VH_ALN8(6) VH_ALN8(7) VH_ALN8(8)
#undef VH_ALN8
    }
    return false;
}

template <typename T, typename TO, int TPR>
void launch_ln_nhwc(const void* x, const float* w, const float* b, void* yv, float* mean,
                    float* rstd, int64_t rows, int C, float eps, hipStream_t s) {
    const unsigned blocks = static_cast<unsigned>((rows + 256 / TPR - 1) / (256 / TPR));
    const int per = (C + TPR - 1) / TPR;
    const T* xp = static_cast<const T*>(x);
    TO* y = static_cast<TO*>(yv);
    if (per <= 4)
        hipLaunchKernelGGL((layernorm_nhwc_kernel<T, TO, TPR, 4>), dim3(blocks), dim3(256), 0, s, xp, w, b,
                           y, mean, rstd, rows, C, eps);
    else if (per <= 8)
        hipLaunchKernelGGL((layernorm_nhwc_kernel<T, TO, TPR, 8>), dim3(blocks), dim3(256), 0, s, xp, w, b,
                           y, mean, rstd, rows, C, eps);
    else if (per <= 16)
        hipLaunchKernelGGL((layernorm_nhwc_kernel<T, TO, TPR, 16>), dim3(blocks), dim3(256), 0, s, xp, w,
                           b, y, mean, rstd, rows, C, eps);
    else if (per <= 32)
        hipLaunchKernelGGL((layernorm_nhwc_kernel<T, TO, TPR, 32>), dim3(blocks), dim3(256), 0, s, xp, w,
                           b, y, mean, rstd, rows, C, eps);
    else
        hipLaunchKernelGGL((layernorm_nhwc_kernel<T, TO, TPR, 64>), dim3(blocks), dim3(256), 0, s, xp, w,
                           b, y, mean, rstd, rows, C, eps);
}

}  // namespace

// ---------------------------------------------------------------------------
// Per-channel bias + optional GELU on a channels-last map, 8 channels per thread:
// out = act(round(x + b)), rounded to the io dtype after each step (the value a
// BatchNorm folded into the preceding convolution produces, then its activation).
// ---------------------------------------------------------------------------
template <typename T, int ACT>
__global__ __launch_bounds__(256) void bias_act8_kernel(const T* __restrict__ x, const float* __restrict__ bias,
                                                       T* __restrict__ out, int64_t vectors, int channels) {
    const int64_t v = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (v >= vectors) return;
    const int64_t at = v * 8;
    const int c = static_cast<int>(at % channels);
    float a[8], b[8];
    load8<T>(x + at, a);
    load8<float>(bias + c, b);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = to_f32(from_f32<T>(a[j] + b[j]));
        if constexpr (ACT == 1) a[j] = gelu_fast(a[j]);
    }
    store8<T>(out + at, a);
}

// GRN statistics from per-slab partial sums of squares partial [B, nslab, C]: gx,
// inv_den and (when scale is not null) scale = 1 + gamma * nx.  Shared with the
// depthwise kernel that produces the partial sums in its epilogue.
int launch_grn_finalize(const float* partial, float* gx, float* inv_den, int64_t B, int64_t C, int64_t nslab,
                        float eps, const float* gamma, float* scale, hipStream_t s) {
    if (B >= 64 || nslab < 64 || C > (int64_t(1) << 30) || nslab > (int64_t(1) << 30)) {
        hipLaunchKernelGGL(grn_finalize_kernel, dim3(static_cast<unsigned>(B)), dim3(kGrnFinalizeThreads), 0, s, partial, gx,
                           inv_den, C, nslab, eps, gamma, scale);
        return check_launch("grn_finalize_kernel");
    }
    // few images with many slabs: the slab sums spread over channel blocks x images
    hipLaunchKernelGGL(grn_gx8_kernel, dim3(static_cast<unsigned>((C + 63) / 64), static_cast<unsigned>(B)), dim3(256), 0, s,
                       partial, gx, static_cast<int>(C), static_cast<int>(nslab));
    hipLaunchKernelGGL(grn_image_scale_kernel, dim3(static_cast<unsigned>(B)), dim3(256), 0, s, gx, inv_den, C, eps, gamma,
                       scale);
    return check_launch("grn statistics kernels");
}

}  // namespace vh

using namespace vh;

extern "C" {

int vh_postprocess_scale_forward(const void* Y, const void* X, int32_t io_dtype, const float* d_skip,
                                 int32_t skip_per_direction, const float* scale, float* out,
                                 int64_t B, int64_t heads, int64_t H, int64_t W, int32_t head_dim,
                                 int32_t channels_last, void* stream) {
    VH_REQUIRE(Y && X && d_skip && scale && out, VH_ERR_ARG, "direction fusion pointers must not be null");
    VH_REQUIRE(B > 0 && heads > 0 && H > 0 && W > 0, VH_ERR_SHAPE,
               "Invalid shape for visionhope_postprocess_scale_forward.");
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    FusionParams fp{Y, X, d_skip, skip_per_direction, scale, out, B, heads, H, W, channels_last};
    const int64_t total = B * heads * head_dim * H * W;
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uintptr_t align = reinterpret_cast<uintptr_t>(Y) | reinterpret_cast<uintptr_t>(X) |
                            reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(d_skip) |
                            reinterpret_cast<uintptr_t>(scale);
    const int64_t groups = H * W * heads * (head_dim / 8);
    if (channels_last && head_dim >= 8 && align % 16 == 0) {
        int th_log2 = 2, tw_log2 = 2;
        int hpb = static_cast<int>(std::min<int64_t>(heads, std::max(1, 96 / head_dim)));
        // fusion_tile override "<log2 TH>x<log2 TW>x<heads per workgroup>" (measurements)
        const Override tile("fusion_tile");
        int ft = 0, fw = 0, fh = 0;
        if (tile.set() && std::sscanf(tile.value, "%dx%dx%d", &ft, &fw, &fh) == 3) {
            // the kernel is built for at most 256 threads (its launch bounds)
            VH_REQUIRE((1 << (ft + fw)) * std::min<int64_t>(fh, heads) * (head_dim / 8) <= 256, VH_ERR_ARG,
                       "fusion_tile override %s needs more than 256 threads per workgroup", tile.value);
            th_log2 = ft;
            tw_log2 = fw;
            hpb = static_cast<int>(std::min<int64_t>(heads, fh));
        }
        const int64_t tiles_w = (W + (1 << tw_log2) - 1) >> tw_log2, tiles_h = (H + (1 << th_log2) - 1) >> th_log2;
        const int64_t chunks = (heads + hpb - 1) / hpb;
        const size_t lds = static_cast<size_t>((1 << (th_log2 + tw_log2)) * hpb * head_dim) * sizeof(float);
        // the channel chunks of one tile are consecutive workgroups (measured 5% faster at
        // 28x28x192 than a chunk per grid z-plane)
        const uint32_t chunks_x = chunks > 1 ? static_cast<uint32_t>(chunks) : 1u;
        const dim3 grid(static_cast<unsigned>(tiles_w * tiles_h * chunks_x), static_cast<unsigned>(B),
                        static_cast<unsigned>(chunks_x > 1 ? 1 : chunks));
        const float inv_g = 1.0f / static_cast<float>(hpb * (head_dim / 8));
        // one thread per (pixel, head, 8-channel group) of a full chunk, in whole waves
        const unsigned threads = static_cast<unsigned>(((1 << (th_log2 + tw_log2)) * hpb * (head_dim / 8) + 63) / 64 * 64);
        int rc = dispatch_d(head_dim, [&](auto dc) {
            constexpr int D = decltype(dc)::value;
            if constexpr (D >= 8) {
                dispatch_t(io_dtype, [&](auto tv) {
                    hipLaunchKernelGGL((direction_fusion_tile_kernel<D, decltype(tv)>), grid, dim3(threads), lds, s, fp,
                                       static_cast<uint32_t>(tiles_w), th_log2, tw_log2, hpb, inv_g, chunks_x);
                });
            }
        });
        if (rc) return rc;
        return check_launch("direction_fusion_tile_kernel");
    }
    if (channels_last && head_dim >= 8 && align % 16 == 0 && groups < (int64_t(1) << 24)) {
        const dim3 grid(static_cast<unsigned>((groups + 255) / 256), static_cast<unsigned>(B));
        const float inv_w = 1.0f / static_cast<float>(W);
        const float inv_g = 1.0f / static_cast<float>(heads * (head_dim / 8));
        int rc = dispatch_d(head_dim, [&](auto dc) {
            constexpr int D = decltype(dc)::value;
            if constexpr (D >= 8) {
                dispatch_t(io_dtype, [&](auto tv) {
                    hipLaunchKernelGGL((direction_fusion8_kernel<D, decltype(tv)>), grid, dim3(256), 0, s, fp,
                                       inv_w, inv_g);
                });
            }
        });
        if (rc) return rc;
        return check_launch("direction_fusion8_kernel");
    }
    int rc = dispatch_d(head_dim, [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        dispatch_t(io_dtype, [&](auto tv) {
            hipLaunchKernelGGL((direction_fusion_kernel<D, decltype(tv)>), dim3(blocks), dim3(256), 0,
                               s, fp);
        });
    });
    if (rc) return rc;
    return check_launch("direction_fusion_kernel");
}

// Slab length of the vectorised GRN statistics: enough slabs for >= ~2048 blocks.
static int64_t grn_rows_per_slab(int64_t B, int64_t S) {
    const int64_t want = std::max<int64_t>(1, 2048 / std::max<int64_t>(B, 1));
    const int64_t nslab = std::min<int64_t>(std::max<int64_t>(1, (S + 7) / 8), want);
    return (S + nslab - 1) / nslab;
}

static bool grn_vectorised(int64_t C, const void* x, const void* y) {
    return C % 8 == 0 && C / 8 <= 256 &&
           (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16 == 0;
}

// Synchronisation header of the one-pass kernel at the start of the workspace (the same
// size for every shape, so no call's partial sums overlap another call's counters).
static size_t grn_sync_bytes() {
    return static_cast<size_t>(kGrnSyncImages) * kGrnSyncWords * 4;
}

// Pieces per image of the one-pass kernel (0 when the map does not qualify): R = 256 / (C/8)
// rows per pass, v rows per thread.  Every piece reads the pieces x C partial sums of its
// image, so the map qualifies only while those reads stay within 1/8 of the piece's own x
// bytes (R v C elem_bytes); wide maps with few rows per piece (e.g. 32x32x1792, 64 pieces
// of 16 rows) take the two-pass kernels instead.
// Pieces per image of the one-pass kernel: at least 5 and as few as 32 rows per thread
// allow, balanced (every piece but the last holds *piece_rows rows, *vrows >= rows per
// thread).  Fewer pieces mean fewer workgroups waiting on each other, more mean more
// workgroups in flight; measured on MI355X (B = 128, bf16 in, FP32 out): 56x56x96 at 5
// pieces (32 rows per thread) 0.78 of the HBM peak against 0.68 at 10 and 0.56 at 19;
// 28x28x192 0.60 / 0.64 / 0.65 / 0.65 at 3 / 4 / 5 / 8.  Returns 0 where the one-pass
// kernel does not apply (fewer than 2 pieces, or the other pieces' partial sums a piece
// reads would not be small next to its own x).
static int64_t grn_onepass_plan(int64_t C, int64_t S, int elem_bytes, int64_t* piece_rows, int* vrows) {
    if (C % 8 != 0 || C / 8 > 256) return 0;
    const int64_t R = 256 / (C / 8);
    int64_t want = std::min<int64_t>(std::max<int64_t>(5, (S + 4 * kGrnVec * R - 1) / (4 * kGrnVec * R)),
                                     (S + R - 1) / R);
    const Override forced("grn_pieces");   // measurements: pieces per image
    if (forced.set()) want = std::min<int64_t>(forced.as_int(), (S + R - 1) / R);
    const int64_t rows = (S + want - 1) / want;
    const int64_t pieces = (S + rows - 1) / rows;
    const int64_t v = (rows + R - 1) / R;
    if (pieces < 2 || pieces > kGrnMaxPieces || v > 4 * kGrnVec || pieces * 4 * 8 > rows * elem_bytes) return 0;
    if (piece_rows) *piece_rows = rows;
    if (vrows) *vrows = v <= kGrnVec ? kGrnVec : v <= 2 * kGrnVec ? 2 * kGrnVec : 4 * kGrnVec;
    return pieces;
}

size_t vh_grn_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W) {
    // Synchronisation words, then enough partial sums for the one-pass, the vectorised or
    // the scalar slab count.
    const int64_t S = H * W;
    const int64_t rows = grn_rows_per_slab(B, S);
    int64_t nslab = std::max<int64_t>((S + rows - 1) / rows, (S + kGrnRowsPerSlab - 1) / kGrnRowsPerSlab);
    // the one-pass kernel's pieces (fp32 qualifies whenever a 16-bit type does)
    nslab = std::max(nslab, grn_onepass_plan(C, S, 4, nullptr, nullptr));
    return grn_sync_bytes() + static_cast<size_t>(B * nslab * C) * sizeof(float);
}

int vh_grn_workspace_fallbacks(const void* workspace, size_t workspace_bytes, void* stream, int64_t* count) {
    VH_REQUIRE(workspace && count, VH_ERR_ARG, "GRN fallback query pointers must not be null");
    VH_REQUIRE(workspace_bytes >= grn_sync_bytes(), VH_ERR_WORKSPACE, "GRN workspace needs at least %zu bytes, got %zu",
               grn_sync_bytes(), workspace_bytes);
    static_assert(kGrnSyncImages * kGrnSyncWords * 4 == 32768, "header size");
    uint32_t words[kGrnSyncImages * kGrnSyncWords];
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(words, workspace, sizeof(words), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return set_error(VH_ERR_LAUNCH, "GRN fallback query: copy of the synchronisation header failed");
    int64_t n = 0;
    for (int i = 0; i < kGrnSyncImages; ++i) n += words[i * kGrnSyncWords + kGrnFallbackWord];
    *count = n;
    return VH_OK;
}

int vh_stream_capture_id(void* stream, int32_t* capturing, uint64_t* id) {
    VH_REQUIRE(capturing && id, VH_ERR_ARG, "capture query pointers must not be null");
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &status, &cid) != hipSuccess)
        return set_error(VH_ERR_LAUNCH, "hipStreamGetCaptureInfo failed");
    *capturing = status == hipStreamCaptureStatusActive ? 1 : 0;
    *id = *capturing ? static_cast<uint64_t>(cid) : 0;
    return VH_OK;
}

int vh_grn_forward(const void* x, int32_t io_dtype, const float* gamma, const float* beta, void* y,
                   int32_t y_dtype, float* gx, float* inv_den, int64_t B, int64_t C, int64_t H,
                   int64_t W, float eps, void* workspace, size_t workspace_bytes, void* stream) {
    VH_REQUIRE(x && gamma && beta && y && gx && inv_den, VH_ERR_ARG, "GRN pointers must not be null");
    VH_REQUIRE(B > 0 && C > 0 && H > 0 && W > 0, VH_ERR_SHAPE, "GRN expects nonempty input");
    VH_REQUIRE(B <= 65535, VH_ERR_SHAPE, "GRN batch must be <= 65535, got %lld", (long long)B);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "GRN supports FP32, FP16 and BF16 input");
    VH_REQUIRE(valid_dtype(y_dtype), VH_ERR_DTYPE, "unsupported GRN output dtype code %d", y_dtype);
    const size_t need = vh_grn_workspace_bytes(B, C, H, W);
    VH_REQUIRE(workspace && workspace_bytes >= need, VH_ERR_WORKSPACE,
               "GRN workspace needs %zu bytes, got %zu", need, workspace ? workspace_bytes : (size_t)0);
    const int64_t S = H * W;
    const int64_t nslab = (S + kGrnRowsPerSlab - 1) / kGrnRowsPerSlab;
    VH_REQUIRE(nslab <= 65535 * 16, VH_ERR_SHAPE, "GRN spatial size too large");
    const int ct = static_cast<int>(std::min<int64_t>(C, 256));
    const size_t lds = static_cast<size_t>(256 / ct) * static_cast<size_t>(C) * sizeof(float);
    VH_REQUIRE(lds <= 64 * 1024, VH_ERR_SHAPE, "GRN channel count %lld too large", (long long)C);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t* sync = static_cast<uint32_t*>(workspace);
    float* partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + grn_sync_bytes());
    const int64_t total = B * S * C;
    int vrows = 0;
    int64_t piece_rows = 0;
    const int64_t pieces = grn_onepass_plan(C, S, dtype_bytes(io_dtype), &piece_rows, &vrows);
    if (pieces > 0 && grn_vectorised(C, x, y) && B * S * C < (int64_t(1) << 31)) {
        const Override forced_spins("grn_spin_limit");
        const uint32_t spin_limit = forced_spins.set() ? static_cast<uint32_t>(forced_spins.as_i64()) : kGrnSpinLimit;
        const int G = static_cast<int>(C / 8);
        const unsigned threads = static_cast<unsigned>((G * (256 / G) + 63) / 64 * 64);
        // [R][C] partial sums (rounded up to 16 bytes), then 2 KB of staging per wave for FP32 output
        const size_t lds = ((static_cast<size_t>(256 / G) * static_cast<size_t>(C) + 3) & ~size_t(3)) * sizeof(float) +
                           static_cast<size_t>(threads / 64) * 2048;
        int rc = dispatch_t(io_dtype, [&](auto tv) {
            using T = decltype(tv);
            dispatch_t(y_dtype, [&](auto ov) {
                using TO = decltype(ov);
                for (int64_t b0 = 0; b0 < B; b0 += kGrnSyncImages) {
                    const int64_t nb = std::min<int64_t>(kGrnSyncImages, B - b0);
                    if (vrows == 4 * kGrnVec)
                        hipLaunchKernelGGL((grn_onepass8_kernel<T, TO, 4 * kGrnVec>), dim3(static_cast<unsigned>(nb * pieces)),
                                           dim3(threads), lds, s, static_cast<const T*>(x), gamma, beta, gx, inv_den,
                                           static_cast<TO*>(y), sync, partial, static_cast<int>(C), static_cast<int>(S),
                                           static_cast<int>(pieces), static_cast<int>(b0), eps, static_cast<int>(piece_rows),
                                           spin_limit);
                    else if (vrows == 2 * kGrnVec)
                        hipLaunchKernelGGL((grn_onepass8_kernel<T, TO, 2 * kGrnVec>), dim3(static_cast<unsigned>(nb * pieces)),
                                           dim3(threads), lds, s, static_cast<const T*>(x), gamma, beta, gx, inv_den,
                                           static_cast<TO*>(y), sync, partial, static_cast<int>(C), static_cast<int>(S),
                                           static_cast<int>(pieces), static_cast<int>(b0), eps, static_cast<int>(piece_rows),
                                           spin_limit);
                    else
                        hipLaunchKernelGGL((grn_onepass8_kernel<T, TO, kGrnVec>), dim3(static_cast<unsigned>(nb * pieces)),
                                           dim3(threads), lds, s, static_cast<const T*>(x), gamma, beta, gx, inv_den,
                                           static_cast<TO*>(y), sync, partial, static_cast<int>(C), static_cast<int>(S),
                                           static_cast<int>(pieces), static_cast<int>(b0), eps, static_cast<int>(piece_rows),
                                           spin_limit);
                }
            });
        });
        if (rc) return rc;
        return check_launch("grn_onepass8_kernel");
    }
    if (grn_vectorised(C, x, y) && B * S * C < (int64_t(1) << 31)) {
        const int G = static_cast<int>(C / 8);
        const int R = std::max(1, 256 / G);
        const int rows = static_cast<int>(grn_rows_per_slab(B, S));
        const int vslab = static_cast<int>((S + rows - 1) / rows);
        const size_t red = static_cast<size_t>(R) * static_cast<size_t>(C) * sizeof(float);
        const int apply_rows = std::max(R, static_cast<int>(std::min<int64_t>(S, std::max(4 * R, 16))));
        const unsigned apply_blocks = static_cast<unsigned>((S + apply_rows - 1) / apply_rows);
        int rc = dispatch_t(io_dtype, [&](auto tv) {
            using T = decltype(tv);
            hipLaunchKernelGGL((grn_partial8_kernel<T>), dim3(static_cast<unsigned>(vslab), static_cast<unsigned>(B)),
                               dim3(G * R), red, s, static_cast<const T*>(x), partial, static_cast<int>(C),
                               static_cast<int>(S), rows, vslab);
            // fold the statistics into the apply pass while each workgroup's extra read of the
            // partial sums (vslab x C floats) stays small next to its share of x
            const bool fold = static_cast<int64_t>(vslab) * C <= 8192;
            if (!fold)
                hipLaunchKernelGGL(grn_gx_kernel, dim3(static_cast<unsigned>((C + 63) / 64), static_cast<unsigned>(B)),
                                   dim3(256), 0, s, partial, gx, static_cast<int>(C), vslab);
            dispatch_t(y_dtype, [&](auto ov) {
                using TO = decltype(ov);
                const dim3 grid(apply_blocks, static_cast<unsigned>(B));
                const size_t lds = static_cast<size_t>(C) * sizeof(float);
                if (fold)
                    hipLaunchKernelGGL((grn_stats_apply8_kernel<T, TO, true>), grid, dim3(256), lds, s,
                                       static_cast<const T*>(x), partial, gamma, beta, gx, inv_den, static_cast<TO*>(y),
                                       static_cast<int>(C), static_cast<int>(S), vslab, apply_rows, eps);
                else
                    hipLaunchKernelGGL((grn_stats_apply8_kernel<T, TO, false>), grid, dim3(256), lds, s,
                                       static_cast<const T*>(x), partial, gamma, beta, gx, inv_den, static_cast<TO*>(y),
                                       static_cast<int>(C), static_cast<int>(S), vslab, apply_rows, eps);
            });
        });
        if (rc) return rc;
        return check_launch("grn vectorised kernels");
    }
    const bool aligned = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16 == 0;
    if (C % 8 == 0 && C / 8 > 256 && aligned && B * S * C < (int64_t(1) << 31)) {
        const int rows = static_cast<int>(grn_rows_per_slab(B, S));
        const int vslab = static_cast<int>((S + rows - 1) / rows);
        const int apply_rows = static_cast<int>(std::min<int64_t>(S, 8));
        const unsigned apply_blocks = static_cast<unsigned>((S + apply_rows - 1) / apply_rows);
        int rc = dispatch_t(io_dtype, [&](auto tv) {
            using T = decltype(tv);
            hipLaunchKernelGGL((grn_partial8_wide_kernel<T>), dim3(static_cast<unsigned>(vslab), static_cast<unsigned>(B)),
                               dim3(256), 0, s, static_cast<const T*>(x), partial, static_cast<int>(C),
                               static_cast<int>(S), rows, vslab);
            hipLaunchKernelGGL(grn_gx_kernel, dim3(static_cast<unsigned>((C + 63) / 64), static_cast<unsigned>(B)),
                               dim3(256), 0, s, partial, gx, static_cast<int>(C), vslab);
            dispatch_t(y_dtype, [&](auto ov) {
                using TO = decltype(ov);
                hipLaunchKernelGGL((grn_apply8_wide_kernel<T, TO>), dim3(apply_blocks, static_cast<unsigned>(B)),
                                   dim3(256), 0, s, static_cast<const T*>(x), gamma, beta, gx, inv_den,
                                   static_cast<TO*>(y), static_cast<int>(C), static_cast<int>(S), apply_rows, eps);
            });
        });
        if (rc) return rc;
        return check_launch("grn wide vectorised kernels");
    }
    int rc = dispatch_t(io_dtype, [&](auto tv) {
        using T = decltype(tv);
        hipLaunchKernelGGL((grn_partial_kernel<T>), dim3(static_cast<unsigned>(nslab), static_cast<unsigned>(B)),
                           dim3(256), lds, s, static_cast<const T*>(x), partial, C, S, nslab);
        hipLaunchKernelGGL(grn_finalize_kernel, dim3(static_cast<unsigned>(B)), dim3(kGrnFinalizeThreads), 0, s, partial,
                           gx, inv_den, C, nslab, eps);
        dispatch_t(y_dtype, [&](auto ov) {
            using TO = decltype(ov);
            hipLaunchKernelGGL((grn_apply_kernel<T, TO>), dim3(grid_for(total, 8192)), dim3(256), 0, s,
                               static_cast<const T*>(x), gamma, beta, gx, inv_den, static_cast<TO*>(y),
                               C, S, total);
        });
    });
    if (rc) return rc;
    return check_launch("grn kernels");
}

int vh_grn_scale_forward(const void* x, int32_t io_dtype, const float* gamma, float* gx, float* inv_den,
                         float* scale, int64_t B, int64_t C, int64_t H, int64_t W, float eps, void* workspace,
                         size_t workspace_bytes, void* stream) {
    VH_REQUIRE(x && gamma && gx && inv_den && scale, VH_ERR_ARG, "GRN statistics pointers must not be null");
    VH_REQUIRE(B > 0 && C > 0 && H > 0 && W > 0, VH_ERR_SHAPE, "GRN expects nonempty input");
    VH_REQUIRE(B <= 65535, VH_ERR_SHAPE, "GRN batch must be <= 65535, got %lld", (long long)B);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "GRN supports FP32, FP16 and BF16 input");
    const int64_t S = H * W;
    VH_REQUIRE(grn_vectorised(C, x, x) && B * S * C < (int64_t(1) << 31), VH_ERR_SHAPE,
               "GRN statistics need C %% 8 == 0, C <= 2048, 16-byte aligned x and B*H*W*C < 2^31");
    const size_t need = vh_grn_workspace_bytes(B, C, H, W);
    VH_REQUIRE(workspace && workspace_bytes >= need, VH_ERR_WORKSPACE,
               "GRN workspace needs %zu bytes, got %zu", need, workspace ? workspace_bytes : (size_t)0);
    hipStream_t s = static_cast<hipStream_t>(stream);
    float* partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + grn_sync_bytes());
    const int G = static_cast<int>(C / 8);
    const int R = std::max(1, 256 / G);
    const int rows = static_cast<int>(grn_rows_per_slab(B, S));
    const int vslab = static_cast<int>((S + rows - 1) / rows);
    const size_t red = static_cast<size_t>(R) * static_cast<size_t>(C) * sizeof(float);
    int rc = dispatch_t(io_dtype, [&](auto tv) {
        using T = decltype(tv);
        hipLaunchKernelGGL((grn_partial8_kernel<T>), dim3(static_cast<unsigned>(vslab), static_cast<unsigned>(B)),
                           dim3(G * R), red, s, static_cast<const T*>(x), partial, static_cast<int>(C),
                           static_cast<int>(S), rows, vslab);
        if (B >= 64) {
            hipLaunchKernelGGL(grn_finalize_kernel, dim3(static_cast<unsigned>(B)), dim3(kGrnFinalizeThreads), 0, s, partial,
                               gx, inv_den, C, static_cast<int64_t>(vslab), eps, gamma, scale);
        } else {
            // few images: the slab sums spread over channel blocks x images (grn_gx8_kernel)
            hipLaunchKernelGGL(grn_gx8_kernel, dim3(static_cast<unsigned>((C + 63) / 64), static_cast<unsigned>(B)),
                               dim3(256), 0, s, partial, gx, static_cast<int>(C), vslab);
            hipLaunchKernelGGL(grn_image_scale_kernel, dim3(static_cast<unsigned>(B)), dim3(256), 0, s, gx, inv_den, C,
                               eps, gamma, scale);
        }
    });
    if (rc) return rc;
    return check_launch("grn statistics kernels");
}

int vh_add_layernorm2d_forward(const void* x, const void* r, int32_t io_dtype, const float* weight,
                               const float* bias, void* x_sum, void* y, int32_t y_dtype, int64_t B, int64_t C,
                               int64_t H, int64_t W, float eps, void* stream) {
    VH_REQUIRE(x && r && weight && bias && x_sum && y, VH_ERR_ARG, "add + LayerNorm2d pointers must not be null");
    VH_REQUIRE(B > 0 && C > 0 && H > 0 && W > 0, VH_ERR_SHAPE, "add + LayerNorm2d expects nonempty input");
    VH_REQUIRE(valid_dtype(io_dtype) && valid_dtype(y_dtype), VH_ERR_DTYPE, "unsupported dtype code");
    VH_REQUIRE(C % 8 == 0 && C <= 64 * 64, VH_ERR_SHAPE, "add + LayerNorm2d needs C %% 8 == 0 and C <= 4096");
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(r) |
                            reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(bias) |
                            reinterpret_cast<uintptr_t>(x_sum) | reinterpret_cast<uintptr_t>(y);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "add + LayerNorm2d tensors must be 16-byte aligned");
    const int64_t ng = C / 8;
    int64_t lg = 0;
    while (lg < 5 && ng % (int64_t(2) << lg) == 0) ++lg;
    VH_REQUIRE((ng >> lg) <= 8, VH_ERR_SHAPE, "add + LayerNorm2d: unsupported channel count %lld", (long long)C);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t rows = B * H * W;
    int rc = dispatch_t(io_dtype, [&](auto tv) {
        dispatch_t(y_dtype, [&](auto ov) {
            launch_add_ln_nhwc8<decltype(tv), decltype(ov)>(x, r, weight, bias, x_sum, y, rows, static_cast<int>(C),
                                                            eps, s);
        });
    });
    if (rc) return rc;
    return check_launch("add + layernorm2d kernel");
}

int vh_layernorm2d_forward(const void* x, int32_t io_dtype, const float* weight, const float* bias,
                           void* y, int32_t y_dtype, float* mean, float* rstd, int64_t B, int64_t C,
                           int64_t H, int64_t W, float eps, int32_t channels_last, void* stream) {
    VH_REQUIRE(x && weight && bias && y, VH_ERR_ARG, "LayerNorm2d pointers must not be null");
    VH_REQUIRE(B > 0 && C > 0 && H > 0 && W > 0, VH_ERR_SHAPE, "LayerNorm2d expects nonempty input");
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "LayerNorm2d supports FP32, FP16 and BF16 input");
    VH_REQUIRE(valid_dtype(y_dtype), VH_ERR_DTYPE, "unsupported LayerNorm2d output dtype code %d", y_dtype);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t rows = B * H * W;
    int rc;
    if (channels_last) {
        VH_REQUIRE(C <= 64 * 64, VH_ERR_SHAPE, "LayerNorm2d supports at most 4096 channels, got %lld",
                   (long long)C);
        const int c = static_cast<int>(C);
        rc = dispatch_t(io_dtype, [&](auto tv) {
            dispatch_t(y_dtype, [&](auto ov) {
                using T = decltype(tv);
                using TO = decltype(ov);
                if (launch_ln_nhwc8<T, TO>(x, weight, bias, y, mean, rstd, rows, c, eps, s)) return;
                if (c <= 16) launch_ln_nhwc<T, TO, 4>(x, weight, bias, y, mean, rstd, rows, c, eps, s);
                else if (c <= 32) launch_ln_nhwc<T, TO, 8>(x, weight, bias, y, mean, rstd, rows, c, eps, s);
                else if (c <= 64) launch_ln_nhwc<T, TO, 16>(x, weight, bias, y, mean, rstd, rows, c, eps, s);
                else if (c <= 128) launch_ln_nhwc<T, TO, 32>(x, weight, bias, y, mean, rstd, rows, c, eps, s);
                else launch_ln_nhwc<T, TO, 64>(x, weight, bias, y, mean, rstd, rows, c, eps, s);
            });
        });
    } else {
        rc = dispatch_t(io_dtype, [&](auto tv) {
            dispatch_t(y_dtype, [&](auto ov) {
                using T = decltype(tv);
                using TO = decltype(ov);
                hipLaunchKernelGGL((layernorm_nchw_kernel<T, TO>),
                                   dim3(static_cast<unsigned>((rows + 255) / 256)), dim3(256), 0, s,
                                   static_cast<const T*>(x), weight, bias, static_cast<TO*>(y), mean,
                                   rstd, B, C, H * W, eps);
            });
        });
    }
    if (rc) return rc;
    return check_launch("layernorm2d kernel");
}

int vh_qnorm_forward(const void* q_raw, int32_t io_dtype, float* q, float* inv_norm, int64_t B,
                     int64_t R, int64_t N, int64_t heads, int32_t head_dim, void* stream) {
    VH_REQUIRE(q_raw && q && inv_norm, VH_ERR_ARG, "qnorm pointers must not be null");
    VH_REQUIRE(B > 0 && R > 0 && N > 0 && heads > 0, VH_ERR_SHAPE, "qnorm expects nonempty input");
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    const int64_t total = B * R * N * heads;
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = dispatch_d(head_dim, [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        dispatch_t(io_dtype, [&](auto tv) {
            using T = decltype(tv);
            hipLaunchKernelGGL((qnorm_kernel<D, T>), dim3(blocks), dim3(256), 0, s,
                               static_cast<const T*>(q_raw), q, inv_norm, B, R, N, heads);
        });
    });
    if (rc) return rc;
    return check_launch("qnorm_kernel");
}

int vh_bias_act_nhwc_forward(const void* x, int32_t io_dtype, const float* bias, int32_t act, void* out,
                             int64_t total, int64_t channels, void* stream) {
    VH_REQUIRE(x && bias && out, VH_ERR_ARG, "bias + activation pointers must not be null");
    VH_REQUIRE(total > 0 && channels > 0 && channels % 8 == 0 && total % channels == 0, VH_ERR_SHAPE,
               "bias + activation needs C %% 8 == 0 and a whole number of pixels");
    VH_REQUIRE(act == 0 || act == 1, VH_ERR_ARG, "unknown activation %d", act);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(bias);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "bias + activation tensors must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t vectors = total / 8;
    const dim3 grid(static_cast<unsigned>((vectors + 255) / 256));
    int rc = dispatch_t(io_dtype, [&](auto tv) {
        using T = decltype(tv);
        if (act == 1)
            hipLaunchKernelGGL((bias_act8_kernel<T, 1>), grid, dim3(256), 0, s, static_cast<const T*>(x), bias,
                               static_cast<T*>(out), vectors, static_cast<int>(channels));
        else
            hipLaunchKernelGGL((bias_act8_kernel<T, 0>), grid, dim3(256), 0, s, static_cast<const T*>(x), bias,
                               static_cast<T*>(out), vectors, static_cast<int>(channels));
    });
    if (rc) return rc;
    return check_launch("bias_act8_kernel");
}

int vh_residual_add_forward(const void* residual, int32_t residual_dtype, const void* branch,
                            int32_t branch_dtype, const float* gamma, const float* drop_scale,
                            float* out, int64_t total, int64_t channels, int64_t spatial,
                            void* stream) {
    VH_REQUIRE(residual && branch && gamma && drop_scale && out, VH_ERR_ARG,
               "residual pointers must not be null");
    VH_REQUIRE(total > 0 && channels > 0 && spatial > 0 && total % (channels * spatial) == 0,
               VH_ERR_SHAPE, "residual add shape mismatch");
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = dispatch_t(residual_dtype, [&](auto rv) {
        dispatch_t(branch_dtype, [&](auto bv) {
            using TR = decltype(rv);
            using TB = decltype(bv);
            hipLaunchKernelGGL((residual_kernel<TR, TB>), dim3(grid_for(total, 8192)), dim3(256), 0, s,
                               static_cast<const TR*>(residual), static_cast<const TB*>(branch), gamma,
                               drop_scale, out, total, channels, spatial);
        });
    });
    if (rc) return rc;
    return check_launch("residual_kernel");
}

}  // extern "C"
