// 3x3 convolutions with padding 1 (stride 1 or 2) on channels-last bf16 maps, as
// implicit GEMMs on the gfx950 matrix cores: the convolutions of the stem and of the
// downsample layers (models/layers.py:85-119), with their eval-mode BatchNorm folded
// into weight and bias and the GELU of the stem fused into the epilogue.
//
// GEMM view: out[m, n] = sum_k A[m, k] w[n, k] + bias[n] with m = (b, oh, ow) the output
// pixel and k = (kh, kw, c) the tap and input channel, so w is the convolution weight in
// channels-last order [N, 3, 3, Cin] and A[m, k] = x[b, s oh - 1 + kh, s ow - 1 + kw, c]
// (zero outside the map).  A is never materialised: each 16-byte chunk of an operand tile
// is read from the input map at the tap's offset.  For Cin % BK == 0 a k tile lies in
// one tap, so a chunk is 8 consecutive channels of one input pixel.  The first stem
// convolution (Cin = 3) takes k = 4 tap + c instead (c = 3 and taps 9..15 are zero
// padding, K = 64) and reads the fp32 or bf16 image directly, rounding to bf16 as autocast
// rounds the image before the convolution.
//
// Under bf16 autocast the reference rounds the convolution output, the BatchNorm output
// and the GELU output to bf16; here the folded sum acc + bias is rounded once and the GELU
// output once (the epilogue of the 1x1 kernels), so results differ from the unfolded
// modules by the one skipped rounding and the rounding of the folded weight.
#include "pw_common.h"

namespace vh {

struct ConvParams {
    PwParams g;        // g.x input map [B, H, W, Cin] (bf16), g.w [N, K], g.bias, g.out [M, N]; M = B Ho Wo
    const float* xf;   // fp32 input map [B, H, W, 3] (Cin = 3 with an fp32 image) or null
    int H, W, Cin, Ho, Wo, stride;
    FastDiv wo, howo;  // division by Wo and by Ho Wo
};

enum ConvMode { CONV_TAPS = 0, CONV_RGB_F32 = 1, CONV_RGB_BF16 = 2 };

// Same tiling as the register-staged 1x1 kernel: a BM x BN output tile per block of 4
// waves, k tiles of BK through two LDS buffers (rows padded to BK + 8 elements), the next
// tile's chunks in registers while the current one feeds the matrix cores.
template <int BM, int BN, int WGM, int BK, int EPI, int MODE, int OCC>
__global__ __launch_bounds__(256, OCC) void conv3x3_kernel(const ConvParams cp) {
    const PwParams& p = cp.g;
    constexpr int LROW = BK + 8;
    constexpr int WGN = 4 / WGM, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
    static_assert(TN % 2 == 0 && TM >= 1, "n tiles come in pairs");
    constexpr int CPR = BK / 8, A_CHUNKS = BM * CPR / 256, B_CHUNKS = (BN * CPR + 255) / 256;
    static_assert(BM * CPR % 256 == 0, "whole A chunks per thread");
    __shared__ __align__(16) bf16_t lds[2][(BM + BN) * LROW];
    __shared__ float gtab[EPI == PW_GELU ? GELU_TAB_N : 1];
    if constexpr (EPI == PW_GELU) gelu_tab_fill(gtab, static_cast<int>(threadIdx.x), 256);   // published by the first barrier

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const int wm = wv % WGM, wn = wv / WGM;
    int64_t m0;
    int n0;
    pw_tile<BM, BN>(p, m0, n0);
    const int K = p.K, ntiles = K / BK, H = cp.H, W = cp.W, Cin = cp.Cin;

    // The rows of this thread's A chunks are the same in every k tile: locate their
    // output pixels once.  pix is the input pixel under tap (0, 0), which may lie in
    // the padding (ih0 or iw0 = -1).
    int ih0[A_CHUNKS], iw0[A_CHUNKS];
    int64_t pix[A_CHUNKS];
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
        const int row = (tid + 256 * i) / CPR;
        const uint32_t m = static_cast<uint32_t>(std::min<int64_t>(m0 + row, p.M - 1));
        const uint32_t b = fast_div(m, cp.howo), rem = m - b * static_cast<uint32_t>(cp.howo.d);
        const uint32_t oh = fast_div(rem, cp.wo), ow = rem - oh * static_cast<uint32_t>(cp.wo.d);
        ih0[i] = static_cast<int>(oh) * cp.stride - 1;
        iw0[i] = static_cast<int>(ow) * cp.stride - 1;
        pix[i] = (static_cast<int64_t>(b) * H + ih0[i]) * W + iw0[i];
    }
    auto inside = [&](int ih, int iw) {
        return static_cast<unsigned>(ih) < static_cast<unsigned>(H) && static_cast<unsigned>(iw) < static_cast<unsigned>(W);
    };
    // One tap (kh, kw) of an RGB pixel as 4 bf16 (c = 0, 1, 2 and a zero).
    auto rgb = [&](int i, int tap) -> uint2 {
        const int kh = tap / 3, kw = tap - 3 * (tap / 3);
        if (tap >= 9 || !inside(ih0[i] + kh, iw0[i] + kw)) return make_uint2(0u, 0u);
        const int64_t at = (pix[i] + kh * W + kw) * 3;
        float v0, v1, v2;
        if constexpr (MODE == CONV_RGB_F32) {
            v0 = cp.xf[at]; v1 = cp.xf[at + 1]; v2 = cp.xf[at + 2];
        } else {
            v0 = to_f32(p.x[at]); v1 = to_f32(p.x[at + 1]); v2 = to_f32(p.x[at + 2]);
        }
        return make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, 0.f));
    };

    uint4 ra[A_CHUNKS], rb[B_CHUNKS];
    auto gload = [&](int t) {
        const int kt = t * BK;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int kc = (tid + 256 * i) % CPR;
            if constexpr (MODE == CONV_TAPS) {
                const int tap = kt / Cin, c0 = kt - tap * Cin + 8 * kc;
                const int kh = tap / 3, kw = tap - 3 * kh;
                ra[i] = inside(ih0[i] + kh, iw0[i] + kw)
                            ? *reinterpret_cast<const uint4*>(p.x + (pix[i] + kh * W + kw) * Cin + c0)
                            : make_uint4(0u, 0u, 0u, 0u);
            } else {
                const int tap = (kt + 8 * kc) / 4;
                const uint2 lo = rgb(i, tap), hi = rgb(i, tap + 1);
                ra[i] = make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = tid + 256 * i, row = c / CPR, kk = kt + 8 * (c % CPR);
            rb[i] = (BN * CPR % 256 == 0 || c < BN * CPR)
                        ? *reinterpret_cast<const uint4*>(p.w + static_cast<int64_t>(n0 + row) * K + kk)
                        : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto lstore = [&](int buf) {
        bf16_t* base = lds[buf];
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4*>(base + (c / CPR) * LROW + 8 * (c % CPR)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            if (BN * CPR % 256 == 0 || c < BN * CPR)
                *reinterpret_cast<uint4*>(base + (BM + c / CPR) * LROW + 8 * (c % CPR)) = rb[i];
        }
    };
    int wrow[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) wrow[tn] = wn * WN + pw_wrow(tn, i16);

    v4f_pw acc[TN][TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = v4f_pw{0.f, 0.f, 0.f, 0.f};

    gload(0);
    lstore(0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) gload(t + 1);
        const bf16_t* base = lds[buf];
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            uint4 af[TN], bfr[TM];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                af[tn] = *reinterpret_cast<const uint4*>(base + (BM + wrow[tn]) * LROW + 32 * ks + 8 * kg);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                bfr[tm] = *reinterpret_cast<const uint4*>(base + (wm * WM + 16 * tm + i16) * LROW + 32 * ks + 8 * kg);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = mfma_16x16x32(af[tn], bfr[tm], acc[tn][tm]);
        }
        if (t + 1 < ntiles) lstore(buf ^ 1);
        __syncthreads();
    }
    pw_epilogue<EPI, TN, TM, WM, WN>(p, m0, n0, wm, wn, kg, i16, acc, EPI == PW_GELU ? gtab : nullptr);
}

// ---------------------------------------------------------------------------
// Band kernel for narrow inputs (Cin = 32 or 64, or the RGB image).  A work item is one
// image's band of TH full-width output rows for BN output channels.  Its input rows
// (S (TH-1) + 3 rows, zero rows outside the image and a zero column either side) are
// copied into LDS once, so every input pixel leaves global memory once per band rather
// than once per tap, and the products read only LDS.  Blocks are persistent: each
// keeps the weight fragments of its channels in registers for the whole launch (one
// wave: 16 channels, all of K) and walks the bands with a stride of the grid, loading
// the next band's rows into registers while the current band computes.  The outputs
// of a band are assembled in LDS and written as contiguous pixel rows.
//
// LDS layout: patch pixel (row r, column p) at slot r PW + pos(p), PW = W + 2; with
// stride 2 the even columns come first and the odd ones after them (pos(p) = p/2 or
// HALF + p/2), so the pixels that one tap reads for consecutive outputs are
// consecutive slots.  A slot holds Cin/8 16-byte chunks plus one spare, so the 16
// slots of a fragment read start in distinct bank groups.  For the image a slot is 8
// bytes: three channels and a zero, rounded to bf16.
//
// The k steps run in the order of conv3x3_kernel (tap-major, 32 channels per step,
// the same operands to the same MFMA), so both kernels produce the same bits.
struct BandParams {
    ConvParams cp;
    int TH, IR, PW, HALF, nbands, nslices, items;   // items = images x bands
    uint32_t patch_bytes;
    FastDiv pw_div, nb_div;
};

template <int CIN, int S, int WGN, int MT, int PRE, int MODE, int EPI>
__global__ __launch_bounds__(256, 2) void conv3x3_band_kernel(const BandParams bp) {
    constexpr bool RGB = MODE != CONV_TAPS;
    static_assert(RGB ? CIN == 4 : (CIN == 32 || CIN == 64), "band kernel channels");
    constexpr int KS = RGB ? 2 : 9 * CIN / 32;            // k steps of 32
    constexpr int CPP = CIN / 8;                          // 16-byte chunks per input pixel
    constexpr int PSTRIDE = RGB ? 8 : (CPP + 1) * 16;     // bytes per patch slot
    constexpr int WGM = 4 / WGN, BN = WGN * 16;
    constexpr int OSTR = 2 * BN + 16;                     // bytes per output-stage pixel
    extern __shared__ __align__(16) unsigned char band_lds[];
    __shared__ float gtab[EPI == PW_GELU ? GELU_TAB_N : 1];
    if constexpr (EPI == PW_GELU) gelu_tab_fill(gtab, static_cast<int>(threadIdx.x), 256);   // published by the first barrier
    unsigned char* const ost = band_lds + bp.patch_bytes;
    const ConvParams& cp = bp.cp;
    const PwParams& p = cp.g;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const int wm = wv % WGM, wn = wv / WGM;
    const int slice = static_cast<int>(blockIdx.x % static_cast<uint32_t>(bp.nslices));
    const int stride_items = static_cast<int>(gridDim.x / static_cast<uint32_t>(bp.nslices));
    const int H = cp.H, W = cp.W, PW = bp.PW, Wo = cp.Wo, TH = bp.TH;
    const int nw = slice * BN + wn * 16;   // this wave's first output channel

    // Weight fragments: channel nw + i16, k = 32 ks + 8 kg .. + 7.
    uint4 wf[KS];
    {
        const bf16_t* wr = p.w + static_cast<int64_t>(nw + i16) * p.K + 8 * kg;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) wf[ks] = *reinterpret_cast<const uint4*>(wr + 32 * ks);
    }
    float bv[4];
    {
        const float4 b4 = p.bias ? *reinterpret_cast<const float4*>(p.bias + nw + 4 * kg) : make_float4(0.f, 0.f, 0.f, 0.f);
        bv[0] = b4.x; bv[1] = b4.y; bv[2] = b4.z; bv[3] = b4.w;
    }

    auto pos = [&](int pc) { return S == 1 ? pc : ((pc & 1) ? bp.HALF + (pc >> 1) : (pc >> 1)); };
    // Staging of one band's input rows: PRE units per thread (16-byte chunks, or image
    // pixels), loaded into registers by fetch and written to the patch by commit.  A
    // unit's patch position is the same in every band; it keeps its LDS destination,
    // its patch row (-1024 for the zero columns, so the row test rejects them) and its
    // byte offset from the band's first input row.
    const int total = RGB ? bp.IR * PW : bp.IR * PW * CPP;
    [[maybe_unused]] uint4 rv[PRE];
    [[maybe_unused]] float rf[PRE][3];
    uint32_t rdst[PRE];
    int rrow[PRE], rrel[PRE];
#pragma unroll
    for (int j = 0; j < PRE; ++j) {
        const int idx = std::min(256 * j + tid, total - 1);
        const int slot = RGB ? idx : idx / CPP, c = RGB ? 0 : idx % CPP;
        const int r = static_cast<int>(fast_div(static_cast<uint32_t>(slot), bp.pw_div)), pc = slot - r * PW;
        const int iw = pc - 1;
        rrow[j] = static_cast<unsigned>(iw) < static_cast<unsigned>(W) ? r : -1024;
        rrel[j] = RGB ? (r * W + iw) * 12 : ((r * W + iw) * CIN + 8 * c) * 2;
        rdst[j] = static_cast<uint32_t>((r * PW + pos(pc)) * PSTRIDE + 16 * c);
    }
    // Image bytes as one buffer: positions outside it read zeros.
    const uint32_t img_bytes = static_cast<uint32_t>(H * W) * (RGB ? (MODE == CONV_RGB_F32 ? 12u : 6u) : 2u * CIN);
    auto fetch = [&](int item) {
        const int b = static_cast<int>(fast_div(static_cast<uint32_t>(item), bp.nb_div));
        const int ih0 = S * (item - b * bp.nbands) * TH - 1;
        if constexpr (!RGB) {
            const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<bf16_t*>(p.x + static_cast<int64_t>(b) * H * W * CIN), 0, img_bytes, 0x00020000);
            const int rowb = ih0 * W * CIN * 2;
#pragma unroll
            for (int j = 0; j < PRE; ++j) {
                const bool ok = static_cast<unsigned>(ih0 + rrow[j]) < static_cast<unsigned>(H);
                const uint32_t off = ok ? static_cast<uint32_t>(rowb + rrel[j]) : 0x80000000u;
                const auto raw = __builtin_amdgcn_raw_buffer_load_b128(xr, static_cast<int>(off), 0, 0);
                rv[j] = make_uint4(raw[0], raw[1], raw[2], raw[3]);
            }
        } else if constexpr (MODE == CONV_RGB_F32) {
            const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(cp.xf + static_cast<int64_t>(b) * H * W * 3), 0, img_bytes, 0x00020000);
            const int rowb = ih0 * W * 12;
#pragma unroll
            for (int j = 0; j < PRE; ++j) {
                const bool ok = static_cast<unsigned>(ih0 + rrow[j]) < static_cast<unsigned>(H);
                const int off = ok ? rowb + rrel[j] : static_cast<int>(0x80000000u);
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    rf[j][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xr, off + 4 * q, 0, 0));
            }
        } else {
            const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<bf16_t*>(p.x + static_cast<int64_t>(b) * H * W * 3), 0, img_bytes, 0x00020000);
            const int rowb = ih0 * W * 6;
#pragma unroll
            for (int j = 0; j < PRE; ++j) {
                const bool ok = static_cast<unsigned>(ih0 + rrow[j]) < static_cast<unsigned>(H);
                const int off = ok ? rowb + rrel[j] / 2 : static_cast<int>(0x80000000u);
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    rf[j][q] = __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(xr, off + 2 * q, 0, 0)) << 16);
            }
        }
    };
    auto commit = [&]() {
#pragma unroll
        for (int j = 0; j < PRE; ++j) {
            if (256 * j + tid >= total) break;
            if constexpr (!RGB)
                *reinterpret_cast<uint4*>(band_lds + rdst[j]) = rv[j];
            else
                *reinterpret_cast<uint2*>(band_lds + rdst[j]) =
                    make_uint2(pack_bf16x2(rf[j][0], rf[j][1]), pack_bf16x2(rf[j][2], 0.f));
        }
    };

    // Byte offset of tap (kh, kw) from the slot of tap (0, 0).
    auto tapoff = [&](int t) {
        const int kh = t / 3, kw = t - 3 * (t / 3);
        return (kh * PW + (S == 1 ? kw : (kw == 1 ? bp.HALF : kw / 2))) * PSTRIDE;
    };
    // The image's k = 4 tap + c: lane kg holds taps 2 kg and 2 kg + 1 in step 0 and
    // tap 8 (kg = 0) or zeros in step 1.
    [[maybe_unused]] int roff0 = 0, roff1 = 0, roff8 = 0;
    if constexpr (RGB) {
        roff0 = tapoff(2 * kg);
        roff1 = tapoff(2 * kg + 1);
        roff8 = tapoff(8);
    }

    int item = static_cast<int>(blockIdx.x / static_cast<uint32_t>(bp.nslices));
    if (item >= bp.items) return;
    fetch(item);
    commit();
    __syncthreads();
    for (; item < bp.items; item += stride_items) {
        const int next = item + stride_items;
        if (next < bp.items) fetch(next);
        const int b = static_cast<int>(fast_div(static_cast<uint32_t>(item), bp.nb_div));
        const int oh0 = (item - b * bp.nbands) * TH;
        const int valid = std::min(TH, cp.Ho - oh0) * Wo;
        const int mtiles = (valid + 15) / 16, per = (mtiles + WGM - 1) / WGM;
        const int mt_end = std::min(mtiles, (wm + 1) * per);
        // A group of CNT pixel tiles (16 consecutive output pixels each, wrapping across
        // rows) starting at tile g: products over all k steps, then the epilogue into
        // the output stage.
        auto group = [&](int g, auto cnt_c) {
            constexpr int CNT = decltype(cnt_c)::value;
            uint32_t vb[CNT];
#pragma unroll
            for (int t = 0; t < CNT; ++t) {
                const int m = std::min((g + t) * 16 + i16, valid - 1);
                const int r = static_cast<int>(fast_div(static_cast<uint32_t>(m), cp.wo)), ow = m - r * Wo;
                vb[t] = static_cast<uint32_t>((S * r * PW + ow) * PSTRIDE + (RGB ? 0 : 16 * kg));
            }
            v4f_pw acc[CNT];
#pragma unroll
            for (int t = 0; t < CNT; ++t) acc[t] = v4f_pw{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                uint4 a[CNT];
#pragma unroll
                for (int t = 0; t < CNT; ++t) {
                    if constexpr (!RGB) {
                        const int tap = CIN == 32 ? ks : ks / 2;
                        const int off = tapoff(tap) + (CIN == 32 ? 0 : 64 * (ks % 2));
                        a[t] = *reinterpret_cast<const uint4*>(band_lds + vb[t] + off);
                    } else if (ks == 0) {
                        const uint2 lo = *reinterpret_cast<const uint2*>(band_lds + vb[t] + roff0);
                        const uint2 hi = *reinterpret_cast<const uint2*>(band_lds + vb[t] + roff1);
                        a[t] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    } else {
                        const uint2 lo = *reinterpret_cast<const uint2*>(band_lds + vb[t] + roff8);
                        a[t] = kg == 0 ? make_uint4(lo.x, lo.y, 0u, 0u) : make_uint4(0u, 0u, 0u, 0u);
                    }
                }
#pragma unroll
                for (int t = 0; t < CNT; ++t) acc[t] = mfma_16x16x32(wf[ks], a[t], acc[t]);
            }
            // Lane holds channels nw + 4 kg .. + 3 of pixel 16 (g + t) + i16.
#pragma unroll
            for (int t = 0; t < CNT; ++t) {
                const int m = (g + t) * 16 + i16;
                if (m >= valid) continue;
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; j += 2) {
                    const uint32_t w = pack_bf16x2(acc[t][j] + bv[j], acc[t][j + 1] + bv[j + 1]);
                    v[j] = bf16_lo(w);
                    v[j + 1] = bf16_hi(w);
                }
                if constexpr (EPI == PW_GELU) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j] = gelu_bf16_tab(v[j], gtab);
                }
                *reinterpret_cast<uint2*>(ost + m * OSTR + 2 * (wn * 16 + 4 * kg)) =
                    make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            }
        };
        int g = wm * per;
        for (; g + MT <= mt_end; g += MT) group(g, std::integral_constant<int, MT>{});
        for (; g < mt_end; ++g) group(g, std::integral_constant<int, 1>{});
        __syncthreads();
        // The band's outputs: valid pixels x BN channels, 16-byte chunks in address order.
        {
            constexpr int CPX = BN / 8;
            bf16_t* out = p.out + ((static_cast<int64_t>(b) * cp.Ho + oh0) * Wo) * p.N + slice * BN;
            for (int c = tid; c < valid * CPX; c += 256) {
                const int m = c / CPX, q = c % CPX;
                *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * p.N + 8 * q) =
                    *reinterpret_cast<const uint4*>(ost + m * OSTR + 16 * q);
            }
        }
        if (next < bp.items) commit();
        __syncthreads();
    }
}

namespace {

template <int EPI, int MODE>
int launch_conv(const ConvParams& cp, hipStream_t s) {
    const PwParams& p = cp.g;
    auto go = [&](auto kern, int rows, int cols) {
        const dim3 grid(static_cast<unsigned>((p.M + rows - 1) / rows * (p.N / cols)));
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, cp);
        return check_launch("conv3x3_kernel");
    };
    if constexpr (MODE != CONV_TAPS) {
        // K = 64 in two k tiles; N = 32 (the Tiny stem) or a multiple of 64.
        if (p.N % 128 == 0) return go(conv3x3_kernel<64, 128, 2, 32, EPI, MODE, 3>, 64, 128);
        if (p.N % 64 == 0) return go(conv3x3_kernel<128, 64, 2, 32, EPI, MODE, 3>, 128, 64);
        return go(conv3x3_kernel<256, 32, 4, 32, EPI, MODE, 2>, 256, 32);
    } else {
        if (cp.Cin % 64 != 0) {   // Cin = 32, 96, ...: k tiles of 32
            if (p.N % 128 == 0) return go(conv3x3_kernel<64, 128, 2, 32, EPI, MODE, 3>, 64, 128);
            if (p.N % 64 == 0) return go(conv3x3_kernel<128, 64, 2, 32, EPI, MODE, 3>, 128, 64);
            return go(conv3x3_kernel<256, 32, 4, 32, EPI, MODE, 2>, 256, 32);
        }
        if (p.N % 128 == 0) return go(conv3x3_kernel<64, 128, 2, 64, EPI, MODE, 2>, 64, 128);
        if (p.N % 64 == 0) return go(conv3x3_kernel<128, 64, 2, 64, EPI, MODE, 2>, 128, 64);
        return go(conv3x3_kernel<256, 32, 4, 64, EPI, MODE, 1>, 256, 32);
    }
}

// Band kernel launch, or -1 when it does not cover the shape (Cin other than 3, 32, 64;
// N not a multiple of 32; more than 64 KB of LDS or 10 staging units per thread) or
// the conv_band override "0" asks for conv3x3_kernel.  The band height aims at 7 pixel tiles per
// wave (one pass of the product loop); the grid is the number of blocks that fit on
// the GPU at once (a multiple of the channel slices).
template <int EPI, int MODE>
int launch_band(const ConvParams& cp, hipStream_t s) {
    const Override band("conv_band");
    if (band.set() && band.value[0] == '0') return -1;
    const int cin = MODE == CONV_TAPS ? cp.Cin : 4;
    if (!(cin == 4 || cin == 32 || cin == 64) || cp.g.N % 32 != 0) return -1;
    if (static_cast<int64_t>(cp.H) * cp.W * (cin == 4 ? 12 : 2 * cin) >= (int64_t(1) << 31)) return -1;
    const int wgn = cp.g.N % 64 == 0 ? 4 : 2, wgm = 4 / wgn, bn = 16 * wgn;
    const int pstride = cin == 4 ? 8 : (cin / 8 + 1) * 16;
    const int units_per_slot = cin == 4 ? 1 : cin / 8;
    BandParams bp{};
    bp.cp = cp;
    bp.PW = cp.W + 2;
    bp.HALF = (bp.PW + 1) / 2;
    auto rows_of = [&](int t) { return cp.stride * (t - 1) + 3; };
    auto lds_of = [&](int t) {
        return static_cast<int64_t>(rows_of(t)) * bp.PW * pstride + static_cast<int64_t>(t) * cp.Wo * (2 * bn + 16);
    };
    auto units_of = [&](int t) { return static_cast<int64_t>(rows_of(t)) * bp.PW * units_per_slot; };
    int th = std::max(1, std::min(cp.Ho, (112 * wgm + cp.Wo - 1) / cp.Wo));
    while (th > 1 && (lds_of(th) > 65536 || units_of(th) > 10 * 256)) --th;
    if (lds_of(th) > 65536 || units_of(th) > 10 * 256) return -1;
    const int pre = static_cast<int>((units_of(th) + 255) / 256);
    bp.TH = th;
    bp.IR = rows_of(th);
    bp.nbands = (cp.Ho + th - 1) / th;
    bp.nslices = cp.g.N / bn;
    const int64_t batch = cp.g.M / (static_cast<int64_t>(cp.Ho) * cp.Wo);
    if (batch * bp.nbands >= (int64_t(1) << 31)) return -1;
    bp.items = static_cast<int>(batch * bp.nbands);
    bp.patch_bytes = static_cast<uint32_t>(static_cast<int64_t>(bp.IR) * bp.PW * pstride);
    bp.pw_div = make_fastdiv(static_cast<uint32_t>(bp.PW));
    bp.nb_div = make_fastdiv(static_cast<uint32_t>(bp.nbands));
    const size_t lds = static_cast<size_t>(lds_of(th));
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    auto go = [&](auto kern) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds) != hipSuccess || per_cu <= 0) per_cu = 1;
        const int64_t streams = std::min<int64_t>(bp.items, static_cast<int64_t>(per_cu) * cus / bp.nslices);
        const dim3 grid(static_cast<unsigned>(std::max<int64_t>(1, streams) * bp.nslices));
        hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, bp);
        return check_launch("conv3x3_band_kernel");
    };
#define VH_BAND(CIN_, S_, WGN_, PRE_)                                                            \
    if (cin == CIN_ && cp.stride == S_ && wgn == WGN_ && pre <= PRE_)                            \
        return go(conv3x3_band_kernel<CIN_, S_, WGN_, 7, PRE_, MODE, EPI>);
    if constexpr (MODE == CONV_TAPS) {
        VH_BAND(32, 1, 2, 8) VH_BAND(32, 1, 4, 8) VH_BAND(32, 2, 2, 10) VH_BAND(32, 2, 4, 10)
        VH_BAND(64, 1, 2, 8) VH_BAND(64, 1, 4, 8) VH_BAND(64, 2, 2, 10) VH_BAND(64, 2, 4, 10)
    } else {
        VH_BAND(4, 1, 2, 5) VH_BAND(4, 1, 4, 5) VH_BAND(4, 2, 2, 5) VH_BAND(4, 2, 4, 5)
    }
#undef VH_BAND
    return -1;
}

template <int MODE>
int launch_conv_act(const ConvParams& cp, int act, hipStream_t s) {
    if (act == 1) {
        const int rc = launch_band<PW_GELU, MODE>(cp, s);
        return rc != -1 ? rc : launch_conv<PW_GELU, MODE>(cp, s);
    }
    const int rc = launch_band<PW_BIAS, MODE>(cp, s);
    return rc != -1 ? rc : launch_conv<PW_BIAS, MODE>(cp, s);
}

}  // namespace
}  // namespace vh

using namespace vh;

extern "C" int vh_conv3x3_nhwc_forward(const void* x, int32_t x_dtype, const void* weight, const float* bias,
                                       int32_t act, void* out, int64_t batch, int64_t height, int64_t width,
                                       int64_t in_channels, int64_t out_channels, int32_t stride, void* stream) {
    VH_REQUIRE(x && weight && bias && out, VH_ERR_ARG, "conv3x3 pointers must not be null");
    VH_REQUIRE(batch > 0 && height > 0 && width > 0 && out_channels > 0, VH_ERR_SHAPE, "conv3x3 expects a nonempty map");
    VH_REQUIRE(stride == 1 || stride == 2, VH_ERR_ARG, "conv3x3 stride must be 1 or 2, got %d", stride);
    VH_REQUIRE(act == 0 || act == 1, VH_ERR_ARG, "conv3x3 activation must be 0 (none) or 1 (GELU), got %d", act);
    const bool rgb = in_channels == 3;
    VH_REQUIRE(rgb || (in_channels % 32 == 0 && in_channels <= 4096), VH_ERR_SHAPE,
               "conv3x3 needs in_channels = 3 or a multiple of 32, got %lld", (long long)in_channels);
    VH_REQUIRE(x_dtype == VH_DTYPE_BF16 || (rgb && x_dtype == VH_DTYPE_F32), VH_ERR_DTYPE,
               "conv3x3 reads a bf16 map (or an fp32 3-channel image), got code %d", x_dtype);
    VH_REQUIRE(out_channels % 32 == 0, VH_ERR_SHAPE, "conv3x3 needs out_channels a multiple of 32, got %lld",
               (long long)out_channels);
    const int64_t ho = (height - 1) / stride + 1, wo = (width - 1) / stride + 1;
    const int64_t m = batch * ho * wo;
    VH_REQUIRE(m < (int64_t(1) << 31) && batch * height * width * std::max<int64_t>(in_channels, 4) < (int64_t(1) << 40),
               VH_ERR_SHAPE, "conv3x3 map too large");
    const uintptr_t align = (rgb ? 0 : reinterpret_cast<uintptr_t>(x)) | reinterpret_cast<uintptr_t>(weight) |
                            reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(bias);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "conv3x3 tensors must be 16-byte aligned (x unless 3-channel)");
    ConvParams cp{};
    cp.g.x = rgb && x_dtype == VH_DTYPE_F32 ? nullptr : static_cast<const bf16_t*>(x);
    cp.g.w = static_cast<const bf16_t*>(weight);
    cp.g.bias = bias;
    cp.g.out = static_cast<bf16_t*>(out);
    cp.g.M = m;
    cp.g.N = static_cast<int>(out_channels);
    cp.g.K = static_cast<int>(rgb ? 64 : 9 * in_channels);
    cp.xf = rgb && x_dtype == VH_DTYPE_F32 ? static_cast<const float*>(x) : nullptr;
    cp.H = static_cast<int>(height);
    cp.W = static_cast<int>(width);
    cp.Cin = static_cast<int>(in_channels);
    cp.Ho = static_cast<int>(ho);
    cp.Wo = static_cast<int>(wo);
    cp.stride = stride;
    cp.wo = make_fastdiv(static_cast<uint32_t>(wo));
    cp.howo = make_fastdiv(static_cast<uint32_t>(ho * wo));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!rgb) return launch_conv_act<CONV_TAPS>(cp, act, s);
    if (cp.xf) return launch_conv_act<CONV_RGB_F32>(cp, act, s);
    return launch_conv_act<CONV_RGB_BF16>(cp, act, s);
}
