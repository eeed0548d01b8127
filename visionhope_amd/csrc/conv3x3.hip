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
    pw_epilogue<EPI, TN, TM, WM, WN>(p, m0, n0, wm, wn, kg, i16, acc);
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

template <int MODE>
int launch_conv_act(const ConvParams& cp, int act, hipStream_t s) {
    return act == 1 ? launch_conv<PW_GELU, MODE>(cp, s) : launch_conv<PW_BIAS, MODE>(cp, s);
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
