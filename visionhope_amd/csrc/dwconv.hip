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
#include <cmath>
#include <cstdlib>

#include "vh_common.h"

namespace vh {

enum DwEpilogue { DW_PLAIN = 0, DW_ADD_INPUT = 1, DW_GATE = 2, DW_ADD_GELU = 3, DW_ACCUM_F32 = 4, DW_ADD_F32_AUX = 5 };

struct DwParams {
    const void* x;
    const float* taps;   // [K*K, C]
    const float* bias;   // [C] or null
    const void* aux;     // gate for DW_GATE (io dtype); fp32 addend for DW_ADD_F32_AUX
    void* out;           // io dtype, or fp32 for DW_ACCUM_F32
    int64_t B, H, W, C;
};

__device__ __forceinline__ float gelu_erf(float v) { return 0.5f * v * (1.f + erff(v * 0.70710678118654752f)); }

// Epilogue of one output vector (8 channels of pixel `at`) from the fp32 conv sum.
template <int EPI, typename T>
__device__ __forceinline__ void dw_epilogue(const DwParams& p, int64_t at, float (&acc)[8]) {
    const T* x = static_cast<const T*>(p.x);
    if constexpr (EPI == DW_ACCUM_F32) {
        float* o = static_cast<float*>(p.out) + at;
        float prev[8];
        load8<float>(o, prev);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = prev[j] + acc[j];
        store8<float>(o, acc);
        return;
    } else {
        if constexpr (EPI == DW_ADD_F32_AUX) {
            float a[8];
            load8<float>(static_cast<const float*>(p.aux) + at, a);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = a[j] + acc[j];
        } else if constexpr (EPI != DW_PLAIN) {
            float xin[8];
            load8<T>(x + at, xin);
            if constexpr (EPI == DW_GATE) {
                float gv[8];
                load8<T>(static_cast<const T*>(p.aux) + at, gv);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = xin[j] + (1.f / (1.f + expf(-gv[j]))) * acc[j];
            } else if constexpr (EPI == DW_ADD_GELU) {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = gelu_erf(xin[j] + acc[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = xin[j] + acc[j];
            }
        }
        store8<T>(static_cast<T*>(p.out) + at, acc);
    }
}

// One thread per (image, row, segment of P pixels, 8 channels): each kernel row loads
// the P+K-1 input vectors of the segment once and reuses them for all K horizontal
// taps of the P outputs, so a K x K window costs (P+K-1)/P input loads per tap row
// instead of K.  Consecutive lanes take consecutive channel groups (coalesced).
template <int K, int EPI, typename T, int P>
__global__ __launch_bounds__(256) void dwconv_nhwc_kernel(const DwParams p, const int segs) {
    constexpr int R = K / 2, NI = P + K - 1;
    const int G = static_cast<int>(p.C / 8);
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= p.B * p.H * segs * G) return;
    const int cg = static_cast<int>(idx % G);
    int64_t t = idx / G;
    const int seg = static_cast<int>(t % segs);
    t /= segs;
    const int h = static_cast<int>(t % p.H);
    const int64_t b = t / p.H;
    const int W = static_cast<int>(p.W), H = static_cast<int>(p.H);
    const int w0 = seg * P;
    const int64_t c = cg * 8;
    const T* x = static_cast<const T*>(p.x);
    const int64_t img = b * p.H * p.W;

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
#pragma unroll
    for (int dy = 0; dy < K; ++dy) {
        const int hh = h + dy - R;
        if (hh < 0 || hh >= H) continue;  // uniform per thread
        float in[NI][8];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int ww = w0 - R + i;
            if (ww >= 0 && ww < W) {
                load8<T>(x + ((img + static_cast<int64_t>(hh) * W + ww) * p.C) + c, in[i]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) in[i][j] = 0.f;
            }
        }
#pragma unroll
        for (int dx = 0; dx < K; ++dx) {
            float tp[8];
            load8<float>(p.taps + (dy * K + dx) * p.C + c, tp);
#pragma unroll
            for (int px = 0; px < P; ++px)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[px][j] += in[px + dx][j] * tp[j];
        }
    }
#pragma unroll
    for (int px = 0; px < P; ++px) {
        if (w0 + px >= W) break;
        dw_epilogue<EPI, T>(p, (img + static_cast<int64_t>(h) * W + w0 + px) * p.C + c, acc[px]);
    }
}

namespace {

// Pixels per thread (register blocking along W).  VH_DW_PIXELS = 1, 2, 4 or 8 overrides
// the default for measurements.
// Measured on MI355X at the Tiny shapes (B=128; W = 56 and 14): 2 pixels for 3x3,
// 4 for 5x5 on wide maps and 2 on narrow ones, 4 for 7x7.
inline int dw_default_pixels(int K, int64_t W) {
    if (K == 3) return 2;
    if (K == 5) return W >= 28 ? 4 : 2;
    return 4;
}

template <int K, typename T, int P>
void launch_dw_p(int epi, const DwParams& dp, hipStream_t s) {
    const int segs = static_cast<int>((dp.W + P - 1) / P);
    const int64_t total = dp.B * dp.H * segs * (dp.C / 8);
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    switch (epi) {
#define VH_DW(E)                                                                                   \
    case E: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, E, T, P>), grid, dim3(256), 0, s, dp, segs); \
        break;
        VH_DW(DW_PLAIN) VH_DW(DW_ADD_INPUT) VH_DW(DW_GATE) VH_DW(DW_ADD_GELU) VH_DW(DW_ACCUM_F32)
        VH_DW(DW_ADD_F32_AUX)
#undef VH_DW
    }
}

template <int K, typename T>
void launch_dw(int epi, const DwParams& dp, hipStream_t s) {
    int px = dw_default_pixels(K, dp.W);
    if (const char* env = std::getenv("VH_DW_PIXELS")) {
        const int v = std::atoi(env);
        if (v == 1 || v == 2 || v == 4 || v == 8) px = v;
    }
    switch (px) {
        case 1: launch_dw_p<K, T, 1>(epi, dp, s); break;
        case 2: launch_dw_p<K, T, 2>(epi, dp, s); break;
        case 4: launch_dw_p<K, T, 4>(epi, dp, s); break;
        default: launch_dw_p<K, T, 8>(epi, dp, s); break;
    }
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
    VH_REQUIRE(H < (int64_t(1) << 30) && W < (int64_t(1) << 30), VH_ERR_SHAPE, "depthwise conv image too large");
    DwParams dp{x, taps, bias, aux, out, B, H, W, C};
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
