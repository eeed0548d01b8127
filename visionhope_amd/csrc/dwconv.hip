// Depthwise KxK convolutions of the VisionHOPE block on channels-last maps, with
// the elementwise work around each convolution fused into its epilogue.
//
// Reference composition (models/block.py:63-107, models/layers.py:73-77):
//   cpe     x + dwconv3(x)                                   (block.py:102-103)
//   local   x + sigmoid(gate) * dwconv7(x)                   (block.py:63-66)
//   lepe    out + dwconv5(x_local)   (out: SRNL NHWC fp32)   (block.py:77-78),
//           accumulated in place (fp32) or written in the io dtype for proj_out
//   ffn     gelu(h + dwconv3(h))                             (layers.py:76-77)
// Each thread computes 8 consecutive channels of one pixel with fp32 accumulation;
// taps are stored taps-major ([K*K][C], fp32) so one tap is two float4 loads.
#include <cmath>

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

template <int K, int EPI, typename T>
__global__ __launch_bounds__(256) void dwconv_nhwc_kernel(const DwParams p) {
    const int64_t groups = p.C / 8;
    const int64_t total = p.B * p.H * p.W * groups;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    const int64_t cg = idx % groups;
    const int64_t pix = idx / groups;
    const int64_t w = pix % p.W;
    const int64_t h = (pix / p.W) % p.H;
    const int64_t b = pix / (p.W * p.H);
    const int64_t c = cg * 8;
    const T* x = static_cast<const T*>(p.x);

    float acc[8];
    if (p.bias) {
        const float4 b0 = *reinterpret_cast<const float4*>(p.bias + c);
        const float4 b1 = *reinterpret_cast<const float4*>(p.bias + c + 4);
        acc[0] = b0.x; acc[1] = b0.y; acc[2] = b0.z; acc[3] = b0.w;
        acc[4] = b1.x; acc[5] = b1.y; acc[6] = b1.z; acc[7] = b1.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    }
    constexpr int R = K / 2;
#pragma unroll
    for (int dy = 0; dy < K; ++dy) {
        const int64_t hh = h + dy - R;
        if (hh < 0 || hh >= p.H) continue;
#pragma unroll
        for (int dx = 0; dx < K; ++dx) {
            const int64_t ww = w + dx - R;
            if (ww < 0 || ww >= p.W) continue;
            float v[8];
            load8<T>(x + ((b * p.H + hh) * p.W + ww) * p.C + c, v);
            const float* tp = p.taps + (dy * K + dx) * p.C + c;
            const float4 t0 = *reinterpret_cast<const float4*>(tp);
            const float4 t1 = *reinterpret_cast<const float4*>(tp + 4);
            acc[0] += v[0] * t0.x; acc[1] += v[1] * t0.y; acc[2] += v[2] * t0.z; acc[3] += v[3] * t0.w;
            acc[4] += v[4] * t1.x; acc[5] += v[5] * t1.y; acc[6] += v[6] * t1.z; acc[7] += v[7] * t1.w;
        }
    }
    const int64_t at = pix * p.C + c;
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

namespace {

template <int K, typename T>
void launch_dw(int epi, const DwParams& dp, unsigned blocks, hipStream_t s) {
    switch (epi) {
        case DW_PLAIN: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, DW_PLAIN, T>), dim3(blocks), dim3(256), 0, s, dp); break;
        case DW_ADD_INPUT: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, DW_ADD_INPUT, T>), dim3(blocks), dim3(256), 0, s, dp); break;
        case DW_GATE: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, DW_GATE, T>), dim3(blocks), dim3(256), 0, s, dp); break;
        case DW_ADD_GELU: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, DW_ADD_GELU, T>), dim3(blocks), dim3(256), 0, s, dp); break;
        case DW_ACCUM_F32: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, DW_ACCUM_F32, T>), dim3(blocks), dim3(256), 0, s, dp); break;
        case DW_ADD_F32_AUX: hipLaunchKernelGGL((dwconv_nhwc_kernel<K, DW_ADD_F32_AUX, T>), dim3(blocks), dim3(256), 0, s, dp); break;
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
    DwParams dp{x, taps, bias, aux, out, B, H, W, C};
    const int64_t total = B * H * W * (C / 8);
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto go = [&](auto tv) {
        using T = decltype(tv);
        if (ksize == 3) launch_dw<3, T>(epilogue, dp, blocks, s);
        else if (ksize == 5) launch_dw<5, T>(epilogue, dp, blocks, s);
        else launch_dw<7, T>(epilogue, dp, blocks, s);
    };
    switch (io_dtype) {
        case VH_DTYPE_F32: go(float{}); break;
        case VH_DTYPE_BF16: go(bf16_t{}); break;
        default: go(f16_t{}); break;
    }
    return check_launch("dwconv_nhwc_kernel");
}
