// Shared pieces of the bf16 matrix-core kernels on channels-last maps (the 1x1
// projections and the 3x3 convolutions): parameters, the MFMA wrapper, the GRN
// operand transform, and the output-tile epilogue.
#pragma once
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "vh_common.h"

namespace vh {

enum PwEpilogue { PW_BIAS = 0, PW_GELU = 1, PW_ADD = 2, PW_SILU = 3,
                  PW_ADD_LN = 4 };   // internal: residual add + LayerNorm of the sum (vh_pointwise_add_layernorm_nhwc_forward)

struct PwParams {
    const bf16_t* x;        // [M, K]
    const bf16_t* w;        // [N, K]
    const float* bias;      // [N] fp32 (values added before the first rounding) or null
    const bf16_t* res;      // [M, N] residual (PW_ADD)
    bf16_t* out;            // [M, N]
    const float* pro_scale; // [images, K] GRN scale 1 + gamma * nx, or null (no prologue)
    const float* pro_shift; // [K] GRN beta
    int64_t M;
    int N, K;
    FastDiv rows_per_image; // pixels per image (prologue)
    // chained product (pointwise_dma_kernel CHAIN): out2 [M, N] = bf16(out @ w2^T + bias2),
    // w2 [N, N] bf16, bias2 [N] fp32 or null
    const bf16_t* w2;
    const float* bias2;
    bf16_t* out2;
    // PW_ADD_LN: out = bf16(res + bf16(x @ w^T + bias)) and ln_out = bf16(LayerNorm(out))
    // over the N channels of each pixel, affine ln_w / ln_b [N] fp32
    const float* ln_w;
    const float* ln_b;
    float ln_eps;
    bf16_t* ln_out;
};

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f_pw __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f_pw mfma_16x16x32(const uint4& a, const uint4& b, v4f_pw c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c,
                                                    0, 0, 0);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// GRN apply on 8 consecutive bf16 of row m: bf16(h * s + beta), s and beta fp32.
__device__ __forceinline__ uint4 grn_apply8(uint4 v, const float* s, const float* beta) {
    const float4 s0 = *reinterpret_cast<const float4*>(s), s1 = *reinterpret_cast<const float4*>(s + 4);
    const float4 b0 = *reinterpret_cast<const float4*>(beta), b1 = *reinterpret_cast<const float4*>(beta + 4);
    uint4 r;
    r.x = pack_bf16x2(bf16_lo(v.x) * s0.x + b0.x, bf16_hi(v.x) * s0.y + b0.y);
    r.y = pack_bf16x2(bf16_lo(v.y) * s0.z + b0.z, bf16_hi(v.y) * s0.w + b0.w);
    r.z = pack_bf16x2(bf16_lo(v.z) * s1.x + b1.x, bf16_hi(v.z) * s1.y + b1.y);
    r.w = pack_bf16x2(bf16_lo(v.w) * s1.z + b1.z, bf16_hi(v.w) * s1.w + b1.w);
    return r;
}


// Epilogue of one tile pair: lane holds channels n .. n+7 (from acc0 = tile 2q,
// acc1 = tile 2q+1) of pixel m.
// gtab: the GELU table (gelu_bf16_tab), required for PW_GELU.
template <int EPI>
__device__ __forceinline__ void pw_store8(const PwParams& p, int64_t m, int n, const float (&bv)[8], const v4f_pw& acc0,
                                          const v4f_pw& acc1, const float* gtab = nullptr) {
    // acc + bias rounded to bf16, two values per conversion.
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
        const uint32_t w0 = pack_bf16x2(acc0[j] + bv[j], acc0[j + 1] + bv[j + 1]);
        const uint32_t w1 = pack_bf16x2(acc1[j] + bv[4 + j], acc1[j + 1] + bv[5 + j]);
        v[j] = bf16_lo(w0); v[j + 1] = bf16_hi(w0);
        v[4 + j] = bf16_lo(w1); v[5 + j] = bf16_hi(w1);
    }
    if constexpr (EPI == PW_GELU) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = gelu_bf16_tab(v[j], gtab);
    } else if constexpr (EPI == PW_SILU) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = v[j] * sigmoid_fast(v[j]);
    } else if constexpr (EPI == PW_ADD) {
        const uint4 r = *reinterpret_cast<const uint4*>(p.res + m * p.N + n);
        v[0] += bf16_lo(r.x); v[1] += bf16_hi(r.x); v[2] += bf16_lo(r.y); v[3] += bf16_hi(r.y);
        v[4] += bf16_lo(r.z); v[5] += bf16_hi(r.z); v[6] += bf16_lo(r.w); v[7] += bf16_hi(r.w);
    }
    *reinterpret_cast<uint4*>(p.out + m * p.N + n) =
        make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
}

__device__ __forceinline__ void pw_bias8(const PwParams& p, int n, float (&bv)[8]) {
    if (p.bias) {
        const float4 b0 = *reinterpret_cast<const float4*>(p.bias + n);
        const float4 b1 = *reinterpret_cast<const float4*>(p.bias + n + 4);
        bv[0] = b0.x; bv[1] = b0.y; bv[2] = b0.z; bv[3] = b0.w; bv[4] = b1.x; bv[5] = b1.y; bv[6] = b1.z; bv[7] = b1.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) bv[j] = 0.f;
    }
}

// PW_ADD_LN epilogue of pixel m from the 2Q accumulator tiles of a lane (all N = 32 Q
// channels of the pixel over the four lanes kg = 0..3 of row i16: channels 32 q + 8 kg + j).
// The sums of the LayerNorm run in the order of layernorm_nhwc8_kernel<..., ADD> over the
// same map (8-channel groups g = 4 q + kg, each summed in channel order from zero, then a
// balanced tree over the groups in index order: kg pairs by lane exchanges, then q pairs in
// the lane), so both outputs carry the bits of that kernel after a bias-epilogue product.
// Every lane takes part in the exchanges; `valid` gates the stores.
template <int Q>
__device__ __forceinline__ void pw_add_ln_store(const PwParams& p, int64_t m, bool valid, int kg, const v4f_pw (&a)[2 * Q]) {
    const int64_t mm = valid ? m : 0;
    float v[Q][8], s[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int n = 32 * q + 8 * kg;
        float bv[8];
        pw_bias8(p, n, bv);
        uint32_t bw[4];   // bf16(acc + bias): the product's output
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            bw[j / 2] = pack_bf16x2(a[2 * q][j] + bv[j], a[2 * q][j + 1] + bv[j + 1]);
            bw[2 + j / 2] = pack_bf16x2(a[2 * q + 1][j] + bv[4 + j], a[2 * q + 1][j + 1] + bv[5 + j]);
        }
        const uint4 r = *reinterpret_cast<const uint4*>(p.res + mm * p.N + n);
        const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
        uint32_t sw[4];
#pragma unroll
        for (int h = 0; h < 4; ++h)
            sw[h] = pack_bf16x2(bf16_lo(rw[h]) + bf16_lo(bw[h]), bf16_hi(rw[h]) + bf16_hi(bw[h]));
        if (valid) *reinterpret_cast<uint4*>(p.out + m * p.N + n) = make_uint4(sw[0], sw[1], sw[2], sw[3]);
        s[q] = 0.f;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            v[q][2 * h] = bf16_lo(sw[h]);
            v[q][2 * h + 1] = bf16_hi(sw[h]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) s[q] += v[q][j];
    }
    auto tree = [&](float (&t)[Q]) {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            t[q] += __shfl_xor(t[q], 16);
            t[q] += __shfl_xor(t[q], 32);
        }
#pragma unroll
        for (int w = 1; w < Q; w *= 2)
#pragma unroll
            for (int q = 0; q < Q; q += 2 * w) t[q] += t[q + w];
        return t[0];
    };
    const float inv_c = 1.f / static_cast<float>(p.N);   // exact for power-of-two N
    const float mean = tree(s) * inv_c;
    float sq[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        sq[q] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[q][j] -= mean;
            sq[q] += v[q][j] * v[q][j];
        }
    }
    const float rstd = __builtin_amdgcn_rsqf(tree(sq) * inv_c + p.ln_eps);
    if (!valid) return;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int n = 32 * q + 8 * kg;
        float wv[8], bv[8], o[8];
        load8<float>(p.ln_w + n, wv);
        load8<float>(p.ln_b + n, bv);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = v[q][j] * rstd * wv[j] + bv[j];
        store8<bf16_t>(p.ln_out + m * p.N + n, o);
    }
}

// Row of w feeding MFMA row i16 of n tile tn.  Output channels are interleaved across
// pairs of 16-row MFMA tiles (tile 2p row r is channel 32p + 8(r/4) + r%4, tile 2p+1
// row r is channel 32p + 8(r/4) + 4 + r%4), so each lane ends with 8 consecutive
// channels of one pixel: one 16-byte store.
__device__ __forceinline__ int pw_wrow(int tn, int i16) { return 32 * (tn / 2) + 8 * (i16 / 4) + 4 * (tn % 2) + (i16 % 4); }

// Output tile of this block.  The grid is flat with the N tiles of one pixel tile
// adjacent; after the XCD remap every XCD owns a contiguous run of them, so the
// blocks that share a pixel tile run together and read its rows from one L2.
template <int BM, int BN>
__device__ __forceinline__ void pw_tile(const PwParams& p, int64_t& m0, int& n0) {
    const uint32_t nt = static_cast<uint32_t>(p.N / BN);
    const uint32_t l = xcd_remap_any(blockIdx.x, gridDim.x);
    m0 = static_cast<int64_t>(l / nt) * BM;
    n0 = static_cast<int>(l % nt) * BN;
}


// Epilogue of a block tile: wave (wm, wn) holds, for each pair q of n tiles, channels
// n0 + wn WN + 32 q + 8 kg + (0..7) of pixel m0 + wm WM + 16 tm + i16.
template <int EPI, int TN, int TM, int WM, int WN>
__device__ __forceinline__ void pw_epilogue(const PwParams& p, int64_t m0, int n0, int wm, int wn, int kg, int i16,
                                            const v4f_pw (&acc)[TN][TM], const float* gtab = nullptr) {
#pragma unroll
    for (int q = 0; q < TN / 2; ++q) {
        const int n = n0 + wn * WN + 32 * q + 8 * kg;
        float bv[8];
        pw_bias8(p, n, bv);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            const int64_t m = m0 + wm * WM + 16 * tm + i16;
            if (m < p.M) pw_store8<EPI>(p, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm], gtab);
        }
    }
}

}  // namespace vh
