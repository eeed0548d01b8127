// 1x1 convolutions of the VisionHOPE block on channels-last bf16 maps, as GEMMs on
// the gfx950 matrix cores, with the elementwise work around each projection fused.
//
// Reference composition (models/block.py:63-107, models/layers.py:67-80):
//   proj_in, local_gate, proj_out, W_q    out = x W^T + b
//   ffn.fc1 + ffn.act                      out = gelu(x W^T + b)
//   ffn.grn + ffn.fc2 + residual           out = r + grn(h) W^T + b, with the GRN apply
//                                          grn(h)[m, k] = h[m, k] * s[img(m), k] + beta[k]
//                                          done on the operand as it is loaded
// Under bf16 autocast every intermediate of the reference is a bf16 tensor; the same
// values are rounded to bf16 at the same points here (the linear output before the
// GELU and before the residual add, the GRN output before the product), so only the
// order of the fp32 accumulation differs.
//
// Layout: x [M, K], w [N, K] (the 1x1 weight as stored), out / residual [M, N], all
// bf16 row-major (NHWC with M = B*H*W pixels).  One v_mfma_f32_16x16x32_bf16 takes
// from lane l the 8 consecutive k of w row (l % 16) as operand A and of x row (l % 16)
// as operand B, and returns D[n][m] for n = 4 (l / 16) + j, m = l % 16: each lane ends
// with 4 consecutive output channels of one pixel (one 8-byte store).  Any order of the
// 32 k inside the instruction gives the same sum, as A and B use the same one.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "vh_common.h"

namespace vh {

enum PwEpilogue { PW_BIAS = 0, PW_GELU = 1, PW_ADD = 2 };

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

__device__ __forceinline__ float round_bf16(float v) {
    return __uint_as_float(static_cast<uint32_t>(from_f32<bf16_t>(v).bits) << 16);
}

// Block tile BM x BN of the output, k in steps of BK = 64 through LDS (two buffers):
// each thread moves 16-byte chunks global -> registers -> LDS (rows of x and w are
// contiguous in k, so 8 consecutive lanes read one 128-byte row segment), and the
// next tile's loads are in flight while the current one feeds the matrix cores.
// The 4 waves split the tile WGM x WGN; a wave owns WM x WN outputs.  LDS rows are
// padded to 72 elements so the 16 rows of one fragment read fall in distinct banks.
// Output channels are interleaved across pairs of 16-row MFMA tiles (tile 2p row r
// is channel 32p + 8(r/4) + r%4, tile 2p+1 row r is channel 32p + 8(r/4) + 4 + r%4),
// so each lane ends with 8 consecutive channels of one pixel: one 16-byte store.
// Epilogue of one tile pair: lane holds channels n .. n+7 (from acc0 = tile 2q,
// acc1 = tile 2q+1) of pixel m.
template <int EPI>
__device__ __forceinline__ void pw_store8(const PwParams& p, int64_t m, int n, const float (&bv)[8], const v4f_pw& acc0,
                                          const v4f_pw& acc1) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[j] = round_bf16(acc0[j] + bv[j]);
        v[4 + j] = round_bf16(acc1[j] + bv[4 + j]);
    }
    if constexpr (EPI == PW_GELU) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = gelu_fast(v[j]);
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

// Row of w feeding MFMA row i16 of n tile tn, for the channel interleave above.
__device__ __forceinline__ int pw_wrow(int tn, int i16) { return 32 * (tn / 2) + 8 * (i16 / 4) + 4 * (tn % 2) + (i16 % 4); }

// PRO: 0 no GRN prologue; 1 GRN applied to each x chunk as it is loaded (scale and
// beta read from global memory per chunk); 2 the k tile's scale rows of the block's
// (at most two) images and beta staged in LDS with the operand tiles and applied to the
// x fragments as they are read (the host takes 2 when an image has at least BM pixels).
template <int BM, int BN, int WGM, int BK, int EPI, int PRO, int OCC = 1>
__global__ __launch_bounds__(256, OCC) void pointwise_gemm_kernel(const PwParams p) {
    constexpr int PW_BK = BK, PW_LDS_ROW = BK + 8;
    static_assert(WGM == 1 || WGM == 2 || WGM == 4, "4 waves");
    constexpr int WGN = 4 / WGM, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
    static_assert(TN % 2 == 0 && TM >= 1, "n tiles come in pairs");
    // 16-byte chunks of a k tile: CPR per row; per thread ceil(total / 256).
    constexpr int CPR = PW_BK / 8, A_TOTAL = BM * CPR, B_TOTAL = BN * CPR;
    constexpr int A_CHUNKS = (A_TOTAL + 255) / 256, B_CHUNKS = (B_TOTAL + 255) / 256;
    __shared__ __align__(16) bf16_t lds[2][(BM + BN) * PW_LDS_ROW];
    __shared__ __align__(16) float grn_s[2][PRO == 2 ? 3 * BK : 4];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const int wm = wv % WGM, wn = wv / WGM;
    const int64_t m0 = static_cast<int64_t>(xcd_remap_any(blockIdx.x, gridDim.x)) * BM;
    const int n0 = static_cast<int>(blockIdx.y) * BN;
    const int K = p.K;
    const int ntiles = (K + PW_BK - 1) / PW_BK;

    [[maybe_unused]] int64_t img0 = 0, last_img = 0;
    [[maybe_unused]] float4 rs = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (PRO == 2) {
        img0 = fast_div(static_cast<uint32_t>(m0), p.rows_per_image);
        last_img = fast_div(static_cast<uint32_t>(p.M - 1), p.rows_per_image);
    }
    // Global chunk c of a tile: row c / CPR, k offset 8 (c % CPR).
    uint4 ra[A_CHUNKS], rb[B_CHUNKS];
    auto gload = [&](int t) {
        const int kt = t * PW_BK;
        if constexpr (PRO == 2) {
            if (tid < 3 * PW_BK / 4) {
                const int which = tid / (PW_BK / 4), kk = kt + 4 * (tid % (PW_BK / 4));
                const float* src = which < 2 ? p.pro_scale + std::min<int64_t>(img0 + which, last_img) * K + kk
                                             : p.pro_shift + kk;
                rs = kk < K ? *reinterpret_cast<const float4*>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int c = tid + 256 * i, row = c / CPR, kk = kt + 8 * (c % CPR);
            const int64_t m = std::min<int64_t>(m0 + row, p.M - 1);
            uint4 v = make_uint4(0u, 0u, 0u, 0u);
            if (kk < K && (A_TOTAL % 256 == 0 || c < A_TOTAL)) {
                v = *reinterpret_cast<const uint4*>(p.x + m * K + kk);
                if constexpr (PRO == 1) {
                    const int64_t img = fast_div(static_cast<uint32_t>(m), p.rows_per_image);
                    v = grn_apply8(v, p.pro_scale + img * K + kk, p.pro_shift + kk);
                }
            }
            ra[i] = v;
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = tid + 256 * i, row = c / CPR, kk = kt + 8 * (c % CPR);
            rb[i] = (kk < K && (B_TOTAL % 256 == 0 || c < B_TOTAL))
                        ? *reinterpret_cast<const uint4*>(p.w + static_cast<int64_t>(n0 + row) * K + kk)
                        : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto lstore = [&](int buf) {
        bf16_t* base = lds[buf];
        if constexpr (PRO == 2) {
            if (tid < 3 * PW_BK / 4)
                *reinterpret_cast<float4*>(&grn_s[buf][(tid / (PW_BK / 4)) * PW_BK + 4 * (tid % (PW_BK / 4))]) = rs;
        }
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            if (A_TOTAL % 256 == 0 || c < A_TOTAL)
                *reinterpret_cast<uint4*>(base + (c / CPR) * PW_LDS_ROW + 8 * (c % CPR)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            if (B_TOTAL % 256 == 0 || c < B_TOTAL)
                *reinterpret_cast<uint4*>(base + (BM + c / CPR) * PW_LDS_ROW + 8 * (c % CPR)) = rb[i];
        }
    };
    // Row of w feeding MFMA row i16 of n tile tn (channel interleave above).
    int wrow[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
        wrow[tn] = wn * WN + pw_wrow(tn, i16);

    // Staged scale row (0: first image of the block, 1: the next) of each x fragment row.
    [[maybe_unused]] int rel[TM];
    if constexpr (PRO == 2) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            const int64_t m = std::min<int64_t>(m0 + wm * WM + 16 * tm + i16, p.M - 1);
            rel[tm] = static_cast<int>(fast_div(static_cast<uint32_t>(m), p.rows_per_image) - img0);
        }
    }

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
        for (int ks = 0; ks < PW_BK / 32; ++ks) {
            uint4 af[TN], bfr[TM];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                af[tn] = *reinterpret_cast<const uint4*>(base + (BM + wrow[tn]) * PW_LDS_ROW + 32 * ks + 8 * kg);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                bfr[tm] = *reinterpret_cast<const uint4*>(base + (wm * WM + 16 * tm + i16) * PW_LDS_ROW + 32 * ks + 8 * kg);
                if constexpr (PRO == 2)
                    bfr[tm] = grn_apply8(bfr[tm], &grn_s[buf][rel[tm] * PW_BK + 32 * ks + 8 * kg],
                                         &grn_s[buf][2 * PW_BK + 32 * ks + 8 * kg]);
            }
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = mfma_16x16x32(af[tn], bfr[tm], acc[tn][tm]);
        }
        if (t + 1 < ntiles) lstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds channels n0 + wn WN + 32 q + 8 kg + (0..7) of pixel
    // m0 + wm WM + 16 tm + i16 for each tile pair q.
#pragma unroll
    for (int q = 0; q < TN / 2; ++q) {
        const int n = n0 + wn * WN + 32 * q + 8 * kg;
        float bv[8];
        pw_bias8(p, n, bv);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            const int64_t m = m0 + wm * WM + 16 * tm + i16;
            if (m < p.M) pw_store8<EPI>(p, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm]);
        }
    }
}

// Narrow outputs (N = 32 or 64) with K <= 256: no LDS.  A wave owns 16 TM pixels and
// every output channel; it issues all loads of its x rows at once (TM * KS 16-byte
// fragments), reads the small weight fragments through L1 and writes each pixel's
// channels once.
template <int KS, int TN, int TM, int EPI, bool PRO>
__global__ __launch_bounds__(256) void pointwise_narrow_kernel(const PwParams p) {
    static_assert(TN % 2 == 0, "n tiles come in pairs");
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, i16 = lane & 15, kg = lane >> 4;
    const int64_t m_wave = (static_cast<int64_t>(xcd_remap_any(blockIdx.x, gridDim.x)) * 4 + wv) * (16 * TM);
    if (m_wave >= p.M) return;
    constexpr int K = 32 * KS;
    uint4 xf[TM][KS];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
        const int64_t m = std::min<int64_t>(m_wave + 16 * tm + i16, p.M - 1);
        const bf16_t* xr = p.x + m * K + 8 * kg;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) xf[tm][ks] = *reinterpret_cast<const uint4*>(xr + 32 * ks);
        if constexpr (PRO) {
            const int64_t img = fast_div(static_cast<uint32_t>(m), p.rows_per_image);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                xf[tm][ks] = grn_apply8(xf[tm][ks], p.pro_scale + img * K + 32 * ks + 8 * kg, p.pro_shift + 32 * ks + 8 * kg);
        }
    }
    v4f_pw acc[TN][TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = v4f_pw{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        uint4 wf[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
            wf[tn] = *reinterpret_cast<const uint4*>(p.w + pw_wrow(tn, i16) * K + 32 * ks + 8 * kg);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = mfma_16x16x32(wf[tn], xf[tm][ks], acc[tn][tm]);
    }
#pragma unroll
    for (int q = 0; q < TN / 2; ++q) {
        const int n = 32 * q + 8 * kg;
        float bv[8];
        pw_bias8(p, n, bv);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            const int64_t m = m_wave + 16 * tm + i16;
            if (m < p.M) pw_store8<EPI>(p, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm]);
        }
    }
}

namespace {

// Narrow outputs (N = 32, 64) with K <= 64 take the LDS-free kernel with 64 pixels per
// wave; the rest the LDS-tiled one with the tile chosen below.  VH_PW_CFG selects a
// variant for measurements: "n<TM>" (narrow, 16 TM pixels per wave, K <= 256),
// "w<BK>" (the earlier fixed tiles, k step 32 or 64) or "t<BM>x<BN>k<BK>o<OCC>".
template <int EPI, bool PRO_ON>
int launch_pw(const PwParams& p, hipStream_t s) {
    constexpr int PRO = PRO_ON ? 1 : 0;
    int narrow_tm = 4, bk = 0;
    bool narrow = (p.N == 32 || p.N == 64) && (p.K == 32 || p.K == 64);
    const bool narrow_ok = (p.N == 32 || p.N == 64) && (p.K == 32 || p.K == 64 || p.K == 128 || p.K == 256);
    if (const char* env = std::getenv("VH_PW_CFG")) {
        if (env[0] == 'n' && narrow_ok) { narrow = true; narrow_tm = std::atoi(env + 1); }
        if (env[0] == 'w') { narrow = false; bk = std::atoi(env + 1); }
    }
    auto go = [&](auto kern, int64_t rows, int cols) {
        const dim3 grid(static_cast<unsigned>((p.M + rows - 1) / rows), static_cast<unsigned>(p.N / cols));
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, p);
        return check_launch("pointwise_gemm_kernel");
    };
    if (narrow) {
        auto pick = [&](auto ks_c) {
            constexpr int KS = decltype(ks_c)::value;
            auto with_tn = [&](auto tn_c) {
                constexpr int TN = decltype(tn_c)::value;
                if (narrow_tm == 1) return go(pointwise_narrow_kernel<KS, TN, 1, EPI, PRO_ON>, 64, p.N);
                if (narrow_tm == 4) return go(pointwise_narrow_kernel<KS, TN, 4, EPI, PRO_ON>, 256, p.N);
                return go(pointwise_narrow_kernel<KS, TN, 2, EPI, PRO_ON>, 128, p.N);
            };
            return p.N == 32 ? with_tn(std::integral_constant<int, 2>{}) : with_tn(std::integral_constant<int, 4>{});
        };
        switch (p.K) {
            case 32: return pick(std::integral_constant<int, 1>{});
            case 64: return pick(std::integral_constant<int, 2>{});
            case 128: return pick(std::integral_constant<int, 4>{});
            default: return pick(std::integral_constant<int, 8>{});
        }
    }
    if (const char* env = std::getenv("VH_PW_CFG")) {
        // t<BM>x<BN>k<BK>o<OCC> (tiled variants for measurements, N % BN == 0)
        int bm = 0, bn = 0, kk = 0, occ = 0;
        if (std::sscanf(env, "t%dx%dk%do%d", &bm, &bn, &kk, &occ) == 4 && p.N % bn == 0) {
#define VH_PWT(BM_, BN_, WGM_, BK_, OCC_)                                                                 \
    if (bm == BM_ && bn == BN_ && kk == BK_ && occ == OCC_)                                              \
        return go(pointwise_gemm_kernel<BM_, BN_, WGM_, BK_, EPI, PRO, OCC_>, BM_, BN_);
            VH_PWT(128, 128, 2, 32, 2) VH_PWT(128, 128, 2, 32, 3) VH_PWT(128, 128, 2, 64, 2)
            VH_PWT(64, 128, 2, 32, 2) VH_PWT(64, 128, 2, 32, 4) VH_PWT(64, 128, 2, 64, 2) VH_PWT(64, 128, 2, 64, 3)
            VH_PWT(128, 64, 2, 32, 4) VH_PWT(256, 128, 4, 32, 2) VH_PWT(128, 256, 2, 32, 1)
#undef VH_PWT
        }
    }
    // The GRN prologue is staged in LDS (PRO 2) when every block spans at most two
    // images (at least BM pixels per image).
    auto tiled = [&](auto bm_c, auto bn_c, auto wgm_c, auto bk_c, auto occ_c) {
        constexpr int BM_ = decltype(bm_c)::value, BN_ = decltype(bn_c)::value, WGM_ = decltype(wgm_c)::value;
        constexpr int BK_ = decltype(bk_c)::value, OCC_ = decltype(occ_c)::value;
        if (PRO_ON && p.rows_per_image.d >= static_cast<uint32_t>(BM_))
            return go(pointwise_gemm_kernel<BM_, BN_, WGM_, BK_, EPI, 2, OCC_>, BM_, BN_);
        return go(pointwise_gemm_kernel<BM_, BN_, WGM_, BK_, EPI, PRO, OCC_>, BM_, BN_);
    };
    if (bk == 0) {
        // Defaults measured on MI355X at the Tiny shapes (B = 128).  Short products want
        // small tiles and many resident blocks (more k tiles in flight per CU); deep
        // ones, 128 x 128 tiles with a 64-deep k step.
        using std::integral_constant;
        if (p.N == 32)
            return tiled(integral_constant<int, 256>{}, integral_constant<int, 32>{}, integral_constant<int, 4>{},
                         integral_constant<int, 32>{}, integral_constant<int, 1>{});
        if (p.N == 64)
            return tiled(integral_constant<int, 128>{}, integral_constant<int, 64>{}, integral_constant<int, 2>{},
                         integral_constant<int, 32>{}, integral_constant<int, 4>{});
        if (p.K <= 128 || (p.K == 256 && p.N >= 512))
            return tiled(integral_constant<int, 64>{}, integral_constant<int, 128>{}, integral_constant<int, 2>{},
                         integral_constant<int, 32>{}, integral_constant<int, 4>{});
        if (p.K == 256)
            return tiled(integral_constant<int, 64>{}, integral_constant<int, 128>{}, integral_constant<int, 2>{},
                         integral_constant<int, 64>{}, integral_constant<int, 2>{});
        return tiled(integral_constant<int, 128>{}, integral_constant<int, 128>{}, integral_constant<int, 2>{},
                     integral_constant<int, 64>{}, integral_constant<int, 2>{});
    }
    if (bk == 32) {
        if (p.N == 32) return go(pointwise_gemm_kernel<256, 32, 4, 32, EPI, PRO>, 256, 32);
        if (p.N == 64) return go(pointwise_gemm_kernel<256, 64, 4, 32, EPI, PRO>, 256, 64);
        return go(pointwise_gemm_kernel<128, 128, 2, 32, EPI, PRO>, 128, 128);
    }
    if (p.N == 32) return go(pointwise_gemm_kernel<256, 32, 4, 64, EPI, PRO>, 256, 32);
    if (p.N == 64) return go(pointwise_gemm_kernel<256, 64, 4, 64, EPI, PRO>, 256, 64);
    return go(pointwise_gemm_kernel<128, 128, 2, 64, EPI, PRO>, 128, 128);
}

}  // namespace
}  // namespace vh

using namespace vh;

extern "C" int vh_pointwise_conv_nhwc_forward(const void* x, int32_t io_dtype, const void* weight,
                                              const float* bias, int32_t epilogue, const void* residual,
                                              const float* grn_scale, const float* grn_beta,
                                              int64_t pixels_per_image, void* out, int64_t M, int64_t N,
                                              int64_t K, void* stream) {
    VH_REQUIRE(x && weight && out, VH_ERR_ARG, "pointwise conv pointers must not be null");
    VH_REQUIRE(io_dtype == VH_DTYPE_BF16, VH_ERR_DTYPE, "pointwise conv supports bf16 tensors only, got code %d",
               io_dtype);
    VH_REQUIRE(M > 0 && N > 0 && K > 0, VH_ERR_SHAPE, "pointwise conv expects nonempty operands");
    VH_REQUIRE(K % 32 == 0 && K <= 65536, VH_ERR_SHAPE, "pointwise conv needs K %% 32 == 0, got %lld", (long long)K);
    VH_REQUIRE(N == 32 || N == 64 || N % 128 == 0, VH_ERR_SHAPE,
               "pointwise conv needs N = 32, 64 or a multiple of 128, got %lld", (long long)N);
    VH_REQUIRE(M * std::max(N, K) < (int64_t(1) << 40), VH_ERR_SHAPE, "pointwise conv operands too large");
    VH_REQUIRE(epilogue >= PW_BIAS && epilogue <= PW_ADD, VH_ERR_ARG, "unknown epilogue %d", epilogue);
    VH_REQUIRE(epilogue != PW_ADD || residual != nullptr, VH_ERR_ARG, "epilogue 2 needs the residual");
    VH_REQUIRE((grn_scale == nullptr) == (grn_beta == nullptr), VH_ERR_ARG,
               "GRN scale and beta must be given together");
    VH_REQUIRE(grn_scale == nullptr || (pixels_per_image > 0 && M % pixels_per_image == 0 && M < (int64_t(1) << 31)),
               VH_ERR_SHAPE, "GRN prologue needs M = images * pixels_per_image < 2^31");
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                            reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(bias) |
                            reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(grn_scale) |
                            reinterpret_cast<uintptr_t>(grn_beta);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "pointwise conv tensors must be 16-byte aligned");
    PwParams p{};
    p.x = static_cast<const bf16_t*>(x);
    p.w = static_cast<const bf16_t*>(weight);
    p.bias = bias;
    p.res = static_cast<const bf16_t*>(residual);
    p.out = static_cast<bf16_t*>(out);
    p.pro_scale = grn_scale;
    p.pro_shift = grn_beta;
    p.M = M;
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.rows_per_image = make_fastdiv(static_cast<uint32_t>(grn_scale ? pixels_per_image : 1));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool pro = grn_scale != nullptr;
    switch (epilogue) {
        case PW_BIAS: return pro ? launch_pw<PW_BIAS, true>(p, s) : launch_pw<PW_BIAS, false>(p, s);
        case PW_GELU: return pro ? launch_pw<PW_GELU, true>(p, s) : launch_pw<PW_GELU, false>(p, s);
        default: return pro ? launch_pw<PW_ADD, true>(p, s) : launch_pw<PW_ADD, false>(p, s);
    }
}
