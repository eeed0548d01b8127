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

#include "pw_common.h"

namespace vh {

// Block tile BM x BN of the output, k in steps of BK = 64 through LDS (two buffers):
// each thread moves 16-byte chunks global -> registers -> LDS (rows of x and w are
// contiguous in k, so 8 consecutive lanes read one 128-byte row segment), and the
// next tile's loads are in flight while the current one feeds the matrix cores.
// The 4 waves split the tile WGM x WGN; a wave owns WM x WN outputs.  LDS rows are
// padded to 72 elements so the 16 rows of one fragment read fall in distinct banks.
// Output channels are interleaved across pairs of 16-row MFMA tiles (tile 2p row r
// is channel 32p + 8(r/4) + r%4, tile 2p+1 row r is channel 32p + 8(r/4) + 4 + r%4),
// so each lane ends with 8 consecutive channels of one pixel: one 16-byte store.
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
    __shared__ float gtab[EPI == PW_GELU ? GELU_TAB_N : 1];
    if constexpr (EPI == PW_GELU) gelu_tab_fill(gtab, static_cast<int>(threadIdx.x), 256);   // published by the first barrier

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const int wm = wv % WGM, wn = wv / WGM;
    int64_t m0;
    int n0;
    pw_tile<BM, BN>(p, m0, n0);
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
            if (m < p.M) pw_store8<EPI>(p, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm], EPI == PW_GELU ? gtab : nullptr);
        }
    }
}

// ---------------------------------------------------------------------------
// Deep products (K % 64 == 0): the operand tiles go global -> LDS directly
// (global_load_lds_dwordx4, no registers), three k tiles in a ring, so two tiles'
// loads are in flight while the third feeds the matrix cores.  Each wave waits for its
// own copies of the next tile (s_waitcnt vmcnt) and a barrier then publishes them to
// the other waves; the copies are issued from inline assembly, so the compiler's own
// wait insertion (which would drain every copy at each barrier) does not apply and the
// counts below are the complete synchronisation.
// LDS layout: 16-byte chunk c (0..7) of tile row r sits at slot 8r + (c ^ (r & 7)), so
// one wave instruction fills 8 rows (8 lanes per 128-byte row, coalesced) and the 16
// rows of a fragment read fall in distinct bank groups.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void lds_dma16(const void* gptr, uint32_t lds_base) {
    // M0 holds the wave's LDS destination; lane i writes 16 bytes at M0 + 16 i.
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_base)
                 : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmem() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// NI > 0: GRN prologue, the k tile's scale rows of the NI images a block can span (at least
// BM / (NI - 1) pixels per image) and beta staged in LDS with the operand tiles.
// CHAIN (N = BN, bias epilogue): the block's output rows, rounded to bf16 and stored, are
// also written to LDS in the operand layout and multiplied by w2 (N x N, its k tiles
// copied into the ring meanwhile) for out2, the next 1x1 projection of the same pixels,
// with the k order and tile layout of a separate launch of this kernel (the same bits).
template <int BM, int BN, int WGM, int EPI, int NI, int OCC, bool CHAIN = false>
__global__ __launch_bounds__(256, OCC) void pointwise_dma_kernel(const PwParams p) {
    constexpr int BK = 64, WGN = 4 / WGM, WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
    constexpr bool PRO = NI > 0;
    static_assert(TN % 2 == 0 && BM % 32 == 0 && BN % 32 == 0 && NI >= 0 && NI <= 3, "tile shape");
    static_assert(!CHAIN || (NI == 0 && EPI == PW_BIAS && BN % 64 == 0 && BN / 64 <= 3), "chained product");
    static_assert(EPI != PW_ADD_LN || (WGM == 4 && NI == 0 && !CHAIN), "add + LayerNorm: whole pixel rows per wave");
    constexpr int A_INS = BM / 32, B_INS = BN / 32;             // wave instructions per operand and stage
    constexpr int D = A_INS + B_INS + (PRO ? 1 : 0);            // copies per wave and stage
    constexpr int GRN_CPW = (NI + 1) * BK / 16;                 // 16-byte GRN chunks per wave and stage
    constexpr int GRN_BYTES = PRO ? (NI + 1) * BK * 4 : 0;
    constexpr int STAGE = (BM + BN) * BK * 2 + GRN_BYTES;
    // PW_ADD_LN launches have at most two k tiles (K <= 128, checked on the host): two stages
    constexpr int NSTAGE = EPI == PW_ADD_LN ? 2 : 3;
    __shared__ __align__(16) unsigned char lds[NSTAGE * STAGE];
    __shared__ float gtab[EPI == PW_GELU ? GELU_TAB_N : 1];
    if constexpr (EPI == PW_GELU) {
        gelu_tab_fill(gtab, static_cast<int>(threadIdx.x), 256);
        __syncthreads();   // before the copies: their waits below are counted by hand
    }

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const int wm = wv % WGM, wn = wv / WGM;
    int64_t m0;
    int n0;
    pw_tile<BM, BN>(p, m0, n0);
    const int K = p.K, ntiles = K / BK;
    typedef __attribute__((address_space(3))) unsigned char lds_byte;
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_byte*)lds));

    // Source of this lane's chunk in each copy instruction (k offset added per tile).
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;
    const bf16_t* asrc[A_INS];
    const bf16_t* bsrc[B_INS];
#pragma unroll
    for (int i = 0; i < A_INS; ++i) {
        const int64_t m = std::min<int64_t>(m0 + (wv * A_INS + i) * 8 + lrow, p.M - 1);
        asrc[i] = p.x + m * K + 8 * lchunk;
    }
    // B rows in fragment order: LDS row wn WN + 16 tn + i16 holds weight row
    // wn WN + pw_wrow(tn, i16), so a fragment reads 16 consecutive swizzled rows (the
    // permuted rows read in place conflict in the LDS banks).
#pragma unroll
    for (int i = 0; i < B_INS; ++i) {
        const int R = (wv * B_INS + i) * 8 + lrow, rn = R / WN, rr = R % WN;
        bsrc[i] = p.w + static_cast<int64_t>(n0 + rn * WN + pw_wrow(rr / 16, rr % 16)) * K + 8 * lchunk;
    }
    [[maybe_unused]] const float* gsrc = nullptr;
    [[maybe_unused]] int64_t img0 = 0;
    if constexpr (PRO) {
        img0 = fast_div(static_cast<uint32_t>(m0), p.rows_per_image);
        const int64_t last_img = fast_div(static_cast<uint32_t>(p.M - 1), p.rows_per_image);
        const int j = GRN_CPW * wv + std::min(lane, GRN_CPW - 1), which = j / 16, off = 4 * (j % 16);
        gsrc = which < NI ? p.pro_scale + std::min<int64_t>(img0 + which, last_img) * K + off : p.pro_shift + off;
    }
    auto issue = [&](int t) {
        const uint32_t sb = lds0 + (t % 3) * STAGE;
        const int kt = t * BK;
#pragma unroll
        for (int i = 0; i < A_INS; ++i)
            lds_dma16(asrc[i] + kt, __builtin_amdgcn_readfirstlane(sb + (wv * A_INS + i) * 1024));
#pragma unroll
        for (int i = 0; i < B_INS; ++i)
            lds_dma16(bsrc[i] + kt, __builtin_amdgcn_readfirstlane(sb + BM * BK * 2 + (wv * B_INS + i) * 1024));
        if constexpr (PRO) {
            // 16 (NI + 1) chunks of scale (NI image rows) and beta: 4 (NI + 1) per wave.
            if (lane < GRN_CPW)
                lds_dma16(gsrc + kt, __builtin_amdgcn_readfirstlane(sb + (BM + BN) * BK * 2 + wv * GRN_CPW * 16));
        }
    };
    auto slot = [](int r, int c) { return (r * 8 + (c ^ (r & 7))) * 16; };
    int brow[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) brow[tn] = wn * WN + 16 * tn + i16;
    [[maybe_unused]] int rel[TM];
    if constexpr (PRO) {
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

    issue(0);
    if (ntiles > 1) issue(1);
    for (int t = 0; t < ntiles; ++t) {
        if (t + 1 < ntiles) wait_vmem<D>();
        else wait_vmem<0>();
        block_barrier();
        if (t + 2 < ntiles) issue(t + 2);
        const unsigned char* sa = lds + (t % 3) * STAGE;
        const unsigned char* sbp = sa + BM * BK * 2;
        [[maybe_unused]] const float* sg = reinterpret_cast<const float*>(sa + (BM + BN) * BK * 2);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int c = 4 * ks + kg;
            uint4 af[TN], bfr[TM];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) af[tn] = *reinterpret_cast<const uint4*>(sbp + slot(brow[tn], c));
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                bfr[tm] = *reinterpret_cast<const uint4*>(sa + slot(wm * WM + 16 * tm + i16, c));
                if constexpr (PRO) bfr[tm] = grn_apply8(bfr[tm], sg + rel[tm] * BK + 8 * c, sg + NI * BK + 8 * c);
            }
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = mfma_16x16x32(af[tn], bfr[tm], acc[tn][tm]);
        }
    }

    if constexpr (EPI == PW_ADD_LN) {
        // one tile across all N = BN channels (n0 = 0): the pixel's LayerNorm in the epilogue
        v4f_pw a[TN];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) a[tn] = acc[tn][0];
        const int64_t m = m0 + wm * WM + i16;
        pw_add_ln_store<TN / 2>(p, m, m < p.M, kg, a);
        return;
    }
    if constexpr (CHAIN) {
        constexpr int NT2 = BN / 64;   // k tiles of the second product
        // Every wave has consumed its last operand reads (their values fed the products
        // above), so after the barrier the ring is free: w2's k tiles go to the B areas of
        // stages 0 .. NT2 - 1 while this block's output rows go to their A areas.
        block_barrier();
        const int K2 = BN;
#pragma unroll
        for (int kt = 0; kt < NT2; ++kt) {
#pragma unroll
            for (int i = 0; i < B_INS; ++i) {
                const int R = (wv * B_INS + i) * 8 + lrow, rn = R / WN, rr = R % WN;
                const bf16_t* src = p.w2 + static_cast<int64_t>(rn * WN + pw_wrow(rr / 16, rr % 16)) * K2 + 8 * lchunk +
                                    kt * BK;
                lds_dma16(src, __builtin_amdgcn_readfirstlane(lds0 + kt * STAGE + BM * BK * 2 + (wv * B_INS + i) * 1024));
            }
        }
#pragma unroll
        for (int q = 0; q < TN / 2; ++q) {
            const int nl = wn * WN + 32 * q + 8 * kg;   // n0 = 0: the block covers all N = BN outputs
            float bv[8];
            pw_bias8(p, nl, bv);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int r = wm * WM + 16 * tm + i16;
                const int64_t m = m0 + r;
                const v4f_pw& a0 = acc[2 * q][tm];
                const v4f_pw& a1 = acc[2 * q + 1][tm];
                // bf16(acc + bias) as pw_store8 rounds it (two values per conversion)
                const uint4 w = make_uint4(pack_bf16x2(a0[0] + bv[0], a0[1] + bv[1]), pack_bf16x2(a0[2] + bv[2], a0[3] + bv[3]),
                                           pack_bf16x2(a1[0] + bv[4], a1[1] + bv[5]), pack_bf16x2(a1[2] + bv[6], a1[3] + bv[7]));
                if (m < p.M) *reinterpret_cast<uint4*>(p.out + m * p.N + nl) = w;
                *reinterpret_cast<uint4*>(lds + (nl / BK) * STAGE + slot(r, (nl % BK) / 8)) = w;
            }
        }
        wait_vmem<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        block_barrier();
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = v4f_pw{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < NT2; ++kt) {
            const unsigned char* sa = lds + kt * STAGE;
            const unsigned char* sbp = sa + BM * BK * 2;
#pragma unroll
            for (int ks = 0; ks < BK / 32; ++ks) {
                const int c = 4 * ks + kg;
                uint4 af[TN], bfr[TM];
#pragma unroll
                for (int tn = 0; tn < TN; ++tn) af[tn] = *reinterpret_cast<const uint4*>(sbp + slot(brow[tn], c));
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) bfr[tm] = *reinterpret_cast<const uint4*>(sa + slot(wm * WM + 16 * tm + i16, c));
#pragma unroll
                for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                    for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = mfma_16x16x32(af[tn], bfr[tm], acc[tn][tm]);
            }
        }
        PwParams p2 = p;
        p2.bias = p.bias2;
        p2.out = p.out2;
#pragma unroll
        for (int q = 0; q < TN / 2; ++q) {
            const int n = wn * WN + 32 * q + 8 * kg;
            float bv[8];
            pw_bias8(p2, n, bv);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int64_t m = m0 + wm * WM + 16 * tm + i16;
                if (m < p.M) pw_store8<PW_BIAS>(p2, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm]);
            }
        }
        return;
    }

#pragma unroll
    for (int q = 0; q < TN / 2; ++q) {
        const int n = n0 + wn * WN + 32 * q + 8 * kg;
        float bv[8];
        pw_bias8(p, n, bv);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            const int64_t m = m0 + wm * WM + 16 * tm + i16;
            if (m < p.M) pw_store8<EPI>(p, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm], EPI == PW_GELU ? gtab : nullptr);
        }
    }
}

// ---------------------------------------------------------------------------
// Resident weights (K = 64 .. 256 in steps of 64, N a multiple of BN, epilogues without
// a residual): a block owns BN output channels and walks pixel tiles of BM rows with a
// stride of the blocks that share its channels.  Each wave keeps the weight fragments
// of its BN/4 channels in registers for the whole launch (TN x K/32 16-byte fragments
// per lane), so per pixel tile only x moves: global -> LDS directly
// (global_load_lds_dwordx4), two tiles in a ring, the copies of tile i+2 issued as soon
// as every wave has read tile i, so they overlap tile i's epilogue and tile i+1's
// products.  Pixel rows past M are clamped to row M - 1 (loads and stores), so every
// lane issues the same stores on every tile and the wait for tile i+1 is an exact
// count: 2 S + D younger operations (S stores per tile, D copies per tile), vector
// memory operations completing in issue order.  The blocks that share a pixel tile
// are adjacent (consecutive on one XCD), so x is read from HBM about once.
// LDS layout as in pointwise_dma_kernel: 16-byte chunk c of tile row r at slot
// K/8 r + ((c & ~X) | ((c ^ r) & X)), X = 15 for rows of 16 or 32 chunks (K = 128, 256),
// else 7: measured on gfx950 (bank-conflict counter, 16 consecutive rows read at one
// chunk), rows of 256 or 512 bytes conflict with the 3-bit swizzle and not with the
// 4-bit one.
// ---------------------------------------------------------------------------
template <int K, int BN, int BM, int EPI>
__global__ __launch_bounds__(256, 2) void pointwise_resident_kernel(const PwParams p, const int blocks_per_slice) {
    static_assert(K % 64 == 0 && K <= 256 && BN % 128 == 0 && BM % 64 == 0, "resident tile shape");
    static_assert(EPI != PW_ADD, "no residual in this kernel");
    constexpr int WN = BN / 4, TN = WN / 16, TM = BM / 16, KS = K / 32, CPR = K / 8;
    constexpr int TILE = BM * K * 2;                 // bytes
    constexpr int D = BM * CPR / 256;                // copies per lane per tile
    constexpr int S = TM * TN / 2;                   // stores per lane per tile
    constexpr int SWZ = CPR % 16 == 0 ? 15 : 7;      // chunk swizzle mask
    static_assert(D * 256 == BM * CPR && D >= 1, "whole copy instructions");
    __shared__ __align__(16) unsigned char lds[2 * TILE];
    __shared__ float gtab[EPI == PW_GELU ? GELU_TAB_N : 1];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, i16 = lane & 15, kg = lane >> 4;
    const uint32_t slices = static_cast<uint32_t>(p.N / BN);
    const uint32_t l = xcd_remap_any(blockIdx.x, gridDim.x);
    const int n0 = static_cast<int>(l % slices) * BN + wv * WN;   // this wave's first channel
    const int64_t g = l / slices;
    const int64_t mtiles = (p.M + BM - 1) / BM;
    const int ntiles = g < mtiles ? static_cast<int>((mtiles - 1 - g) / blocks_per_slice + 1) : 0;
    if (ntiles == 0) return;   // uniform per block, before any barrier

    // Weights and bias of the wave's channels, held for the whole launch.
    uint4 wf[TN][KS];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            wf[tn][ks] = *reinterpret_cast<const uint4*>(p.w + static_cast<int64_t>(n0 + pw_wrow(tn, i16)) * K +
                                                          32 * ks + 8 * kg);
    float bv[TN / 2][8];
#pragma unroll
    for (int q = 0; q < TN / 2; ++q) pw_bias8(p, n0 + 32 * q + 8 * kg, bv[q]);
    if constexpr (EPI == PW_GELU) {
        gelu_tab_fill(gtab, tid, 256);
        __syncthreads();
    }

    typedef __attribute__((address_space(3))) unsigned char lds_byte;
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_byte*)lds));
    auto issue = [&](int i) {   // copies of this block's i-th tile into ring slot i % 2
        const int64_t m0 = (g + static_cast<int64_t>(i) * blocks_per_slice) * BM;
        const uint32_t sb = lds0 + (i & 1) * TILE;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int slot = (wv * D + d) * 64 + lane, r = slot / CPR, sc = slot % CPR;
            const int c = (sc & ~SWZ) | ((sc ^ r) & SWZ);
            const int64_t m = std::min<int64_t>(m0 + r, p.M - 1);
            lds_dma16(p.x + m * K + 8 * c, __builtin_amdgcn_readfirstlane(sb + (wv * D + d) * 1024));
        }
    };
    auto slot = [](int r, int c) { return (r * CPR + ((c & ~SWZ) | ((c ^ r) & SWZ))) * 16; };

    // Weights and bias in registers before the copies start: the empty statements make
    // the compiler wait for these loads here, outside the loop (it does not see the
    // copies, which the waits below count by hand).
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            asm volatile("" ::"v"(wf[tn][ks].x), "v"(wf[tn][ks].y), "v"(wf[tn][ks].z), "v"(wf[tn][ks].w));
#pragma unroll
    for (int q = 0; q < TN / 2; ++q)
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" ::"v"(bv[q][j]));
    issue(0);
    if (ntiles > 1) issue(1);
    for (int i = 0; i < ntiles; ++i) {
        // Wait for tile i's copies.  Younger operations: for i = 0 tile 1's copies; for
        // i = 1 tile 2's copies and tile 0's stores; for i >= 2 tile i-2's stores, tile
        // i+1's copies and tile i-1's stores (copies only where those tiles exist).
        if (i == 0) {
            if (ntiles > 1) wait_vmem<D>();
            else wait_vmem<0>();
        } else if (i == 1) {
            if (ntiles > 2) wait_vmem<S + D>();
            else wait_vmem<S>();
        } else {
            if (i + 1 < ntiles) wait_vmem<2 * S + D>();
            else wait_vmem<2 * S>();
        }
        block_barrier();
        const unsigned char* a = lds + (i & 1) * TILE;
        v4f_pw acc[TN][TM];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = v4f_pw{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 xf[TM];
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) xf[tm] = *reinterpret_cast<const uint4*>(a + slot(16 * tm + i16, 4 * ks + kg));
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = mfma_16x16x32(wf[tn][ks], xf[tm], acc[tn][tm]);
        }
        if (i + 2 < ntiles) {
            block_barrier();   // every wave has read slot i % 2
            issue(i + 2);
        }
        const int64_t m0 = (g + static_cast<int64_t>(i) * blocks_per_slice) * BM;
#pragma unroll
        for (int q = 0; q < TN / 2; ++q)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int64_t m = std::min<int64_t>(m0 + 16 * tm + i16, p.M - 1);
                pw_store8<EPI>(p, m, n0 + 32 * q + 8 * kg, bv[q], acc[2 * q][tm], acc[2 * q + 1][tm],
                               EPI == PW_GELU ? gtab : nullptr);
            }
    }
}

// Narrow outputs (N = 32 or 64) with K <= 256: no LDS.  A wave owns 16 TM pixels and
// every output channel; it issues all loads of its x rows at once (TM * KS 16-byte
// fragments), reads the small weight fragments through L1 and writes each pixel's
// channels once.
// CHAIN (bias epilogue): out2 = bf16(out @ w2^T + bias2) too, w2 N x N.  A lane ends the
// first product with 8 consecutive channels of one pixel, 32 q + 8 kg .. + 7, which is
// the operand fragment of k step q of the second product for that pixel, so the packed
// bf16 output feeds it directly (the bits a separate launch would load).
template <int KS, int TN, int TM, int EPI, bool PRO, bool CHAIN = false>
__global__ __launch_bounds__(256) void pointwise_narrow_kernel(const PwParams p) {
    static_assert(TN % 2 == 0, "n tiles come in pairs");
    static_assert(!CHAIN || (EPI == PW_BIAS && !PRO), "chained product: bias epilogue, no prologue");
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
    if constexpr (EPI == PW_ADD_LN) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            v4f_pw a[TN];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) a[tn] = acc[tn][tm];
            const int64_t m = m_wave + 16 * tm + i16;
            pw_add_ln_store<TN / 2>(p, m, m < p.M, kg, a);
        }
        return;
    }
    if constexpr (CHAIN) {
        constexpr int K2 = 16 * TN;   // = N
        uint4 yf[TN / 2][TM];         // bf16 output fragments: k step q of the second product
#pragma unroll
        for (int q = 0; q < TN / 2; ++q) {
            const int n = 32 * q + 8 * kg;
            float bv[8];
            pw_bias8(p, n, bv);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const v4f_pw& a0 = acc[2 * q][tm];
                const v4f_pw& a1 = acc[2 * q + 1][tm];
                // bf16(acc + bias) as pw_store8 rounds it (two values per conversion)
                yf[q][tm] = make_uint4(pack_bf16x2(a0[0] + bv[0], a0[1] + bv[1]), pack_bf16x2(a0[2] + bv[2], a0[3] + bv[3]),
                                       pack_bf16x2(a1[0] + bv[4], a1[1] + bv[5]), pack_bf16x2(a1[2] + bv[6], a1[3] + bv[7]));
                const int64_t m = m_wave + 16 * tm + i16;
                if (m < p.M) *reinterpret_cast<uint4*>(p.out + m * p.N + n) = yf[q][tm];
            }
        }
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = v4f_pw{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < TN / 2; ++ks) {
            uint4 wf[TN];
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
                wf[tn] = *reinterpret_cast<const uint4*>(p.w2 + pw_wrow(tn, i16) * K2 + 32 * ks + 8 * kg);
#pragma unroll
            for (int tn = 0; tn < TN; ++tn)
#pragma unroll
                for (int tm = 0; tm < TM; ++tm) acc[tn][tm] = mfma_16x16x32(wf[tn], yf[ks][tm], acc[tn][tm]);
        }
        PwParams p2 = p;
        p2.bias = p.bias2;
        p2.out = p.out2;
#pragma unroll
        for (int q = 0; q < TN / 2; ++q) {
            const int n = 32 * q + 8 * kg;
            float bv[8];
            pw_bias8(p2, n, bv);
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const int64_t m = m_wave + 16 * tm + i16;
                if (m < p.M) pw_store8<PW_BIAS>(p2, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm]);
            }
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < TN / 2; ++q) {
        const int n = 32 * q + 8 * kg;
        float bv[8];
        pw_bias8(p, n, bv);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) {
            const int64_t m = m_wave + 16 * tm + i16;
            if (m < p.M) pw_store8<EPI>(p, m, n, bv, acc[2 * q][tm], acc[2 * q + 1][tm], EPI == PW_GELU ? gelu_tail_table : nullptr);
        }
    }
}

namespace {

// Narrow outputs (N = 32, 64) with K <= 64 take the LDS-free kernel with 64 pixels per
// wave; the rest the LDS-tiled one with the tile chosen below.  The pw_cfg override
// selects a variant for measurements: "n<TM>" (narrow, 16 TM pixels per wave, K <= 256),
// "w<BK>" (the earlier fixed tiles, k step 32 or 64) or "t<BM>x<BN>k<BK>o<OCC>".
template <int EPI, bool PRO_ON>
int launch_pw(const PwParams& p, hipStream_t s) {
    constexpr int PRO = PRO_ON ? 1 : 0;
    int narrow_tm = 4, bk = 0;
    bool narrow = (p.N == 32 || p.N == 64) && (p.K == 32 || p.K == 64);
    const bool narrow_ok = (p.N == 32 || p.N == 64) && (p.K == 32 || p.K == 64 || p.K == 128 || p.K == 256);
    const Override cfg("pw_cfg");
    const char* const env = cfg.set() ? cfg.value : nullptr;
    if (env) {
        if (env[0] == 'n' && narrow_ok) { narrow = true; narrow_tm = std::atoi(env + 1); }
        if (env[0] == 'w') { narrow = false; bk = std::atoi(env + 1); }
    }
    auto go = [&](auto kern, int64_t rows, int cols) {
        const dim3 grid(static_cast<unsigned>((p.M + rows - 1) / rows * (p.N / cols)));
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
    if (env) {
        // d<BM>x<BN>o<OCC>[w<WGM>]: LDS-copy ring kernel (K % 64 == 0, N % BN == 0), the
        // four waves as WGM x (4 / WGM) (default 2, 4 for BM = 256)
        int dm = 0, dn = 0, docc = 0, dw = 0;
        const int dfields = std::sscanf(env, "d%dx%do%dw%d", &dm, &dn, &docc, &dw);
        if (dfields >= 3 && p.N % dn == 0 && p.K % 64 == 0) {
            if (dfields == 3) dw = dm == 256 ? 4 : 2;
            const bool stage_grn = PRO_ON && p.rows_per_image.d >= static_cast<uint32_t>(dm);
#define VH_PWD(BM_, BN_, WGM_, OCC_)                                                                     \
    if (dm == BM_ && dn == BN_ && docc == OCC_ && dw == WGM_ && (stage_grn || !PRO_ON))                  \
        return go(pointwise_dma_kernel<BM_, BN_, WGM_, EPI, PRO_ON ? 2 : 0, OCC_>, BM_, BN_);
            VH_PWD(128, 128, 2, 1) VH_PWD(128, 128, 2, 2) VH_PWD(64, 128, 2, 2) VH_PWD(64, 128, 2, 3)
            VH_PWD(128, 64, 2, 2) VH_PWD(128, 64, 2, 3) VH_PWD(256, 128, 4, 1)
            VH_PWD(64, 128, 4, 2) VH_PWD(64, 128, 4, 3) VH_PWD(128, 128, 4, 2) VH_PWD(128, 64, 4, 3)
#undef VH_PWD
        }
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
    // Resident weights for the shallow products without residual or GRN prologue
    // (fc1 + GELU, the projections): K = 64 .. 256, N a multiple of 128.  Channel
    // slices of 256 up to K = 128, else 128 (the weight fragments take 64 VGPRs), and
    // about 512 blocks (two per CU, one round).  It pays when every block streams a
    // few pixel tiles past its weights: measured on MI355X (Tiny, B = 128) fc1 + GELU
    // 56x56 98 -> 86 us, 28x28 56 -> 49 us, 14x14 42 -> 35 us, proj_out 28x28 11.5 ->
    // 9.6 us, but slower where the pixel tiles x channel slices are fewer than 1024
    // (14x14 and 7x7 projections: the weights are loaded for one or two tiles).
    // The pw_resident override "0" turns it off, "2" takes it wherever the shape allows
    // (tests).
    if constexpr (!PRO_ON && EPI != PW_ADD) {
        const Override res("pw_resident");
        const bool res_off = res.set() && res.value[0] == '0', res_all = res.set() && res.value[0] == '2';
        if (!res_off && bk == 0 && p.K % 64 == 0 && p.K <= 256 && p.N % 128 == 0) {
            const bool wide = p.N % 256 == 0 && p.K <= 128;
            const int64_t slices = p.N / (wide ? 256 : 128), mtiles = (p.M + 63) / 64;
            const int64_t bps = std::max<int64_t>(1, std::min<int64_t>(mtiles, 512 / std::max<int64_t>(1, slices)));
            if ((res_all || mtiles * slices >= 1024) && slices * bps < (int64_t(1) << 31)) {
                const dim3 grid(static_cast<unsigned>(slices * bps));
                auto run = [&](auto kern) {
                    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, p, static_cast<int>(bps));
                    return check_launch("pointwise_resident_kernel");
                };
                switch (p.K) {
                    case 64: return wide ? run(pointwise_resident_kernel<64, 256, 64, EPI>)
                                         : run(pointwise_resident_kernel<64, 128, 64, EPI>);
                    case 128: return wide ? run(pointwise_resident_kernel<128, 256, 64, EPI>)
                                          : run(pointwise_resident_kernel<128, 128, 64, EPI>);
                    case 192: return run(pointwise_resident_kernel<192, 128, 64, EPI>);
                    default: return run(pointwise_resident_kernel<256, 128, 64, EPI>);
                }
            }
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
    if (bk == 0 && p.K % 64 == 0 && p.K >= 128 &&
        ((p.N % 128 != 0 && p.N % 64 == 0) || (p.N % 128 == 0 && (p.K >= 256 || p.N <= 256)))) {
        // Deep products: the LDS-copy ring (measured on MI355X at the Tiny shapes,
        // B = 128: 5-40 % faster than the register-staged tiles from K = 128 up, except
        // K = 128 with N = 512, where the wide output favours the 4-resident tiles).
        // Widths that are multiples of 64 but not of 128 take 64-channel tiles.
        // With the GRN prologue the four waves split the tile 4 x 1 (each wave owns whole
        // pixel rows, so each x fragment is transformed once per block instead of twice),
        // and the block stages the scale rows of the two or three images it can span
        // (measured on MI355X: Tiny 14x14 fc2 34.2 -> 32.0 us, Base 512^2 fc2 at 64x64x768 ->
        // 192 29.9 -> 25.1 us and 32x32x1792 -> 448 36.7 -> 29.1 us; Tiny 7x7 fc2, 49
        // pixels per image, 76 us on the register-staged kernel).
        const bool n64 = p.N % 128 != 0;
        const uint32_t bm = n64 ? 128u : 64u, rpi = p.rows_per_image.d;
        if (!PRO_ON) {
            if (n64) return go(pointwise_dma_kernel<128, 64, 2, EPI, 0, 3>, 128, 64);
            if (p.K >= 1024) return go(pointwise_dma_kernel<64, 128, 2, EPI, 0, 2>, 64, 128);
            return go(pointwise_dma_kernel<64, 128, 2, EPI, 0, 3>, 64, 128);
        }
        if (rpi >= bm) {
            if (n64) return go(pointwise_dma_kernel<128, 64, 4, EPI, 2, 3>, 128, 64);
            return go(pointwise_dma_kernel<64, 128, 4, EPI, 2, 3>, 64, 128);
        }
        if (2 * rpi >= bm) {
            if (n64) return go(pointwise_dma_kernel<128, 64, 4, EPI, 3, 3>, 128, 64);
            return go(pointwise_dma_kernel<64, 128, 4, EPI, 3, 3>, 64, 128);
        }
    }
    if (bk == 0) {
        // Shorter products: register-staged tiles.  They want small tiles and many
        // resident blocks (more k tiles in flight per CU).  Widths that are not multiples
        // of 128 take 32- or 64-channel tiles.
        using std::integral_constant;
        if (p.N % 64 != 0)
            return tiled(integral_constant<int, 256>{}, integral_constant<int, 32>{}, integral_constant<int, 4>{},
                         integral_constant<int, 32>{}, integral_constant<int, 1>{});
        if (p.N % 128 != 0)
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
        if (p.N % 64 != 0) return go(pointwise_gemm_kernel<256, 32, 4, 32, EPI, PRO>, 256, 32);
        if (p.N % 128 != 0) return go(pointwise_gemm_kernel<256, 64, 4, 32, EPI, PRO>, 256, 64);
        return go(pointwise_gemm_kernel<128, 128, 2, 32, EPI, PRO>, 128, 128);
    }
    if (p.N % 64 != 0) return go(pointwise_gemm_kernel<256, 32, 4, 64, EPI, PRO>, 256, 32);
    if (p.N % 128 != 0) return go(pointwise_gemm_kernel<256, 64, 4, 64, EPI, PRO>, 256, 64);
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
    VH_REQUIRE(N % 32 == 0, VH_ERR_SHAPE, "pointwise conv needs N %% 32 == 0, got %lld", (long long)N);
    VH_REQUIRE(M * std::max(N, K) < (int64_t(1) << 40), VH_ERR_SHAPE, "pointwise conv operands too large");
    VH_REQUIRE(epilogue >= PW_BIAS && epilogue <= PW_SILU, VH_ERR_ARG, "unknown epilogue %d", epilogue);
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
        case PW_SILU: return pro ? launch_pw<PW_SILU, true>(p, s) : launch_pw<PW_SILU, false>(p, s);
        default: return pro ? launch_pw<PW_ADD, true>(p, s) : launch_pw<PW_ADD, false>(p, s);
    }
}

extern "C" int vh_pointwise_chain_nhwc_forward(const void* x, const void* weight, const float* bias,
                                               const void* weight2, const float* bias2, void* out, void* out2,
                                               int64_t M, int64_t N, int64_t K, void* stream) {
    VH_REQUIRE(x && weight && weight2 && out && out2, VH_ERR_ARG, "chained pointwise conv pointers must not be null");
    VH_REQUIRE(M > 0 && M < (int64_t(1) << 31), VH_ERR_SHAPE, "chained pointwise conv expects 0 < M < 2^31");
    VH_REQUIRE(((N == 64 || N == 128) && K % 64 == 0 && K >= 64 && K <= 65536) || (N == 32 && (K == 32 || K == 64)),
               VH_ERR_SHAPE, "chained pointwise conv takes N = 64 or 128 with K %% 64 == 0, or N = 32 with K = 32 or 64; "
               "got N = %lld, K = %lld", (long long)N, (long long)K);
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                            reinterpret_cast<uintptr_t>(weight2) | reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(out2) | reinterpret_cast<uintptr_t>(bias) |
                            reinterpret_cast<uintptr_t>(bias2);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "chained pointwise conv tensors must be 16-byte aligned");
    PwParams p{};
    p.x = static_cast<const bf16_t*>(x);
    p.w = static_cast<const bf16_t*>(weight);
    p.bias = bias;
    p.out = static_cast<bf16_t*>(out);
    p.M = M;
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.rows_per_image = make_fastdiv(1u);
    p.w2 = static_cast<const bf16_t*>(weight2);
    p.bias2 = bias2;
    p.out2 = static_cast<bf16_t*>(out2);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The tiles of the separate launches at these widths (64 x 128, 128 x 64 for N = 64, and
    // the LDS-free kernel with 64 pixels per wave for N = 32).
    if (N == 32) {
        const dim3 grid(static_cast<unsigned>((M + 255) / 256));
        if (K == 32) hipLaunchKernelGGL((pointwise_narrow_kernel<1, 2, 4, PW_BIAS, false, true>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((pointwise_narrow_kernel<2, 2, 4, PW_BIAS, false, true>), grid, dim3(256), 0, s, p);
    } else if (N == 128) {
        hipLaunchKernelGGL((pointwise_dma_kernel<64, 128, 2, PW_BIAS, 0, 3, true>),
                           dim3(static_cast<unsigned>((M + 63) / 64)), dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL((pointwise_dma_kernel<128, 64, 2, PW_BIAS, 0, 3, true>),
                           dim3(static_cast<unsigned>((M + 127) / 128)), dim3(256), 0, s, p);
    }
    return check_launch("pointwise_dma_kernel (chained)");
}

extern "C" int vh_pointwise_add_layernorm_nhwc_forward(const void* x, const void* weight, const float* bias,
                                                       const void* residual, const float* ln_weight,
                                                       const float* ln_bias, float eps, void* out_sum, void* out_norm,
                                                       int64_t M, int64_t N, int64_t K, void* stream) {
    VH_REQUIRE(x && weight && residual && ln_weight && ln_bias && out_sum && out_norm, VH_ERR_ARG,
               "pointwise conv + add + LayerNorm pointers must not be null");
    VH_REQUIRE(M > 0 && M < (int64_t(1) << 31), VH_ERR_SHAPE, "pointwise conv + add + LayerNorm expects 0 < M < 2^31");
    VH_REQUIRE((N == 64 && (K == 32 || K == 64)) || ((N == 128 || N == 256) && (K == 64 || K == 128)), VH_ERR_SHAPE,
               "pointwise conv + add + LayerNorm takes N = 64 with K = 32 or 64, or N = 128 or 256 with K = 64 or 128; "
               "got N = %lld, K = %lld", (long long)N, (long long)K);
    VH_REQUIRE(eps > 0.f, VH_ERR_ARG, "LayerNorm eps must be positive");
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                            reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(residual) |
                            reinterpret_cast<uintptr_t>(ln_weight) | reinterpret_cast<uintptr_t>(ln_bias) |
                            reinterpret_cast<uintptr_t>(out_sum) | reinterpret_cast<uintptr_t>(out_norm);
    VH_REQUIRE(align % 16 == 0, VH_ERR_ARG, "pointwise conv + add + LayerNorm tensors must be 16-byte aligned");
    PwParams p{};
    p.x = static_cast<const bf16_t*>(x);
    p.w = static_cast<const bf16_t*>(weight);
    p.bias = bias;
    p.res = static_cast<const bf16_t*>(residual);
    p.out = static_cast<bf16_t*>(out_sum);
    p.M = M;
    p.N = static_cast<int>(N);
    p.K = static_cast<int>(K);
    p.rows_per_image = make_fastdiv(1u);
    p.ln_w = ln_weight;
    p.ln_b = ln_bias;
    p.ln_eps = eps;
    p.ln_out = static_cast<bf16_t*>(out_norm);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (N == 64) {
        // the LDS-free kernel, 64 pixels per wave: all 64 channels of a pixel in four lanes
        const dim3 grid(static_cast<unsigned>((M + 255) / 256));
        if (K == 32) hipLaunchKernelGGL((pointwise_narrow_kernel<1, 4, 4, PW_ADD_LN, false>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((pointwise_narrow_kernel<2, 4, 4, PW_ADD_LN, false>), grid, dim3(256), 0, s, p);
    } else if (N == 128) {
        hipLaunchKernelGGL((pointwise_dma_kernel<64, 128, 4, PW_ADD_LN, 0, 3>), dim3(static_cast<unsigned>((M + 63) / 64)),
                           dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL((pointwise_dma_kernel<64, 256, 4, PW_ADD_LN, 0, 2>), dim3(static_cast<unsigned>((M + 63) / 64)),
                           dim3(256), 0, s, p);
    }
    return check_launch("pointwise conv + add + LayerNorm");
}
