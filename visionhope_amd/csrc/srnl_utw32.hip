// SRNL chunk scan for head_dim 32 (bf16, fp16 or FP32 activations) in the block form: the algebra of
// srnl_ut.hip (same operand arithmetic) with the 32-wide matrices cut into 2 x 2 tiles of
// 16 x 16 matrix-core products, and the layout of srnl_utw.hip (one workgroup per line, the
// chunk's 16-token blocks spread over its waves).  Reference recurrence:
// models/srnl_core/csrc/inference_recurrence.cuh:32-135, memory.cuh:219-233.
//
//   * one workgroup per line, W waves (the chunk's 16-slot blocks rounded up to a power of
//     two, at most 4: chunks of up to 64 tokens); wave w forms the affine map (X_w, Y_w) of
//     block w: k_t = normalise(M_k x_t), v_t = M_v x_t and the gate pre-activations as two
//     16-feature steps of bf16 products, the triangle L = diag(rho) K^T K diag(kappa) over
//     the 32 features, Z = (I + L)^-1 W K^T by back substitution (32 columns, one lane
//     each), then the four 16 x 16 tiles of X_w = a_15 I - (K D_a) Z and of Y_w^T = -(Delta Z)^T;
//   * the maps compose in order, G^T <- X_w^T G^T + Y_w^T, with tile (I, J) =
//     sum_K (X_w^T)[I][K] (G^T)[K][J] + (Y_w^T)[I][J] on wave 2I + J (mod W), one barrier per
//     block;
//   * the state S = [M_m; M_v; M_k; e; a; 0] (98 rows padded to 112, 32 columns, FP32) lives
//     in LDS; the refresh S <- S G (reference :119-133) runs by 16-row blocks over the waves.
//
// Tiles pass between waves in the accumulator layout (lane 16 q + j: rows 4q..4q+3 of column
// j), which the receiving lane reads back as it was written.  The accumulator layout of a
// tile C is the A-operand layout of C^T and the B-operand layout of C, so X_w's tile (K, I)
// is the A operand of (X_w^T)[I][K].  Slots past the chunk act as the identity.  The
// chunk-start M_m goes to the workspace for the readout, split into bf16 hi + lo pairs for
// spatial maps (p.split_states).
#include "srnl_block_form.h"

namespace vh {
using namespace blockform;

namespace {

// The wave's own LDS writes become visible to its other lanes (wave-private tables).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void st4(float* p, const v4f& v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ void split4(const float4& v, v4s& hi, v4s& lo) {
    const float a[4] = {v.x, v.y, v.z, v.w};
    blockform::split4(a, hi, lo);
}

}  // namespace

template <typename T, int W, bool SPATIAL>
__global__ __launch_bounds__(64 * W) void srnl_scan32_utw_kernel(const ScanParams p) {
    using XQ = XQuad<T>;
    // Row strides are padded (keys 20, L and Z 20, state and G 36 floats) so that the 16-byte
    // loads of 16 lanes down a column of rows fall in different LDS banks; the hand-over
    // tiles are read back by the lane that wrote them, so they are stored lane-major.
    constexpr int D = 32, DKS = 20, TS = 20, SD = 36;
    constexpr int SR = 112;           // state rows: M_m 0-31, M_v 32-63, M_k 64-95, e 96, a 97, zero
    constexpr int XW = W > 1 ? W - 1 : 1;
    __shared__ __align__(16) float kT[W][D * DKS];    // normalised keys [feature][slot]
    __shared__ __align__(16) float ndT[W][D * DKS];   // v - k [feature][slot]
    __shared__ __align__(16) float tk[W][64];         // per slot: rho, kappa, -a_{t-1}, w
    __shared__ __align__(16) float LZ[W][D * TS];     // L[s][t] at [t][s], then Z[s][f] at [f][s]
    __shared__ __align__(16) float Xt[XW][4 * 256];   // waves 1..: X_w tile (K, I) at [2K + I], lane-major
    __shared__ __align__(16) float Yt[XW][4 * 256];   // waves 1..: Y_w^T tile (I, J) at [2I + J], lane-major
    __shared__ __align__(16) float St[SR * SD];       // state rows
    __shared__ __align__(16) float Gr[D * SD];        // chunk gain G, by rows
    __shared__ __align__(16) float G0[4 * 256];       // wave 0: (X_0 + Y_0)^T tile (I, J) at [2I + J], lane-major

    const int tid = static_cast<int>(threadIdx.x);
    const int wv = tid >> 6, lane = tid & 63, i16 = lane & 15, q = lane >> 4;
    const int64_t lines = p.B * p.R * p.heads;
    const int64_t line = xcd_remap(blockIdx.x, lines);
    const int64_t head = line % p.heads;
    const int r = static_cast<int>((line / p.heads) % p.R);
    const int64_t b = line / (p.heads * p.R);
    const int64_t sidx = p.per_line_state ? line : r * p.heads + head;

    for (int idx = tid; idx < SR * D / 4; idx += 64 * W) {
        const int row = idx >> 3, c4 = (idx & 7) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row < 32) v = ld4(p.Mm + sidx * D * D + row * D + c4);
        else if (row < 64) v = ld4(p.Mv + sidx * D * D + (row - 32) * D + c4);
        else if (row < 96) v = ld4(p.Mk + sidx * D * D + (row - 64) * D + c4);
        else if (row == 96) v = ld4(p.Me + sidx * D + c4);
        else if (row == 97) v = ld4(p.Ma + sidx * D + c4);
        *reinterpret_cast<float4*>(St + row * SD + c4) = v;
    }

    const int C = chunk_of(p.chunk, r);
    const int64_t nc = (p.L + C - 1) / C;
    const int nblk = (C + 15) / 16;
    const T* xcol = static_cast<const T*>(p.x.ptr) + b * p.x.sb + r * p.x.sr + head * p.x.sh + 4 * q;
    int pa = 0, pb = 0, pc = 0, pst = 0;
    if constexpr (SPATIAL) {
        const int Wd = static_cast<int>(p.x.W), L = static_cast<int>(p.x.H * p.x.W);
        pa = r == 0 ? Wd : r == 1 ? -Wd : r == 2 ? 1 : -1;
        pb = r == 0 ? 1 : r == 1 ? -1 : r == 2 ? Wd : -Wd;
        pc = (r & 1) ? L - 1 : 0;
        pst = static_cast<int>(p.x.st);
    }
    // x of token (chunk cc, slot 16 wv + i16), features 4q..4q+3 and 16+4q..16+4q+3, as raw
    // bits; slots past the chunk read the line's first token and are zeroed when decoded
    auto load_x = [&](int64_t cc, typename XQ::Raw (&raw)[2], bool& ok) {
        const int slot = 16 * wv + i16;
        const int64_t tok = cc * C + slot;
        ok = slot < C && tok < p.L;
        int64_t off = 0;
        if (ok) {
            if (SPATIAL && p.aligned) off = static_cast<int64_t>(pa * static_cast<int>(cc) + pb * slot + pc) * pst;
            else off = token_offset<SPATIAL>(p.x, r, tok);
        }
        raw[0] = XQ::load(xcol + off);
        raw[1] = XQ::load(xcol + off + 16);
    };
    float* const kTw = kT[wv];
    float* const ndTw = ndT[wv];
    float* const tkw = tk[wv];
    float* const LZw = LZ[wv];

    // x is always loaded one computing chunk ahead, so the only loads in flight when a chunk
    // starts are its own x, issued before the chunk-start store: the wait for them leaves
    // that store outstanding.
    typename XQ::Raw xr[2] = {};
    bool xok = false;
    if (wv < nblk && nc > 1) load_x(0, xr, xok);
    __syncthreads();
    for (int64_t c = 0; c < nc; ++c) {
        // chunk-start M_m for the readout (FP32 or split, p.split_states), a fixed number of
        // stores per thread
#pragma unroll
        for (int k = 0; k < D * D / 4 / (64 * W); ++k) {
            const int idx = tid + 64 * W * k;
            store_state4(p.states + (line * p.max_chunks + c) * D * D + idx * 4, ld4(St + (idx >> 3) * SD + (idx & 7) * 4),
                         p.split_states);
        }
        if (c == nc - 1) break;

        if (wv < nblk) {
            const bool valid = 16 * wv + i16 < C;   // slot inside the chunk (every such token is < L here)
            // ---- token phase: [M_k; M_v] x and (x.e, x.a), two 16-feature steps each ----
            v4s xh[2], xl[2];
            XQ::operands(xr[0], xok, xh[0], xl[0]);
            XQ::operands(xr[1], xok, xh[1], xl[1]);
            // (both 16-feature steps in one 16x16x32 product: the lane's two quads as 8 k)
            v4f kacc[2], vacc[2], gacc;
            const bool on = (i16 & 3) < 2;   // operand rows 4q' + 0 / 4q' + 1: e / a, others zero
            const v4f z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int RB = 0; RB < 2; ++RB) {
                v4s h[2], l[2];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) split4(ld4(St + (64 + 16 * RB + i16) * SD + 16 * kk + 4 * q), h[kk], l[kk]);
                kacc[RB] = XQ::mma_k2(h, l, xh, xl, z4);
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) split4(ld4(St + (32 + 16 * RB + i16) * SD + 16 * kk + 4 * q), h[kk], l[kk]);
                vacc[RB] = XQ::mma_k2(h, l, xh, xl, z4);
            }
            {
                v4s h[2], l[2];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    float4 g4 = ld4(St + (96 + (i16 & 1)) * SD + 16 * kk + 4 * q);
                    if (!on) g4 = make_float4(0.f, 0.f, 0.f, 0.f);
                    split4(g4, h[kk], l[kk]);
                }
                gacc = XQ::mma_k2(h, l, xh, xl, z4);
            }
            // the next computing chunk's x, in flight during the rest of this chunk
            if (c + 1 < nc - 1) load_x(c + 1, xr, xok);
            float kn = 0.f;
#pragma unroll
            for (int RB = 0; RB < 2; ++RB)
#pragma unroll
                for (int j = 0; j < 4; ++j) kn += kacc[RB][j] * kacc[RB][j];
            kn = xor16_32_sum(kn);
            // ||k||^2 of the normalised key is ||k~||^2 / (||k~||^2 + 1e-6)
            const float inv = rsqrtf(kn + 1e-6f);
            const float ksq = kn * inv * inv;
            float kn4[2][4], dsq = 0.f;
#pragma unroll
            for (int RB = 0; RB < 2; ++RB)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float kv = kacc[RB][j] * inv, nd = vacc[RB][j] - kv;
                    kn4[RB][j] = kv;
                    dsq += nd * nd;
                    kTw[(16 * RB + 4 * q + j) * DKS + i16] = kv;
                    ndTw[(16 * RB + 4 * q + j) * DKS + i16] = nd;
                }
            dsq = xor16_32_sum(dsq);
            float alpha, eff;
            token_gates_fast(p.k, gacc[0], gacc[1], dsq, ksq, alpha, eff);   // every lane: token i16
            // Per-slot scalars (srnl_ut.hip): cl = inclusive prefix of log2 alpha over the
            // 16-lane row, a_15 = 2^cl_15, and the triangle's ratio a_{t-1} / a_s split into
            // rho_s = eta^_s 2^(m - cl_s) and kappa_t = 2^(clx_t - m) about m = cl_15 / 2.
            const float la = valid ? __builtin_amdgcn_logf(alpha) : 0.f;
            const float eh = valid ? eff : 0.f;
            float cl = la;
            cl += row_shr<1>(cl);
            cl += row_shr<2>(cl);
            cl += row_shr<4>(cl);
            cl += row_shr<8>(cl);
            const float tot = readlane_f(cl, 15);
            const float decay = __builtin_amdgcn_exp2f(tot), mid = 0.5f * tot, clx = cl - la;
            if (lane < 16) {
                tkw[lane] = eh * __builtin_amdgcn_exp2f(mid - cl);        // rho
                tkw[16 + lane] = __builtin_amdgcn_exp2f(clx - mid);       // kappa
                tkw[32 + lane] = -__builtin_amdgcn_exp2f(clx);            // -a_{t-1}
                tkw[48 + lane] = eh * __builtin_amdgcn_exp2f(tot - cl);   // w
            }
            wave_sync();
            // ---- L = diag(rho) K^T K diag(kappa) over 32 features, strict upper triangle,
            //      by columns ----
            {
                // the Gram tile from the keys split once, scaled after the product
                const float kap = tkw[16 + i16];
                const float4 r4 = ld4(tkw + 4 * q);   // rho of rows 4q..4q+3
                const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
                v4s kh[2], kl[2];
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) blockform::split4(kn4[kk], kh[kk], kl[kk]);
                const v4f P = mma3k2(kh, kl, kh, kl, v4f{0.f, 0.f, 0.f, 0.f});
                float lv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) lv[j] = (4 * q + j < i16) ? (P[j] * rr[j]) * kap : 0.f;
                *reinterpret_cast<float4*>(LZw + i16 * TS + 4 * q) = make_float4(lv[0], lv[1], lv[2], lv[3]);
            }
            wave_sync();
            // ---- Z = (I + L)^-1 W K^T: lane 16 q + i (q < 2) solves column f = 16 q + i from
            //      the last row up, Z[s][f] = w_s k_s[f] - sum_{v > s} L[s][v] Z[v][f]; Z
            //      overwrites L once every lane has read it (one wave, program order) ----
            if (q < 2) {
                const int f = 16 * q + i16;
                float acc[16], zc[16];
#pragma unroll
                for (int s0 = 0; s0 < 16; s0 += 4) {
                    const float4 k4 = ld4(kTw + f * DKS + s0);
                    const float4 w4 = ld4(tkw + 48 + s0);
                    acc[s0] = k4.x * w4.x; acc[s0 + 1] = k4.y * w4.y;
                    acc[s0 + 2] = k4.z * w4.z; acc[s0 + 3] = k4.w * w4.w;
                }
                float lA[4][16], lB[4][16];
                auto load_group = [&](int v0, float (&buf)[4][16]) {
#pragma unroll
                    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
                        for (int s0 = 0; s0 < v0 + dv; s0 += 4) {
                            const float4 l4 = ld4(LZw + (v0 + dv) * TS + s0);
                            buf[dv][s0] = l4.x; buf[dv][s0 + 1] = l4.y; buf[dv][s0 + 2] = l4.z; buf[dv][s0 + 3] = l4.w;
                        }
                };
                auto solve_group = [&](int v0, const float (&buf)[4][16]) {
#pragma unroll
                    for (int dv = 3; dv >= 0; --dv) {
                        const int v = v0 + dv;
                        zc[v] = acc[v];
#pragma unroll
                        for (int s2 = 0; s2 < v; ++s2) acc[s2] -= buf[dv][s2] * zc[v];
                    }
                };
                load_group(12, lA);
                load_group(8, lB);
                solve_group(12, lA);
                load_group(4, lA);
                solve_group(8, lB);
                load_group(0, lB);
                solve_group(4, lA);
                solve_group(0, lB);
#pragma unroll
                for (int s = 0; s < 16; s += 4)
                    *reinterpret_cast<float4*>(LZw + f * TS + s) = make_float4(zc[s], zc[s + 1], zc[s + 2], zc[s + 3]);
            }
            wave_sync();
            // ---- the block's map, tile by tile: X = a_15 I - (K D_a) Z, Y = -Delta Z; wave 0
            //      (the first block, entered with G = I) keeps (X_0 + Y_0)^T, the others hand
            //      over X_w and Y_w^T ----
            {
                const float4 a4 = ld4(tkw + 32 + 4 * q);
                v4s zh[2], zl[2];
                float nka[2][4], ndl[2][4];
#pragma unroll
                for (int F = 0; F < 2; ++F) {
                    split4(ld4(LZw + (16 * F + i16) * TS + 4 * q), zh[F], zl[F]);   // Z[4q + j][16F + i16]
                    const float4 k4 = ld4(kTw + (16 * F + i16) * DKS + 4 * q);
                    const float4 d4 = ld4(ndTw + (16 * F + i16) * DKS + 4 * q);
                    nka[F][0] = k4.x * a4.x; nka[F][1] = k4.y * a4.y; nka[F][2] = k4.z * a4.z; nka[F][3] = k4.w * a4.w;
                    ndl[F][0] = d4.x; ndl[F][1] = d4.y; ndl[F][2] = d4.z; ndl[F][3] = d4.w;
                }
                const v4f dI = diag4(decay, q, i16), z0 = {0.f, 0.f, 0.f, 0.f};
                if (wv == 0) {
                    v4s nbh[2], nbl[2];
#pragma unroll
                    for (int F = 0; F < 2; ++F) {
                        const float nb[4] = {nka[F][0] + ndl[F][0], nka[F][1] + ndl[F][1], nka[F][2] + ndl[F][2],
                                             nka[F][3] + ndl[F][3]};
                        blockform::split4(nb, nbh[F], nbl[F]);
                    }
#pragma unroll
                    for (int I = 0; I < 2; ++I)
#pragma unroll
                        for (int J = 0; J < 2; ++J) {
                            const v4f gT = mma3(zh[I], zl[I], nbh[J], nbl[J], I == J ? dI : z0);   // (X_0 + Y_0)^T
                            // one block: G itself (lane (j, q) of tile (I, J) holds
                            // G[16J + j][16I + 4q..16I + 4q + 3]); else the composition's start
                            if (nblk == 1) st4(Gr + (16 * J + i16) * SD + 16 * I + 4 * q, gT);
                            else st4(G0 + (2 * I + J) * 256 + 4 * lane, gT);
                        }
                } else {
                    v4s kah[2], kal[2], dlh[2], dll[2];
#pragma unroll
                    for (int F = 0; F < 2; ++F) {
                        blockform::split4(nka[F], kah[F], kal[F]);
                        blockform::split4(ndl[F], dlh[F], dll[F]);
                    }
                    float* const xt = Xt[wv - 1];
                    float* const yt = Yt[wv - 1];
#pragma unroll
                    for (int A = 0; A < 2; ++A)
#pragma unroll
                        for (int B = 0; B < 2; ++B) {
                            // X_w tile (A, B); Y_w^T tile (A, B)
                            st4(xt + (2 * A + B) * 256 + 4 * lane, mma3(kah[A], kal[A], zh[B], zl[B], A == B ? dI : z0));
                            st4(yt + (2 * A + B) * 256 + 4 * lane, mma3(zh[A], zl[A], dlh[B], dll[B], z0));
                        }
                }
            }
        }
        __syncthreads();
        // ---- composition, tile (I, J) of G^T on wave 2I + J (mod W):
        //      (G^T)[I][J] <- sum_K (X_w^T)[I][K] (G^T)[K][J] + (Y_w^T)[I][J], one barrier per
        //      block.  Step w writes its tiles over Y_w's (each read only by the wave that
        //      owns the tile); the last step writes G by rows. ----
        {
            const float* gprev = G0;
            for (int w = 1; w < nblk; ++w) {
                if (w > 1) __syncthreads();   // step w - 1's tiles written
                float* const ynext = Yt[w - 1];
                for (int t = wv; t < 4; t += W) {
                    const int I = t >> 1, J = t & 1;
                    v4s gh[2], gl[2], xh[2], xl[2];
#pragma unroll
                    for (int K = 0; K < 2; ++K) {
                        split4(ld4(gprev + (2 * K + J) * 256 + 4 * lane), gh[K], gl[K]);
                        // (X_w^T)[I][K] is the transpose of X_w's tile (K, I)
                        split4(ld4(Xt[w - 1] + (2 * K + I) * 256 + 4 * lane), xh[K], xl[K]);
                    }
                    const float4 y4 = ld4(ynext + t * 256 + 4 * lane);
                    const v4f gT = mma3k2(xh, xl, gh, gl, v4f{y4.x, y4.y, y4.z, y4.w});
                    if (w == nblk - 1) st4(Gr + (16 * J + i16) * SD + 16 * I + 4 * q, gT);
                    else st4(ynext + t * 256 + 4 * lane, gT);
                }
                gprev = ynext;
            }
        }
        __syncthreads();
        // ---- refresh: S <- S G, 16-row blocks over the waves (A: S rows; B: G columns) ----
        {
            v4s gh[2][2], gl[2][2];   // [K][FC]: G[16K + 4q + k][16FC + i16]
#pragma unroll
            for (int K = 0; K < 2; ++K)
#pragma unroll
                for (int FC = 0; FC < 2; ++FC) {
                    float gv[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) gv[k] = Gr[(16 * K + 4 * q + k) * SD + 16 * FC + i16];
                    blockform::split4(gv, gh[K][FC], gl[K][FC]);
                }
            for (int R = wv; R < SR / 16; R += W) {
                v4s sh[2], sl[2];
#pragma unroll
                for (int K = 0; K < 2; ++K) split4(ld4(St + (16 * R + i16) * SD + 16 * K + 4 * q), sh[K], sl[K]);
                v4f sn[2];
#pragma unroll
                for (int FC = 0; FC < 2; ++FC) {
                    const v4s bh[2] = {gh[0][FC], gh[1][FC]}, bl[2] = {gl[0][FC], gl[1][FC]};
                    sn[FC] = mma3k2(sh, sl, bh, bl, v4f{0.f, 0.f, 0.f, 0.f});
                }
#pragma unroll
                for (int FC = 0; FC < 2; ++FC)
#pragma unroll
                    for (int k = 0; k < 4; ++k) St[(16 * R + 4 * q + k) * SD + 16 * FC + i16] = sn[FC][k];
            }
        }
        __syncthreads();
    }
}

// Waves per line of the head_dim-32 block-form scan: the chunk's 16-slot blocks rounded up to
// a power of two; 0 when a chunk exceeds 4 blocks (64 tokens) or the input rows are not
// aligned for vector loads.
int scan32_utw_waves(const ScanParams& sp) {
    int max_chunk = 0;
    for (int r = 0; r < sp.R; ++r) max_chunk = std::max(max_chunk, sp.chunk[r]);
    const int blocks = (max_chunk + 15) / 16;
    if (blocks > 4 || !sp.x_vec) return 0;
    int w = 1;
    while (w < blocks) w *= 2;
    return w;
}

template <typename T>
bool launch_scan32_utw(const ScanParams& sp, hipStream_t stream) {
    const int waves = scan32_utw_waves(sp);
    if (waves == 0) return false;
    const unsigned grid = static_cast<unsigned>(sp.B * sp.R * sp.heads);
    auto go = [&](auto wc, auto spc) {
        constexpr int WV = decltype(wc)::value;
        hipLaunchKernelGGL((srnl_scan32_utw_kernel<T, WV, decltype(spc)::value>), dim3(grid), dim3(64 * WV), 0, stream,
                           sp);
    };
    auto pick = [&](auto spc) {
        switch (waves) {
            case 1: go(std::integral_constant<int, 1>{}, spc); break;
            case 2: go(std::integral_constant<int, 2>{}, spc); break;
            default: go(std::integral_constant<int, 4>{}, spc); break;
        }
    };
    if (sp.x.spatial) pick(std::true_type{});
    else pick(std::false_type{});
    return true;
}

template bool launch_scan32_utw<bf16_t>(const ScanParams&, hipStream_t);
template bool launch_scan32_utw<f16_t>(const ScanParams&, hipStream_t);
template bool launch_scan32_utw<float>(const ScanParams&, hipStream_t);

}  // namespace vh
