// SRNL recurrence for gfx950: chunk scan + readout.
//
// The recurrence (reference: models/srnl_core/csrc/inference_recurrence.cuh:3-137,
// memory.cuh:219-233) per line (batch b, direction r, head h), head_dim D:
//   state  M_m, M_v, M_k (D x D), e, a (D), all fp32
//   chunk c, token t (chunk-start state):
//     k~ = M_k x, v = M_v x, k = k~ / sqrt(|k~|^2 + 1e-6)
//     eta = s * softplus(clamp(x.e)), alpha = amin + (1-amin) sigmoid(clamp(x.a + bias))
//     eta^ = soft cap of eta by mu (1-alpha) / (|k-v| + 1e-6), clamped to 2m alpha/|k|^2
//     y_t = M_m q_t / max(|q_t|, 1e-12)
//   gain  G = I;  G <- alpha G - eta^ (G k + k - v) k^T  (serial over the chunk)
//   refresh  M <- M G  for m, v, k;  e <- G^T e;  a <- G^T a
//
// MI355X decomposition:
//   * srnl_scan_kernel — one workgroup of 4*D threads per line.  The gain
//     recurrence is row-parallel: row i of G only needs the shared key stream,
//     so each row lives in 4 lanes (D/4 entries each) and a step costs one
//     4-lane butterfly.  Keys/values/gates of a token tile are produced first
//     from the chunk-start state, then consumed by the serial loop.  The scan
//     writes the chunk-start content memory M_m^c of every chunk to the
//     workspace instead of computing y.
//   * readout kernels — y = M_m^c q_hat for every token, fully parallel.  For
//     the spatial operator the readout also restores the four scan orders and
//     fuses sum_r w_r (y_r + skip_r x) per pixel, so no per-direction output
//     ever reaches HBM and no atomics are used.  head_dim 16, and 32 with fp32
//     or bf16 activations, with row/column chunks use 16x16-pixel MFMA tiles
//     (srnl_readout_tile_kernel); every other case one thread per output in the
//     reference's summation order.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <type_traits>

#include "srnl_device.h"

namespace vh {

template <int D>
struct ScanCfg {
    static constexpr int NT = 4 * D;                            // threads per line
    static constexpr int E = D / 4;                             // G entries per thread (4 lanes per row)
    static constexpr int TT = D <= 8 ? NT : (D == 64 ? 32 : 64);  // tokens per tile
    static constexpr int TPT = NT / TT;                         // token-phase threads per token
    static constexpr int RPT = D / TPT;                         // key/value rows per token-phase thread
    static constexpr int ROWS = 3 * D + 2;                      // M_m, M_v, M_k rows, then e, a
    static constexpr int GS = D + 1;                            // padded stride of the gain staging
    static constexpr int NCOLG = NT / D;                        // refresh column groups
    static constexpr int NOUT = (ROWS + NCOLG - 1) / NCOLG;     // refresh rows per thread
};

// Row of D elements starting at p, as fp32.  `vec`: p is 16-byte aligned (8-byte for
// D = 4 with 16-bit elements) so whole rows move with vector loads.
template <typename T, int D>
__device__ __forceinline__ void load_row(const T* p, bool vec, float (&out)[D]) {
    if (vec) {
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int j = 0; j < D; j += 4) {
                const float4 v = *reinterpret_cast<const float4*>(p + j);
                out[j] = v.x; out[j + 1] = v.y; out[j + 2] = v.z; out[j + 3] = v.w;
            }
            return;
        } else if constexpr (D % 8 == 0) {
#pragma unroll
            for (int j = 0; j < D; j += 8) {
                const uint4 v = *reinterpret_cast<const uint4*>(p + j);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    out[j + 2 * h] = to_f32(T{static_cast<uint16_t>(w[h] & 0xffffu)});
                    out[j + 2 * h + 1] = to_f32(T{static_cast<uint16_t>(w[h] >> 16)});
                }
            }
            return;
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(p);
            out[0] = to_f32(T{static_cast<uint16_t>(v.x & 0xffffu)});
            out[1] = to_f32(T{static_cast<uint16_t>(v.x >> 16)});
            out[2] = to_f32(T{static_cast<uint16_t>(v.y & 0xffffu)});
            out[3] = to_f32(T{static_cast<uint16_t>(v.y >> 16)});
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < D; ++j) out[j] = to_f32(p[j]);
}

template <int D>
__device__ __forceinline__ float dot_lds(const float* row, const float (&x)[D]) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < D; j += 4) {
        const float4 s = *reinterpret_cast<const float4*>(row + j);
        acc += s.x * x[j];
        acc += s.y * x[j + 1];
        acc += s.z * x[j + 2];
        acc += s.w * x[j + 3];
    }
    return acc;
}

// Sum over the N consecutive lanes of a group (N a power of two, N <= 8).
template <int N>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = 1; off < N; off <<= 1) v += __shfl_xor(v, off);
    return v;
}

template <int D, typename T>
__global__ __launch_bounds__(4 * D) void srnl_scan_kernel(const ScanParams p) {
    using Cfg = ScanCfg<D>;
    constexpr int NT = Cfg::NT, E = Cfg::E, TT = Cfg::TT, TPT = Cfg::TPT, RPT = Cfg::RPT;
    constexpr int ROWS = Cfg::ROWS, GS = Cfg::GS, NCOLG = Cfg::NCOLG, NOUT = Cfg::NOUT;
    __shared__ __align__(16) float S[ROWS * D];   // state rows
    __shared__ __align__(16) float Gs[D * GS];    // chunk gain staging
    __shared__ __align__(16) float kk[TT * D];    // normalised keys of the tile
    __shared__ __align__(16) float dk[TT * D];    // k - v of the tile
    __shared__ float al_s[TT], et_s[TT];         // retention, projected step

    const int64_t lines = p.B * p.R * p.heads;
    const int64_t line = xcd_remap(blockIdx.x, lines);
    const int64_t head = line % p.heads;
    const int r = static_cast<int>((line / p.heads) % p.R);
    const int64_t b = line / (p.heads * p.R);
    const int64_t s = p.per_line_state ? line : r * p.heads + head;
    const int tid = threadIdx.x;

    for (int idx = tid; idx < D * D; idx += NT) {
        S[idx] = p.Mm[s * D * D + idx];
        S[D * D + idx] = p.Mv[s * D * D + idx];
        S[2 * D * D + idx] = p.Mk[s * D * D + idx];
    }
    for (int idx = tid; idx < D; idx += NT) {
        S[3 * D * D + idx] = p.Me[s * D + idx];
        S[(3 * D + 1) * D + idx] = p.Ma[s * D + idx];
    }

    const int C = chunk_of(p.chunk, r);
    const int64_t nc = (p.L + C - 1) / C;
    const int grow = tid / 4;                 // recurrence: row of G held by this thread
    const int c0 = (tid % 4) * E;             // recurrence: first column held
    const int t_loc = tid / TPT;              // token phase: token of this thread
    const int sub = tid % TPT;                // token phase: row phase of this thread
    const int gcol = tid % D;                 // refresh: column of G held
    const int ggrp = tid / D;                 // refresh: row group
    float* out_states = p.states + line * p.max_chunks * D * D;
    // One wave holds a whole line and owns token t in lane t: gates travel by readlane.
    constexpr bool kLaneGates = TPT == 1 && NT <= 64;
    // Registers for the next tile's x rows (skipped where they would spill).
    constexpr bool kPrefetch = D <= 32;
    float xnext[D];
    bool have_next = false;

    for (int64_t c = 0; c < nc; ++c) {
        __syncthreads();
        for (int idx = tid * 4; idx < D * D; idx += NT * 4)
            store_state4(out_states + c * D * D + idx, *reinterpret_cast<const float4*>(S + idx), p.split_states);
        // The last chunk's gain only feeds a refresh that no output reads.
        if (c == nc - 1) break;

        float g[E];
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = (c0 + e == grow) ? 1.f : 0.f;

        for (int base = 0; base < C; base += TT) {
            const int cnt = min(TT, C - base);
            // ---- token phase: keys, values, gates from the chunk-start state ----
            float xr[D];
            if (kPrefetch && have_next) {
#pragma unroll
                for (int j = 0; j < D; ++j) xr[j] = xnext[j];
            } else {
                const int64_t tok = c * C + base + t_loc;
                if (t_loc < cnt && tok < p.L) load_row<T, D>(line_ptr<T>(p.x, b, r, head, tok), p.x_vec, xr);
                else {
#pragma unroll
                    for (int j = 0; j < D; ++j) xr[j] = 0.f;
                }
            }
            float my_alpha, my_eff;
            {
                float kr[RPT], vr[RPT];
                float kn = 0.f;
#pragma unroll
                for (int m = 0; m < RPT; ++m) {
                    const int i = sub + TPT * m;
                    kr[m] = dot_lds<D>(S + (2 * D + i) * D, xr);
                    vr[m] = dot_lds<D>(S + (D + i) * D, xr);
                    kn += kr[m] * kr[m];
                }
                kn = group_sum<TPT>(kn);
                const float den = sqrtf(kn + 1e-6f);
                float dsq = 0.f, ksq = 0.f;
#pragma unroll
                for (int m = 0; m < RPT; ++m) {
                    const float kv = kr[m] / den;
                    kr[m] = kv;
                    vr[m] = kv - vr[m];
                    dsq += vr[m] * vr[m];
                    ksq += kv * kv;
                }
                dsq = group_sum<TPT>(dsq);
                ksq = group_sum<TPT>(ksq);
                float ep = dot_lds<D>(S + 3 * D * D, xr);
                float ap = dot_lds<D>(S + (3 * D + 1) * D, xr);
                ep = fminf(10.f, fmaxf(-10.f, ep));
                ap = fminf(10.f, fmaxf(-10.f, ap + p.k.alpha_bias));
                const float sp = ep > 20.f ? ep : logf(1.f + expf(ep));
                const float eta = p.k.eta_scale * sp;
                const float alpha = p.k.alpha_min + (1.f - p.k.alpha_min) * (1.f / (1.f + expf(-ap)));
                const float dn = sqrtf(dsq + 1e-12f);
                const float cap = p.k.stab_mu * (1.f - alpha) / (dn + 1e-6f);
                float eff = cap * (-expm1f(-(eta / cap)));
                if (p.k.clamp) eff = fminf(eff, nextafterf(p.k.factor * alpha / fmaxf(ksq, 1e-20f), 0.f));
                my_alpha = alpha;
                my_eff = eff;
                if (t_loc < cnt) {
#pragma unroll
                    for (int m = 0; m < RPT; ++m) {
                        kk[t_loc * D + sub + TPT * m] = kr[m];
                        dk[t_loc * D + sub + TPT * m] = vr[m];
                    }
                    if (!kLaneGates && sub == 0) {
                        al_s[t_loc] = alpha;
                        et_s[t_loc] = eff;
                    }
                }
            }
            // ---- prefetch the x rows of the next tile (the next chunk's first tile
            //      if this is the last one); their loads overlap the recurrence ----
            if constexpr (kPrefetch) {
                int64_t nc_idx = c, nbase = base + TT;
                if (nbase >= C) { nc_idx = c + 1; nbase = 0; }
                have_next = nc_idx < nc - 1;
                if (have_next) {
                    const int ncnt = min(TT, C - static_cast<int>(nbase));
                    const int64_t tok = nc_idx * C + nbase + t_loc;
                    if (t_loc < ncnt && tok < p.L)
                        load_row<T, D>(line_ptr<T>(p.x, b, r, head, tok), p.x_vec, xnext);
                    else {
#pragma unroll
                        for (int j = 0; j < D; ++j) xnext[j] = 0.f;
                    }
                }
            }
            __syncthreads();
            // ---- serial gain recurrence: 4 lanes per row of G; operands of the next
            //      U tokens are read from LDS while the current U are processed ----
            constexpr int U = 4;
            float kvb[U][E], dfb[U], alb[U], etb[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int t = min(u, cnt - 1);
#pragma unroll
                for (int e = 0; e < E; ++e) kvb[u][e] = kk[t * D + c0 + e];
                dfb[u] = dk[t * D + grow];
                if constexpr (!kLaneGates) {
                    alb[u] = al_s[t];
                    etb[u] = et_s[t];
                }
            }
            for (int t0 = 0; t0 < cnt; t0 += U) {
                float kvn[U][E], dfn[U], aln[U], etn[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int t = min(t0 + U + u, cnt - 1);
#pragma unroll
                    for (int e = 0; e < E; ++e) kvn[u][e] = kk[t * D + c0 + e];
                    dfn[u] = dk[t * D + grow];
                    if constexpr (!kLaneGates) {
                        aln[u] = al_s[t];
                        etn[u] = et_s[t];
                    }
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if (t0 + u < cnt) {
                        float alpha, eta;
                        if constexpr (kLaneGates) {
                            // token t0+u was produced by lane t0+u: broadcast to all lanes
                            alpha = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_alpha), t0 + u));
                            eta = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_eff), t0 + u));
                        } else {
                            alpha = alb[u];
                            eta = etb[u];
                        }
                        float dot = 0.f;
#pragma unroll
                        for (int e = 0; e < E; ++e) dot += g[e] * kvb[u][e];
                        dot += quad_swap1(dot);
                        dot += quad_swap2(dot);
                        const float coef = eta * (dfb[u] + dot);
#pragma unroll
                        for (int e = 0; e < E; ++e) g[e] = alpha * g[e] - coef * kvb[u][e];
                    }
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
#pragma unroll
                    for (int e = 0; e < E; ++e) kvb[u][e] = kvn[u][e];
                    dfb[u] = dfn[u];
                    alb[u] = aln[u];
                    etb[u] = etn[u];
                }
            }
            __syncthreads();
        }
        // ---- refresh: S <- S G (all 3D+2 rows) ----
#pragma unroll
        for (int e = 0; e < E; ++e) Gs[grow * GS + c0 + e] = g[e];
        __syncthreads();
        float outv[NOUT];
        if constexpr (D <= 16) {
            // Column of G in registers, state rows as LDS broadcasts.
            float gc[D];
#pragma unroll
            for (int l = 0; l < D; ++l) gc[l] = Gs[l * GS + gcol];
#pragma unroll
            for (int m = 0; m < NOUT; ++m) {
                const int rr = ggrp + NCOLG * m;
                outv[m] = rr < ROWS ? dot_lds<D>(S + rr * D, gc) : 0.f;
            }
        } else {
            // Large heads: both operands from LDS (a register copy of the column spills).
#pragma unroll
            for (int m = 0; m < NOUT; ++m) outv[m] = 0.f;
#pragma unroll 4
            for (int l = 0; l < D; ++l) {
                const float gl = Gs[l * GS + gcol];
#pragma unroll
                for (int m = 0; m < NOUT; ++m) {
                    const int rr = ggrp + NCOLG * m;
                    if (rr < ROWS) outv[m] += S[rr * D + l] * gl;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < NOUT; ++m) {
            const int rr = ggrp + NCOLG * m;
            if (rr < ROWS) S[rr * D + gcol] = outv[m];
        }
    }
}

// ---------------------------------------------------------------------------
// head_dim 16: one wave per line, projections and refresh on MFMA.
//
// v_mfma_f32_16x16x4_f32 lane layout (wave64): lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; the 16x16 result lands in lane l as rows 4(l/16)..4(l/16)+3 of
// column l%16.  A K=16 product runs as 4 steps; step s takes logical index
// 4(l/16)+s from lane l, so every lane reads 4 consecutive values of a row.
//
//   token phase  [K~ ; V] (32 x 64 tokens) = [M_k ; M_v] (32 x 16) . X (16 x 64)
//                -> lane l ends up with rows 4q..4q+3 (q = l/16) of tokens
//                   16T + l%16, T = 0..3: norms reduce over the 4 lane groups.
//   refresh      S (64 x 16, 50 rows used) <- S . G
// The serial gain recurrence stays on the VALU (4 lanes per row of G).
// ---------------------------------------------------------------------------
// NL lines per wave (NL in {1, 2, 4}) and TCW column tiles of 16 token slots per wave
// (TCW in {2, 4}, NL <= TCW): the NL lines share (b, r) and take consecutive heads.
// Each tile gives every line S = 16 TCW / NL token slots; lane l < 16 TCW owns slot
// l % S of line l / S for the per-token work (the other lanes idle there), and MFMA
// column tile tc belongs to line tc / (TCW / NL).  G of every line is spread over 64/NL
// lanes, RL = 4/NL lanes per row, E = 4 NL entries per lane, so a row dot needs
// log2(RL) DPP steps.  Packing lines lets short chunks (row length 14 or 7) fill the
// token slots; two tiles per wave instead of four halve the wave's token work and
// double the number of waves, so two waves share each SIMD and hide each other's
// latency when the lines would otherwise give one wave per SIMD.
template <typename T, int NL, int TCW, bool SPATIAL>
__global__ __launch_bounds__(64) void srnl_scan16_kernel(const ScanParams p) {
    static_assert((TCW == 2 || TCW == 4) && NL <= TCW, "tile packing");
    constexpr int D = 16, TT = 16 * TCW, ROWS = 3 * D + 2, GS = D + 1, DKS = TT + 4;
    constexpr int S = TT / NL, TPL = TCW / NL, RL = 4 / NL, E = D / RL, SR = 64 * D;
    constexpr int NU = NL == 1 ? 1 : TCW;   // state sets the column tiles read
    __shared__ __align__(16) float St[NL * SR];       // per line: 50 state rows + zero rows
    __shared__ __align__(16) float Gs[NL * D * GS];
    __shared__ __align__(16) float kk[TT * D];        // normalised keys [slot][16]
    __shared__ __align__(16) float dkT[D * DKS];      // (k - v)[row][slot]
    __shared__ __align__(16) float cf[TT * 8];        // block coefficients per slot

    const int64_t groups = p.B * p.R * p.heads / NL;
    const int64_t line0 = xcd_remap(blockIdx.x, groups) * NL;
    const int64_t head0 = line0 % p.heads;
    const int r = static_cast<int>((line0 / p.heads) % p.R);
    const int64_t b = line0 / (p.heads * p.R);
    const int lane = threadIdx.x;
    const int i16 = lane & 15, q = lane >> 4;

#pragma unroll
    for (int lam = 0; lam < NL; ++lam) {
        const int64_t s = p.per_line_state ? line0 + lam : r * p.heads + head0 + lam;
        float* Sl = St + lam * SR;
        for (int idx = lane; idx < D * D; idx += 64) {
            Sl[idx] = p.Mm[s * D * D + idx];
            Sl[D * D + idx] = p.Mv[s * D * D + idx];
            Sl[2 * D * D + idx] = p.Mk[s * D * D + idx];
        }
        if (lane < D) {
            Sl[3 * D * D + lane] = p.Me[s * D + lane];
            Sl[(3 * D + 1) * D + lane] = p.Ma[s * D + lane];
        }
        for (int idx = ROWS * D + lane; idx < SR; idx += 64) Sl[idx] = 0.f;
    }

    const int C = chunk_of(p.chunk, r);
    const int64_t nc = (p.L + C - 1) / C;
    const int lam_g = lane / (16 * RL);                 // recurrence layout
    const int grow = (lane % (16 * RL)) / RL, c0 = (lane % RL) * E;
    const int my_slot = lane % S;
    const bool slot_lane = lane < TT;
    const T* xcol[TCW];
#pragma unroll
    for (int tc = 0; tc < TCW; ++tc)
        xcol[tc] = static_cast<const T*>(p.x.ptr) + b * p.x.sb + r * p.x.sr + (head0 + tc / TPL) * p.x.sh + 4 * q;

    // x operands of a tile move as raw bits: the loads are issued without a branch
    // (invalid slots read their line's first token) and decoded only where used, so a
    // prefetch never waits for memory before the work it overlaps.
    using Raw = typename std::conditional<sizeof(T) == 4, uint4, uint2>::type;
    Raw xr_next[TCW];
    unsigned valid_next = 0;
    bool have_next = false;
    // Row/column chunks (the spatial operator): token i of chunk cc of scan r is pixel
    // pa*cc + pb*i + pc, an affine map with per-scan constants (no division, no branch).
    // 32-bit: the host enables row/column addressing only when H*W*pixel_stride < 2^31.
    int pa = 0, pb = 0, pc = 0, pst = 0;
    if constexpr (SPATIAL) {
        const int W = static_cast<int>(p.x.W), L = static_cast<int>(p.x.H * p.x.W);
        pa = r == 0 ? W : r == 1 ? -W : r == 2 ? 1 : -1;
        pb = r == 0 ? 1 : r == 1 ? -1 : r == 2 ? W : -W;
        pc = (r & 1) ? L - 1 : 0;
        pst = static_cast<int>(p.x.st);
    }
    auto issue_tile = [&](int64_t cc, int base, int cnt, Raw (&raw)[TCW], unsigned& valid) {
        valid = 0;
        int64_t offs[TCW];
        if (SPATIAL && p.aligned) {
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                const int slot = (tc % TPL) * 16 + i16;
                const bool ok = slot < cnt && cc * C + base + slot < p.L;
                valid |= ok ? (1u << tc) : 0u;
                offs[tc] = ok ? (pa * static_cast<int>(cc) + pb * (base + slot) + pc) * pst : 0;
            }
        } else {
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                const int slot = (tc % TPL) * 16 + i16;
                const int64_t tok = cc * C + base + slot;
                const bool ok = slot < cnt && tok < p.L;
                valid |= ok ? (1u << tc) : 0u;
                offs[tc] = ok ? token_offset<SPATIAL>(p.x, r, tok) : 0;   // invalid: the line's first token
            }
        }
        if (p.x_vec) {
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) raw[tc] = *reinterpret_cast<const Raw*>(xcol[tc] + offs[tc]);
        } else {
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                const T* src = xcol[tc] + offs[tc];
                if constexpr (sizeof(T) == 4) {
                    raw[tc] = make_uint4(__float_as_uint(src[0]), __float_as_uint(src[1]), __float_as_uint(src[2]),
                                         __float_as_uint(src[3]));
                } else {
                    raw[tc] = make_uint2(static_cast<uint32_t>(src[0].bits) | (static_cast<uint32_t>(src[1].bits) << 16),
                                         static_cast<uint32_t>(src[2].bits) | (static_cast<uint32_t>(src[3].bits) << 16));
                }
            }
        }
    };
    auto decode_tile = [&](const Raw (&raw)[TCW], unsigned valid, float (&xo)[TCW][4]) {
#pragma unroll
        for (int tc = 0; tc < TCW; ++tc) {
            float v[4];
            if constexpr (sizeof(T) == 4) {
                v[0] = __uint_as_float(raw[tc].x); v[1] = __uint_as_float(raw[tc].y);
                v[2] = __uint_as_float(raw[tc].z); v[3] = __uint_as_float(raw[tc].w);
            } else {
                v[0] = to_f32(T{static_cast<uint16_t>(raw[tc].x & 0xffffu)});
                v[1] = to_f32(T{static_cast<uint16_t>(raw[tc].x >> 16)});
                v[2] = to_f32(T{static_cast<uint16_t>(raw[tc].y & 0xffffu)});
                v[3] = to_f32(T{static_cast<uint16_t>(raw[tc].y >> 16)});
            }
            const bool ok = (valid >> tc) & 1u;
#pragma unroll
            for (int j = 0; j < 4; ++j) xo[tc][j] = ok ? v[j] : 0.f;
        }
    };

    for (int64_t c = 0; c < nc; ++c) {
        __syncthreads();
#pragma unroll
        for (int lam = 0; lam < NL; ++lam)
            store_state4(p.states + ((line0 + lam) * p.max_chunks + c) * D * D + lane * 4,
                         *reinterpret_cast<const float4*>(St + lam * SR + lane * 4), p.split_states);
        if (c == nc - 1) break;

        float g[E];
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = (c0 + e == grow) ? 1.f : 0.f;

        for (int base = 0; base < C; base += S) {
            const int cnt = min(S, C - base);
            float xo[TCW][4];
            if (!have_next) issue_tile(c, base, cnt, xr_next, valid_next);
            decode_tile(xr_next, valid_next, xo);
            // ---- projections on MFMA, norms per token; then each lane computes the
            //      gates of its own slot ----
            // All four column tiles at once (no control flow between them), so their
            // MFMA chains and reductions overlap instead of running back to back.  A
            // column tile without tokens sees x = 0 and yields zero keys and differences.
            float ak[NU][4], av[NU][4], ev[NU][4], aa[NU][4];
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const float* Sl = St + (u / TPL) * SR;
                const float4 k4 = *reinterpret_cast<const float4*>(Sl + (2 * D + i16) * D + 4 * q);
                const float4 v4 = *reinterpret_cast<const float4*>(Sl + (D + i16) * D + 4 * q);
                const float4 e4 = *reinterpret_cast<const float4*>(Sl + 3 * D * D + 4 * q);
                const float4 a4 = *reinterpret_cast<const float4*>(Sl + (3 * D + 1) * D + 4 * q);
                ak[u][0] = k4.x; ak[u][1] = k4.y; ak[u][2] = k4.z; ak[u][3] = k4.w;
                av[u][0] = v4.x; av[u][1] = v4.y; av[u][2] = v4.z; av[u][3] = v4.w;
                ev[u][0] = e4.x; ev[u][1] = e4.y; ev[u][2] = e4.z; ev[u][3] = e4.w;
                aa[u][0] = a4.x; aa[u][1] = a4.y; aa[u][2] = a4.z; aa[u][3] = a4.w;
            }
            v4f kacc[TCW], vacc[TCW];
            float pe[TCW], pa[TCW];
            // bf16: the gate pre-activations x.e and x.a come from a third product whose
            // operand rows 4q and 4q+1 are e and a (the rest zero), so every lane of token
            // column i16 receives them in accumulator entries 0 and 1, with no reduction.
            constexpr bool kMfmaBf16 = std::is_same<T, bf16_t>::value;
            [[maybe_unused]] v4s akh[NU], akl[NU], avh[NU], avl[NU], gh[NU], gl[NU];
            if constexpr (kMfmaBf16) {
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    split_bf16(ak[u], akh[u], akl[u]);
                    split_bf16(av[u], avh[u], avl[u]);
                    // state rows 48 (e), 49 (a) and 50 (zero) by the lane's operand row i16
                    const float4 g4 = *reinterpret_cast<const float4*>(
                        St + (u / TPL) * SR + (3 * D + min(i16 & 3, 2)) * D + 4 * q);
                    const float ga[4] = {g4.x, g4.y, g4.z, g4.w};
                    split_bf16(ga, gh[u], gl[u]);
                }
            }
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                const int u = NU == 1 ? 0 : tc;
                kacc[tc] = v4f{0.f, 0.f, 0.f, 0.f};
                vacc[tc] = v4f{0.f, 0.f, 0.f, 0.f};
                if constexpr (std::is_same<T, bf16_t>::value) {
                    // x is bf16 (exact); M_k, M_v enter as hi + lo.  xr_next still holds this tile.
                    const v4s xs = ((valid_next >> tc) & 1u) ? bf16x4_bits(xr_next[tc]) : v4s{0, 0, 0, 0};
                    kacc[tc] = mfma_bf16(akh[u], xs, kacc[tc]);
                    vacc[tc] = mfma_bf16(avh[u], xs, vacc[tc]);
                    kacc[tc] = mfma_bf16(akl[u], xs, kacc[tc]);
                    vacc[tc] = mfma_bf16(avl[u], xs, vacc[tc]);
                    v4f gacc = mfma_bf16(gh[u], xs, v4f{0.f, 0.f, 0.f, 0.f});
                    gacc = mfma_bf16(gl[u], xs, gacc);
                    pe[tc] = gacc[0];
                    pa[tc] = gacc[1];
                } else {
#pragma unroll
                    for (int st = 0; st < 4; ++st) {
                        kacc[tc] = mfma4(ak[u][st], xo[tc][st], kacc[tc]);
                        vacc[tc] = mfma4(av[u][st], xo[tc][st], vacc[tc]);
                    }
                    pe[tc] = ev[u][0] * xo[tc][0] + ev[u][1] * xo[tc][1] + ev[u][2] * xo[tc][2] + ev[u][3] * xo[tc][3];
                    pa[tc] = aa[u][0] * xo[tc][0] + aa[u][1] * xo[tc][1] + aa[u][2] * xo[tc][2] + aa[u][3] * xo[tc][3];
                }
            }
            float kn[TCW];
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                kn[tc] = kacc[tc][0] * kacc[tc][0] + kacc[tc][1] * kacc[tc][1] + kacc[tc][2] * kacc[tc][2] +
                         kacc[tc][3] * kacc[tc][3];
                kn[tc] = xor16_32_sum(kn[tc]);
                if constexpr (!kMfmaBf16) {
                    pe[tc] = xor16_32_sum(pe[tc]);
                    pa[tc] = xor16_32_sum(pa[tc]);
                }
            }
            // ||k||^2 of the normalised key is ||k~||^2 / (||k~||^2 + 1e-6), taken from the
            // reduced norm instead of a second reduction.
            float dsq[TCW], ksq[TCW];
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                const float inv = rsqrtf(kn[tc] + 1e-6f);
                float kv[4], df[4];
                dsq[tc] = 0.f;
                ksq[tc] = kn[tc] * inv * inv;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    kv[j] = kacc[tc][j] * inv;
                    df[j] = kv[j] - vacc[tc][j];
                    dsq[tc] += df[j] * df[j];
                }
                const int t = 16 * tc + i16;
                *reinterpret_cast<float4*>(kk + t * D + 4 * q) = make_float4(kv[0], kv[1], kv[2], kv[3]);
#pragma unroll
                for (int j = 0; j < 4; ++j) dkT[(4 * q + j) * DKS + t] = df[j];
            }
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) dsq[tc] = xor16_32_sum(dsq[tc]);
            // Lane 16 tc + i16 owns the token of column i16 of tile tc (lanes past the
            // tiles take tile 0's values and are masked below).
#define VH_OWN(v) (TCW == 4 ? (q == 0 ? v[0] : q == 1 ? v[1] : q == 2 ? v[2 % TCW] : v[3 % TCW]) \
                             : (q == 1 ? v[1] : v[0]))
            const float tok_ksq = VH_OWN(ksq), tok_dsq = VH_OWN(dsq), tok_ep = VH_OWN(pe), tok_ap = VH_OWN(pa);
#undef VH_OWN
            float my_alpha, my_eff;
            {
                float alpha, eff;
                token_gates_fast(p.k, tok_ep, tok_ap, tok_dsq, tok_ksq, alpha, eff);
                my_alpha = alpha;
                my_eff = eff;
            }
            // ---- prefetch the next tile's x operands ----
            {
                int64_t ncc = c;
                int nbase = base + S;
                if (nbase >= C) { ncc = c + 1; nbase = 0; }
                have_next = ncc < nc - 1;
                if (have_next) issue_tile(ncc, nbase, min(S, C - nbase), xr_next, valid_next);
            }
            __syncthreads();
            // ---- block coefficients: slots 4u..4u+3 of a line are the lanes of one DPP
            //      quad.  With A_j = prod_{s<=j} alpha_s inside the block,
            //        r_j = A_{j-1} (g.k_j) + delta_j - sum_{s<j} beta_sj r_s
            //        g  <- A_3 g - sum_s w_s r_s k_s
            //      beta_sj = (A_{j-1}/A_s) eta_s (k_s.k_j), w_s = (A_3/A_s) eta_s.
            //      Slots past the chunk act as the identity (alpha 1, eta 0). ----
            {
                const bool valid = slot_lane && my_slot < cnt;
                const float al_t = valid ? my_alpha : 1.f;
                const float et_t = valid ? my_eff : 0.f;
                const int j = lane & 3;
                const float pa1 = quad_perm<0x90>(al_t), pa2 = quad_perm<0x40>(al_t), pa3 = quad_perm<0x00>(al_t);
                const float pe1 = quad_perm<0x90>(et_t), pe2 = quad_perm<0x40>(et_t), pe3 = quad_perm<0x00>(et_t);
                const float na1 = quad_perm<0xF9>(al_t), na2 = quad_perm<0xFE>(al_t), na3 = quad_perm<0xFF>(al_t);
                float kd1 = 0.f, kd2 = 0.f, kd3 = 0.f;
                {
                    const int t0 = min(lane, TT - 1);
                    const int t1 = max(t0 - 1, 0), t2 = max(t0 - 2, 0), t3 = max(t0 - 3, 0);
#pragma unroll
                    for (int e = 0; e < D; e += 4) {
                        const float4 k0 = *reinterpret_cast<const float4*>(kk + t0 * D + e);
                        const float4 k1 = *reinterpret_cast<const float4*>(kk + t1 * D + e);
                        const float4 k2 = *reinterpret_cast<const float4*>(kk + t2 * D + e);
                        const float4 k3 = *reinterpret_cast<const float4*>(kk + t3 * D + e);
                        kd1 += k0.x * k1.x + k0.y * k1.y + k0.z * k1.z + k0.w * k1.w;
                        kd2 += k0.x * k2.x + k0.y * k2.y + k0.z * k2.z + k0.w * k2.w;
                        kd3 += k0.x * k3.x + k0.y * k3.y + k0.z * k3.z + k0.w * k3.w;
                    }
                }
                float cf_a = 1.f;
                if (j >= 1) cf_a *= pa1;
                if (j >= 2) cf_a *= pa2;
                if (j >= 3) cf_a *= pa3;
                const float cf_b1 = pe1 * kd1;
                const float cf_b2 = pe2 * kd2 * pa1;
                const float cf_b3 = pe3 * kd3 * pa2 * pa1;
                float cf_w = et_t;
                if (j <= 2) cf_w *= na1;
                if (j <= 1) cf_w *= na2;
                if (j == 0) cf_w *= na3;
                const float cf_A3 = quad_perm<0x00>(al_t) * quad_perm<0x55>(al_t) * quad_perm<0xAA>(al_t) *
                                    quad_perm<0xFF>(al_t);
                if (slot_lane) {
                    *reinterpret_cast<float4*>(cf + lane * 8) = make_float4(cf_a, cf_b1, cf_b2, cf_b3);
                    *reinterpret_cast<float4*>(cf + lane * 8 + 4) = make_float4(cf_w, cf_A3, 0.f, 0.f);
                }
            }
            __syncthreads();
            // ---- serial recurrence, 4 tokens per step; the operands of the next step
            //      are read from LDS while the current one computes (two register sets
            //      used alternately, so no copies between steps) ----
            struct StepOps {
                float kv[4][E];
                float df[4];
                float c0v[4][4];   // slots 1..3: a, beta_{j-1,j}, beta_{j-2,j}, beta_{j-3,j}
                float c1v[4][2];   // every slot: w; slot 0: A_3 of the block
            };
            StepOps opA, opB;
            auto fetch = [&](int t, StepOps& o) {
                const int tn = lam_g * S + min(t, S - 4);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
#pragma unroll
                    for (int e = 0; e < E; e += 4) {
                        const float4 k4 = *reinterpret_cast<const float4*>(kk + (tn + u) * D + c0 + e);
                        o.kv[u][e] = k4.x; o.kv[u][e + 1] = k4.y; o.kv[u][e + 2] = k4.z; o.kv[u][e + 3] = k4.w;
                    }
                    if (u > 0) {
                        const float4 a4 = *reinterpret_cast<const float4*>(cf + (tn + u) * 8);
                        o.c0v[u][0] = a4.x; o.c0v[u][1] = a4.y; o.c0v[u][2] = a4.z; o.c0v[u][3] = a4.w;
                    }
                    const float2 w2 = *reinterpret_cast<const float2*>(cf + (tn + u) * 8 + 4);
                    o.c1v[u][0] = w2.x; o.c1v[u][1] = w2.y;
                }
                const float4 d4 = *reinterpret_cast<const float4*>(dkT + grow * DKS + tn);
                o.df[0] = d4.x; o.df[1] = d4.y; o.df[2] = d4.z; o.df[3] = d4.w;
            };
            auto step = [&](const StepOps& o) {
                float pdot[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    float d;
                    if constexpr (E <= 4) {
                        d = g[0] * o.kv[u][0];
#pragma unroll
                        for (int e = 1; e < E; ++e) d += g[e] * o.kv[u][e];
                    } else {
                        float d0 = g[0] * o.kv[u][0];
                        float d1 = g[1] * o.kv[u][1];
#pragma unroll
                        for (int e = 2; e < E; e += 2) {
                            d0 += g[e] * o.kv[u][e];
                            d1 += g[e + 1] * o.kv[u][e + 1];
                        }
                        d = d0 + d1;
                    }
                    if constexpr (RL >= 2) d += quad_swap1(d);
                    if constexpr (RL == 4) d += quad_swap2(d);
                    pdot[u] = d;
                }
                const float r0 = pdot[0] + o.df[0];
                const float r1 = o.c0v[1][0] * pdot[1] + o.df[1] - o.c0v[1][1] * r0;
                const float r2 = o.c0v[2][0] * pdot[2] + o.df[2] - o.c0v[2][2] * r0 - o.c0v[2][1] * r1;
                const float r3 = o.c0v[3][0] * pdot[3] + o.df[3] - o.c0v[3][3] * r0 - o.c0v[3][2] * r1 -
                                 o.c0v[3][1] * r2;
                const float A3 = o.c1v[0][1];
                const float c0r = o.c1v[0][0] * r0, c1r = o.c1v[1][0] * r1, c2r = o.c1v[2][0] * r2,
                            c3r = o.c1v[3][0] * r3;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    float v = A3 * g[e] - c0r * o.kv[0][e];
                    v -= c1r * o.kv[1][e];
                    v -= c2r * o.kv[2][e];
                    g[e] = v - c3r * o.kv[3][e];
                }
            };
            // Pin freshly read operands in registers once the step between has run, so
            // the compiler cannot turn them back into LDS reads next to their use.
            auto pin = [&](StepOps& o) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
#pragma unroll
                    for (int e = 0; e < E; ++e) asm volatile("" : "+v"(o.kv[u][e]));
#pragma unroll
                    for (int m = 0; m < 4; ++m) asm volatile("" : "+v"(o.c0v[u][m]));
                    asm volatile("" : "+v"(o.c1v[u][0]), "+v"(o.c1v[u][1]), "+v"(o.df[u]));
                }
            };
            fetch(0, opA);
            for (int t0 = 0; t0 < cnt; t0 += 8) {
                fetch(t0 + 4, opB);
                __builtin_amdgcn_sched_barrier(0);
                step(opA);
                pin(opB);
                if (t0 + 4 >= cnt) break;
                fetch(t0 + 8, opA);
                __builtin_amdgcn_sched_barrier(0);
                step(opB);
                pin(opA);
            }
            __syncthreads();
        }
        // ---- refresh on MFMA: S <- S G for every line ----
#pragma unroll
        for (int e = 0; e < E; ++e) Gs[lam_g * D * GS + grow * GS + c0 + e] = g[e];
        __syncthreads();
        v4f acc[NL][4];
#pragma unroll
        for (int lam = 0; lam < NL; ++lam) {
            float bg[4];
#pragma unroll
            for (int st = 0; st < 4; ++st) bg[st] = Gs[lam * D * GS + (4 * q + st) * GS + i16];
#pragma unroll
            for (int R = 0; R < 4; ++R) {
                const float4 a4 = *reinterpret_cast<const float4*>(St + lam * SR + (16 * R + i16) * D + 4 * q);
                const float a[4] = {a4.x, a4.y, a4.z, a4.w};
                acc[lam][R] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4; ++st) acc[lam][R] = mfma4(a[st], bg[st], acc[lam][R]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int lam = 0; lam < NL; ++lam)
#pragma unroll
            for (int R = 0; R < 4; ++R)
#pragma unroll
                for (int j = 0; j < 4; ++j) St[lam * SR + (16 * R + 4 * q + j) * D + i16] = acc[lam][R][j];
    }
}

// ---------------------------------------------------------------------------
// Spatial readout + four-direction fusion, one thread per output element.
// ---------------------------------------------------------------------------
template <int D, typename T, typename TO>
__global__ __launch_bounds__(256) void srnl_fuse_readout_kernel(const FuseParams p) {
    const int64_t L = p.H * p.W;
    const int64_t total = p.B * L * p.C;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    const int64_t c = idx % p.C;
    const int64_t pix = (idx / p.C) % L;
    const int64_t b = idx / (L * p.C);
    const int64_t head = c / D;
    const int i = static_cast<int>(c % D);
    const int64_t h = pix / p.W, w = pix % p.W;
    const T* xq = static_cast<const T*>(p.x);
    const T* qq = static_cast<const T*>(p.q);

    float qv[D];
    float qinv = 0.f;
    float xval = 0.f;
    if (!p.per_direction) {
        const T* qrow = qq + (b * L + pix) * p.C + head * D;
        float qn = 0.f;
#pragma unroll
        for (int j = 0; j < D; ++j) {
            qv[j] = to_f32(qrow[j]);
            qn += qv[j] * qv[j];
        }
        qinv = 1.f / fmaxf(sqrtf(qn), 1e-12f);
        xval = to_f32(xq[(b * L + pix) * p.C + c]);
    }
    float acc = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t t = pixel_to_scan(r, h, w, p.H, p.W);
        if (p.per_direction) {
            const T* qrow = qq + ((b * 4 + r) * L + t) * p.C + head * D;
            float qn = 0.f;
#pragma unroll
            for (int j = 0; j < D; ++j) {
                qv[j] = to_f32(qrow[j]);
                qn += qv[j] * qv[j];
            }
            qinv = 1.f / fmaxf(sqrtf(qn), 1e-12f);
            xval = to_f32(xq[((b * 4 + r) * L + t) * p.C + c]);
        }
        const int64_t ch = t / chunk_of(p.chunk, r);
        const float* m = p.states + (((b * 4 + r) * p.heads + head) * p.max_chunks + ch) * D * D + i * D;
        float dot = 0.f;
        if (p.split_states) {
#pragma unroll
            for (int j = 0; j < D; ++j) dot += split_state_at(m, j) * qv[j];
        } else {
#pragma unroll
            for (int j = 0; j < D; ++j) dot += m[j] * qv[j];
        }
        const float y = dot * qinv;
        const float contrib = y + p.skip[(p.skip_per_dir ? r * p.C : 0) + c] * xval;
        const float weighted = p.wgt[r * p.C + c] * contrib;
        acc = r == 0 ? weighted : acc + weighted;
    }
    if (p.aux) acc += to_f32(static_cast<const T*>(p.aux)[idx]);
    static_cast<TO*>(p.out)[idx] = from_f32<TO>(acc);
}

// ---------------------------------------------------------------------------
// Spatial readout + fusion for head_dim 16 with row/column chunks (W, W, H, H).
//
// One workgroup of four waves per 16x16-pixel tile of one (image, head).  Every
// pixel of a tile row reads the same direction-0/1 states (chunks h and H-1-h) and
// every pixel of a tile column the same direction-2/3 states (chunks w and W-1-w),
// so each y = M q over 16 pixels is one 16x16x16 product on the matrix cores:
//   step m of four 16x16x4 MFMAs: lane l = 16g + n supplies A = M[n][4g+m] and
//   B = q[pixel n][4g+m] (k permuted so both operands are 4-vector loads) and
//   receives D[4g+j][n], channels 4g..4g+3 of pixel n.
// Wave v takes tile columns 4v..4v+3 (directions 2, 3) and then tile rows 4v..4v+3
// (directions 0, 1); column contributions go through LDS to move pixels onto the
// row layout; each output is then (c0 + c1) + (c2 + c3) with c_r = w_r (y_r +
// skip_r x), stored once.  Loads are branch-free (positions past the image edge
// read the edge pixel and are never stored), so every load of a wave's four
// columns or rows is in flight at once, and the row loads are issued before the
// column work.
// ---------------------------------------------------------------------------
template <typename T>
struct Pix4 {   // 4 channels of one pixel as raw bits
    using Raw = typename std::conditional<sizeof(T) == 4, uint4, uint2>::type;
};

template <typename T>
__device__ __forceinline__ void raw4_to_f32(const typename Pix4<T>::Raw& r, float (&v)[4]) {
    if constexpr (sizeof(T) == 4) {
        v[0] = __uint_as_float(r.x); v[1] = __uint_as_float(r.y); v[2] = __uint_as_float(r.z); v[3] = __uint_as_float(r.w);
    } else {
        v[0] = to_f32(T{static_cast<uint16_t>(r.x & 0xffffu)});
        v[1] = to_f32(T{static_cast<uint16_t>(r.x >> 16)});
        v[2] = to_f32(T{static_cast<uint16_t>(r.y & 0xffffu)});
        v[3] = to_f32(T{static_cast<uint16_t>(r.y >> 16)});
    }
}

// Sum of squares of a lane's D/4 query channels (raw bits).
template <typename T, int D>
__device__ __forceinline__ float xraw_sumsq(const XRaw<T, D>& r) {
    float s = 0.f;
    float v[D / 4];
    decode_x<T, D>(r, v);
#pragma unroll
    for (int j = 0; j < D / 4; ++j) s += v[j] * v[j];
    return s;
}

// y = M q~ for 16 pixels on the matrix cores: lane l = 16 g + n gives M row n (of the
// 16-channel half) and pixel n's query over the K-range [g D/4, (g+1) D/4), and receives
// channels 4g..4g+3 of the half for pixel n.  bf16: M as hi + lo, q exact.
// SPLIT (bf16, D = 16 or 32): m holds the bits of the stored bf16 hi[4], lo[4] pairs (one
// pair per 4 entries).
template <typename T, int D, bool SPLIT = false>
__device__ __forceinline__ v4f readout_mfma(const float (&m)[D / 4], const XRaw<T, D>& qr) {
    v4f y = {0.f, 0.f, 0.f, 0.f};
    if constexpr (SPLIT && D == 16) {
        static_assert(std::is_same<T, bf16_t>::value, "split states: bf16");
        const v4s hi = __builtin_bit_cast(v4s, make_uint2(__float_as_uint(m[0]), __float_as_uint(m[1])));
        const v4s lo = __builtin_bit_cast(v4s, make_uint2(__float_as_uint(m[2]), __float_as_uint(m[3])));
        const v4s qs = bf16x4_bits(qr.v);
        y = mfma_bf16x2(hi, lo, qs, qs, y);   // (hi + lo) q in one 16x16x32 product
    } else if constexpr (SPLIT) {
        static_assert(std::is_same<T, bf16_t>::value && D == 32, "split states: bf16, head_dim 16 or 32");
        // entries 8g..8g+3 then 8g+4..8g+7: hi of both groups, then lo of both
        const v8bf hi = __builtin_bit_cast(v8bf, make_uint4(__float_as_uint(m[0]), __float_as_uint(m[1]),
                                                            __float_as_uint(m[4]), __float_as_uint(m[5])));
        const v8bf lo = __builtin_bit_cast(v8bf, make_uint4(__float_as_uint(m[2]), __float_as_uint(m[3]),
                                                            __float_as_uint(m[6]), __float_as_uint(m[7])));
        const auto qs = BfOp<32>::exact(qr);
        y = BfOp<32>::mma(lo, qs, BfOp<32>::mma(hi, qs, y));   // two 16x16x32 products
    } else if constexpr (std::is_same<T, bf16_t>::value) {
        using Bf = BfOp<D>;
        typename Bf::type hi, lo;
        Bf::split(m, hi, lo);
        const auto qs = Bf::exact(qr);
        y = Bf::mma_pair(hi, lo, qs, qs, y);
    } else {
        float qv[D / 4];
        decode_x<T, D>(qr, qv);
#pragma unroll
        for (int j = 0; j < D / 4; ++j) y = mfma4(m[j], qv[j], y);
    }
    return y;
}

// ---------------------------------------------------------------------------
// Spatial readout + fusion for head_dim 16 or 32 with row/column chunks (W, W, H, H).
//
// One workgroup of four waves per 16x16-pixel tile of one (image, head).  Every pixel of
// a tile row reads the same direction-0/1 states (chunks h and H-1-h) and every pixel of
// a tile column the same direction-2/3 states (chunks w and W-1-w), so each y = M q over
// 16 pixels and a 16-channel half of the head is one matrix-core product (K = head_dim).
// Wave v takes tile columns 4v..4v+3 (directions 2, 3) and then tile rows 4v..4v+3
// (directions 0, 1); column contributions go through LDS to move pixels onto the row
// layout; each output is (c0 + c1) + (c2 + c3) with c_r = w_r (y_r + skip_r x), stored
// once.  Loads are branch-free (positions past the image edge read the edge pixel and
// are never stored), so every load of a wave's four columns or rows is in flight at
// once, and the row loads are issued before the column work.  head_dim 32 runs the two
// 16-channel halves in two workgroups.  TP = 8 (maps of at most 8 x 8): 8 x 8-pixel tiles,
// two rows and two columns per wave, so a 7 x 7 map issues half the loads of a 16 x 16
// tile (the 16-pixel product still runs; the lanes past the tile store nothing).
//
// LEPE: the block's local position encoding, a 5x5 depthwise convolution of x (zero
// padding) plus bias, rounded to T and added to the result, is computed here instead of
// in a separate pass (models/block.py:77-78).  The tile's 16 channels of x with a
// two-pixel halo are loaded at the start (held in registers over the column pass) and
// staged raw in LDS; thread (channel, tile column) then convolves TP or TP / 2 rows with
// its channel's 25 taps in registers, each output accumulated from the bias in tap-row
// order, left to right (the order of the depthwise kernels, so the value is the one
// they store), and hands the rounded results to the row pass through the same LDS.
// ---------------------------------------------------------------------------
template <typename T, typename TO, int D, bool SPLIT = false, int TP = 16, bool LEPE = false>
__global__ __launch_bounds__(256) void srnl_readout_tile_kernel(const FuseParams p, const int64_t tiles_h,
                                                                const int64_t tiles_w) {
    static_assert(TP == 16 || TP == 8, "tile size");
    constexpr int REC = 20, PER = TP / 4, KQ = D / 4;   // 16 channels + 4 padding floats per pixel record
    using Raw = typename Pix4<T>::Raw;
    __shared__ __align__(16) float col[256 * REC];
    // LEPE: halo tile of HP x HP pixels x 16 channels (raw T), later the rounded results
    constexpr int HP = TP + 4, HALO_Q = HP * HP * 4, HALO_IT = (HALO_Q + 255) / 256;
    constexpr int LRP = TP * TP / 16;              // rows per thread in the convolution
    __shared__ __align__(16) Raw halo[LEPE ? HALO_Q : 1];
    // Tile indices fit 32 bits (the host checks the grid size).  head_dim 32: two
    // workgroups per tile, one per 16-channel half (the halves' registers do not share a
    // wave, so more waves stay resident).
    constexpr int NH = D / 16;
    const uint32_t thw = static_cast<uint32_t>(tiles_h * tiles_w), ntw = static_cast<uint32_t>(tiles_w);
    const uint32_t wg = xcd_remap_any(blockIdx.x, gridDim.x);
    const uint32_t tile = wg / NH;
    const int my_half = static_cast<int>(wg % NH);
    const uint32_t bh = tile / thw, in_img = tile - bh * thw;
    const uint32_t th = in_img / ntw, tw = in_img - th * ntw;
    const uint32_t heads = static_cast<uint32_t>(p.heads);
    const int64_t head = bh % heads, b = bh / heads;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, n = lane & 15, g = lane >> 4;
    const int H = static_cast<int>(p.H), W = static_cast<int>(p.W);
    const int64_t C = p.C, L = p.H * p.W;
    const int Ci = static_cast<int>(C);
    const int h0 = static_cast<int>(th) * TP, w0 = static_cast<int>(tw) * TP;
    // Workgroup-uniform bases and 32-bit lane offsets (the host requires H * W * C < 2^31
    // and per-line state blocks below 2^31 floats), so loads take a scalar base.
    const int64_t img = b * L * C + head * D;
    const T* qb = static_cast<const T*>(p.q) + img;
    const float* st[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) st[r] = p.states + ((b * 4 + r) * p.heads + head) * p.max_chunks * (D * D);
    auto pix = [&](int h, int w) { return (h * W + w) * Ci; };
    auto load_q = [&](int h, int w) { return load_xraw<T, D>(qb + (pix(h, w) + KQ * g)); };
    auto load_m = [&](const float* base, int chunk, int row, float (&m)[KQ]) {
        const float* src = base + (chunk * (D * D) + row * D + KQ * g);
#pragma unroll
        for (int j = 0; j < KQ; j += 4) {
            const float4 f = *reinterpret_cast<const float4*>(src + j);
            m[j] = f.x; m[j + 1] = f.y; m[j + 2] = f.z; m[j + 3] = f.w;
        }
    };
    const int wr = min(w0 + n, W - 1), hc = min(h0 + n, H - 1);
    {
        const int half = my_half;
        const int64_t cbase = head * D + 16 * half + 4 * g;   // this lane's 4 output channels
        const int cl = 16 * half + 4 * g;                      // ... relative to the head
        const T* xb = static_cast<const T*>(p.x) + img;
        const int mrow = 16 * half + n;                        // M row of this lane (A operand)

        // LEPE halo: quad e % 4 of pixel e / 4 of the HP x HP tile, zeros outside the image.
        [[maybe_unused]] Raw hraw[LEPE ? HALO_IT : 1];
        if constexpr (LEPE) {
#pragma unroll
            for (int i = 0; i < HALO_IT; ++i) {
                const int e = static_cast<int>(threadIdx.x) + 256 * i, px = e >> 2;
                const int hy = h0 - 2 + px / HP, wx = w0 - 2 + px % HP;
                hraw[i] = Raw{};
                if (e < HALO_Q && hy >= 0 && hy < H && wx >= 0 && wx < W)
                    hraw[i] = *reinterpret_cast<const Raw*>(xb + (pix(hy, wx) + 16 * half + 4 * (e & 3)));
            }
        }
        // Row pass operands (directions 0, 1): tile row hh = 4 wv + k, lane n holds pixel
        // (h0 + hh, w0 + n).  Issued first; consumed after the column pass.
        XRaw<T, D> rq[PER];
        Raw rx[PER];
        float m0[PER][KQ], m1[PER][KQ];
        [[maybe_unused]] Raw ra[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int h = min(h0 + PER * wv + k, H - 1);
            rq[k] = load_q(h, wr);
            rx[k] = *reinterpret_cast<const Raw*>(xb + (pix(h, wr) + cl));
            load_m(st[0], h, mrow, m0[k]);
            load_m(st[1], H - 1 - h, mrow, m1[k]);
            if (!LEPE && p.aux) ra[k] = *reinterpret_cast<const Raw*>(static_cast<const T*>(p.aux) + img + (pix(h, wr) + cl));
        }

        // Column pass (directions 2, 3): tile column ww = 4 wv + k, lane n holds pixel
        // (h0 + n, w0 + ww).
        float wt[4][4], sk[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float4 w4 = *reinterpret_cast<const float4*>(p.wgt + r * C + cbase);
            const float4 s4 = *reinterpret_cast<const float4*>(p.skip + (p.skip_per_dir ? r * C : 0) + cbase);
            wt[r][0] = w4.x; wt[r][1] = w4.y; wt[r][2] = w4.z; wt[r][3] = w4.w;
            sk[r][0] = s4.x; sk[r][1] = s4.y; sk[r][2] = s4.z; sk[r][3] = s4.w;
        }
        {
            XRaw<T, D> cq[PER];
            Raw cx[PER];
            float m2[PER][KQ], m3[PER][KQ];
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int w = min(w0 + PER * wv + k, W - 1);
                cq[k] = load_q(hc, w);
                cx[k] = *reinterpret_cast<const Raw*>(xb + (pix(hc, w) + cl));
                load_m(st[2], w, mrow, m2[k]);
                load_m(st[3], W - 1 - w, mrow, m3[k]);
            }
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                float xv[4];
                raw4_to_f32<T>(cx[k], xv);
                // 1 / max(|q|, 1e-12) = rsqrt(max(|q|^2, 1e-24)) (hardware reciprocal square root)
                const float inv = __builtin_amdgcn_rsqf(fmaxf(xor16_32_sum(xraw_sumsq<T, D>(cq[k])), 1e-24f));
                const v4f y2 = readout_mfma<T, D, SPLIT>(m2[k], cq[k]);
                const v4f y3 = readout_mfma<T, D, SPLIT>(m3[k], cq[k]);
                float c23[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    c23[j] = wt[2][j] * (y2[j] * inv + sk[2][j] * xv[j]) + wt[3][j] * (y3[j] * inv + sk[3][j] * xv[j]);
                *reinterpret_cast<float4*>(col + ((PER * wv + k) * 16 + n) * REC + 4 * g) =
                    make_float4(c23[0], c23[1], c23[2], c23[3]);
            }
        }
        if constexpr (LEPE) {
#pragma unroll
            for (int i = 0; i < HALO_IT; ++i) {
                const int e = static_cast<int>(threadIdx.x) + 256 * i;
                if (e < HALO_Q) halo[e] = hraw[i];
            }
        }
        __syncthreads();
        [[maybe_unused]] float lepe[PER][4];
        if constexpr (LEPE) {
            // Thread t: channel c = t % 16 of the half, tile column x = (t / 16) % TP, rows
            // LRP (t / 16 / TP) .. + LRP - 1.  Halo row r feeds output row k through tap
            // row r - k, so visiting r in order adds each output's terms row by row.
            const int c = static_cast<int>(threadIdx.x) & 15, rest = static_cast<int>(threadIdx.x) >> 4;
            const int x = rest % TP, r0 = LRP * (rest / TP);
            const int64_t cg = head * D + 16 * half + c;
            float tap[25];
#pragma unroll
            for (int i = 0; i < 25; ++i) tap[i] = p.lepe_taps[i * C + cg];
            const float bias = p.lepe_bias ? p.lepe_bias[cg] : 0.f;
            float acc[LRP];
#pragma unroll
            for (int k = 0; k < LRP; ++k) acc[k] = bias;
            const auto* hv = reinterpret_cast<const std::conditional_t<sizeof(T) == 4, float, uint16_t>*>(halo);
#pragma unroll
            for (int r = 0; r < LRP + 4; ++r) {
                float v[5];
#pragma unroll
                for (int dx = 0; dx < 5; ++dx) {
                    const auto u = hv[((r0 + r) * HP + x + dx) * 16 + c];
                    if constexpr (sizeof(T) == 4) v[dx] = u;
                    else v[dx] = to_f32(T{u});
                }
#pragma unroll
                for (int k = 0; k < LRP; ++k) {
                    const int dy = r - k;
                    if (dy >= 0 && dy < 5) {
#pragma unroll
                        for (int dx = 0; dx < 5; ++dx) acc[k] = fmaf(v[dx], tap[dy * 5 + dx], acc[k]);
                    }
                }
            }
            __syncthreads();   // every halo read done: the results overwrite it
            auto* res = reinterpret_cast<std::conditional_t<sizeof(T) == 4, float, uint16_t>*>(halo);
#pragma unroll
            for (int k = 0; k < LRP; ++k) {
                const int at = ((r0 + k) * TP + x) * 16 + c;
                if constexpr (sizeof(T) == 4) {
                    res[at] = acc[k];
                } else {
                    // the FP32 sum first, then T (as the depthwise kernel stores it): the
                    // empty asm keeps the last multiply-add from fusing with the conversion
                    // into one multiply-add that rounds to fp16 directly
                    float a = acc[k];
                    asm volatile("" : "+v"(a));
                    res[at] = from_f32<T>(a).bits;
                }
            }
            __syncthreads();
            // this lane's 4 channels of its row-pass pixels (lanes past an 8-wide tile read
            // column TP - 1 and store nothing)
            const int xn = min(n, TP - 1);
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const Raw rr = *reinterpret_cast<const Raw*>(res + ((PER * wv + k) * TP + xn) * 16 + 4 * g);
                raw4_to_f32<T>(rr, lepe[k]);
            }
        }

        const int w = w0 + n;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int hh = PER * wv + k, h = h0 + hh;
            float xv[4];
            raw4_to_f32<T>(rx[k], xv);
            const float inv = __builtin_amdgcn_rsqf(fmaxf(xor16_32_sum(xraw_sumsq<T, D>(rq[k])), 1e-24f));
            const v4f y0 = readout_mfma<T, D, SPLIT>(m0[k], rq[k]);
            const v4f y1 = readout_mfma<T, D, SPLIT>(m1[k], rq[k]);
            const float4 c23 = *reinterpret_cast<const float4*>(col + (n * 16 + hh) * REC + 4 * g);
            const float c23v[4] = {c23.x, c23.y, c23.z, c23.w};
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = (wt[0][j] * (y0[j] * inv + sk[0][j] * xv[j]) + wt[1][j] * (y1[j] * inv + sk[1][j] * xv[j])) +
                       c23v[j];
            if constexpr (LEPE) {
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] += lepe[k][j];
            } else if (p.aux) {
                float a[4];
                raw4_to_f32<T>(ra[k], a);
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] += a[j];
            }
            if (h < H && w < W && n < TP) {
                const int64_t at = img + (pix(h, w) + cl);
                if constexpr (sizeof(TO) == 4) {
                    *reinterpret_cast<float4*>(static_cast<float*>(p.out) + at) = make_float4(o[0], o[1], o[2], o[3]);
                } else if constexpr (std::is_same<TO, bf16_t>::value) {
                    *reinterpret_cast<uint2*>(static_cast<TO*>(p.out) + at) =
                        make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
                } else {
                    const uint32_t lo = static_cast<uint32_t>(from_f32<TO>(o[0]).bits) |
                                        (static_cast<uint32_t>(from_f32<TO>(o[1]).bits) << 16);
                    const uint32_t hi = static_cast<uint32_t>(from_f32<TO>(o[2]).bits) |
                                        (static_cast<uint32_t>(from_f32<TO>(o[3]).bits) << 16);
                    *reinterpret_cast<uint2*>(static_cast<TO*>(p.out) + at) = make_uint2(lo, hi);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Packed readout: y[b, r, head, t, :] = M_m^(t / chunk_r) q_hat_t.
// ---------------------------------------------------------------------------
struct PackedParams {
    LineInput q;
    int q_raw;
    const float* states;
    int64_t max_chunks;
    void* out;  // [B, R, heads, N, D]
    int64_t B, R, heads, N;
    int chunk[4];
};

template <int D, typename TQ, typename TO>
__global__ __launch_bounds__(256) void srnl_packed_readout_kernel(const PackedParams p) {
    const int64_t lines = p.B * p.R * p.heads;
    const int64_t total = lines * p.N * D;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    const int i = static_cast<int>(idx % D);
    const int64_t t = (idx / D) % p.N;
    const int64_t line = idx / (D * p.N);
    const int64_t head = line % p.heads;
    const int r = static_cast<int>((line / p.heads) % p.R);
    const int64_t b = line / (p.heads * p.R);
    const TQ* qrow = line_ptr<TQ>(p.q, b, r, head, t);
    float qv[D];
    float qn = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) {
        qv[j] = to_f32(qrow[j]);
        qn += qv[j] * qv[j];
    }
    const float qinv = p.q_raw ? 1.f / fmaxf(sqrtf(qn), 1e-12f) : 1.f;
    const float* m = p.states + (line * p.max_chunks + t / chunk_of(p.chunk, r)) * D * D + i * D;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) dot += m[j] * qv[j];
    static_cast<TO*>(p.out)[idx] = from_f32<TO>(dot * qinv);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

Consts make_consts(const vh_srnl_consts* k) {
    return Consts{k->step_scale, k->min_retention, k->retention_bias, k->injection_margin,
                  k->spectral_clamp, k->spectral_factor};
}

int check_memories(const float* a, const float* b, const float* c, const float* d, const float* e) {
    VH_REQUIRE(a && b && c && d && e, VH_ERR_ARG, "SRNL memories must not be null");
    return VH_OK;
}

template <typename T>
constexpr int dtype_code_of() {
    return std::is_same<T, float>::value ? VH_DTYPE_F32 : std::is_same<T, bf16_t>::value ? VH_DTYPE_BF16 : VH_DTYPE_F16;
}

// Waves per line of the wide scan for this call: 0 = use the single-wave kernels.  Every
// head_dim-32 scan and head_dim-16 scans with fewer lines than SIMDs use it.  The
// scan_wide override (0 | 1 | 2 | 4) forces the choice (1 only for head_dim 16); a
// scan_pack override (a forced head_dim-16 packing) selects the single-wave kernels.
int wide_waves(int64_t lines, int d) {
    const Override forced("scan_wide");
    if (forced.set()) {
        const int w = forced.as_int();
        if (w == 0) return 0;
        if (w == 2 || w == 4 || (w == 1 && d == 16)) return w;
    }
    if (Override("scan_pack").set()) return 0;   // a forced single-wave packing
    if (d == 32 || (d == 16 && lines < 1024)) return scan_wide_waves(lines, d);
    return 0;
}

void scan16_ut_packing(int64_t lines, int64_t heads, int* nl, int* tcw);

// Format of the chunk-start states in the workspace.  Spatial scans of bf16 maps with
// head_dim 16 or 32 store them split into bf16 hi + lo pairs (split_state_at), the operands
// of the matrix-core readout; every other scan stores FP32.  The format is a function of
// these arguments alone: every scan kernel that can run for such a call (block form,
// stepped, wide, under any dispatch override) stores it, so the readout, which decides
// it from the same arguments, always decodes what the scan wrote.
bool scan_ut_enabled() {
    const Override ut("scan_ut");
    return !(ut.set() && ut.value[0] == '0');
}
bool state_split_bf16(int io_dtype, int d, bool spatial) {
    return io_dtype == VH_DTYPE_BF16 && (d == 16 || d == 32) && spatial;
}

template <int D, typename T>
void launch_scan(const ScanParams& sp, hipStream_t stream) {
    const int64_t lines = sp.B * sp.R * sp.heads;
    if constexpr (D == 16 || D == 32) {
        const int waves = wide_waves(lines, D);
        // Token blocks (head_dim 16, chunks of 64 tokens or more, several waves): measured
        // faster than the row split there, slower for shorter chunks and for head_dim 32.
        // The scan_tb override (1 | 2) forces the row split or the blocks.
        int max_chunk = 0;
        for (int r = 0; r < sp.R; ++r) max_chunk = std::max(max_chunk, sp.chunk[r]);
        int token_blocks = (D == 16 && max_chunk >= 64) ? 2 : 1;
        const Override tb("scan_tb");
        if (tb.set()) token_blocks = tb.as_int() == 1 ? 1 : 2;
        if constexpr (D == 16) {
            // Few lines: the block form with a chunk's blocks spread over the waves of one
            // workgroup per line (srnl_utw.hip), unless a dispatch override forces the wide
            // scan or the stepped form.
            const Override utw("scan_utw");   // "1": whenever the chunks allow, "0": never
            const bool utw_on = utw.set() ? utw.value[0] == '1' : waves > 0;
            if (utw_on && scan_ut_enabled() && !Override("scan_wide").set() && launch_scan16_utw<T>(sp, stream))
                return;
        }
        if constexpr (D == 32) {
            // head_dim 32: the block form with one workgroup per line (srnl_utw32.hip) for
            // chunks of up to 64 tokens, unless an override forces the wide scan (scan_wide),
            // the stepped forms (scan_ut "0") or turns it off (scan_utw "0").
            const Override utw("scan_utw");
            const bool utw_on = !(utw.set() && utw.value[0] == '0');
            if (utw_on && scan_ut_enabled() && !Override("scan_wide").set() && launch_scan32_utw<T>(sp, stream))
                return;
        }
        if (waves > 0 && launch_scan_wide(sp, dtype_code_of<T>(), D, waves, token_blocks, stream)) return;
    }
    if constexpr (D == 16) {
        // The block form (srnl_ut.hip).  The scan_ut override "0" selects the stepped form
        // below instead.
        if (scan_ut_enabled()) {
            ScanParams up = sp;
            scan16_ut_packing(lines, sp.heads, &up.lines_per_wave, &up.tiles_per_wave);
            if (launch_scan16_ut<T>(up, stream)) return;
        }
    }
    if constexpr (D == 16) {
        const int nl = sp.lines_per_wave, tcw = sp.tiles_per_wave;
        const unsigned grid = static_cast<unsigned>(lines / nl);
        auto go = [&](auto nlc, auto tcc, auto spc) {
            hipLaunchKernelGGL((srnl_scan16_kernel<T, decltype(nlc)::value, decltype(tcc)::value,
                                                   decltype(spc)::value>),
                               dim3(grid), dim3(64), 0, stream, sp);
        };
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        using S4 = std::integral_constant<int, 4>;
        auto pack = [&](auto spc) {
            if (tcw == 2) {
                if (nl == 2) go(S2{}, S2{}, spc);
                else go(S1{}, S2{}, spc);
            } else {
                if (nl == 4) go(S4{}, S4{}, spc);
                else if (nl == 2) go(S2{}, S4{}, spc);
                else go(S1{}, S4{}, spc);
            }
        };
        if (sp.x.spatial) pack(std::true_type{});
        else pack(std::false_type{});
    } else
        hipLaunchKernelGGL((srnl_scan_kernel<D, T>), dim3(static_cast<unsigned>(lines)),
                           dim3(ScanCfg<D>::NT), 0, stream, sp);
}

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
    return set_error(VH_ERR_DTYPE, "unsupported io dtype code %d", t);
}

int64_t max_chunk_count(int64_t length, const int64_t* chunks, int64_t R) {
    int64_t m = 0;
    for (int64_t r = 0; r < R; ++r) m = std::max(m, (length + chunks[r] - 1) / chunks[r]);
    return m;
}

// Shared validation + scan launch for every SRNL entry point.
// Packing of the head_dim-16 scan: NL lines and TCW 16-slot column tiles per wave.
// Packing lines multiplies the useful work of the token phase for chunks of at most
// 16 TCW / NL tokens and shortens every row dot, but divides the number of waves.  The
// scan is latency-bound, so two waves per SIMD (2048 on MI355X) beat fuller tiles with
// one: measured on MI355X at the Tiny stages (B = 128), 2 lines x 2 tiles for 4096 and
// 8192 lines (chunks 14 and 7) is 12-15 % faster than 4 x 4, and 1 line x 4 tiles for
// 2048 lines (chunk 28) 13 % faster than 2 x 4.  The lines of a wave share (b, r), so NL
// divides heads.  The scan_pack override "<NL>x<TCW>" forces a packing (when heads
// allows it).
void scan16_packing(int64_t lines, int64_t heads, int* nl, int* tcw) {
    const Override forced("scan_pack");
    if (forced.set()) {
        int fl = 0, ft = 0;
        if (std::sscanf(forced.value, "%dx%d", &fl, &ft) == 2 && (fl == 1 || fl == 2 || fl == 4) && (ft == 2 || ft == 4) &&
            fl <= ft && heads % fl == 0) {
            *nl = fl;
            *tcw = ft;
            return;
        }
    }
    if (heads % 2 == 0 && lines >= 4 * 1024) {
        *nl = 2;
        *tcw = 2;
    } else {
        *nl = 1;
        *tcw = 4;
    }
}

// Packing of the block-form scan (srnl_ut.hip, 200-310 VGPRs: one or two waves per SIMD).
// Measured on MI355X at the Tiny stages (B = 128, scan launches alone): 1 x 4 for 1024
// lines (chunk 56: 270 us; 1 x 2 301 us), 1 x 2 for 2048 (chunk 28: 104 us; 1 x 4 217 us),
// 2 x 2 for 4096 and 8192 (chunks 14 and 7: 56.5 and 53 us; 4 x 4 71 and 68 us).
// The scan_pack override applies as for the stepped form.
void scan16_ut_packing(int64_t lines, int64_t heads, int* nl, int* tcw) {
    if (Override("scan_pack").set()) {
        scan16_packing(lines, heads, nl, tcw);
        return;
    }
    if (heads % 2 == 0 && lines >= 4 * 1024) {
        *nl = 2;
        *tcw = 2;
    } else if (lines >= 2 * 1024) {
        *nl = 1;
        *tcw = 2;
    } else {
        *nl = 1;
        *tcw = 4;
    }
}

int run_scan(const LineInput& x, int io_dtype, const float* Mm, const float* Mv, const float* Mk,
             const float* Me, const float* Ma, int64_t B, int64_t R, int64_t heads, int64_t L,
             int d, const int64_t* chunks, const vh_srnl_consts* consts, void* workspace,
             size_t workspace_bytes, hipStream_t stream, ScanParams* out_params,
             int per_line_state = 0) {
    VH_REQUIRE(valid_head_dim(d), VH_ERR_HEAD_DIM,
               "head_dim must be one of 4, 8, 16, 32, 64; got %d", d);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    VH_REQUIRE(B > 0 && heads > 0 && L > 0, VH_ERR_SHAPE,
               "SRNL requires nonempty batches and sequences (B=%lld heads=%lld L=%lld)",
               (long long)B, (long long)heads, (long long)L);
    VH_REQUIRE(R == 1 || R == 2 || R == 4, VH_ERR_SHAPE, "directions must be 1, 2 or 4, got %lld",
               (long long)R);
    VH_REQUIRE(chunks != nullptr, VH_ERR_ARG, "chunk lengths must not be null");
    for (int64_t r = 0; r < R; ++r)
        VH_REQUIRE(chunks[r] > 0 && chunks[r] <= (int64_t)1 << 30, VH_ERR_ARG,
                   "invalid chunk length %lld for direction %lld", (long long)chunks[r], (long long)r);
    int rc = check_srnl_consts(consts);
    if (rc) return rc;
    rc = check_memories(Mm, Mv, Mk, Me, Ma);
    if (rc) return rc;
    VH_REQUIRE(x.ptr != nullptr, VH_ERR_ARG, "SRNL input must not be null");
    const int64_t lines = B * R * heads;
    VH_REQUIRE(lines < ((int64_t)1 << 31), VH_ERR_SHAPE, "too many SRNL lines (%lld)", (long long)lines);
    const int64_t mc = max_chunk_count(L, chunks, R);
    const size_t need = vh_srnl_workspace_bytes(lines, mc, d);
    VH_REQUIRE(workspace != nullptr && workspace_bytes >= need, VH_ERR_WORKSPACE,
               "SRNL workspace needs %zu bytes, got %zu", need, workspace ? workspace_bytes : (size_t)0);
    ScanParams sp{};
    sp.x = x;
    sp.Mm = Mm; sp.Mv = Mv; sp.Mk = Mk; sp.Me = Me; sp.Ma = Ma;
    sp.B = B; sp.R = R; sp.heads = heads; sp.L = L;
    for (int r = 0; r < 4; ++r) sp.chunk[r] = static_cast<int>(chunks[r < R ? r : 0]);
    sp.max_chunks = mc;
    sp.states = static_cast<float*>(workspace);
    sp.per_line_state = per_line_state;
    {
        // Vector loads need every row start aligned: base pointer and all strides.
        const size_t elem = static_cast<size_t>(dtype_bytes(io_dtype));
        const size_t align = (elem == 2 && d == 4) ? 8 : 16;
        const uintptr_t base = reinterpret_cast<uintptr_t>(x.ptr);
        bool ok = base % align == 0;
        for (int64_t st : {x.sb, x.sr, x.sh, x.st}) ok = ok && (static_cast<size_t>(st) * elem) % align == 0;
        sp.x_vec = ok ? 1 : 0;
    }
    sp.k = make_consts(consts);
    scan16_packing(lines, heads, &sp.lines_per_wave, &sp.tiles_per_wave);
    sp.aligned = x.spatial && R == 4 && chunks[0] == x.W && chunks[1] == x.W && chunks[2] == x.H &&
                 chunks[3] == x.H && x.H * x.W * x.st < (int64_t(1) << 31);
    sp.split_states = state_split_bf16(io_dtype, d, x.spatial != 0) ? 1 : 0;
    rc = dispatch_d(d, [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        dispatch_t(io_dtype, [&](auto tv) { launch_scan<D, decltype(tv)>(sp, stream); });
    });
    if (rc) return rc;
    *out_params = sp;
    return check_launch("srnl_scan_kernel");
}

int run_fuse(const ScanParams& sp, const void* x, const void* q, int per_direction, int io_dtype,
             const float* skip, int skip_per_dir, const float* wgt, void* out, int64_t H,
             int64_t W, int64_t C, int d, hipStream_t stream, const void* aux = nullptr,
             int out_dtype = VH_DTYPE_F32, const float* lepe_taps = nullptr, const float* lepe_bias = nullptr) {
    VH_REQUIRE(skip && wgt && out && q, VH_ERR_ARG, "SRNL fusion arguments must not be null");
    VH_REQUIRE(out_dtype == VH_DTYPE_F32 || out_dtype == io_dtype, VH_ERR_DTYPE,
               "SRNL fused output must be fp32 or the io dtype");
    const bool lepe = lepe_taps != nullptr;
    VH_REQUIRE(!lepe || (out_dtype == io_dtype && !aux && !per_direction), VH_ERR_ARG,
               "the position encoding is fused only into a spatial readout to the io dtype, without aux");
    FuseParams fp{};
    fp.x = x; fp.q = q; fp.per_direction = per_direction;
    fp.states = sp.states; fp.max_chunks = sp.max_chunks;
    fp.skip = skip; fp.skip_per_dir = skip_per_dir; fp.wgt = wgt; fp.out = out; fp.aux = aux;
    fp.lepe_taps = lepe_taps; fp.lepe_bias = lepe_bias;
    fp.B = sp.B; fp.H = H; fp.W = W; fp.C = C; fp.heads = sp.heads;
    for (int r = 0; r < 4; ++r) fp.chunk[r] = sp.chunk[r];
    fp.split_states = sp.split_states;
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(q) |
                            reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(sp.states) |
                            reinterpret_cast<uintptr_t>(aux) | reinterpret_cast<uintptr_t>(skip) |
                            reinterpret_cast<uintptr_t>(wgt);
    const bool out_f32 = out_dtype == VH_DTYPE_F32;
    VH_REQUIRE(fp.split_states == ((io_dtype == VH_DTYPE_BF16 && (d == 16 || d == 32) && !per_direction) ? 1 : 0), VH_ERR_ARG,
               "SRNL readout: state format does not match the scan's");
    if ((d == 16 || (d == 32 && io_dtype != VH_DTYPE_F16)) && !per_direction && sp.chunk[0] == W &&
        sp.chunk[1] == W && sp.chunk[2] == H && sp.chunk[3] == H && align % 16 == 0 && C % 16 == 0 &&
        H * W * C < (int64_t(1) << 31) && sp.max_chunks * d * d < (int64_t(1) << 31)) {
        // 8 x 8 tiles for maps of at most 8 x 8 (the Tiny 7 x 7 stage), else 16 x 16; the
        // readout_tile override forces either
        const Override rt("readout_tile");
        const bool small = rt.set() ? rt.value[0] == '8' : (H <= 8 && W <= 8);
        const int64_t tp = small ? 8 : 16;
        const int64_t tiles_h = (H + tp - 1) / tp, tiles_w = (W + tp - 1) / tp;
        // one workgroup per tile and 16-channel half
        const int64_t n_tiles = sp.B * sp.heads * tiles_h * tiles_w * (d / 16);
        VH_REQUIRE(n_tiles <= 0x7fffffff, VH_ERR_SHAPE, "SRNL readout grid too large");
        auto go = [&](auto tv, auto dc) {
            using T = decltype(tv);
            constexpr int DD = decltype(dc)::value;
            // bf16 maps always carry split states here (state_split_bf16)
            constexpr bool SPLIT = std::is_same<T, bf16_t>::value;
            auto run = [&](auto tpc) {
                constexpr int TPV = decltype(tpc)::value;
                if (lepe)
                    hipLaunchKernelGGL((srnl_readout_tile_kernel<T, T, DD, SPLIT, TPV, true>),
                                       dim3(static_cast<unsigned>(n_tiles)), dim3(256), 0, stream, fp, tiles_h, tiles_w);
                else if (out_f32)
                    hipLaunchKernelGGL((srnl_readout_tile_kernel<T, float, DD, SPLIT, TPV>),
                                       dim3(static_cast<unsigned>(n_tiles)), dim3(256), 0, stream, fp, tiles_h, tiles_w);
                else
                    hipLaunchKernelGGL((srnl_readout_tile_kernel<T, T, DD, SPLIT, TPV>),
                                       dim3(static_cast<unsigned>(n_tiles)), dim3(256), 0, stream, fp, tiles_h, tiles_w);
            };
            if (small) run(std::integral_constant<int, 8>{});
            else run(std::integral_constant<int, 16>{});
        };
        int rc;
        if (d == 16) rc = dispatch_t(io_dtype, [&](auto tv) { go(tv, std::integral_constant<int, 16>{}); });
        else if (io_dtype == VH_DTYPE_BF16) rc = (go(bf16_t{}, std::integral_constant<int, 32>{}), VH_OK);
        else rc = (go(float{}, std::integral_constant<int, 32>{}), VH_OK);
        if (rc) return rc;
        return check_launch("srnl_readout_tile_kernel");
    }
    if (lepe) {
        // The encoding goes to `out` first (the depthwise kernel, the same bits), and the
        // per-element readout adds it in place (each thread reads its own element first).
        const int rc = vh_dwconv2d_nhwc_forward(x, io_dtype, lepe_taps, lepe_bias, 5, 0, nullptr, out, sp.B, H, W, C,
                                                stream);
        if (rc) return rc;
        fp.aux = out;
    }
    const int64_t total = sp.B * H * W * C;
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
    int rc = dispatch_d(d, [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        dispatch_t(io_dtype, [&](auto tv) {
            using T = decltype(tv);
            if (out_f32)
                hipLaunchKernelGGL((srnl_fuse_readout_kernel<D, T, float>), dim3(blocks), dim3(256), 0, stream, fp);
            else
                hipLaunchKernelGGL((srnl_fuse_readout_kernel<D, T, T>), dim3(blocks), dim3(256), 0, stream, fp);
        });
    });
    if (rc) return rc;
    return check_launch("srnl_fuse_readout_kernel");
}

template <typename TQ>
int run_packed(const ScanParams& sp, const LineInput& q, int q_raw, int io_dtype, void* out, int d,
               hipStream_t stream) {
    VH_REQUIRE(out != nullptr && q.ptr != nullptr, VH_ERR_ARG, "SRNL output/query must not be null");
    PackedParams pp{};
    pp.q = q; pp.q_raw = q_raw;
    pp.states = sp.states; pp.max_chunks = sp.max_chunks;
    pp.out = out;
    pp.B = sp.B; pp.R = sp.R; pp.heads = sp.heads; pp.N = sp.L;
    for (int r = 0; r < 4; ++r) pp.chunk[r] = sp.chunk[r];
    const int64_t total = sp.B * sp.R * sp.heads * sp.L * d;
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
    int rc = dispatch_d(d, [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        dispatch_t(io_dtype, [&](auto tv) {
            using TO = decltype(tv);
            using TQQ = typename std::conditional<std::is_same<TQ, void>::value, TO, TQ>::type;
            hipLaunchKernelGGL((srnl_packed_readout_kernel<D, TQQ, TO>), dim3(blocks), dim3(256), 0,
                               stream, pp);
        });
    });
    if (rc) return rc;
    return check_launch("srnl_packed_readout_kernel");
}

}  // namespace

int check_spatial_shape(int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim) {
    VH_REQUIRE(H > 0 && W > 0 && C > 0 && B > 0, VH_ERR_SHAPE, "spatial SRNL needs nonempty [B,H,W,C]");
    VH_REQUIRE(valid_head_dim(head_dim), VH_ERR_HEAD_DIM,
               "head_dim must be one of 4, 8, 16, 32, 64; got %d", head_dim);
    VH_REQUIRE(C % head_dim == 0, VH_ERR_SHAPE, "C=%lld is not a multiple of head_dim=%d",
               (long long)C, head_dim);
    VH_REQUIRE(H * W < (int64_t(1) << 24), VH_ERR_SHAPE, "spatial SRNL supports H*W < 2^24 pixels, got %lld",
               (long long)(H * W));
    return VH_OK;
}

int srnl_spatial_forward_ws(const void* x, const void* q, int32_t io_dtype, const float* M_m, const float* M_v,
                            const float* M_k, const float* M_eta, const float* M_alpha, const float* d_skip,
                            int32_t skip_per_direction, const float* dir_weight, float* out, int64_t B, int64_t H,
                            int64_t W, int64_t C, int32_t head_dim, const int64_t chunks[4],
                            const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
    int rc = check_spatial_shape(B, H, W, C, head_dim);
    if (rc) return rc;
    const int64_t heads = C / head_dim;
    LineInput xin{x, H * W * C, 0, head_dim, C, 1, H, W, 1.0f / static_cast<float>(H)};
    ScanParams sp{};
    rc = run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, 4, heads, H * W, head_dim, chunks, consts,
                  workspace, workspace_bytes, stream, &sp);
    if (rc) return rc;
    return run_fuse(sp, x, q, 0, io_dtype, d_skip, skip_per_direction, dir_weight, out, H, W, C, head_dim, stream);
}

}  // namespace vh

namespace vh {
// vh_srnl_spatial_readout, with the position encoding fused when lepe_taps is not null
int spatial_readout_impl(const void* x, const void* q, int32_t io_dtype, const float* d_skip,
                         int32_t skip_per_direction, const float* dir_weight, const void* aux, void* out,
                         int32_t out_dtype, int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim,
                         const int64_t chunks[4], const void* workspace, size_t workspace_bytes, void* stream,
                         const float* lepe_taps, const float* lepe_bias);
}  // namespace vh

using namespace vh;

extern "C" {

size_t vh_srnl_workspace_bytes(int64_t lines, int64_t max_chunks, int32_t head_dim) {
    if (lines <= 0 || max_chunks <= 0 || head_dim <= 0) return 0;
    return static_cast<size_t>(lines) * static_cast<size_t>(max_chunks) *
           static_cast<size_t>(head_dim) * static_cast<size_t>(head_dim) * sizeof(float);
}

int vh_srnl_spatial_forward(const void* x, const void* q, int32_t io_dtype, const float* M_m,
                            const float* M_v, const float* M_k, const float* M_eta,
                            const float* M_alpha, const float* d_skip, int32_t skip_per_direction,
                            const float* dir_weight, float* out, int64_t B, int64_t H, int64_t W,
                            int64_t C, int32_t head_dim, const int64_t chunks[4],
                            const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes,
                            void* stream) {
    return srnl_spatial_forward_ws(x, q, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, d_skip, skip_per_direction,
                                   dir_weight, out, B, H, W, C, head_dim, chunks, consts, workspace, workspace_bytes,
                                   static_cast<hipStream_t>(stream));
}

int vh_srnl_spatial_scan(const void* x, int32_t io_dtype, const float* M_m, const float* M_v, const float* M_k,
                         const float* M_eta, const float* M_alpha, int64_t B, int64_t H, int64_t W, int64_t C,
                         int32_t head_dim, const int64_t chunks[4], const vh_srnl_consts* consts, void* workspace,
                         size_t workspace_bytes, void* stream) {
    VH_REQUIRE(H > 0 && W > 0 && C > 0 && B > 0, VH_ERR_SHAPE, "spatial SRNL needs nonempty [B,H,W,C]");
    VH_REQUIRE(valid_head_dim(head_dim), VH_ERR_HEAD_DIM,
               "head_dim must be one of 4, 8, 16, 32, 64; got %d", head_dim);
    VH_REQUIRE(C % head_dim == 0, VH_ERR_SHAPE, "C=%lld is not a multiple of head_dim=%d",
               (long long)C, head_dim);
    VH_REQUIRE(H * W < (int64_t(1) << 24), VH_ERR_SHAPE, "spatial SRNL supports H*W < 2^24 pixels, got %lld",
               (long long)(H * W));
    LineInput xin{x, H * W * C, 0, head_dim, C, 1, H, W, 1.0f / static_cast<float>(H)};
    ScanParams sp{};
    return run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, 4, C / head_dim, H * W, head_dim, chunks,
                    consts, workspace, workspace_bytes, static_cast<hipStream_t>(stream), &sp);
}

int vh_srnl_spatial_readout(const void* x, const void* q, int32_t io_dtype, const float* d_skip,
                            int32_t skip_per_direction, const float* dir_weight, const void* aux, void* out,
                            int32_t out_dtype, int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim,
                            const int64_t chunks[4], const void* workspace, size_t workspace_bytes,
                            void* stream) {
    return spatial_readout_impl(x, q, io_dtype, d_skip, skip_per_direction, dir_weight, aux, out, out_dtype, B, H, W,
                                C, head_dim, chunks, workspace, workspace_bytes, stream, nullptr, nullptr);
}

}  // extern "C"

namespace vh {
int spatial_readout_impl(const void* x, const void* q, int32_t io_dtype, const float* d_skip,
                         int32_t skip_per_direction, const float* dir_weight, const void* aux, void* out,
                         int32_t out_dtype, int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim,
                         const int64_t chunks[4], const void* workspace, size_t workspace_bytes, void* stream,
                         const float* lepe_taps, const float* lepe_bias) {
    VH_REQUIRE(x && q && workspace && chunks, VH_ERR_ARG, "spatial SRNL readout pointers must not be null");
    VH_REQUIRE(H > 0 && W > 0 && C > 0 && B > 0, VH_ERR_SHAPE, "spatial SRNL needs nonempty [B,H,W,C]");
    VH_REQUIRE(valid_head_dim(head_dim), VH_ERR_HEAD_DIM,
               "head_dim must be one of 4, 8, 16, 32, 64; got %d", head_dim);
    VH_REQUIRE(C % head_dim == 0, VH_ERR_SHAPE, "C=%lld is not a multiple of head_dim=%d",
               (long long)C, head_dim);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    for (int r = 0; r < 4; ++r)
        VH_REQUIRE(chunks[r] > 0 && chunks[r] <= (int64_t)1 << 30, VH_ERR_ARG, "invalid chunk length %lld",
                   (long long)chunks[r]);
    ScanParams sp{};
    sp.B = B; sp.R = 4; sp.heads = C / head_dim; sp.L = H * W;
    for (int r = 0; r < 4; ++r) sp.chunk[r] = static_cast<int>(chunks[r]);
    sp.max_chunks = max_chunk_count(H * W, chunks, 4);
    const size_t need = vh_srnl_workspace_bytes(B * 4 * sp.heads, sp.max_chunks, head_dim);
    VH_REQUIRE(workspace_bytes >= need, VH_ERR_WORKSPACE, "SRNL workspace needs %zu bytes, got %zu", need,
               workspace_bytes);
    sp.states = const_cast<float*>(static_cast<const float*>(workspace));
    sp.split_states = state_split_bf16(io_dtype, head_dim, true) ? 1 : 0;
    return run_fuse(sp, x, q, 0, io_dtype, d_skip, skip_per_direction, dir_weight, out, H, W, C, head_dim,
                    static_cast<hipStream_t>(stream), aux, out_dtype, lepe_taps, lepe_bias);
}
}  // namespace vh

extern "C" {

int vh_srnl_spatial_readout_lepe(const void* x, const void* q, int32_t io_dtype, const float* d_skip,
                                 int32_t skip_per_direction, const float* dir_weight, const float* lepe_taps,
                                 const float* lepe_bias, void* out, int64_t B, int64_t H, int64_t W, int64_t C,
                                 int32_t head_dim, const int64_t chunks[4], const void* workspace,
                                 size_t workspace_bytes, void* stream) {
    VH_REQUIRE(lepe_taps, VH_ERR_ARG, "position encoding taps must not be null");
    VH_REQUIRE(H * W * C < (int64_t(1) << 31), VH_ERR_SHAPE, "position encoding: one image must be below 2^31 elements");
    return spatial_readout_impl(x, q, io_dtype, d_skip, skip_per_direction, dir_weight, nullptr, out, io_dtype, B, H,
                                W, C, head_dim, chunks, workspace, workspace_bytes, stream, lepe_taps, lepe_bias);
}

int vh_srnl_line_forward_seq_noatomic(const void* X, const void* Q_raw, int32_t io_dtype,
                                      const float* M_m, const float* M_v, const float* M_k,
                                      const float* M_eta, const float* M_alpha,
                                      const float* d_skip, int32_t skip_per_direction,
                                      const float* dir_weight, float* out, int64_t B, int64_t H,
                                      int64_t W, int64_t C, int32_t head_dim,
                                      const vh_srnl_consts* consts, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    VH_REQUIRE(H > 0 && W > 0 && B > 0 && C > 0, VH_ERR_SHAPE,
               "line fused SRNL needs nonempty [B, 4, H*W, C] stacks");
    VH_REQUIRE(valid_head_dim(head_dim), VH_ERR_HEAD_DIM,
               "line fused HOPE supports head_dim in {4, 8, 16, 32, 64}; got %d", head_dim);
    VH_REQUIRE(C % head_dim == 0, VH_ERR_SHAPE, "C=%lld is not a multiple of head_dim=%d",
               (long long)C, head_dim);
    const int64_t heads = C / head_dim;
    const int64_t L = H * W;
    const int64_t chunks[4] = {W, W, H, H};
    LineInput xin{X, 4 * L * C, L * C, head_dim, C, 0, 0, 0, 0.f};
    ScanParams sp{};
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, 4, heads, L, head_dim,
                      chunks, consts, workspace, workspace_bytes, s, &sp);
    if (rc) return rc;
    return run_fuse(sp, X, Q_raw, 1, io_dtype, d_skip, skip_per_direction, dir_weight, out, H, W,
                    C, head_dim, s);
}

int vh_srnl_sequence_forward(const void* X, const void* Q_raw, int32_t io_dtype, const float* M_m,
                             const float* M_v, const float* M_k, const float* M_eta,
                             const float* M_alpha, int32_t memories_per_line, void* out, int64_t B,
                             int64_t R, int64_t heads, int64_t N, int32_t head_dim,
                             const int64_t* chunks, const vh_srnl_consts* consts, void* workspace,
                             size_t workspace_bytes, void* stream) {
    const int64_t d = head_dim;
    LineInput xin{X, R * heads * N * d, heads * N * d, N * d, d, 0, 0, 0, 0.f};
    ScanParams sp{};
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, R, heads, N, head_dim, chunks,
                      consts, workspace, workspace_bytes, s, &sp, memories_per_line ? 1 : 0);
    if (rc) return rc;
    const int64_t C = heads * d;
    LineInput qin{Q_raw, R * N * C, N * C, d, C, 0, 0, 0, 0.f};
    return run_packed<void>(sp, qin, 1, io_dtype, out, head_dim, s);
}

int vh_srnl_forward(const void* X, int32_t io_dtype, const float* Q, const float* M_m,
                    const float* M_v, const float* M_k, const float* M_eta, const float* M_alpha,
                    int32_t memories_per_line, void* out, int64_t B, int64_t R, int64_t heads,
                    int64_t N, int32_t head_dim, const int64_t* chunks,
                    const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes,
                    void* stream) {
    const int64_t d = head_dim;
    LineInput xin{X, R * heads * N * d, heads * N * d, N * d, d, 0, 0, 0, 0.f};
    ScanParams sp{};
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, R, heads, N, head_dim, chunks,
                      consts, workspace, workspace_bytes, s, &sp, memories_per_line ? 1 : 0);
    if (rc) return rc;
    LineInput qin{Q, R * heads * N * d, heads * N * d, N * d, d, 0, 0, 0, 0.f};
    return run_packed<float>(sp, qin, 0, io_dtype, out, head_dim, s);
}

}  // extern "C"
