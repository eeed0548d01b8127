// SRNL chunk scan for head_dim 16 (bf16, fp16 or FP32 activations): the block form of the
// gain recurrence, with the serial part reduced to one matrix-core product per 16 tokens.
//
// Reference recurrence (models/srnl_core/csrc/inference_recurrence.cuh:32-135, memory.cuh:
// 219-233), per line and chunk, from the chunk-start state M_m, M_v, M_k, e, a:
//   k_t = normalise(M_k x_t), v_t = M_v x_t, gates alpha_t, eta^_t of x.e, x.a, |k - v|, |k|
//   G = I;  for t: G <- alpha_t G - eta^_t (G k_t + k_t - v_t) k_t^T      (serial, :92-106)
//   M_{m,v,k} <- M G;  e <- G^T e;  a <- G^T a                               (:119-133)
//
// Block form.  Cut the chunk into blocks of 16 token slots (one MFMA tile each; slots past
// the chunk act as the identity: alpha = 1, eta^ = 0, k = v = 0).  Inside a block entered
// with gain G_b, let a_t = prod_{s<=t} alpha_s (block-local).  The correction vectors
// r_t = G_{t-1} k_t + delta_t (delta = k - v) then satisfy
//     r_t = a_{t-1} G_b k_t + delta_t - sum_{s<t} L[s][t] r_s,
//     L[s][t] = eta^_s (a_{t-1} / a_s) (k_s . k_t)              (s < t, strictly upper),
// so R (I + L) = G_b K D_a + Delta with D_a = diag(a_{t-1}), and the block's exit gain is
//     G_{b+1} = a_15 G_b - R W K^T,     W = diag(w_s),  w_s = eta^_s a_15 / a_s.
// With Z = (I + L)^-1 W K^T (16 tokens x 16 features) this is an affine map of G_b:
//     G_{b+1} = G_b X_b + Y_b,   X_b = a_15 I - (K D_a) Z,   Y_b = -Delta Z.
// X_b and Y_b depend only on the block's own keys and gates, so every block's pair is
// formed off the serial path; the chain across the chunk's blocks is one product per
// block.  This regroups the serial update exactly (rounding differs by reassociation).
//
// MI355X mapping (one wave per NL lines, TCW tiles of 16 slots; tile tc is block tc % TPL
// of line tc / TPL):
//   * state S = [M_m; M_v; M_k; e; a; 0] (64 x 16 FP32) stays in registers in the MFMA
//     A-operand layout (lane 16 q + i: row 16 R + i, columns 4q..4q+3);
//   * projections [M_k; M_v] X and the gate pre-activations on bf16 MFMAs (bf16 x exact,
//     fp16 / FP32 x and the FP32 state as bf16 hi + lo), norms by row-swap permutes, gates
//     per token lane;
//   * per-slot scalars through one DPP prefix sum per tile: cl_t = sum log2 alpha, so
//     a_t / a_s = 2^(cl_t - cl_s) (every ratio used is <= 1; no overflow for any alpha);
//   * Gram tiles K^T K and the triangle L on the matrix cores (bf16 hi + lo operands,
//     three bf16 products with the lo x lo term dropped);
//   * Z by back substitution on the VALU: lane 16 b + f solves column f of tile b;
//   * X_b, Y_b and the composition on the matrix cores.  Operand layouts are chosen so
//     that every product consumes what the previous one leaves in registers: with K as
//     the projections leave it (slot across lanes, features in entries), K^T K needs no
//     movement; Z, the feature-major key/difference operands and G alternate between the
//     accumulator layout of M and of M^T, and the composition keeps G^T until the chunk's
//     last block, which yields G itself, the operand the refresh S^T <- G^T S^T needs;
//   * the refresh keeps S in its A-operand layout (it is the B operand of S^T).
// The chunk-start M_m of every chunk goes to the workspace for the readout (srnl.hip).
#include "srnl_block_form.h"

namespace vh {
using namespace blockform;

// Two-tile packings run two waves per SIMD (their line counts give 2048 or more waves), so
// they are held to 256 VGPRs; four-tile packings run one wave per SIMD.
template <typename T, int NL, int TCW, bool SPATIAL>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(TCW == 2 ? 2 : 1)))
void srnl_scan16_ut_kernel(const ScanParams p) {
    using XQ = XQuad<T>;
    static_assert((TCW == 2 || TCW == 4) && NL <= TCW, "tile packing");
    constexpr int D = 16, TT = 16 * TCW, S = TT / NL, TPL = TCW / NL, DKS = TT + 4;
    __shared__ __align__(16) float kT[D * DKS];     // normalised keys [feature][slot]
    __shared__ __align__(16) float ndT[D * DKS];    // v - k [feature][slot]
    __shared__ __align__(16) float tk[4 * TT];      // per slot: rho, kappa, -a_{t-1}, w
    // L and Z rows are padded to LS = 20 floats, so that 16-byte accesses of 16 lanes down a
    // column of rows fall in different LDS banks.
    constexpr int LS = 20;
    __shared__ __align__(16) float Lc[TCW * 16 * LS];   // per tile: L[s][t] at [t][s]
    __shared__ __align__(16) float Zs[TCW * 16 * LS];   // per tile: Z[s][f] at [f][s]
    __shared__ __align__(16) float gr[NL * 2 * D];  // per line: e, a (gate operand rows)

    const int64_t groups = p.B * p.R * p.heads / NL;
    const int64_t line0 = xcd_remap(blockIdx.x, groups) * NL;
    const int64_t head0 = line0 % p.heads;
    const int r = static_cast<int>((line0 / p.heads) % p.R);
    const int64_t b = line0 / (p.heads * p.R);
    const int lane = threadIdx.x;
    const int i16 = lane & 15, q = lane >> 4;
    // Four-tile packings: reserve the whole 256-entry architected VGPR file, so that two
    // waves of this kernel never share a SIMD (more than 256 of its 512 registers each).
    // With fewer registers the workgroup dispatcher was seen to put two waves on ~90 SIMDs
    // and leave as many idle, which made the launch 20 % longer (the doubled waves finish
    // last); waves of other kernels can still share the SIMD.
    if constexpr (TCW == 4) asm volatile("" ::: "v255");

    // State in A-operand layout: sA[lam][R][j] = S[16 R + i16][4 q + j].
    float sA[NL][4][4];
#pragma unroll
    for (int lam = 0; lam < NL; ++lam) {
        const int64_t s = p.per_line_state ? line0 + lam : r * p.heads + head0 + lam;
        const float4 mm = ld4(p.Mm + s * D * D + i16 * D + 4 * q);
        const float4 mv = ld4(p.Mv + s * D * D + i16 * D + 4 * q);
        const float4 mk = ld4(p.Mk + s * D * D + i16 * D + 4 * q);
        float4 ea = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i16 == 0) ea = ld4(p.Me + s * D + 4 * q);
        if (i16 == 1) ea = ld4(p.Ma + s * D + 4 * q);
        const float4 rows[4] = {mm, mv, mk, ea};
#pragma unroll
        for (int R = 0; R < 4; ++R) {
            sA[lam][R][0] = rows[R].x; sA[lam][R][1] = rows[R].y;
            sA[lam][R][2] = rows[R].z; sA[lam][R][3] = rows[R].w;
        }
        if (i16 < 2) *reinterpret_cast<float4*>(gr + (lam * 2 + i16) * D + 4 * q) = ea;
    }

    const int C = chunk_of(p.chunk, r);
    const int64_t nc = (p.L + C - 1) / C;
    const int my_slot = lane % S;
    const bool slot_lane = lane < TT;
    const T* xcol[TCW];
#pragma unroll
    for (int tc = 0; tc < TCW; ++tc)
        xcol[tc] = static_cast<const T*>(p.x.ptr) + b * p.x.sb + r * p.x.sr + (head0 + tc / TPL) * p.x.sh + 4 * q;
    // Row/column chunks of the spatial operator: token i of chunk cc of scan r is pixel
    // pa*cc + pb*i + pc (32-bit; the host enables this only when H*W*pixel_stride < 2^31).
    int pa = 0, pb = 0, pc = 0, pst = 0;
    if constexpr (SPATIAL) {
        const int W = static_cast<int>(p.x.W), L = static_cast<int>(p.x.H * p.x.W);
        pa = r == 0 ? W : r == 1 ? -W : r == 2 ? 1 : -1;
        pb = r == 0 ? 1 : r == 1 ? -1 : r == 2 ? W : -W;
        pc = (r & 1) ? L - 1 : 0;
        pst = static_cast<int>(p.x.st);
    }
    // x operands move as raw bits, loaded without a branch (invalid slots read their
    // line's first token and are zeroed when decoded).
    auto issue_tile = [&](int64_t cc, int base, int cnt, typename XQ::Raw (&raw)[TCW], unsigned& valid) {
        valid = 0;
        int64_t offs[TCW];
#pragma unroll
        for (int tc = 0; tc < TCW; ++tc) {
            const int slot = (tc % TPL) * 16 + i16;
            const int64_t tok = cc * C + base + slot;
            const bool ok = slot < cnt && tok < p.L;
            valid |= ok ? (1u << tc) : 0u;
            if (SPATIAL && p.aligned)
                offs[tc] = ok ? (pa * static_cast<int>(cc) + pb * (base + slot) + pc) * pst : 0;
            else
                offs[tc] = ok ? token_offset<SPATIAL>(p.x, r, tok) : 0;
        }
        if (p.x_vec) {
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) raw[tc] = XQ::load(xcol[tc] + offs[tc]);
        } else {
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) raw[tc] = XQ::load_scalar(xcol[tc] + offs[tc]);
        }
    };

    typename XQ::Raw xr[TCW];
    unsigned xvalid = 0;
    bool have_next = false;

    for (int64_t c = 0; c < nc; ++c) {
#pragma unroll
        for (int lam = 0; lam < NL; ++lam) {
            // FP32, or bf16 hi[4] then lo[4]: the readout's matrix-core operands, no split there
            store_state4(p.states + ((line0 + lam) * p.max_chunks + c) * D * D + i16 * D + 4 * q,
                         make_float4(sA[lam][0][0], sA[lam][0][1], sA[lam][0][2], sA[lam][0][3]), p.split_states);
        }
        if (c == nc - 1) break;

        // Composition state: gT = G^T (accumulator layout) until the chunk's last block,
        // which leaves gD = G.
        v4f gT[NL], gD[NL];
        bool g_identity = true;

        for (int base = 0; base < C; base += S) {
            const int cnt = min(S, C - base);
            const bool last_pass = base + S >= C;
            if (!have_next) issue_tile(c, base, cnt, xr, xvalid);
            // ---- token phase: [M_k; M_v] X and (x.e, x.a) on the matrix cores ----
            v4s akh[NL], akl[NL], avh[NL], avl[NL], gah[NL], gal[NL];
#pragma unroll
            for (int lam = 0; lam < NL; ++lam) {
                split4(sA[lam][2], akh[lam], akl[lam]);
                split4(sA[lam][1], avh[lam], avl[lam]);
                // operand rows 4q' + 0 / 4q' + 1 are e / a, the rest zero, so every lane of
                // a token column gets x.e and x.a in accumulator entries 0 and 1
                float4 g4 = ld4(gr + (lam * 2 + (i16 & 1)) * D + 4 * q);
                const bool on = (i16 & 3) < 2;
                const float ga[4] = {on ? g4.x : 0.f, on ? g4.y : 0.f, on ? g4.z : 0.f, on ? g4.w : 0.f};
                split4(ga, gah[lam], gal[lam]);
            }
            v4f kacc[TCW], vacc[TCW];
            float pe[TCW], pq[TCW];
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                const int lam = tc / TPL;
                v4s xh, xl;
                XQ::operands(xr[tc], (xvalid >> tc) & 1u, xh, xl);
                const v4f z4 = {0.f, 0.f, 0.f, 0.f};
                kacc[tc] = XQ::mma(akh[lam], akl[lam], xh, xl, z4);
                vacc[tc] = XQ::mma(avh[lam], avl[lam], xh, xl, z4);
                const v4f gacc = XQ::mma(gah[lam], gal[lam], xh, xl, z4);
                pe[tc] = gacc[0];
                pq[tc] = gacc[1];
            }
            float kn[TCW], dsq[TCW], ksq[TCW], kn4[TCW][4];
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                kn[tc] = kacc[tc][0] * kacc[tc][0] + kacc[tc][1] * kacc[tc][1] + kacc[tc][2] * kacc[tc][2] +
                         kacc[tc][3] * kacc[tc][3];
                kn[tc] = xor16_32_sum(kn[tc]);
            }
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                // ||k||^2 of the normalised key is ||k~||^2 / (||k~||^2 + 1e-6)
                const float inv = rsqrtf(kn[tc] + 1e-6f);
                ksq[tc] = kn[tc] * inv * inv;
                dsq[tc] = 0.f;
                const int t = 16 * tc + i16;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float kv = kacc[tc][j] * inv, nd = vacc[tc][j] - kv;
                    kn4[tc][j] = kv;
                    dsq[tc] += nd * nd;
                    kT[(4 * q + j) * DKS + t] = kv;
                    ndT[(4 * q + j) * DKS + t] = nd;
                }
            }
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) dsq[tc] = xor16_32_sum(dsq[tc]);
            // lane 16 tc + i16 owns the token of column i16 of tile tc
#define VH_OWN(v) (TCW == 4 ? (q == 0 ? v[0] : q == 1 ? v[1] : q == 2 ? v[2 % TCW] : v[3 % TCW]) \
                             : (q == 1 ? v[1 % TCW] : v[0]))
            float alpha, eff;
            token_gates_fast(p.k, VH_OWN(pe), VH_OWN(pq), VH_OWN(dsq), VH_OWN(ksq), alpha, eff);
            // Per-slot scalars.  A tile is one DPP row, where cl is the inclusive prefix sum
            // of log2 alpha; the block decay a_15 is 2^cl at its last slot (tot).  The
            // triangle's ratio a_{t-1} / a_s = 2^(clx_t - cl_s) (clx = cl - log2 alpha) is
            // split into a row factor rho_s = eta^_s 2^(m - cl_s) and a column factor
            // kappa_t = 2^(clx_t - m) about the block's midpoint m = tot / 2: both exponents
            // stay within |tot| / 2 <= 116 (alpha >= sigmoid(-10) per token), so neither
            // factor overflows.
            const bool valid = slot_lane && my_slot < cnt;
            const float la = valid ? __builtin_amdgcn_logf(alpha) : 0.f;
            const float eh = valid ? eff : 0.f;
            float cl = la;
            cl += row_shr<1>(cl);
            cl += row_shr<2>(cl);
            cl += row_shr<4>(cl);
            cl += row_shr<8>(cl);
            float decay[TCW], tots[TCW];
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                tots[tc] = readlane_f(cl, 16 * tc + 15);
                decay[tc] = __builtin_amdgcn_exp2f(tots[tc]);
            }
            const float tot = VH_OWN(tots), mid = 0.5f * tot, clx = cl - la;
#undef VH_OWN
            if (slot_lane) {
                tk[lane] = eh * __builtin_amdgcn_exp2f(mid - cl);            // rho
                tk[TT + lane] = __builtin_amdgcn_exp2f(clx - mid);           // kappa
                tk[2 * TT + lane] = -__builtin_amdgcn_exp2f(clx);            // -a_{t-1}
                tk[3 * TT + lane] = eh * __builtin_amdgcn_exp2f(tot - cl);   // w
            }
            // prefetch the next tile's x operands
            {
                int64_t ncc = c;
                int nbase = base + S;
                if (nbase >= C) { ncc = c + 1; nbase = 0; }
                have_next = ncc < nc - 1;
                if (have_next) issue_tile(ncc, nbase, min(S, C - nbase), xr, xvalid);
            }
            __syncthreads();
            // ---- L = diag(rho) K^T K diag(kappa), strict upper triangle (lane 16 q + t,
            //      entry j: L[4q + j][t]), stored by columns: Lc[tc][t][s] = L[s][t].  The
            //      Gram tile K^T K takes the keys split once (the same registers are its A
            //      and B operands); row and column factors scale it after the product
            //      (rho_s P kappa_t <= 1 for s < t, each factor below 2^117) ----
#pragma unroll
            for (int tc = 0; tc < TCW; ++tc) {
                const float kap = tk[TT + 16 * tc + i16];
                const float4 r4 = ld4(tk + 16 * tc + 4 * q);   // rho of rows 4q..4q+3
                const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
                v4s kh, kl;
                split4(kn4[tc], kh, kl);
                const v4f P = mma3(kh, kl, kh, kl, v4f{0.f, 0.f, 0.f, 0.f});
                float lv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) lv[j] = (4 * q + j < i16) ? (P[j] * rr[j]) * kap : 0.f;
                *reinterpret_cast<float4*>(Lc + (16 * tc + i16) * LS + 4 * q) = make_float4(lv[0], lv[1], lv[2], lv[3]);
            }
            __syncthreads();
            // ---- Z = (I + L)^-1 W K^T: lane 16 b + f solves column f of tile b from the last
            //      row up, Z[s][f] = w_s k_s[f] - sum_{v > s} L[s][v] Z[v][f] ----
            if (q < TCW) {
                float acc[16], zc[16];
#pragma unroll
                for (int s0 = 0; s0 < 16; s0 += 4) {
                    const float4 k4 = ld4(kT + i16 * DKS + 16 * q + s0);
                    const float4 w4 = ld4(tk + 3 * TT + 16 * q + s0);
                    acc[s0] = k4.x * w4.x; acc[s0 + 1] = k4.y * w4.y;
                    acc[s0 + 2] = k4.z * w4.z; acc[s0 + 3] = k4.w * w4.w;
                }
                // four columns of L at a time (rows s < v of column v); the next group's
                // loads are issued before the current group's arithmetic
                float lA[4][16], lB[4][16];
                auto load_group = [&](int v0, float (&buf)[4][16]) {
#pragma unroll
                    for (int dv = 0; dv < 4; ++dv)
#pragma unroll
                        for (int s0 = 0; s0 < v0 + dv; s0 += 4) {
                            const float4 l4 = ld4(Lc + (16 * q + v0 + dv) * LS + s0);
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
                __builtin_amdgcn_sched_barrier(0);
                solve_group(12, lA);
                __builtin_amdgcn_sched_barrier(0);
                load_group(4, lA);
                __builtin_amdgcn_sched_barrier(0);
                solve_group(8, lB);
                __builtin_amdgcn_sched_barrier(0);
                load_group(0, lB);
                __builtin_amdgcn_sched_barrier(0);
                solve_group(4, lA);
                solve_group(0, lB);
                float* dst = Zs + (16 * q + i16) * LS;
#pragma unroll
                for (int s = 0; s < 16; s += 4)
                    *reinterpret_cast<float4*>(dst + s) = make_float4(zc[s], zc[s + 1], zc[s + 2], zc[s + 3]);
            }
            __syncthreads();
            // ---- per block X_b (and Y_b or Y_b^T) on the matrix cores, all tiles at once;
            //      then the composition G <- G X_b + Y_b, the only serial step.  ONE: the
            //      chunk is this single full pass (first block: tile 0 of each line, last:
            //      tile TPL - 1), so each block's products are fixed at compile time. ----
            const int nblk = (cnt + 15) / 16;
            auto blocks = [&](auto one_c) {
            constexpr bool ONE = decltype(one_c)::value;
            // block bt's X/Y products are issued right before its composition step, so they
            // overlap the previous step's matrix-core latency
#pragma unroll
            for (int bt = 0; bt < TPL; ++bt) {
                if (!ONE && bt >= nblk) break;
                const bool first = ONE ? bt == 0 : (g_identity && bt == 0);
                const bool last = ONE ? bt == TPL - 1 : (last_pass && bt == nblk - 1);
                v4s xh[NL], xl[NL];
                v4f yc[NL];
#pragma unroll
                for (int lam = 0; lam < NL; ++lam) {
                    const int tc = lam * TPL + bt;
                    // D(Z): lane 16 q + f holds Z[4q + j][f]; feature-major operands of the
                    // block (slot 4q + j, feature f): -(k a_{t-1}) and -delta
                    const float4 z4 = ld4(Zs + (16 * tc + i16) * LS + 4 * q);
                    const float4 k4 = ld4(kT + i16 * DKS + 16 * tc + 4 * q);
                    const float4 d4 = ld4(ndT + i16 * DKS + 16 * tc + 4 * q);
                    const float4 a4 = ld4(tk + 2 * TT + 16 * tc + 4 * q);
                    const float zv[4] = {z4.x, z4.y, z4.z, z4.w};
                    const float nka[4] = {k4.x * a4.x, k4.y * a4.y, k4.z * a4.z, k4.w * a4.w};
                    const float ndl[4] = {d4.x, d4.y, d4.z, d4.w};
                    v4s zh, zl;
                    split4(zv, zh, zl);
                    const v4f dI = diag4(decay[tc], q, i16);
                    if (first) {
                        // G_b = I: G_{b+1} = X_b + Y_b = a_15 I - (K D_a + Delta) Z, or its transpose
                        const float nb[4] = {nka[0] + ndl[0], nka[1] + ndl[1], nka[2] + ndl[2], nka[3] + ndl[3]};
                        v4s nbh, nbl;
                        split4(nb, nbh, nbl);
                        if (last) gD[lam] = mma3(nbh, nbl, zh, zl, dI);
                        else gT[lam] = mma3(zh, zl, nbh, nbl, dI);
                    } else {
                        v4s kah, kal, dlh, dll;
                        split4(nka, kah, kal);
                        split4(ndl, dlh, dll);
                        split4(mma3(kah, kal, zh, zl, dI), xh[lam], xl[lam]);               // D(X_b)
                        if (last) yc[lam] = mma3(dlh, dll, zh, zl, v4f{0.f, 0.f, 0.f, 0.f});    // D(Y_b)
                        else yc[lam] = mma3(zh, zl, dlh, dll, v4f{0.f, 0.f, 0.f, 0.f});         // D(Y_b^T)
                    }
                }
                if (first) continue;
#pragma unroll
                for (int lam = 0; lam < NL; ++lam) {
                    v4s gh, gl;
                    split4(gT[lam], gh, gl);
                    if (last) gD[lam] = mma3(gh, gl, xh[lam], xl[lam], yc[lam]);      // G_b X_b + Y_b
                    else gT[lam] = mma3(xh[lam], xl[lam], gh, gl, yc[lam]);           // X_b^T G_b^T + Y_b^T
                }
            }
            };
            if (g_identity && last_pass && nblk == TPL) blocks(std::true_type{});
            else blocks(std::false_type{});
            g_identity = false;
            __syncthreads();
        }
        // ---- refresh: S^T <- G^T S^T (A: G in its accumulator layout; B: S as held) ----
#pragma unroll
        for (int lam = 0; lam < NL; ++lam) {
            v4s gh, gl;
            split4(gD[lam], gh, gl);
#pragma unroll
            for (int R = 0; R < 4; ++R) {
                v4s sh, sl;
                split4(sA[lam][R], sh, sl);
                const v4f o = mma3(gh, gl, sh, sl, v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int j = 0; j < 4; ++j) sA[lam][R][j] = o[j];
            }
            if (i16 < 2)
                *reinterpret_cast<float4*>(gr + (lam * 2 + i16) * D + 4 * q) =
                    make_float4(sA[lam][3][0], sA[lam][3][1], sA[lam][3][2], sA[lam][3][3]);
        }
        __syncthreads();
    }
}

template <typename T>
bool launch_scan16_ut(const ScanParams& sp, hipStream_t stream) {
    const int64_t lines = sp.B * sp.R * sp.heads;
    const int nl = sp.lines_per_wave, tcw = sp.tiles_per_wave;
    const unsigned grid = static_cast<unsigned>(lines / nl);
    auto go = [&](auto nlc, auto tcc, auto spc) {
        hipLaunchKernelGGL((srnl_scan16_ut_kernel<T, decltype(nlc)::value, decltype(tcc)::value, decltype(spc)::value>),
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
    return true;
}
template bool launch_scan16_ut<bf16_t>(const ScanParams&, hipStream_t);
template bool launch_scan16_ut<f16_t>(const ScanParams&, hipStream_t);
template bool launch_scan16_ut<float>(const ScanParams&, hipStream_t);

}  // namespace vh
