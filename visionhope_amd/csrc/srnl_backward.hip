// SRNL backward: gradients of the packed forward (y = readout of every token from the
// chunk-start memory) with respect to x, the queries and the five initial memories.
//
// The forward it differentiates (reference chunk.cu:252-509, memory.cuh:219-233), per
// line (b, r, head) with state S = (M_m, M_v, M_k, e, a) shared over the batch:
//   token t of chunk c:  q^ = q / max(|q|, 1e-12); y = M_m q^;  k~ = M_k x, v = M_v x,
//     k = k~ / sqrt(|k~|^2 + 1e-6); eta = ETA softplus(clamp(e.x)); alpha = AMIN +
//     (1 - AMIN) sigmoid(clamp(a.x + BIAS)); eta^ = softcap(eta, alpha, |k - v|) and the
//     spectral clamp;  G <- alpha G - eta^ (G k + k - v) k^T from G = I;
//   after the chunk: M_* <- M_* G, e <- G^T e, a <- G^T a.
// The backward follows the reference's subgradient conventions (chunk.cu:511-1057,
// memory.cuh:253-352): clamps pass the gradient for |pre-activation| <= 10, the spectral
// clamp routes it to alpha and |k|^2 only when it binds, and the query normalisation
// drops its projection below the epsilon.
//
// Structure (one workgroup of D lanes per line, lane i holding row i of the d x d
// matrices; all math fp32):
//   1. forward state pass: the chunk-start state of every chunk goes to the workspace;
//   2. chunks in reverse: the chunk's keys, values and gates are recomputed from its
//      start state, the gain trajectory G_0..G_{C-1} is stored (workspace), the upstream
//      state gradient dS' gives dG_C = sum M^T dM' + e de'^T + a da'^T and the start-state
//      gradient M' G^T, G de', then tokens run backwards through
//        G_{t+1} = alpha G_t - eta^ r k^T,  r = G_t k + k - v
//      with dG_t = alpha dG_{t+1} + r_bar k^T, r_bar = -eta^ dG_{t+1} k, and the gate,
//      normalisation and projection chains down to dx, dq and the start-state gradient;
//   3. per-line gradients of the initial memories, summed over the batch in line order
//      by a second kernel (deterministic).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "vh_common.h"

namespace vh {

constexpr int kBwdMaxChunk = 64;     // chunks up to this length use the small-LDS variant
constexpr int kBwdLongChunk = 256;   // longest chunk of the backward (lines.cu:252-760 range)

// The chunk buffers of a workgroup hold CMAX tokens: 64, or 256 when a direction's chunk
// is longer (the long-line backward; about 42 KB of LDS more at d = 16).
inline int bwd_cmax(int64_t max_chunk) { return max_chunk <= kBwdMaxChunk ? kBwdMaxChunk : kBwdLongChunk; }

struct BwdParams {
    const void* x;      // [B, R, heads, N, D] io dtype
    const void* q;      // raw: [B, R, N, heads * D] io dtype; else fp32 [B, R, heads, N, D]
    const float* dy;    // [B, R, heads, N, D]
    const float* m0[5]; // M_m, M_v, M_k [S, D, D]; M_eta, M_alpha [S, D]; S = R * heads, or one per line
    int per_line;       // 1: state s = line; 0: s = line % (R * heads), shared over the batch
    float* dx;          // [B, R, heads, N, D]
    float* dq;          // layout of q, fp32
    float* dline;       // [lines, 3 D^2 + 2 D] per-line gradient of the initial state
    float* states;      // [lines, nc, 3 D^2 + 2 D] chunk-start states
    float* gtraj;       // [lines, CMAX, D, D] gain trajectory of the current chunk
    int64_t B, R, heads, N, nc;
    int chunk[4];
    vh_srnl_consts k;
};

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum over the D-lane group of this lane, on the VALU (DPP and the gfx950 row swap; no LDS
// round trip).  Every step adds lane pairs that exchange values (row mirror, half-row
// mirror, quad xor 1 and 2, row xor), so all lanes of a group end with the same bits.
template <int D>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(D == 4 || D == 8 || D == 16 || D == 32, "group of 4, 8, 16 or 32 lanes");
    if constexpr (D >= 16) v += dpp_f<0x140>(v);   // row_mirror: lane l <-> 15 - l
    if constexpr (D >= 8) v += dpp_f<0x141>(v);    // row_half_mirror: l <-> 7 - l in each 8
    v += dpp_f<0xB1>(v);                           // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4E>(v);                           // quad_perm [2, 3, 0, 1]
    if constexpr (D == 32) {
        const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
    }
    return v;
}

// Keeps the compiler from moving LDS loads across this point (so the matrix products
// below load operands where they are used instead of holding whole matrices in registers).
__device__ __forceinline__ void lds_fence() { asm volatile("" ::: "memory"); }

template <typename T>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
    return to_f32(static_cast<const T*>(p)[i]);
}

// d(eta^)/d(cap) of eta^ = cap (1 - exp(-u)), u = eta / cap: (1 - e^-u) - u e^-u, by its
// series u^2 (1/2 - u/3 + u^2/8 - u^3/30 + u^4/144) below u = 1e-3 (cancellation).
__device__ __forceinline__ float softcap_dcap(float u, float e_neg) {
    if (u < 1e-3f) return u * u * (0.5f + u * (-1.f / 3.f + u * (1.f / 8.f + u * (-1.f / 30.f + u / 144.f))));
    return -expm1f(-u) - u * e_neg;
}

// LPW lines per workgroup, D lanes each (lines ln = LPW blockIdx.x + sub share (b, r), so
// they run the same chunk schedule and meet every barrier together).
template <int D, typename T, bool QRAW, int CMAX, int LPW>
__global__ __launch_bounds__(D * LPW) void srnl_backward_kernel(const BwdParams p) {
    constexpr int SD = 3 * D * D + 2 * D, P = D + 1;
    __shared__ float Ms_[LPW][3][D][P];     // chunk-start M_m, M_v, M_k
    __shared__ float Ev_[LPW][2][D];        // chunk-start e, a
    __shared__ float Gs_[LPW][D][P];        // a gain matrix (rows by lane)
    __shared__ float BG_[LPW][D][P];        // dG rows
    __shared__ float Up_[LPW][3][D][P];     // upstream state gradient dM'
    __shared__ float UpV_[LPW][2][D];       // upstream de', da'
    __shared__ float Kc_[LPW][CMAX][D], Vc_[LPW][CMAX][D];
    __shared__ float Sc_[LPW][CMAX][5];     // eta, alpha, d eta/d pre, d alpha/d pre, 1/|k~|
    __shared__ float Vec_[LPW][6][D];       // x, dy, q^, r, r_bar / dk~, dv
    const int sub = static_cast<int>(threadIdx.x) / D;
    float(&Ms)[3][D][P] = Ms_[sub];
    float(&Ev)[2][D] = Ev_[sub];
    float(&Gs)[D][P] = Gs_[sub];
    float(&BG)[D][P] = BG_[sub];
    float(&Up)[3][D][P] = Up_[sub];
    float(&UpV)[2][D] = UpV_[sub];
    float(&Kc)[CMAX][D] = Kc_[sub];
    float(&Vc)[CMAX][D] = Vc_[sub];
    float(&Sc)[CMAX][5] = Sc_[sub];
    float(&Vec)[6][D] = Vec_[sub];

    const int i = static_cast<int>(threadIdx.x) % D;
    const int64_t ln = static_cast<int64_t>(blockIdx.x) * LPW + sub;
    const int64_t RH = p.R * p.heads;
    const int64_t s = p.per_line ? ln : ln % RH;
    const int r_dir = static_cast<int>((ln / p.heads) % p.R);
    const int64_t b = ln / RH, head = ln % p.heads;
    const int C = p.chunk[r_dir];
    const int64_t N = p.N, nc = (N + C - 1) / C;
    const int64_t nc_alloc = p.nc;
    const float ETA = p.k.step_scale, AMIN = p.k.min_retention, BIAS = p.k.retention_bias, MU = p.k.injection_margin;
    const float FAC = p.k.spectral_factor;
    const bool CLAMP = p.k.spectral_clamp != 0;

    const int64_t xbase = ln * N * D;   // packed [B, R, heads, N, D] == line-major
    auto x_at = [&](int64_t t) { return t < N ? ld<T>(p.x, xbase + t * D + i) : 0.f; };
    auto q_index = [&](int64_t t) -> int64_t {
        if constexpr (QRAW) return ((b * p.R + r_dir) * N + t) * (p.heads * D) + head * D + i;
        else return xbase + t * D + i;
    };
    auto q_at = [&](int64_t t) {
        if constexpr (QRAW) return t < N ? ld<T>(p.q, q_index(t)) : 1.f;
        else return t < N ? static_cast<const float*>(p.q)[q_index(t)] : 1.f;
    };

    // ---- state in LDS: lane i writes row i -------------------------------------------
    auto load_state = [&](const float* src) {   // src: [3 D^2 + 2 D] (rows of M_m, M_v, M_k, then e, a)
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int j = 0; j < D; ++j) Ms[m][i][j] = src[m * D * D + i * D + j];
        Ev[0][i] = src[3 * D * D + i];
        Ev[1][i] = src[3 * D * D + D + i];
    };
    auto store_state = [&](float* dst) {
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int j = 0; j < D; ++j) dst[m * D * D + i * D + j] = Ms[m][i][j];
        dst[3 * D * D + i] = Ev[0][i];
        dst[3 * D * D + D + i] = Ev[1][i];
    };
    float* my_states = p.states + ln * nc_alloc * SD;
    float* my_traj = p.gtraj + ln * CMAX * D * D;

    // Keys, values and gates of the tokens of chunk c from the state in Ms / Ev.
    auto token_data = [&](int64_t c) {
        for (int tl = 0; tl < C; ++tl) {
            const int64_t t = c * C + tl;
            const float xi = x_at(t);
            Vec[0][i] = xi;
            __syncthreads();
            float kr = 0.f, vv = 0.f;
#pragma unroll
            for (int j = 0; j < D; ++j) {
                kr += Ms[2][i][j] * Vec[0][j];
                vv += Ms[1][i][j] * Vec[0][j];
            }
            const float pe_raw = group_sum<D>(Ev[0][i] * xi);
            const float pa_raw = group_sum<D>(Ev[1][i] * xi) + BIAS;
            const float inv_k = rsqrtf(group_sum<D>(kr * kr) + 1e-6f);
            Kc[tl][i] = kr * inv_k;
            Vc[tl][i] = vv;
            if (i == 0) {
                const float ep = fminf(10.f, fmaxf(-10.f, pe_raw));
                const float ap = fminf(10.f, fmaxf(-10.f, pa_raw));
                const float sp = ep > 20.f ? ep : logf(1.f + expf(ep));
                const float sg = 1.f / (1.f + expf(-ap));
                Sc[tl][0] = ETA * sp;
                Sc[tl][1] = AMIN + (1.f - AMIN) * sg;
                Sc[tl][2] = fabsf(pe_raw) <= 10.f ? ETA * (ep > 20.f ? 1.f : 1.f / (1.f + expf(-ep))) : 0.f;
                Sc[tl][3] = fabsf(pa_raw) <= 10.f ? (1.f - AMIN) * sg * (1.f - sg) : 0.f;
                Sc[tl][4] = inv_k;
            }
            __syncthreads();
        }
    };
    // eta^ of token tl (with its derivatives when wanted); every lane gets the values.
    struct Gate {
        float eff, deff_deta, deff_dcap, deff_dalpha, deff_dksq, cap, denom, dn, ksq;
    };
    auto gate = [&](int tl) {
        Gate o;
        const float ki = Kc[tl][i], di = ki - Vc[tl][i];
        o.dn = sqrtf(group_sum<D>(di * di) + 1e-12f);
        o.ksq = group_sum<D>(ki * ki);
        const float eta = Sc[tl][0], alpha = Sc[tl][1];
        o.denom = o.dn + 1e-6f;
        o.cap = MU * (1.f - alpha) / o.denom;
        const float u = eta / o.cap, e_neg = expf(-u);
        o.eff = o.cap * (-expm1f(-u));
        o.deff_deta = e_neg;
        o.deff_dcap = softcap_dcap(u, e_neg);
        o.deff_dalpha = 0.f;
        o.deff_dksq = 0.f;
        if (CLAMP) {
            const float den = fmaxf(o.ksq, 1e-20f);
            const float lim = nextafterf(FAC * alpha / den, 0.f);
            if (o.eff > lim) {
                o.eff = lim;
                o.deff_deta = 0.f;
                o.deff_dcap = 0.f;
                o.deff_dalpha = FAC / den;
                if (o.ksq > 1e-20f) o.deff_dksq = -FAC * alpha / (den * den);
            }
        }
        return o;
    };

    // ---- 1. forward state pass ---------------------------------------------------------
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
        for (int j = 0; j < D; ++j) Ms[m][i][j] = p.m0[m][s * D * D + i * D + j];
    Ev[0][i] = p.m0[3][s * D + i];
    Ev[1][i] = p.m0[4][s * D + i];
    __syncthreads();
    for (int64_t c = 0; c < nc; ++c) {
        store_state(my_states + c * SD);
        if (c == nc - 1) break;
        token_data(c);
        float gr[D];
#pragma unroll
        for (int j = 0; j < D; ++j) gr[j] = i == j ? 1.f : 0.f;
        for (int tl = 0; tl < C; ++tl) {
            const Gate o = gate(tl);
            float ri = Kc[tl][i] - Vc[tl][i];
#pragma unroll
            for (int j = 0; j < D; ++j) ri += gr[j] * Kc[tl][j];
            const float alpha = Sc[tl][1];
#pragma unroll
            for (int j = 0; j < D; ++j) gr[j] = alpha * gr[j] - o.eff * ri * Kc[tl][j];
        }
#pragma unroll
        for (int j = 0; j < D; ++j) Gs[i][j] = gr[j];
        __syncthreads();
        // S <- S G (row i of each matrix, through Up as scratch), e <- G^T e, a <- G^T a
#pragma unroll 1
        for (int m = 0; m < 3; ++m) {
            // out = row_i(M_m) G, accumulated over the rows l of G: row l is one broadcast
            // read of D consecutive floats for every lane, so its loads issue back to back
            float out[D];
#pragma unroll
            for (int j = 0; j < D; ++j) out[j] = 0.f;
#pragma unroll
            for (int l = 0; l < D; ++l) {
                const float r = Ms[m][i][l];
#pragma unroll
                for (int j = 0; j < D; ++j) out[j] += r * Gs[l][j];
            }
#pragma unroll
            for (int j = 0; j < D; ++j) Up[m][i][j] = out[j];
        }
        float ne = 0.f, na = 0.f;
#pragma unroll
        for (int l = 0; l < D; ++l) {
            ne += Gs[l][i] * Ev[0][l];
            na += Gs[l][i] * Ev[1][l];
        }
        __syncthreads();
#pragma unroll 1
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int j = 0; j < D; ++j) Ms[m][i][j] = Up[m][i][j];
        Ev[0][i] = ne;
        Ev[1][i] = na;
        __syncthreads();
    }

    // ---- 2. chunks in reverse ----------------------------------------------------------
#pragma unroll
    for (int m = 0; m < 3; ++m)
#pragma unroll
        for (int j = 0; j < D; ++j) Up[m][i][j] = 0.f;
    UpV[0][i] = 0.f;
    UpV[1][i] = 0.f;
    __syncthreads();
    for (int64_t c = nc - 1; c >= 0; --c) {
        load_state(my_states + c * SD);
        __syncthreads();
        token_data(c);
        // Gain trajectory: G_t (row i) for every token, then G_C.
        float gr[D];
#pragma unroll
        for (int j = 0; j < D; ++j) gr[j] = i == j ? 1.f : 0.f;
        for (int tl = 0; tl < C; ++tl) {
#pragma unroll
            for (int j = 0; j < D; ++j) my_traj[(tl * D + i) * D + j] = gr[j];
            const Gate o = gate(tl);
            float ri = Kc[tl][i] - Vc[tl][i];
#pragma unroll
            for (int j = 0; j < D; ++j) ri += gr[j] * Kc[tl][j];
            const float alpha = Sc[tl][1];
#pragma unroll
            for (int j = 0; j < D; ++j) gr[j] = alpha * gr[j] - o.eff * ri * Kc[tl][j];
        }
#pragma unroll
        for (int j = 0; j < D; ++j) Gs[i][j] = gr[j];
        __syncthreads();
        // dG_C row i: sum_m (M_m^T dM'_m)[i][j] + e_i de'_j + a_i da'_j (reads every row of
        // the upstream gradient, so before it is replaced below).
        float bg[D];
#pragma unroll
        for (int j = 0; j < D; ++j) bg[j] = Ev[0][i] * UpV[0][j] + Ev[1][i] * UpV[1][j];
#pragma unroll 1
        for (int m = 0; m < 3; ++m) {
            // bg += column_i(M_m)^T dM'_m, over the rows l of dM'_m (broadcast row reads)
#pragma unroll
            for (int l = 0; l < D; ++l) {
                const float cl = Ms[m][l][i];
#pragma unroll
                for (int j = 0; j < D; ++j) bg[j] += cl * Up[m][l][j];
            }
        }
        float acc_e = 0.f, acc_a = 0.f;
#pragma unroll
        for (int l = 0; l < D; ++l) {
            acc_e += Gs[i][l] * UpV[0][l];
            acc_a += Gs[i][l] * UpV[1][l];
        }
        __syncthreads();
        // Start-state gradient from the refresh S' = S G: dM = dM' G^T (row i from row i
        // of dM', in place; the tokens below add to it), de = G de'.
#pragma unroll 1
        for (int m = 0; m < 3; ++m) {
            float out[D];
#pragma unroll
            for (int j = 0; j < D; ++j) out[j] = 0.f;
#pragma unroll
            for (int l = 0; l < D; ++l) {   // column l of G: a broadcast read for every lane
                const float r = Up[m][i][l];
#pragma unroll
                for (int j = 0; j < D; ++j) out[j] += r * Gs[j][l];
            }
#pragma unroll
            for (int j = 0; j < D; ++j) Up[m][i][j] = out[j];
        }
        __syncthreads();

        const int64_t t_end = min(static_cast<int64_t>(C), N - c * C);   // real tokens of the chunk
        for (int tl = static_cast<int>(t_end) - 1; tl >= 0; --tl) {
            const int64_t t = c * C + tl;
            float gt[D];
#pragma unroll
            for (int j = 0; j < D; ++j) gt[j] = my_traj[(tl * D + i) * D + j];
            const float xi = x_at(t), dyi = p.dy[xbase + t * D + i];
            const float q_raw = q_at(t);
            const float qinv = QRAW ? 1.f / fmaxf(sqrtf(group_sum<D>(q_raw * q_raw)), 1e-12f) : 1.f;
            const float qi = q_raw * qinv;
            const float ki = Kc[tl][i], vi = Vc[tl][i], di = ki - vi;
            const float alpha = Sc[tl][1];
            float ri = di;
#pragma unroll
            for (int j = 0; j < D; ++j) ri += gt[j] * Kc[tl][j];
            const Gate o = gate(tl);
            Vec[0][i] = xi;
            Vec[1][i] = dyi;
            Vec[2][i] = qi;
            Vec[3][i] = ri;
#pragma unroll
            for (int j = 0; j < D; ++j) {
                Gs[i][j] = gt[j];
                BG[i][j] = bg[j];
            }
            __syncthreads();
            // Readout: dM_m += dy q^T; dq^ = M_m^T dy.
#pragma unroll
            for (int j = 0; j < D; ++j) Up[0][i][j] += dyi * Vec[2][j];
            float dqh = 0.f;
#pragma unroll
            for (int l = 0; l < D; ++l) dqh += Ms[0][l][i] * Vec[1][l];
            // Recurrence step.
            float part_alpha = 0.f, hk = 0.f;
#pragma unroll
            for (int j = 0; j < D; ++j) {
                part_alpha += bg[j] * gt[j];
                hk += bg[j] * Kc[tl][j];
            }
            float d_alpha = group_sum<D>(part_alpha);
            const float d_eff = -group_sum<D>(ri * hk);
            const float rbar = -o.eff * hk;
            Vec[4][i] = rbar;
            __syncthreads();
            float htr = 0.f, gtrbar = 0.f;
#pragma unroll
            for (int l = 0; l < D; ++l) {
                htr += BG[l][i] * Vec[3][l];
                gtrbar += Gs[l][i] * Vec[4][l];
            }
            const float d_eta = d_eff * o.deff_deta;
            const float d_cap = d_eff * o.deff_dcap;
            d_alpha += d_cap * (-MU / o.denom) + d_eff * o.deff_dalpha;
            const float d_dn = d_cap * (-o.cap / o.denom);
            const float d_ksq = d_eff * o.deff_dksq;
            float dk = -o.eff * htr + gtrbar + rbar + d_dn * di / o.dn + 2.f * d_ksq * ki;
            const float dv = -rbar - d_dn * di / o.dn;
#pragma unroll
            for (int j = 0; j < D; ++j) bg[j] = alpha * bg[j] + rbar * Kc[tl][j];
            const float kdot = group_sum<D>(dk * ki);
            const float dkr = (dk - kdot * ki) * Sc[tl][4];
            const float d_apre = d_alpha * Sc[tl][3];
            const float d_epre = d_eta * Sc[tl][2];
            __syncthreads();   // every lane has read r and r_bar
#pragma unroll
            for (int j = 0; j < D; ++j) {
                Up[1][i][j] += dv * Vec[0][j];
                Up[2][i][j] += dkr * Vec[0][j];
            }
            acc_e += xi * d_epre;
            acc_a += xi * d_apre;
            Vec[5][i] = dv;
            Vec[4][i] = dkr;   // r_bar was consumed above
            __syncthreads();
            float dxi = d_epre * Ev[0][i] + d_apre * Ev[1][i];
#pragma unroll
            for (int l = 0; l < D; ++l) dxi += Ms[1][l][i] * Vec[5][l] + Ms[2][l][i] * Vec[4][l];
            float dqi = dqh;
            if constexpr (QRAW) {
                const float qdot = group_sum<D>(dqh * qi);
                dqi = qinv > 9.999e11f ? dqh * qinv : (dqh - qi * qdot) * qinv;
            }
            p.dx[xbase + t * D + i] = dxi;
            p.dq[q_index(t)] = dqi;
            __syncthreads();
        }
        // The start-state gradient (in Up) becomes the upstream gradient of chunk c - 1.
        UpV[0][i] = acc_e;
        UpV[1][i] = acc_a;
        __syncthreads();
    }
    {
        float* dst = p.dline + ln * SD;
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int j = 0; j < D; ++j) dst[m * D * D + i * D + j] = Up[m][i][j];
        dst[3 * D * D + i] = UpV[0][i];
        dst[3 * D * D + D + i] = UpV[1][i];
    }
}

// dM[s] = sum over b of the per-line gradients of lines b * S + s, in b order.
__global__ __launch_bounds__(256) void srnl_backward_reduce_kernel(const float* dline, int64_t batch, int64_t S,
                                                                   int d, float* dmm, float* dmv, float* dmk,
                                                                   float* dme, float* dma) {
    const int64_t SD = 3 * d * d + 2 * d;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= S * SD) return;
    const int64_t s = idx / SD, e = idx % SD;
    float acc = 0.f;
    for (int64_t b = 0; b < batch; ++b) acc += dline[(b * S + s) * SD + e];
    const int64_t dd = static_cast<int64_t>(d) * d;
    if (e < dd) dmm[s * dd + e] = acc;
    else if (e < 2 * dd) dmv[s * dd + e - dd] = acc;
    else if (e < 3 * dd) dmk[s * dd + e - 2 * dd] = acc;
    else if (e < 3 * dd + d) dme[s * d + e - 3 * dd] = acc;
    else dma[s * d + e - 3 * dd - d] = acc;
}

namespace {

struct BwdLayout {
    int64_t lines, nc, sd, cmax;
    size_t states, traj, dline, total;
};

BwdLayout bwd_layout(int64_t B, int64_t R, int64_t heads, int64_t N, int d, const int64_t* chunks) {
    BwdLayout l{};
    l.lines = B * R * heads;
    l.nc = 0;
    for (int64_t r = 0; r < R; ++r) l.nc = std::max<int64_t>(l.nc, (N + chunks[r] - 1) / chunks[r]);
    l.sd = 3 * int64_t(d) * d + 2 * d;
    auto round = [](size_t v) { return (v + 63) / 64 * 64; };
    l.states = round(static_cast<size_t>(l.lines * l.nc * l.sd));
    int64_t cmax = 0;
    for (int64_t r = 0; r < R; ++r) cmax = std::max<int64_t>(cmax, chunks[r]);
    l.cmax = bwd_cmax(cmax);
    l.traj = round(static_cast<size_t>(l.lines * l.cmax * d * d));
    l.dline = round(static_cast<size_t>(l.lines * l.sd));
    l.total = (l.states + l.traj + l.dline) * sizeof(float);
    return l;
}

}  // namespace
}  // namespace vh

using namespace vh;

extern "C" {

size_t vh_srnl_backward_workspace_bytes(int64_t B, int64_t R, int64_t heads, int64_t N, int32_t head_dim,
                                        const int64_t* chunks) {
    if (B <= 0 || R <= 0 || R > 4 || heads <= 0 || N <= 0 || chunks == nullptr) return 0;
    if (head_dim != 4 && head_dim != 8 && head_dim != 16 && head_dim != 32) return 0;
    for (int64_t r = 0; r < R; ++r)
        if (chunks[r] <= 0 || chunks[r] > kBwdLongChunk) return 0;
    return bwd_layout(B, R, heads, N, head_dim, chunks).total;
}

int vh_srnl_backward(const void* x, const void* q, int32_t io_dtype, int32_t q_raw, const float* dy,
                     const float* M_m, const float* M_v, const float* M_k, const float* M_eta, const float* M_alpha,
                     int32_t memories_per_line, float* dx, float* dq, float* dM_m, float* dM_v, float* dM_k, float* dM_eta, float* dM_alpha,
                     int64_t B, int64_t R, int64_t heads, int64_t N, int32_t head_dim, const int64_t* chunks,
                     const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes, void* stream) {
    VH_REQUIRE(x && q && dy && M_m && M_v && M_k && M_eta && M_alpha && dx && dq && dM_m && dM_v && dM_k &&
                   dM_eta && dM_alpha && chunks && consts,
               VH_ERR_ARG, "SRNL backward pointers must not be null");
    VH_REQUIRE(B > 0 && heads > 0 && N > 0, VH_ERR_SHAPE, "SRNL backward needs nonempty [B, R, heads, N] lines");
    VH_REQUIRE(R == 1 || R == 2 || R == 4, VH_ERR_SHAPE, "directions must be 1, 2 or 4, got %lld", (long long)R);
    {
        const int rc = check_srnl_consts(consts);
        if (rc) return rc;
    }
    VH_REQUIRE(head_dim == 4 || head_dim == 8 || head_dim == 16 || head_dim == 32, VH_ERR_HEAD_DIM,
               "SRNL backward supports head_dim 4, 8, 16 and 32; got %d", head_dim);
    VH_REQUIRE(valid_dtype(io_dtype), VH_ERR_DTYPE, "unsupported io dtype code %d", io_dtype);
    for (int64_t r = 0; r < R; ++r)
        VH_REQUIRE(chunks[r] > 0 && chunks[r] <= kBwdLongChunk, VH_ERR_ARG,
                   "SRNL backward chunk lengths must be in [1, %d], got %lld", kBwdLongChunk, (long long)chunks[r]);
    const BwdLayout lay = bwd_layout(B, R, heads, N, head_dim, chunks);
    VH_REQUIRE(workspace && workspace_bytes >= lay.total, VH_ERR_WORKSPACE,
               "SRNL backward workspace needs %zu bytes, got %zu", lay.total, workspace ? workspace_bytes : (size_t)0);
    VH_REQUIRE(lay.lines * lay.nc * lay.sd < (int64_t(1) << 40), VH_ERR_SHAPE, "SRNL backward problem too large");
    BwdParams bp{};
    bp.x = x; bp.q = q; bp.dy = dy; bp.per_line = memories_per_line ? 1 : 0;
    bp.m0[0] = M_m; bp.m0[1] = M_v; bp.m0[2] = M_k; bp.m0[3] = M_eta; bp.m0[4] = M_alpha;
    bp.dx = dx; bp.dq = dq;
    float* ws = static_cast<float*>(workspace);
    bp.states = ws;
    bp.gtraj = ws + lay.states;
    bp.dline = ws + lay.states + lay.traj;
    bp.B = B; bp.R = R; bp.heads = heads; bp.N = N; bp.nc = lay.nc;
    for (int r = 0; r < 4; ++r) bp.chunk[r] = static_cast<int>(chunks[r < R ? r : R - 1]);
    bp.k = *consts;
    hipStream_t s = static_cast<hipStream_t>(stream);
    VH_REQUIRE(lay.lines < (int64_t(1) << 31), VH_ERR_SHAPE, "SRNL backward: too many lines");
    // Lines per workgroup: consecutive heads of one (b, r), as many as LDS allows (one line
    // of d = 16 with 64-token buffers needs about 19 KB; 256-token buffers 43 KB; d = 32
    // about 52 and 105 KB).
    auto launch = [&](auto kern, int lpw, int d) {
        hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(lay.lines / lpw)), dim3(d * lpw), 0, s, bp);
    };
    auto go = [&](auto dc, auto tv) {
        constexpr int D = decltype(dc)::value;
        using T = decltype(tv);
        constexpr int LS = D <= 16 ? 4 : 2;   // 64-token buffers
        constexpr int LL = D <= 16 ? 2 : 1;   // 256-token buffers
        if (lay.cmax == kBwdMaxChunk) {
            const bool packed = heads % LS == 0;
            if (q_raw) {
                if (packed) launch(srnl_backward_kernel<D, T, true, kBwdMaxChunk, LS>, LS, D);
                else launch(srnl_backward_kernel<D, T, true, kBwdMaxChunk, 1>, 1, D);
            } else {
                if (packed) launch(srnl_backward_kernel<D, T, false, kBwdMaxChunk, LS>, LS, D);
                else launch(srnl_backward_kernel<D, T, false, kBwdMaxChunk, 1>, 1, D);
            }
        } else {
            const bool packed = heads % LL == 0;
            if (q_raw) {
                if (packed) launch(srnl_backward_kernel<D, T, true, kBwdLongChunk, LL>, LL, D);
                else launch(srnl_backward_kernel<D, T, true, kBwdLongChunk, 1>, 1, D);
            } else {
                if (packed) launch(srnl_backward_kernel<D, T, false, kBwdLongChunk, LL>, LL, D);
                else launch(srnl_backward_kernel<D, T, false, kBwdLongChunk, 1>, 1, D);
            }
        }
    };
    auto by_type = [&](auto dc) {
        switch (io_dtype) {
            case VH_DTYPE_F32: go(dc, float{}); break;
            case VH_DTYPE_BF16: go(dc, bf16_t{}); break;
            default: go(dc, f16_t{}); break;
        }
    };
    switch (head_dim) {
        case 4: by_type(std::integral_constant<int, 4>{}); break;
        case 8: by_type(std::integral_constant<int, 8>{}); break;
        case 16: by_type(std::integral_constant<int, 16>{}); break;
        default: by_type(std::integral_constant<int, 32>{}); break;
    }
    int rc = check_launch("srnl_backward_kernel");
    if (rc) return rc;
    // Shared states: sum the B lines of each; one state per line: copy.
    const int64_t S = memories_per_line ? lay.lines : R * heads, batch = memories_per_line ? 1 : B;
    const int64_t total = S * lay.sd;
    hipLaunchKernelGGL(srnl_backward_reduce_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, s,
                       bp.dline, batch, S, head_dim, dM_m, dM_v, dM_k, dM_eta, dM_alpha);
    return check_launch("srnl_backward_reduce_kernel");
}

}  // extern "C"
