// SRNL scan with one line per workgroup of W waves (head_dim 16 and 32), for gfx950.
//
// The recurrence of a line (batch b, direction r, head h) is serial over its chunks; inside
// a chunk every token's key, value and gates come from the chunk-start state, and the gain
// G <- alpha G - eta^ (G k + k - v) k^T is serial over tokens but independent per ROW of G.
// This kernel spreads one line over W waves (one per SIMD of a CU) along those two
// parallel dimensions:
//
//   token phase   each wave takes its share of the chunk's 16-token tiles: [M_k; M_v] x and
//                 the gate pre-activations on the matrix cores, key norms by lane-group
//                 reductions, gates per token, and the 4-token block coefficients from
//                 neighbouring keys (DPP row shifts, no LDS round trip);
//   recurrence    wave w owns rows [w D/W, (w+1) D/W) of G and walks all tokens of the
//                 chunk in blocks of 4 (the exact regrouping of the serial update used by
//                 the single-wave scan): no communication between waves inside a chunk;
//   refresh       [M_m; M_v; M_k; e; a] <- [...] G on the matrix cores, 16-row tiles split
//                 over the waves.
//
// Keys, differences and coefficients of a 64-token segment are double-buffered in LDS, so
// one barrier separates a segment's token phase from its recurrence; the state is
// double-buffered, so the refresh needs two barriers per chunk.  Used when there are too
// few lines to give every SIMD a wave of its own (VisionHOPE-Base at 512^2, the d = 32
// operator of config 3) and for every head_dim-32 scan.
//
// Operands of the matrix products: lane l = 16 q + n supplies, for column n (a token, or
// a column of G), the K-range [q D/4, (q+1) D/4), and receives rows 4q..4q+3 of column n
// (the v_mfma_f32_16x16x{4,16,32} layouts).  bf16 activations enter exactly; fp32 state
// enters as hi + lo bf16 parts (|v - hi - lo| <= 2^-16 |v|).  fp32 activations use the
// fp32 matrix cores throughout.
#include "srnl_device.h"

namespace vh {
namespace {

// TB token blocks: TB = 1 splits the rows of G over the W waves (every wave walks every
// token); TB > 1 also splits the tokens of a segment into TB contiguous blocks, one per
// group of W/TB waves.  The gain update is linear in (G, k - v), so block b maps the gain at
// its start to G X_b + Y_b, where X_b is the recurrence over the block started from the
// identity with k - v taken as zero and Y_b the recurrence started from zero with the
// actual k - v: both are the same row recurrence on 2D rows (rows of G are independent),
// computed for every block at once.  The blocks are then composed in order,
// G <- G X_b + Y_b, as D x D products on the fp32 matrix cores, which shortens the serial
// chain of a segment by the factor TB.
template <typename T, int D, int W, int TB, bool SPATIAL>
__global__ __launch_bounds__(64 * W) void srnl_scanw_kernel(const ScanParams p) {
    static_assert((D == 16 || D == 32) && (W == 1 || W == 2 || W == 4) && W % TB == 0, "scan shape");
    constexpr int KQ = D / 4;                       // K-range of a lane group
    constexpr int NRT = D / 16;                     // 16-row tiles of a D x D matrix
    constexpr int ROWS = 3 * D + 2;                 // M_m, M_v, M_k rows, then e, a
    constexpr int RT = (ROWS + 1 + 15) / 16;        // state row tiles, with a zero row after a
    constexpr int SR = RT * 16 * D;                 // floats of one state buffer
    constexpr int SEG = (TB > 1 && D == 16) ? 128 : 64;   // tokens per segment
    constexpr int NBUF = TB > 1 ? 1 : 2;            // segment buffers (double-buffered rows mode)
    constexpr int TPW = SEG / 16 / W;               // tiles per wave per segment
    constexpr int RB = W / TB;                      // row groups
    constexpr int RW = (TB > 1 ? 2 * D : D) / RB;   // recurrence rows per wave (X and Y rows when TB > 1)
    constexpr int RL = 64 / RW, E = D / RL;         // lanes per row, entries per lane
    static_assert(RL >= 2 && RL <= 16 && E >= 1, "recurrence layout");
    constexpr int GS = D + 1, DKS = SEG + 4;
    constexpr bool kBf16 = std::is_same<T, bf16_t>::value;
    constexpr bool kRefreshBf16 = kBf16 && D == 32;
    using Bf = BfOp<D>;
    using Half = typename Bf::type;

    __shared__ __align__(16) float St[2 * SR];          // state, double-buffered across chunks
    __shared__ __align__(16) float Gs[2][D * GS];       // the chunk's gain (TB > 1: ping-pong while composing)
    __shared__ __align__(16) float kk[NBUF][SEG * D];   // normalised keys [slot][D]
    __shared__ __align__(16) float dkT[NBUF][D * DKS];  // (k - v)[row][slot]
    __shared__ __align__(16) float cf[NBUF][SEG * 8];   // block coefficients per slot
    __shared__ __align__(16) float XY[TB > 1 ? TB * 2 * D * GS : 1];   // X_b rows, then Y_b rows, per block

    const int64_t lines = p.B * p.R * p.heads;
    const int64_t line = xcd_remap(blockIdx.x, lines);
    const int64_t head = line % p.heads;
    const int r = static_cast<int>((line / p.heads) % p.R);
    const int64_t b = line / (p.heads * p.R);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, i16 = lane & 15, q = lane >> 4;
    {
        const int64_t s = p.per_line_state ? line : r * p.heads + head;
        for (int idx = tid; idx < D * D; idx += 64 * W) {
            St[idx] = p.Mm[s * D * D + idx];
            St[D * D + idx] = p.Mv[s * D * D + idx];
            St[2 * D * D + idx] = p.Mk[s * D * D + idx];
        }
        for (int idx = tid; idx < D; idx += 64 * W) {
            St[3 * D * D + idx] = p.Me[s * D + idx];
            St[(3 * D + 1) * D + idx] = p.Ma[s * D + idx];
        }
        for (int idx = ROWS * D + tid; idx < SR; idx += 64 * W) {
            St[idx] = 0.f;
            St[SR + idx] = 0.f;
        }
    }
    __syncthreads();

    const int C = chunk_of(p.chunk, r);
    const int64_t nc = (p.L + C - 1) / C;
    // Recurrence layout: lane -> (row, first column).  TB = 1: row grow of G.  TB > 1: wave
    // (tb, rb) holds pseudo-row prow of block tb: X_b row prow (< D) or Y_b row prow - D.
    const int tb = wv % TB, prow = (wv / TB) * RW + lane / RL, c0 = (lane % RL) * E;
    const int grow = TB > 1 ? prow % D : prow;                   // row of G (and of k - v) it follows
    const bool use_dk = TB == 1 || prow >= D;                    // X rows see k - v as zero
    const T* xcol = static_cast<const T*>(p.x.ptr) + b * p.x.sb + r * p.x.sr + head * p.x.sh + q * KQ;
    // Row/column chunks (spatial operator): token i of chunk cc is pixel pa*cc + pb*i + pc
    // (32-bit: the host allows this only when H*W*pixel_stride < 2^31).
    int pa = 0, pb = 0, pc = 0, pst = 0;
    if constexpr (SPATIAL) {
        const int Wd = static_cast<int>(p.x.W), L = static_cast<int>(p.x.H * p.x.W);
        pa = r == 0 ? Wd : r == 1 ? -Wd : r == 2 ? 1 : -1;
        pb = r == 0 ? 1 : r == 1 ? -1 : r == 2 ? Wd : -Wd;
        pc = (r & 1) ? L - 1 : 0;
        pst = static_cast<int>(p.x.st);
    }
    // x of this wave's tiles of segment (cc, sbase): loads issued without a branch (invalid
    // slots read the line's first token and are zeroed on use).
    XRaw<T, D> xr[TPW];
    unsigned vmask = 0;
    auto issue = [&](int64_t cc, int sbase, int scnt) {
        vmask = 0;
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const int slot = (wv + W * tt) * 16 + i16;
            const int64_t tok = cc * C + sbase + slot;
            const bool ok = slot < scnt && tok < p.L;
            vmask |= ok ? (1u << tt) : 0u;
            int64_t off = 0;
            if (ok) {
                if (SPATIAL && p.aligned) off = (pa * static_cast<int>(cc) + pb * (sbase + slot) + pc) * pst;
                else off = token_offset<SPATIAL>(p.x, r, tok);
            }
            xr[tt] = load_xraw<T, D>(xcol + off);
        }
    };

    // Token phase of one 16-token tile (slots s0..s0+15 of the segment buffers).
    auto token_tile = [&](const float* Sc, const XRaw<T, D>& raw, bool valid, int s0, int buf) {
        v4f kacc[NRT], vacc[NRT], gacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < NRT; ++t) kacc[t] = vacc[t] = v4f{0.f, 0.f, 0.f, 0.f};
        const int grow_row = 3 * D + min(i16 & 3, 2);   // e, a, then a zero row
        if constexpr (kBf16) {
            const Half xs = valid ? Bf::exact(raw) : Half{};
#pragma unroll
            for (int t = 0; t < NRT; ++t) {
                float ak[KQ], av[KQ];
                lds_vec<KQ>(Sc + (2 * D + 16 * t + i16) * D + q * KQ, ak);
                lds_vec<KQ>(Sc + (D + 16 * t + i16) * D + q * KQ, av);
                Half kh, kl, vh, vl;
                Bf::split(ak, kh, kl);
                Bf::split(av, vh, vl);
                kacc[t] = Bf::mma(kh, xs, kacc[t]);
                vacc[t] = Bf::mma(vh, xs, vacc[t]);
                kacc[t] = Bf::mma(kl, xs, kacc[t]);
                vacc[t] = Bf::mma(vl, xs, vacc[t]);
            }
            float ag[KQ];
            lds_vec<KQ>(Sc + grow_row * D + q * KQ, ag);
            Half gh, gl;
            Bf::split(ag, gh, gl);
            gacc = Bf::mma(gh, xs, gacc);
            gacc = Bf::mma(gl, xs, gacc);
        } else {
            float xv[KQ];
            decode_x<T, D>(raw, xv);
#pragma unroll
            for (int j = 0; j < KQ; ++j) xv[j] = valid ? xv[j] : 0.f;
#pragma unroll
            for (int t = 0; t < NRT; ++t) {
                float ak[KQ], av[KQ];
                lds_vec<KQ>(Sc + (2 * D + 16 * t + i16) * D + q * KQ, ak);
                lds_vec<KQ>(Sc + (D + 16 * t + i16) * D + q * KQ, av);
#pragma unroll
                for (int j = 0; j < KQ; ++j) {
                    kacc[t] = mfma4(ak[j], xv[j], kacc[t]);
                    vacc[t] = mfma4(av[j], xv[j], vacc[t]);
                }
            }
            float ag[KQ];
            lds_vec<KQ>(Sc + grow_row * D + q * KQ, ag);
#pragma unroll
            for (int j = 0; j < KQ; ++j) gacc = mfma4(ag[j], xv[j], gacc);
        }
        // Lane 16q + n now holds rows 4q..4q+3 of every 16-row tile for token n.
        float kn = 0.f;
#pragma unroll
        for (int t = 0; t < NRT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) kn += kacc[t][j] * kacc[t][j];
        kn = xor16_32_sum(kn);
        const float inv = rsqrtf(kn + 1e-6f);
        float kv[NRT][4], dsq = 0.f;
#pragma unroll
        for (int t = 0; t < NRT; ++t) {
            float df[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kv[t][j] = kacc[t][j] * inv;
                df[j] = kv[t][j] - vacc[t][j];
                dsq += df[j] * df[j];
            }
            const int slot = s0 + i16;
            *reinterpret_cast<float4*>(&kk[buf][slot * D + 16 * t + 4 * q]) = make_float4(kv[t][0], kv[t][1], kv[t][2], kv[t][3]);
#pragma unroll
            for (int j = 0; j < 4; ++j) dkT[buf][(16 * t + 4 * q + j) * DKS + slot] = df[j];
        }
        dsq = xor16_32_sum(dsq);
        // dots with the previous 1, 2, 3 tokens (same 4-token block: lanes of one quad)
        float kd1 = 0.f, kd2 = 0.f, kd3 = 0.f;
#pragma unroll
        for (int t = 0; t < NRT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kd1 += kv[t][j] * row_shr<1>(kv[t][j]);
                kd2 += kv[t][j] * row_shr<2>(kv[t][j]);
                kd3 += kv[t][j] * row_shr<3>(kv[t][j]);
            }
        kd1 = xor16_32_sum(kd1);
        kd2 = xor16_32_sum(kd2);
        kd3 = xor16_32_sum(kd3);
        float alpha, eff;
        token_gates_fast(p.k, gacc[0], gacc[1], dsq, kn * inv * inv, alpha, eff);
        // Slots past the chunk or the line act as the identity (alpha 1, eta^ 0).
        const float al_t = valid ? alpha : 1.f, et_t = valid ? eff : 0.f;
        // Block coefficients, with A_j the product of alpha over the block's slots <= j:
        //   r_j = A_{j-1} (g.k_j) + delta_j - sum_{s<j} beta_sj r_s,  g <- A_3 g - sum_s w_s r_s k_s
        //   beta_sj = (A_{j-1}/A_s) eta_s (k_s.k_j),  w_s = (A_3/A_s) eta_s.
        const int j = lane & 3;
        const float pa1 = quad_perm<0x90>(al_t), pa2 = quad_perm<0x40>(al_t), pa3 = quad_perm<0x00>(al_t);
        const float pe1 = quad_perm<0x90>(et_t), pe2 = quad_perm<0x40>(et_t), pe3 = quad_perm<0x00>(et_t);
        const float na1 = quad_perm<0xF9>(al_t), na2 = quad_perm<0xFE>(al_t), na3 = quad_perm<0xFF>(al_t);
        float cf_a = 1.f;
        if (j >= 1) cf_a *= pa1;
        if (j >= 2) cf_a *= pa2;
        if (j >= 3) cf_a *= pa3;
        const float cf_b1 = pe1 * kd1, cf_b2 = pe2 * kd2 * pa1, cf_b3 = pe3 * kd3 * pa2 * pa1;
        float cf_w = et_t;
        if (j <= 2) cf_w *= na1;
        if (j <= 1) cf_w *= na2;
        if (j == 0) cf_w *= na3;
        const float cf_A3 = quad_perm<0x00>(al_t) * quad_perm<0x55>(al_t) * quad_perm<0xAA>(al_t) *
                            quad_perm<0xFF>(al_t);
        if (q == 0) {
            float* c = &cf[buf][(s0 + i16) * 8];
            *reinterpret_cast<float4*>(c) = make_float4(cf_a, cf_b1, cf_b2, cf_b3);
            *reinterpret_cast<float4*>(c + 4) = make_float4(cf_w, cf_A3, 0.f, 0.f);
        }
    };

    // Serial recurrence over `cnt` slots for this wave's rows of G, 4 tokens per step; the
    // next step's operands are read while the current one computes.
    struct StepOps {
        float kv[4][E];
        float df[4];
        float c0v[4][4];   // slots 1..3: a, beta_{j-1,j}, beta_{j-2,j}, beta_{j-3,j}
        float c1v[4][2];   // every slot: w; slot 0: A_3 of the block
    };
    auto fetch = [&](int buf, int t, StepOps& o) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float* kr = &kk[buf][(t + u) * D + c0];
            if constexpr (E % 4 == 0) {
#pragma unroll
                for (int e = 0; e < E; e += 4) {
                    const float4 k4 = *reinterpret_cast<const float4*>(kr + e);
                    o.kv[u][e] = k4.x; o.kv[u][e + 1] = k4.y; o.kv[u][e + 2] = k4.z; o.kv[u][e + 3] = k4.w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) o.kv[u][e] = kr[e];
            }
            if (u > 0) {
                const float4 a4 = *reinterpret_cast<const float4*>(&cf[buf][(t + u) * 8]);
                o.c0v[u][0] = a4.x; o.c0v[u][1] = a4.y; o.c0v[u][2] = a4.z; o.c0v[u][3] = a4.w;
            }
            const float2 w2 = *reinterpret_cast<const float2*>(&cf[buf][(t + u) * 8 + 4]);
            o.c1v[u][0] = w2.x; o.c1v[u][1] = w2.y;
        }
        const float4 d4 = *reinterpret_cast<const float4*>(&dkT[buf][grow * DKS + t]);
        o.df[0] = use_dk ? d4.x : 0.f; o.df[1] = use_dk ? d4.y : 0.f;
        o.df[2] = use_dk ? d4.z : 0.f; o.df[3] = use_dk ? d4.w : 0.f;
    };
    auto step = [&](float (&g)[E], const StepOps& o) {
        float pdot[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            float d0 = g[0] * o.kv[u][0];
            if constexpr (E >= 2) {
                float d1 = g[1] * o.kv[u][1];
#pragma unroll
                for (int e = 2; e < E; e += 2) {
                    d0 += g[e] * o.kv[u][e];
                    d1 += g[e + 1] * o.kv[u][e + 1];
                }
                d0 += d1;
            }
            pdot[u] = row_group_sum<RL>(d0);
        }
        const float r0 = pdot[0] + o.df[0];
        const float r1 = o.c0v[1][0] * pdot[1] + o.df[1] - o.c0v[1][1] * r0;
        const float r2 = o.c0v[2][0] * pdot[2] + o.df[2] - o.c0v[2][2] * r0 - o.c0v[2][1] * r1;
        const float r3 = o.c0v[3][0] * pdot[3] + o.df[3] - o.c0v[3][3] * r0 - o.c0v[3][2] * r1 - o.c0v[3][1] * r2;
        const float A3 = o.c1v[0][1];
        const float w0 = o.c1v[0][0] * r0, w1 = o.c1v[1][0] * r1, w2 = o.c1v[2][0] * r2, w3 = o.c1v[3][0] * r3;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            float v = A3 * g[e] - w0 * o.kv[0][e];
            v -= w1 * o.kv[1][e];
            v -= w2 * o.kv[2][e];
            g[e] = v - w3 * o.kv[3][e];
        }
    };
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

    // G <- Gin X_bb + Y_bb (or X_0 + Y_0 when Gin is null): the 16x16 output tiles over the
    // waves (head_dim 16: one tile, wave 0), fp32 matrix cores.
    // `first`, `stride`: the threads taking part (one wave: lane, 64; the workgroup: tid, 64 W).
    auto compose = [&](const float* Gin, int bb, float* Gout, int first, int stride) {
        const float* X = XY + bb * 2 * D * GS;
        const float* Y = X + D * GS;
        if (Gin == nullptr) {
            for (int idx = first; idx < D * D; idx += stride) {
                const int rr = idx / D, cc = idx - rr * D;
                Gout[rr * GS + cc] = X[rr * GS + cc] + Y[rr * GS + cc];
            }
            return;
        }
        for (int tile = wv; tile < NRT * NRT; tile += W) {
            const int rt = tile / NRT, ct = tile - rt * NRT;
            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kh = 0; kh < NRT; ++kh)
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const int k = 16 * kh + 4 * q + st;
                    acc = mfma4(Gin[(16 * rt + i16) * GS + k], X[k * GS + 16 * ct + i16], acc);
                }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int rr = 16 * rt + 4 * q + j, cc = 16 * ct + i16;
                Gout[rr * GS + cc] = acc[j] + Y[rr * GS + cc];
            }
        }
    };

    bool have_next = false;
    int buf = 0;
    for (int64_t c = 0; c < nc; ++c) {
        const float* Sc = St + (c & 1) * SR;
        float* Sn = St + ((c + 1) & 1) * SR;
        {   // chunk-start content memory -> workspace (read by the readout)
            float* dst = p.states + (line * p.max_chunks + c) * D * D;
            for (int idx = tid * 4; idx < D * D; idx += 64 * W * 4)
                store_state4(dst + idx, *reinterpret_cast<const float4*>(Sc + idx), p.split_states);
        }
        // The last chunk's gain only feeds a refresh that no output reads.
        if (c == nc - 1) break;
        float g[E];
        int gcur = -1;   // TB > 1: buffer of Gs holding the composed gain so far (-1: identity)
        if constexpr (TB == 1) {
#pragma unroll
            for (int e = 0; e < E; ++e) g[e] = (c0 + e == grow) ? 1.f : 0.f;
        }
        for (int sbase = 0; sbase < C; sbase += SEG) {
            const int scnt = min(SEG, C - sbase);
            if (!have_next) issue(c, sbase, scnt);
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                const int s0 = (wv + W * tt) * 16;
                if (s0 < scnt) token_tile(Sc, xr[tt], (vmask >> tt) & 1u, s0, buf);
            }
            {   // x of this wave's next tiles (the next chunk's first segment after the last)
                int64_t ncc = c;
                int nbase = sbase + SEG;
                if (nbase >= C) { ncc = c + 1; nbase = 0; }
                have_next = ncc < nc - 1;
                if (have_next) issue(ncc, nbase, min(SEG, C - nbase));
            }
            __syncthreads();
            // Slots [t_begin, t_end) of this wave's block, in 4-slot steps (slots past the
            // segment's count act as the identity, so the count rounds up to a multiple of 4).
            int t_begin = 0, t_end = scnt;
            if constexpr (TB > 1) {
                const int cnt4 = (scnt + 3) & ~3;
                const int span = ((cnt4 + 4 * TB - 1) / (4 * TB)) * 4;
                t_begin = min(tb * span, cnt4);
                t_end = min(t_begin + span, cnt4);
#pragma unroll
                for (int e = 0; e < E; ++e) g[e] = (prow < D && c0 + e == prow) ? 1.f : 0.f;
            }
            if (t_begin < t_end) {
                StepOps opA, opB;
                fetch(buf, t_begin, opA);
                for (int t0 = t_begin; t0 < t_end; t0 += 8) {
                    fetch(buf, min(t0 + 4, SEG - 4), opB);
                    __builtin_amdgcn_sched_barrier(0);
                    step(g, opA);
                    pin(opB);
                    if (t0 + 4 >= t_end) break;
                    fetch(buf, min(t0 + 8, SEG - 4), opA);
                    __builtin_amdgcn_sched_barrier(0);
                    step(g, opB);
                    pin(opA);
                }
            }
            if constexpr (TB > 1) {
                // block maps to LDS, then compose them onto the gain so far
#pragma unroll
                for (int e = 0; e < E; ++e) XY[(tb * 2 * D + prow) * GS + c0 + e] = g[e];
                __syncthreads();
                if constexpr (NRT == 1) {
                    // One 16x16 tile: wave 0 composes every block with the gain held transposed
                    // in accumulator layout (lane 16q + n holds G[n][4q..4q+3]):
                    //   G X + Y  ->  (G X + Y)^T = X^T G^T + Y^T,
                    // so G^T is the B operand as it stands and only X and Y are read from LDS
                    // (independent of the chain, all issued up front).
                    if (wv == 0) {
                        float xa[TB][4], yt[TB][4];
#pragma unroll
                        for (int bb = 0; bb < TB; ++bb) {
                            const float* X = XY + bb * 2 * D * GS;
#pragma unroll
                            for (int st = 0; st < 4; ++st) {
                                xa[bb][st] = X[(4 * q + st) * GS + i16];          // X^T[n][4q + st]
                                yt[bb][st] = X[(D + i16) * GS + 4 * q + st];      // Y^T[4q + st][n]
                            }
                        }
                        v4f gt;
                        int bb0 = 0;
                        if (gcur < 0) {
                            const float* X0 = XY;
#pragma unroll
                            for (int j = 0; j < 4; ++j) gt[j] = X0[i16 * GS + 4 * q + j] + yt[0][j];
                            bb0 = 1;
                        } else {
#pragma unroll
                            for (int j = 0; j < 4; ++j) gt[j] = Gs[gcur][i16 * GS + 4 * q + j];
                        }
#pragma unroll
                        for (int bb = 0; bb < TB; ++bb) {
                            if (bb < bb0) continue;
                            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int st = 0; st < 4; ++st) acc = mfma4(xa[bb][st], gt[st], acc);
#pragma unroll
                            for (int j = 0; j < 4; ++j) gt[j] = acc[j] + yt[bb][j];
                        }
                        const int out = gcur < 0 ? 0 : gcur ^ 1;
#pragma unroll
                        for (int j = 0; j < 4; ++j) Gs[out][i16 * GS + 4 * q + j] = gt[j];
                    }
                    gcur = gcur < 0 ? 0 : gcur ^ 1;
                } else {
                    for (int bb = 0; bb < TB; ++bb) {
                        const int out = gcur < 0 ? 0 : gcur ^ 1;
                        compose(gcur < 0 ? nullptr : Gs[gcur], bb, Gs[out], tid, 64 * W);
                        gcur = out;
                        __syncthreads();
                    }
                }
                if constexpr (NRT == 1) __syncthreads();
            } else {
                buf ^= 1;
            }
        }
        // ---- refresh: Sn <- Sc G, 16-row tiles over the waves ----
        const float* Gf = Gs[TB > 1 ? gcur : 0];
        if constexpr (TB == 1) {
#pragma unroll
            for (int e = 0; e < E; ++e) Gs[0][grow * GS + c0 + e] = g[e];
            __syncthreads();
        }
        // The columns of G this lane supplies (K-range of its lane group), read and split once.
        float bg[NRT][KQ];
        [[maybe_unused]] Half bh[NRT], bl[NRT];
#pragma unroll
        for (int ct = 0; ct < NRT; ++ct) {
#pragma unroll
            for (int s = 0; s < KQ; ++s) bg[ct][s] = Gf[(q * KQ + s) * GS + 16 * ct + i16];
            if constexpr (kRefreshBf16) Bf::split(bg[ct], bh[ct], bl[ct]);
        }
        for (int rt = wv; rt < RT; rt += W) {
            float a[KQ];
            lds_vec<KQ>(Sc + (16 * rt + i16) * D + q * KQ, a);
            [[maybe_unused]] Half ah, al;
            if constexpr (kRefreshBf16) Bf::split(a, ah, al);
#pragma unroll
            for (int ct = 0; ct < NRT; ++ct) {
                v4f acc = {0.f, 0.f, 0.f, 0.f};
                if constexpr (kRefreshBf16) {
                    acc = Bf::mma(ah, bh[ct], acc);
                    acc = Bf::mma(al, bh[ct], acc);
                    acc = Bf::mma(ah, bl[ct], acc);
                } else {
#pragma unroll
                    for (int s = 0; s < KQ; ++s) acc = mfma4(a[s], bg[ct][s], acc);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) Sn[(16 * rt + 4 * q + j) * D + 16 * ct + i16] = acc[j];
            }
        }
        __syncthreads();
    }
}

template <typename T, int D, bool SPATIAL>
void launch_w(const ScanParams& sp, int waves, int token_blocks, hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(sp.B * sp.R * sp.heads);
    auto go = [&](auto wc, auto tc) {
        constexpr int Wc = decltype(wc)::value, TBc = decltype(tc)::value;
        hipLaunchKernelGGL((srnl_scanw_kernel<T, D, Wc, TBc, SPATIAL>), dim3(grid), dim3(64 * Wc), 0, stream, sp);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    if constexpr (D == 16) {
        if (waves == 1) go(I1{}, I1{});
        else if (waves == 2) token_blocks > 1 ? go(I2{}, I2{}) : go(I2{}, I1{});
        else token_blocks > 1 ? go(I4{}, I4{}) : go(I4{}, I1{});
    } else {
        if (waves <= 2) go(I2{}, I1{});
        else token_blocks > 1 ? go(I4{}, I2{}) : go(I4{}, I1{});
    }
}

template <typename T, int D>
void launch_t(const ScanParams& sp, int waves, int token_blocks, hipStream_t stream) {
    if (sp.x.spatial) launch_w<T, D, true>(sp, waves, token_blocks, stream);
    else launch_w<T, D, false>(sp, waves, token_blocks, stream);
}

}  // namespace

int scan_wide_waves(int64_t lines, int head_dim) {
    // Enough waves per line for about two per SIMD (1024 SIMDs on MI355X); head_dim 32
    // keeps at least two (16 G entries per lane with one would not fit the registers).
    int w = lines <= 512 ? 4 : lines <= 1024 ? 2 : 1;
    if (head_dim == 32 && w < 2) w = 2;
    return w;
}

bool launch_scan_wide(const ScanParams& sp, int io_dtype, int head_dim, int waves, int token_blocks,
                      hipStream_t stream) {
    if (!sp.x_vec || (head_dim != 16 && head_dim != 32) || io_dtype == VH_DTYPE_F16) return false;
    if (head_dim == 16) {
        if (io_dtype == VH_DTYPE_BF16) launch_t<bf16_t, 16>(sp, waves, token_blocks, stream);
        else launch_t<float, 16>(sp, waves, token_blocks, stream);
    } else {
        if (io_dtype == VH_DTYPE_BF16) launch_t<bf16_t, 32>(sp, waves, token_blocks, stream);
        else launch_t<float, 32>(sp, waves, token_blocks, stream);
    }
    return true;
}

}  // namespace vh
