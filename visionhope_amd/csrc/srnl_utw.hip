// SRNL chunk scan for head_dim 16 (bf16, fp16 or FP32 activations) when the lines are few (fewer than
// the GPU's 1024 SIMDs: VisionHOPE-Base at 512^2 has 96 to 640 lines per launch, with chunks
// of 128 down to 16 tokens).  It is the block form of srnl_ut.hip (same algebra, same
// operand arithmetic) with the blocks of a chunk spread over the waves of a workgroup:
//
//   * one workgroup per line, W waves (W = the chunk's 16-slot blocks rounded up to a power
//     of two, at most 8); wave w forms the affine map (X_w, Y_w) of block w of the current
//     chunk -- token projections, gates, the triangle L, Z = (I + L)^-1 W K^T by back
//     substitution, X_w = a_15 I - (K D_a) Z, Y_w = -Delta Z -- exactly as srnl_ut.hip forms
//     one tile's map (reference recurrence: inference_recurrence.cuh:32-135, memory.cuh:
//     219-233);
//   * the maps compose in order on wave 0 (srnl_ut.hip's chain): wave 0 forms G^T =
//     (X_0 + Y_0)^T in registers, the other waves hand X_w and Y_w^T over through LDS, and
//     G^T <- X_w^T G^T + Y_w^T follows block by block -- one barrier, no transposes (a tree
//     of log2 W levels measured 3,800 of 8,600 cycles per chunk at W = 8, against about
//     1,200 for the chain);
//   * the state S = [M_m; M_v; M_k; e; a; 0] (64 x 16 FP32) lives in LDS; the refresh
//     S <- S G (the reference's M <- M G and e <- G^T e, a <- G^T a, :119-133) is split over
//     the waves by 16-row blocks.
//
// Matrices pass between waves in LDS in the accumulator layout of lane 16 q + j (rows
// 4q..4q+3 of column j), read back by the lane that wrote them: X_w is then the A operand of
// X_w^T and Y_w^T the addend, one 16-byte load each.  Slots past the chunk act as the identity.
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

}  // namespace

template <typename T, int W, bool SPATIAL>
__global__ __launch_bounds__(64 * W) void srnl_scan16_utw_kernel(const ScanParams p) {
    using XQ = XQuad<T>;
    // Row strides are padded to 20 floats (keys, L, Z, state, G) so that the 16-byte loads of
    // 16 lanes down a column of rows fall in different LDS banks; the hand-over maps are read
    // back by the lane that wrote them, so they are stored lane-major.
    constexpr int D = 16, DKS = 20, TS = 20, SD = 20;
    __shared__ __align__(16) float kT[W][D * DKS];    // normalised keys [feature][slot]
    __shared__ __align__(16) float ndT[W][D * DKS];   // v - k [feature][slot]
    __shared__ __align__(16) float tk[W][64];         // per slot: rho, kappa, -a_{t-1}, w
    __shared__ __align__(16) float Lc[W][16 * TS];    // L[s][t] at [t][s]
    __shared__ __align__(16) float Zs[W][16 * TS];    // Z[s][f] at [f][s]
    __shared__ __align__(16) float Xt[W][256];        // X_w, accumulator layout, lane-major
    __shared__ __align__(16) float Yt[W][256];        // Y_w^T, accumulator layout, lane-major
    __shared__ __align__(16) float St[64 * SD];       // state rows
    __shared__ __align__(16) float Gr[16 * SD];       // chunk gain G, by rows

    const int tid = static_cast<int>(threadIdx.x);
    const int wv = tid >> 6, lane = tid & 63, i16 = lane & 15, q = lane >> 4;
    const int64_t lines = p.B * p.R * p.heads;
    const int64_t line = xcd_remap(blockIdx.x, lines);
    const int64_t head = line % p.heads;
    const int r = static_cast<int>((line / p.heads) % p.R);
    const int64_t b = line / (p.heads * p.R);
    const int64_t sidx = p.per_line_state ? line : r * p.heads + head;

    // initial state: rows 0-15 M_m, 16-31 M_v, 32-47 M_k, 48 e, 49 a, 50-63 zero
    for (int idx = tid; idx < 16 * D; idx += 64 * W) {
        const int row = idx >> 2, c4 = (idx & 3) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row < 16) v = ld4(p.Mm + sidx * D * D + row * D + c4);
        else if (row < 32) v = ld4(p.Mv + sidx * D * D + (row - 16) * D + c4);
        else if (row < 48) v = ld4(p.Mk + sidx * D * D + (row - 32) * D + c4);
        else if (row == 48) v = ld4(p.Me + sidx * D + c4);
        else if (row == 49) v = ld4(p.Ma + sidx * D + c4);
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
    // x of token (chunk cc, slot 16 wv + i16), features 4q..4q+3, as raw bits; slots past the
    // chunk read the line's first token and are zeroed when decoded
    auto load_x = [&](int64_t cc, typename XQ::Raw& raw, bool& ok) {
        const int slot = 16 * wv + i16;
        const int64_t tok = cc * C + slot;
        ok = slot < C && tok < p.L;
        int64_t off = 0;
        if (ok) {
            if (SPATIAL && p.aligned) off = static_cast<int64_t>(pa * static_cast<int>(cc) + pb * slot + pc) * pst;
            else off = token_offset<SPATIAL>(p.x, r, tok);
        }
        raw = XQ::load(xcol + off);
    };
    float* const kTw = kT[wv];
    float* const ndTw = ndT[wv];
    float* const tkw = tk[wv];
    float* const Lcw = Lc[wv];
    float* const Zsw = Zs[wv];

    typename XQ::Raw xr{};
    bool xok = false, have = false;
    __syncthreads();
    for (int64_t c = 0; c < nc; ++c) {
        if (wv == 0)   // chunk-start M_m for the readout
            store_state4(p.states + (line * p.max_chunks + c) * D * D + i16 * D + 4 * q,
                         ld4(St + i16 * SD + 4 * q), p.split_states);
        if (c == nc - 1) break;

        v4f gT = {0.f, 0.f, 0.f, 0.f};   // wave 0: G^T of the blocks composed so far
        if (wv < nblk) {
            if (!have) load_x(c, xr, xok);
            const bool valid = 16 * wv + i16 < C;   // slot inside the chunk (every such token is < L here)
            // ---- token phase: [M_k; M_v] x and (x.e, x.a) on the matrix cores ----
            v4s akh, akl, avh, avl, gah, gal;
            {
                const float4 mk = ld4(St + (32 + i16) * SD + 4 * q);
                const float4 mv = ld4(St + (16 + i16) * SD + 4 * q);
                const float4 g4 = ld4(St + (48 + (i16 & 1)) * SD + 4 * q);
                const bool on = (i16 & 3) < 2;   // operand rows 4q' + 0 / 4q' + 1: e / a, others zero
                const float ak[4] = {mk.x, mk.y, mk.z, mk.w};
                const float av[4] = {mv.x, mv.y, mv.z, mv.w};
                const float ga[4] = {on ? g4.x : 0.f, on ? g4.y : 0.f, on ? g4.z : 0.f, on ? g4.w : 0.f};
                split4(ak, akh, akl);
                split4(av, avh, avl);
                split4(ga, gah, gal);
            }
            v4s xh, xl;
            XQ::operands(xr, xok, xh, xl);
            const v4f z4 = {0.f, 0.f, 0.f, 0.f};
            const v4f kacc = XQ::mma(akh, akl, xh, xl, z4);
            const v4f vacc = XQ::mma(avh, avl, xh, xl, z4);
            const v4f gacc = XQ::mma(gah, gal, xh, xl, z4);
            // the next computing chunk's x, in flight during the rest of this chunk
            have = c + 1 < nc - 1;
            if (have) load_x(c + 1, xr, xok);
            float kn = kacc[0] * kacc[0] + kacc[1] * kacc[1] + kacc[2] * kacc[2] + kacc[3] * kacc[3];
            kn = xor16_32_sum(kn);
            // ||k||^2 of the normalised key is ||k~||^2 / (||k~||^2 + 1e-6)
            const float inv = rsqrtf(kn + 1e-6f);
            const float ksq = kn * inv * inv;
            float kn4[4], dsq = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float kv = kacc[j] * inv, nd = vacc[j] - kv;
                kn4[j] = kv;
                dsq += nd * nd;
                kTw[(4 * q + j) * DKS + i16] = kv;
                ndTw[(4 * q + j) * DKS + i16] = nd;
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
            // ---- L = diag(rho) K^T K diag(kappa), strict upper triangle, by columns (the
            //      Gram tile from the keys split once, scaled after the product) ----
            {
                const float kap = tkw[16 + i16];
                const float4 r4 = ld4(tkw + 4 * q);   // rho of rows 4q..4q+3
                const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
                v4s kh, kl;
                split4(kn4, kh, kl);
                const v4f P = mma3(kh, kl, kh, kl, v4f{0.f, 0.f, 0.f, 0.f});
                float lv[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) lv[j] = (4 * q + j < i16) ? (P[j] * rr[j]) * kap : 0.f;
                *reinterpret_cast<float4*>(Lcw + i16 * TS + 4 * q) = make_float4(lv[0], lv[1], lv[2], lv[3]);
            }
            wave_sync();
            // ---- Z = (I + L)^-1 W K^T: lane f (of the first 16) solves column f from the last
            //      row up, Z[s][f] = w_s k_s[f] - sum_{v > s} L[s][v] Z[v][f] ----
            if (q == 0) {
                float acc[16], zc[16];
#pragma unroll
                for (int s0 = 0; s0 < 16; s0 += 4) {
                    const float4 k4 = ld4(kTw + i16 * DKS + s0);
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
                            const float4 l4 = ld4(Lcw + (v0 + dv) * TS + s0);
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
                    *reinterpret_cast<float4*>(Zsw + i16 * TS + s) = make_float4(zc[s], zc[s + 1], zc[s + 2], zc[s + 3]);
            }
            wave_sync();
            // ---- the block's map: X = a_15 I - (K D_a) Z, Y = -Delta Z; wave 0 (the first
            //      block, entered with G = I) keeps (X_0 + Y_0)^T, the others hand over X_w
            //      and Y_w^T (accumulator layouts) ----
            {
                const float4 z4f = ld4(Zsw + i16 * TS + 4 * q);
                const float4 k4 = ld4(kTw + i16 * DKS + 4 * q);
                const float4 d4 = ld4(ndTw + i16 * DKS + 4 * q);
                const float4 a4 = ld4(tkw + 32 + 4 * q);
                const float zv[4] = {z4f.x, z4f.y, z4f.z, z4f.w};
                const float nka[4] = {k4.x * a4.x, k4.y * a4.y, k4.z * a4.z, k4.w * a4.w};
                const float ndl[4] = {d4.x, d4.y, d4.z, d4.w};
                v4s zh, zl, kah, kal, dlh, dll;
                split4(zv, zh, zl);
                if (wv == 0) {
                    const float nb[4] = {nka[0] + ndl[0], nka[1] + ndl[1], nka[2] + ndl[2], nka[3] + ndl[3]};
                    v4s nbh, nbl;
                    split4(nb, nbh, nbl);
                    gT = mma3(zh, zl, nbh, nbl, diag4(decay, q, i16));   // (X_0 + Y_0)^T
                } else {
                    split4(nka, kah, kal);
                    split4(ndl, dlh, dll);
                    st4(Xt[wv] + 4 * lane, mma3(kah, kal, zh, zl, diag4(decay, q, i16)));   // X_w
                    st4(Yt[wv] + 4 * lane, mma3(zh, zl, dlh, dll, v4f{0.f, 0.f, 0.f, 0.f}));  // Y_w^T
                }
            }
        }
        __syncthreads();
        // ---- composition on wave 0: G^T <- X_w^T G^T + Y_w^T, then G row-major ----
        if (wv == 0) {
            for (int w = 1; w < nblk; ++w) {
                const float4 x4 = ld4(Xt[w] + 4 * lane);   // A operand of X_w^T
                const float4 y4 = ld4(Yt[w] + 4 * lane);   // Y_w^T
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
                v4s xh, xl, gh, gl;
                split4(xv, xh, xl);
                split4(gT, gh, gl);
                gT = mma3(xh, xl, gh, gl, v4f{y4.x, y4.y, y4.z, y4.w});
            }
            st4(Gr + i16 * SD + 4 * q, gT);   // lane (j, q) holds G[j][4q..4q+3]
        }
        __syncthreads();
        // ---- refresh: S <- S G, one 16-row block per wave ----
        for (int R = wv; R < 4; R += W) {
            const float4 s4 = ld4(St + (16 * R + i16) * SD + 4 * q);   // A operand: row 16R + i16
            const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
            float gv[4];                                              // B operand: column i16 of G
#pragma unroll
            for (int k = 0; k < 4; ++k) gv[k] = Gr[(4 * q + k) * SD + i16];
            v4s sh, sl, gh, gl;
            split4(sv, sh, sl);
            split4(gv, gh, gl);
            const v4f sn = mma3(sh, sl, gh, gl, v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int k = 0; k < 4; ++k) St[(16 * R + 4 * q + k) * SD + i16] = sn[k];
        }
        __syncthreads();
    }
}

// Waves per line of the few-line block-form scan: the chunk's 16-slot blocks rounded up to
// a power of two; 0 when a chunk exceeds 8 blocks (128 tokens) or the input rows are not
// aligned for vector loads.
int scan16_utw_waves(const ScanParams& sp) {
    int max_chunk = 0;
    for (int r = 0; r < sp.R; ++r) max_chunk = std::max(max_chunk, sp.chunk[r]);
    const int blocks = (max_chunk + 15) / 16;
    if (blocks > 8 || !sp.x_vec) return 0;
    int w = 1;
    while (w < blocks) w *= 2;
    return w;
}

template <typename T>
bool launch_scan16_utw(const ScanParams& sp, hipStream_t stream) {
    const int waves = scan16_utw_waves(sp);
    if (waves == 0) return false;
    const unsigned grid = static_cast<unsigned>(sp.B * sp.R * sp.heads);
    auto go = [&](auto wc, auto spc) {
        constexpr int WV = decltype(wc)::value;
        hipLaunchKernelGGL((srnl_scan16_utw_kernel<T, WV, decltype(spc)::value>), dim3(grid), dim3(64 * WV), 0, stream,
                           sp);
    };
    auto pick = [&](auto spc) {
        switch (waves) {
            case 1: go(std::integral_constant<int, 1>{}, spc); break;
            case 2: go(std::integral_constant<int, 2>{}, spc); break;
            case 4: go(std::integral_constant<int, 4>{}, spc); break;
            default: go(std::integral_constant<int, 8>{}, spc); break;
        }
    };
    if (sp.x.spatial) pick(std::true_type{});
    else pick(std::false_type{});
    return true;
}

template bool launch_scan16_utw<bf16_t>(const ScanParams&, hipStream_t);
template bool launch_scan16_utw<f16_t>(const ScanParams&, hipStream_t);
template bool launch_scan16_utw<float>(const ScanParams&, hipStream_t);

}  // namespace vh
