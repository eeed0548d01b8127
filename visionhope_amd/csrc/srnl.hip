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
//     fuses sum_r w_r (y_r + skip_r x) per pixel in the reference's summation
//     order, so no per-direction output ever reaches HBM and no atomics are used.
#include <cmath>

#include "vh_common.h"

namespace vh {

struct Consts {
    float eta_scale, alpha_min, alpha_bias, stab_mu;
    int clamp;
    float factor;
};

// Element (b, r, head, t, i) of a line-major input.  spatial = 1: t is a scan
// index of direction r, mapped to a pixel of a channels-last image whose pixel
// stride is st; otherwise st is the token stride of direction r.
struct LineInput {
    const void* ptr;
    int64_t sb, sr, sh, st;
    int spatial;
    int64_t H, W;
};

template <typename T>
__device__ __forceinline__ const T* line_ptr(const LineInput& in, int64_t b, int r, int64_t head,
                                             int64_t t) {
    const T* base = static_cast<const T*>(in.ptr);
    if (in.spatial) return base + b * in.sb + scan_to_pixel(r, t, in.H, in.W) * in.st + head * in.sh;
    return base + b * in.sb + r * in.sr + head * in.sh + t * in.st;
}

struct ScanParams {
    LineInput x;
    const float *Mm, *Mv, *Mk, *Me, *Ma;
    int64_t B, R, heads, L;
    int chunk[4];
    int64_t max_chunks;
    float* states;  // [lines, max_chunks, D, D]: chunk-start M_m
    int per_line_state;  // 1: memories hold one state per line (chunk.cu:287, StateCount == N)
    Consts k;
};

template <int D>
struct ScanCfg {
    static constexpr int NT = 4 * D;             // threads per line
    static constexpr int E = D / 4;              // G entries per thread (4 lanes per row)
    static constexpr int TT = D == 64 ? 32 : 64; // tokens per tile
    static constexpr int SD = D + 1;             // padded LDS row
    static constexpr int ROWS = 3 * D + 2;       // M_m, M_v, M_k rows, then e, a
    static constexpr int NOUT = (ROWS * D + NT - 1) / NT;
};

template <int D, typename T>
__global__ __launch_bounds__(4 * D) void srnl_scan_kernel(const ScanParams p) {
    using Cfg = ScanCfg<D>;
    constexpr int NT = Cfg::NT, E = Cfg::E, TT = Cfg::TT, SD = Cfg::SD, ROWS = Cfg::ROWS;
    __shared__ float S[ROWS * SD];
    __shared__ float Gs[D * SD];
    __shared__ float xs[TT * SD];
    __shared__ float kk[TT * SD];
    __shared__ float vd[TT * SD];
    __shared__ float ep_s[TT], ap_s[TT], al_s[TT], et_s[TT];

    const int64_t lines = p.B * p.R * p.heads;
    const int64_t line = xcd_remap(blockIdx.x, lines);
    const int64_t head = line % p.heads;
    const int r = static_cast<int>((line / p.heads) % p.R);
    const int64_t b = line / (p.heads * p.R);
    const int64_t s = p.per_line_state ? line : r * p.heads + head;
    const int tid = threadIdx.x;

    for (int idx = tid; idx < D * D; idx += NT) {
        const int row = idx / D, col = idx % D;
        S[row * SD + col] = p.Mm[s * D * D + idx];
        S[(D + row) * SD + col] = p.Mv[s * D * D + idx];
        S[(2 * D + row) * SD + col] = p.Mk[s * D * D + idx];
    }
    for (int idx = tid; idx < D; idx += NT) {
        S[3 * D * SD + idx] = p.Me[s * D + idx];
        S[(3 * D + 1) * SD + idx] = p.Ma[s * D + idx];
    }

    const int C = p.chunk[r];
    const int64_t nc = (p.L + C - 1) / C;
    const int grow = tid / 4;       // row of G held by this thread
    const int c0 = (tid % 4) * E;   // first column of G held by this thread
    float* out_states = p.states + line * p.max_chunks * D * D;

    for (int64_t c = 0; c < nc; ++c) {
        __syncthreads();
        for (int idx = tid; idx < D * D; idx += NT)
            out_states[c * D * D + idx] = S[(idx / D) * SD + idx % D];
        // The last chunk's gain only feeds a refresh no output reads.
        if (c == nc - 1) break;

        float g[E];
#pragma unroll
        for (int e = 0; e < E; ++e) g[e] = (c0 + e == grow) ? 1.f : 0.f;

        for (int base = 0; base < C; base += TT) {
            const int cnt = min(TT, C - base);
            for (int idx = tid; idx < cnt * D; idx += NT) {
                const int t = idx / D, j = idx % D;
                const int64_t tok = c * C + base + t;
                xs[t * SD + j] = tok < p.L ? to_f32(line_ptr<T>(p.x, b, r, head, tok)[j]) : 0.f;
            }
            __syncthreads();
            // values (rows D..2D-1), raw keys (2D..3D-1), gate pre-activations (3D, 3D+1)
            for (int idx = tid; idx < (2 * D + 2) * cnt; idx += NT) {
                const int t = idx / (2 * D + 2), rr = idx % (2 * D + 2);
                const float* srow = &S[(D + rr) * SD];
                const float* xt = &xs[t * SD];
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < D; ++j) acc += srow[j] * xt[j];
                if (rr < D) vd[t * SD + rr] = acc;
                else if (rr < 2 * D) kk[t * SD + rr - D] = acc;
                else if (rr == 2 * D) ep_s[t] = acc;
                else ap_s[t] = acc;
            }
            __syncthreads();
            // per-token normalisation and gates
            for (int t = tid; t < cnt; t += NT) {
                float kn = 0.f;
#pragma unroll
                for (int j = 0; j < D; ++j) kn += kk[t * SD + j] * kk[t * SD + j];
                const float den = sqrtf(kn + 1e-6f);
                float dsq = 0.f, ksq = 0.f;
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    const float kv = kk[t * SD + j] / den;
                    kk[t * SD + j] = kv;
                    const float diff = kv - vd[t * SD + j];
                    vd[t * SD + j] = diff;
                    dsq += diff * diff;
                    ksq += kv * kv;
                }
                const float ep = fminf(10.f, fmaxf(-10.f, ep_s[t]));
                const float ap = fminf(10.f, fmaxf(-10.f, ap_s[t] + p.k.alpha_bias));
                const float sp = ep > 20.f ? ep : logf(1.f + expf(ep));
                const float eta = p.k.eta_scale * sp;
                const float alpha = p.k.alpha_min + (1.f - p.k.alpha_min) * (1.f / (1.f + expf(-ap)));
                const float dn = sqrtf(dsq + 1e-12f);
                const float cap = p.k.stab_mu * (1.f - alpha) / (dn + 1e-6f);
                float eff = cap * (-expm1f(-(eta / cap)));
                if (p.k.clamp) {
                    const float lim = nextafterf(p.k.factor * alpha / fmaxf(ksq, 1e-20f), 0.f);
                    eff = fminf(eff, lim);
                }
                al_s[t] = alpha;
                et_s[t] = eff;
            }
            __syncthreads();
            // serial gain recurrence; rows are independent, 4 lanes per row
            for (int t = 0; t < cnt; ++t) {
                const float* kt = &kk[t * SD];
                float dot = 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) dot += g[e] * kt[c0 + e];
                dot += __shfl_xor(dot, 1);
                dot += __shfl_xor(dot, 2);
                const float rv = vd[t * SD + grow] + dot;
                const float alpha = al_s[t];
                const float coef = et_s[t] * rv;
#pragma unroll
                for (int e = 0; e < E; ++e) g[e] = alpha * g[e] - coef * kt[c0 + e];
            }
            __syncthreads();
        }
        // refresh: S <- S G (all 3D+2 rows)
#pragma unroll
        for (int e = 0; e < E; ++e) Gs[grow * SD + c0 + e] = g[e];
        __syncthreads();
        float buf[Cfg::NOUT];
#pragma unroll
        for (int q = 0; q < Cfg::NOUT; ++q) {
            const int idx = tid + q * NT;
            float acc = 0.f;
            if (idx < ROWS * D) {
                const int row = idx / D, col = idx % D;
#pragma unroll
                for (int l = 0; l < D; ++l) acc += S[row * SD + l] * Gs[l * SD + col];
            }
            buf[q] = acc;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < Cfg::NOUT; ++q) {
            const int idx = tid + q * NT;
            if (idx < ROWS * D) S[(idx / D) * SD + idx % D] = buf[q];
        }
    }
}

// ---------------------------------------------------------------------------
// Spatial readout + four-direction fusion, one thread per output element.
// ---------------------------------------------------------------------------
struct FuseParams {
    const void* x;
    const void* q;
    int per_direction;  // 1: x, q are serialized stacks [B, 4, L, C]; 0: channels-last [B, L, C]
    const float* states;
    int64_t max_chunks;
    const float* skip;
    int skip_per_dir;
    const float* wgt;
    float* out;
    int64_t B, H, W, C, heads;
    int chunk[4];
};

template <int D, typename T>
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
        const int64_t ch = t / p.chunk[r];
        const float* m = p.states + (((b * 4 + r) * p.heads + head) * p.max_chunks + ch) * D * D + i * D;
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < D; ++j) dot += m[j] * qv[j];
        const float y = dot * qinv;
        const float contrib = y + p.skip[(p.skip_per_dir ? r * p.C : 0) + c] * xval;
        const float weighted = p.wgt[r * p.C + c] * contrib;
        acc = r == 0 ? weighted : acc + weighted;
    }
    p.out[idx] = acc;
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
    const float* m = p.states + (line * p.max_chunks + t / p.chunk[r]) * D * D + i * D;
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

int check_consts(const vh_srnl_consts* k) {
    VH_REQUIRE(k != nullptr, VH_ERR_ARG, "SRNL constants must not be null");
    VH_REQUIRE(k->min_retention >= 0.f && k->min_retention < 1.f, VH_ERR_ARG,
               "MIN_RETENTION must be in [0, 1), got %g", (double)k->min_retention);
    VH_REQUIRE(k->injection_margin > 0.f && k->injection_margin < 1.f, VH_ERR_ARG,
               "INJECTION_MARGIN must be in (0, 1), got %g", (double)k->injection_margin);
    VH_REQUIRE(k->step_scale > 0.f, VH_ERR_ARG, "STEP_SCALE must be positive, got %g",
               (double)k->step_scale);
    return VH_OK;
}

int check_memories(const float* a, const float* b, const float* c, const float* d, const float* e) {
    VH_REQUIRE(a && b && c && d && e, VH_ERR_ARG, "SRNL memories must not be null");
    return VH_OK;
}

template <int D, typename T>
void launch_scan(const ScanParams& sp, hipStream_t stream) {
    const int64_t lines = sp.B * sp.R * sp.heads;
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
    int rc = check_consts(consts);
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
    sp.k = make_consts(consts);
    rc = dispatch_d(d, [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        dispatch_t(io_dtype, [&](auto tv) { launch_scan<D, decltype(tv)>(sp, stream); });
    });
    if (rc) return rc;
    *out_params = sp;
    return check_launch("srnl_scan_kernel");
}

int run_fuse(const ScanParams& sp, const void* x, const void* q, int per_direction, int io_dtype,
             const float* skip, int skip_per_dir, const float* wgt, float* out, int64_t H,
             int64_t W, int64_t C, int d, hipStream_t stream) {
    VH_REQUIRE(skip && wgt && out && q, VH_ERR_ARG, "SRNL fusion arguments must not be null");
    FuseParams fp{};
    fp.x = x; fp.q = q; fp.per_direction = per_direction;
    fp.states = sp.states; fp.max_chunks = sp.max_chunks;
    fp.skip = skip; fp.skip_per_dir = skip_per_dir; fp.wgt = wgt; fp.out = out;
    fp.B = sp.B; fp.H = H; fp.W = W; fp.C = C; fp.heads = sp.heads;
    for (int r = 0; r < 4; ++r) fp.chunk[r] = sp.chunk[r];
    const int64_t total = sp.B * H * W * C;
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256);
    int rc = dispatch_d(d, [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        dispatch_t(io_dtype, [&](auto tv) {
            hipLaunchKernelGGL((srnl_fuse_readout_kernel<D, decltype(tv)>), dim3(blocks), dim3(256),
                               0, stream, fp);
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
    VH_REQUIRE(H > 0 && W > 0 && C > 0 && B > 0, VH_ERR_SHAPE, "spatial SRNL needs nonempty [B,H,W,C]");
    VH_REQUIRE(valid_head_dim(head_dim), VH_ERR_HEAD_DIM,
               "head_dim must be one of 4, 8, 16, 32, 64; got %d", head_dim);
    VH_REQUIRE(C % head_dim == 0, VH_ERR_SHAPE, "C=%lld is not a multiple of head_dim=%d",
               (long long)C, head_dim);
    const int64_t heads = C / head_dim;
    LineInput xin{x, H * W * C, 0, head_dim, C, 1, H, W};
    ScanParams sp{};
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, 4, heads, H * W, head_dim,
                      chunks, consts, workspace, workspace_bytes, s, &sp);
    if (rc) return rc;
    return run_fuse(sp, x, q, 0, io_dtype, d_skip, skip_per_direction, dir_weight, out, H, W, C,
                    head_dim, s);
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
    LineInput xin{X, 4 * L * C, L * C, head_dim, C, 0, 0, 0};
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
    LineInput xin{X, R * heads * N * d, heads * N * d, N * d, d, 0, 0, 0};
    ScanParams sp{};
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, R, heads, N, head_dim, chunks,
                      consts, workspace, workspace_bytes, s, &sp, memories_per_line ? 1 : 0);
    if (rc) return rc;
    const int64_t C = heads * d;
    LineInput qin{Q_raw, R * N * C, N * C, d, C, 0, 0, 0};
    return run_packed<void>(sp, qin, 1, io_dtype, out, head_dim, s);
}

int vh_srnl_forward(const void* X, int32_t io_dtype, const float* Q, const float* M_m,
                    const float* M_v, const float* M_k, const float* M_eta, const float* M_alpha,
                    int32_t memories_per_line, void* out, int64_t B, int64_t R, int64_t heads,
                    int64_t N, int32_t head_dim, const int64_t* chunks,
                    const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes,
                    void* stream) {
    const int64_t d = head_dim;
    LineInput xin{X, R * heads * N * d, heads * N * d, N * d, d, 0, 0, 0};
    ScanParams sp{};
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = run_scan(xin, io_dtype, M_m, M_v, M_k, M_eta, M_alpha, B, R, heads, N, head_dim, chunks,
                      consts, workspace, workspace_bytes, s, &sp, memories_per_line ? 1 : 0);
    if (rc) return rc;
    LineInput qin{Q, R * heads * N * d, heads * N * d, N * d, d, 0, 0, 0};
    return run_packed<float>(sp, qin, 0, io_dtype, out, head_dim, s);
}

}  // extern "C"
