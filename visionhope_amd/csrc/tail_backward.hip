// Backward of the SRNL operator's tail for gfx950: direction fusion, GRN, LayerNorm over
// channels, the query normalisation and the residual add.
//
// Every parameter gradient is a sum over pixels (and images).  Each kernel writes one fp32
// partial row per workgroup (or per image) into the caller's workspace and a column-sum
// kernel adds the rows in a fixed order, so the result does not depend on scheduling
// (no atomics).  Upstream gradients are fp32; input gradients are stored in the dtype of
// the input they belong to.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "vh_common.h"

namespace vh {
namespace {

template <typename F>
int dispatch_io(int t, F&& f) {
    switch (t) {
        case VH_DTYPE_F32: f(float{}); return VH_OK;
        case VH_DTYPE_BF16: f(bf16_t{}); return VH_OK;
        case VH_DTYPE_F16: f(f16_t{}); return VH_OK;
    }
    return set_error(VH_ERR_DTYPE, "unsupported dtype code %d", t);
}

size_t round256(size_t v) { return (v + 255) / 256 * 256; }

// out_a[j] = sum_p part[p][j] for j < na, out_b[j - na] for na <= j < width.  A workgroup
// covers 16 columns with 16 thread rows; row q sums the parts p = q, q + 16, ... into four
// interleaved accumulators (four loads in flight), then the 16 rows are added in order, so
// the result does not depend on scheduling.
__global__ __launch_bounds__(256) void column_sum_kernel(const float* __restrict__ part, int64_t parts,
                                                         int64_t width, int64_t na, float* __restrict__ out_a,
                                                         float* __restrict__ out_b) {
    __shared__ float red[16][17];
    const int lc = threadIdx.x & 15, row = threadIdx.x >> 4;
    const int64_t col = static_cast<int64_t>(blockIdx.x) * 16 + lc;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (col < width) {
        int64_t p = row;
        for (; p + 48 < parts; p += 64) {
            a0 += part[p * width + col];
            a1 += part[(p + 16) * width + col];
            a2 += part[(p + 32) * width + col];
            a3 += part[(p + 48) * width + col];
        }
        for (; p < parts; p += 16) a0 += part[p * width + col];
    }
    red[row][lc] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    if (row == 0 && col < width) {
        float v = 0.f;
#pragma unroll
        for (int q = 0; q < 16; ++q) v += red[q][lc];
        if (col < na) out_a[col] = v;
        else out_b[col - na] = v;
    }
}

void launch_column_sum(const float* part, int64_t parts, int64_t width, int64_t na, float* out_a, float* out_b,
                       hipStream_t s) {
    hipLaunchKernelGGL(column_sum_kernel, dim3(static_cast<unsigned>((width + 15) / 16)), dim3(256), 0, s, part,
                       parts, width, na, out_a, out_b);
}

// Threads of a 256-thread workgroup over (pixel, channel): for C <= 256, PPB = 256 / C
// pixels per step with channel t % C; above, one pixel per step and channel chunks of 256.
struct PixelChannelMap {
    int ppb, c0, pix;
    bool active;
    __device__ PixelChannelMap(int C, int chunk_base) {
        const int t = static_cast<int>(threadIdx.x);
        if (C <= 256) {
            ppb = 256 / C;
            pix = t / C;
            c0 = t % C;
            active = pix < ppb;
        } else {
            ppb = 1;
            pix = 0;
            c0 = chunk_base + t;
            active = c0 < C;
        }
    }
};

// ---------------------------------------------------------------------------
// Direction fusion backward (reference direction_fusion.cu:123-250, :585-691):
//   out[b, c, pixel] = sum_r s_r[c] (y_r[t_r] + k_r[c] x_r[t_r])
//   dy_r = g s_r, dx_r = g s_r k_r, dk_r = sum g s_r x_r, ds_r = sum g (y_r + k_r x_r)
// with g = dout[b, c, pixel] and t_r the scan position of the pixel in direction r.
// Grid (segments, B); partial rows [B * segments][nk * C + 4 C].
// ---------------------------------------------------------------------------
struct FusionBwdParams {
    const float* dout;
    const void* y;
    const void* x;
    const float* skip;
    const float* scale;
    void* dy;
    void* dx;
    float* part;
    int64_t heads, H, W, D, seg_len;
    int skip_per_dir, channels_last;
};

template <typename T>
__global__ __launch_bounds__(256) void fusion_backward_kernel(const FusionBwdParams p) {
    const int64_t b = blockIdx.y, seg = blockIdx.x;
    const int C = static_cast<int>(p.heads * p.D), D = static_cast<int>(p.D);
    const int64_t L = p.H * p.W;
    const int64_t l_begin = seg * p.seg_len, l_end = std::min<int64_t>(L, l_begin + p.seg_len);
    const int nk = p.skip_per_dir ? 4 : 1, width = (nk + 4) * C;
    float* prow = p.part + (b * gridDim.x + seg) * width;
    const int64_t stride_dir = p.heads * L * p.D;
    const T* y = static_cast<const T*>(p.y);
    const T* x = static_cast<const T*>(p.x);
    T* dy = static_cast<T*>(p.dy);
    T* dx = static_cast<T*>(p.dx);
    __shared__ float red[8][256];
    for (int chunk = 0; chunk < C; chunk += 256) {
        const PixelChannelMap m(C, chunk);
        const int c = m.c0;
        float acc_k[4] = {0.f, 0.f, 0.f, 0.f}, acc_s[4] = {0.f, 0.f, 0.f, 0.f};
        if (m.active) {
            const int head = c / D, di = c - head * D;
            float s[4], k[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] = p.scale[r * C + c];
                k[r] = p.skip[(p.skip_per_dir ? r * C : 0) + c];
            }
            const int64_t base = (b * 4 * p.heads + head) * L * p.D + di;
            for (int64_t l = l_begin + m.pix; l < l_end; l += m.ppb) {
                const int64_t h = l / p.W, w = l - h * p.W;
                const int64_t wh = w * p.H + h;
                const int64_t pos[4] = {l, L - 1 - l, wh, L - 1 - wh};
                const float g = p.channels_last ? p.dout[(b * L + l) * C + c] : p.dout[(b * C + c) * L + l];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t i = base + r * stride_dir + pos[r] * p.D;
                    const float xv = to_f32(x[i]), yv = to_f32(y[i]);
                    const float gs = g * s[r];
                    dy[i] = from_f32<T>(gs);
                    dx[i] = from_f32<T>(gs * k[r]);
                    acc_k[r] += gs * xv;
                    acc_s[r] += g * (yv + k[r] * xv);
                }
            }
        }
        // sum the PPB pixel rows of each channel in pixel order
        const int t = static_cast<int>(threadIdx.x);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            red[r][t] = acc_k[r];
            red[4 + r][t] = acc_s[r];
        }
        __syncthreads();
        if (m.active && m.pix == 0) {
            float sk[4], ss[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sk[r] = 0.f;
                ss[r] = 0.f;
            }
            for (int j = 0; j < m.ppb; ++j) {
                const int src = (C <= 256) ? j * C + c : t;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sk[r] += red[r][src];
                    ss[r] += red[4 + r][src];
                }
            }
            if (nk == 4) {
#pragma unroll
                for (int r = 0; r < 4; ++r) prow[r * C + c] = sk[r];
            } else {
                prow[c] = ((sk[0] + sk[1]) + sk[2]) + sk[3];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) prow[(nk + r) * C + c] = ss[r];
        }
        __syncthreads();
    }
}

// Tiled variant for D >= 8 (16-byte accesses): one workgroup per (image, band of 4 pixel
// rows, group of at most 96 channels) walks the band's 4x4 tiles.  Each tile's dout block
// is staged in LDS; the row scans (directions 0, 1) are visited with the tile's pixels in
// row-major order and the column scans (2, 3) in column-major order, so consecutive lanes
// touch consecutive tokens of one head in both (the access pattern of the tiled forward).
// Thread t keeps channel group t % G for the whole band and sums in registers; the pixel
// rows of the workgroup are added in LDS in a fixed order.  Partial rows [B * bands][width].
template <int D, typename T>
__global__ __launch_bounds__(256) void fusion_backward_tile_kernel(const FusionBwdParams p, const int heads_per_block) {
    constexpr int GD = D / 8;
    const int64_t b = blockIdx.y, band = blockIdx.x;
    const int C = static_cast<int>(p.heads) * D;
    const int head0 = static_cast<int>(blockIdx.z) * heads_per_block;
    const int nh = min(heads_per_block, static_cast<int>(p.heads) - head0);
    const int CB = nh * D, G = nh * GD, PPB = 256 / G;
    const int64_t L = p.H * p.W, stride_dir = p.heads * L * D;
    const int nk = p.skip_per_dir ? 4 : 1, width = (nk + 4) * C;
    const int t = static_cast<int>(threadIdx.x);
    const int cg = t % G, pr = t / G;
    const bool active = pr < PPB;
    const int hl = cg / GD, gi = cg % GD, head = head0 + hl;
    const int c0 = head * D + gi * 8;
    const T* y = static_cast<const T*>(p.y);
    const T* x = static_cast<const T*>(p.x);
    T* dy = static_cast<T*>(p.dy);
    T* dx = static_cast<T*>(p.dx);
    extern __shared__ float lds[];
    float* gt = lds;              // [16 pixels][CB] dout of the current tile
    float* red = lds + 16 * CB;   // [PPB][CB] reduction rows
    float s[4][8], k[4][8], acc_k[4][8], acc_s[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            s[r][j] = active ? p.scale[r * C + c0 + j] : 0.f;
            k[r][j] = active ? p.skip[(p.skip_per_dir ? r * C : 0) + c0 + j] : 0.f;
            acc_k[r][j] = 0.f;
            acc_s[r][j] = 0.f;
        }
    const int64_t base = (b * 4 * p.heads + head) * L * D + gi * 8;
    const int64_t h0 = band * 4;
    const int64_t tiles_w = (p.W + 3) / 4;
    for (int64_t tw = 0; tw < tiles_w; ++tw) {
        const int64_t w0 = tw * 4;
        for (int e = t; e < 16 * CB; e += 256) {
            const int q = e / CB, c = e % CB;
            const int64_t h = h0 + (q >> 2), w = w0 + (q & 3);
            float g = 0.f;
            if (h < p.H && w < p.W) {
                const int64_t l = h * p.W + w, ch = head0 * D + c;
                g = p.channels_last ? p.dout[(b * L + l) * C + ch] : p.dout[(b * C + ch) * L + l];
            }
            gt[q * CB + c] = g;
        }
        __syncthreads();
#pragma unroll
        for (int phase = 0; phase < 2; ++phase) {
            for (int q = pr; active && q < 16; q += PPB) {
                const int ph = phase == 0 ? q >> 2 : q & 3, pw = phase == 0 ? q & 3 : q >> 2;
                const int64_t h = h0 + ph, w = w0 + pw;
                if (h >= p.H || w >= p.W) continue;
                const float* g8 = gt + (ph * 4 + pw) * CB + hl * D + gi * 8;
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    const int r = 2 * phase + rr;
                    const int64_t at = base + r * stride_dir + pixel_to_scan(r, h, w, p.H, p.W) * D;
                    float yv[8], xv[8], oy[8], ox[8];
                    load8<T>(y + at, yv);
                    load8<T>(x + at, xv);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float gs = g8[j] * s[r][j];
                        oy[j] = gs;
                        ox[j] = gs * k[r][j];
                        acc_k[r][j] += gs * xv[j];
                        acc_s[r][j] += g8[j] * (yv[j] + k[r][j] * xv[j]);
                    }
                    store8<T>(dy + at, oy);
                    store8<T>(dx + at, ox);
                }
            }
        }
        __syncthreads();
    }
    float* prow = p.part + (b * gridDim.x + band) * width;
    for (int r = 0; r < 4; ++r) {
        for (int kind = 0; kind < 2; ++kind) {
            if (active) {
#pragma unroll
                for (int j = 0; j < 8; ++j) red[pr * CB + hl * D + gi * 8 + j] = kind == 0 ? acc_k[r][j] : acc_s[r][j];
            }
            __syncthreads();
            if (active && pr == 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float v = 0.f;
                    for (int q = 0; q < PPB; ++q) v += red[q * CB + hl * D + gi * 8 + j];
                    if (kind == 1) prow[(nk + r) * C + c0 + j] = v;
                    else if (nk == 4) prow[r * C + c0 + j] = v;
                    else acc_k[r][j] = v;   // shared skip: the four directions are added below
                }
            }
            __syncthreads();
        }
    }
    if (nk == 1 && active && pr == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) prow[c0 + j] = ((acc_k[0][j] + acc_k[1][j]) + acc_k[2][j]) + acc_k[3][j];
    }
}

// ---------------------------------------------------------------------------
// GRN backward (reference grn_cuda.cu:126-265; utils/grn.py:31-38 for the formula):
//   y = x (1 + gamma nx) + beta, nx_c = gx_c inv, gx_c = ||x_c||_2 over pixels,
//   inv = 1 / (mean_c gx_c + eps).  With P_c = sum dout x, s_c = gamma_c P_c:
//   dx = dout (1 + gamma nx) + x (s_c inv - inv^2 sum_c' s_c' gx_c' / C) / gx_c
//   (the last term is 0 where gx_c = 0), dgamma = sum_b P_c nx_c, dbeta = sum dout.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void grn_backward_partial_kernel(const float* __restrict__ dout,
                                                                   const T* __restrict__ x,
                                                                   float* __restrict__ part, int64_t S, int C,
                                                                   int64_t slab) {
    const int64_t b = blockIdx.y, sl = blockIdx.x;
    const int64_t s_begin = sl * slab, s_end = std::min<int64_t>(S, s_begin + slab);
    float* prow = part + (b * gridDim.x + sl) * 2 * C;
    __shared__ float red[2][256];
    for (int chunk = 0; chunk < C; chunk += 256) {
        const PixelChannelMap m(C, chunk);
        float sdx = 0.f, sd = 0.f;
        if (m.active) {
            for (int64_t s = s_begin + m.pix; s < s_end; s += m.ppb) {
                const int64_t i = (b * S + s) * C + m.c0;
                const float g = dout[i];
                sdx += g * to_f32(x[i]);
                sd += g;
            }
        }
        red[0][threadIdx.x] = sdx;
        red[1][threadIdx.x] = sd;
        __syncthreads();
        if (m.active && m.pix == 0) {
            float a = 0.f, d = 0.f;
            for (int j = 0; j < m.ppb; ++j) {
                const int src = (C <= 256) ? j * C + m.c0 : static_cast<int>(threadIdx.x);
                a += red[0][src];
                d += red[1][src];
            }
            prow[m.c0] = a;
            prow[C + m.c0] = d;
        }
        __syncthreads();
    }
}

// 16-byte variants (C % 8 == 0, C / 8 <= 256, aligned): thread t owns channel group t % G of
// pixel rows t / G, t / G + 256 / G, ... of the slab (partial sums), or one 8-channel group
// of one pixel (dx).
template <typename T>
__global__ __launch_bounds__(256) void grn_backward_partial8_kernel(const float* __restrict__ dout,
                                                                    const T* __restrict__ x, float* __restrict__ part,
                                                                    int64_t S, int C, int64_t slab) {
    const int64_t b = blockIdx.y, sl = blockIdx.x;
    const int64_t s_begin = sl * slab, s_end = std::min<int64_t>(S, s_begin + slab);
    const int G = C / 8, R = 256 / G;
    const int t = static_cast<int>(threadIdx.x), g = t % G, rr = t / G;
    float sdx[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, sd[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (rr < R) {
        for (int64_t s = s_begin + rr; s < s_end; s += R) {
            const int64_t i = (b * S + s) * C + g * 8;
            float d[8], xv[8];
            load8<float>(dout + i, d);
            load8<T>(x + i, xv);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sdx[j] += d[j] * xv[j];
                sd[j] += d[j];
            }
        }
    }
    __shared__ float red[2][256 * 8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        red[0][t * 8 + j] = sdx[j];
        red[1][t * 8 + j] = sd[j];
    }
    __syncthreads();
    if (t < G) {
        float* prow = part + (b * gridDim.x + sl) * 2 * C;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float a = 0.f, d = 0.f;
            for (int q = 0; q < R; ++q) {
                a += red[0][(q * G + t) * 8 + j];
                d += red[1][(q * G + t) * 8 + j];
            }
            prow[t * 8 + j] = a;
            prow[C + t * 8 + j] = d;
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void grn_backward_dx8_kernel(const float* __restrict__ dout, const T* __restrict__ x,
                                                               const float* __restrict__ coef, T* __restrict__ dx,
                                                               int64_t groups, int64_t S, int C) {
    const int G = C / 8;
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; q < groups;
         q += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t g = q % G, b = q / (S * G);
        const float* cf = coef + b * 2 * C + g * 8;
        float d[8], xv[8], a[8], c2[8], o[8];
        load8<float>(dout + q * 8, d);
        load8<T>(x + q * 8, xv);
        load8<float>(cf, a);
        load8<float>(cf + C, c2);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = d[j] * a[j] + c2[j] * xv[j];
        store8<T>(dx + q * 8, o);
    }
}

// One workgroup per image: per-channel sums over the slabs, then the coefficients of dx
// (coef[b][0][c] = 1 + gamma nx, coef[b][1][c] = the x factor) and the per-image parameter
// partials pp[b] = (P_c nx_c, sum dout).
__global__ __launch_bounds__(256) void grn_backward_finalize_kernel(const float* __restrict__ part,
                                                                    const float* __restrict__ gamma,
                                                                    const float* __restrict__ gx,
                                                                    const float* __restrict__ inv_den,
                                                                    float* __restrict__ coef, float* __restrict__ pp,
                                                                    int64_t nslab, int C) {
    const int64_t b = blockIdx.x;
    const float inv = inv_den[b];
    const float* prow = part + b * nslab * 2 * C;
    float* cf = coef + b * 2 * C;
    float* pb = pp + b * 2 * C;
    float sg = 0.f;
    for (int c = threadIdx.x; c < C; c += 256) {
        float a = 0.f, d = 0.f;
        for (int64_t j = 0; j < nslab; ++j) {
            a += prow[j * 2 * C + c];
            d += prow[j * 2 * C + C + c];
        }
        const float g = gx[b * C + c];
        const float nx = g * inv;
        const float sc = gamma[c] * a;
        cf[c] = 1.f + gamma[c] * nx;
        cf[C + c] = sc;   // s_c, finished below
        pb[c] = a * nx;
        pb[C + c] = d;
        sg += sc * g;
    }
    __shared__ float red[256];
    red[threadIdx.x] = sg;
    __syncthreads();
    for (int off = 128; off > 0; off >>= 1) {
        if (static_cast<int>(threadIdx.x) < off) red[threadIdx.x] += red[threadIdx.x + off];
        __syncthreads();
    }
    const float sum_sg = red[0];
    for (int c = threadIdx.x; c < C; c += 256) {
        const float g = gx[b * C + c];
        const float dg = cf[C + c] * inv - (sum_sg * inv * inv) / static_cast<float>(C);
        cf[C + c] = g > 0.f ? dg / g : 0.f;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void grn_backward_dx_kernel(const float* __restrict__ dout, const T* __restrict__ x,
                                                              const float* __restrict__ coef, T* __restrict__ dx,
                                                              int64_t total, int64_t S, int C) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t c = i % C, b = i / (S * C);
        const float* cf = coef + b * 2 * C;
        dx[i] = from_f32<T>(dout[i] * cf[c] + cf[C + c] * to_f32(x[i]));
    }
}

// ---------------------------------------------------------------------------
// LayerNorm over channels backward (reference layer_norm_cuda.py:59-121), channels-last
// rows of C: x^ = (x - mean) rstd, g = dy w,
//   dx = (g - mean_c(g) - x^ mean_c(g x^)) rstd,  dw = sum dy x^,  db = sum dy.
// TPR lanes per row, MAXV channels per lane (c = lane + k TPR); the per-lane parameter
// sums run over a grid-stride loop of rows, then over the rows of the workgroup.
// ---------------------------------------------------------------------------
template <typename T, int TPR, int MAXV>
__global__ __launch_bounds__(256) void layernorm_backward_kernel(const float* __restrict__ dy, const T* __restrict__ x,
                                                                 const float* __restrict__ w,
                                                                 const float* __restrict__ mean,
                                                                 const float* __restrict__ rstd, T* __restrict__ dx,
                                                                 float* __restrict__ part, int64_t rows, int C) {
    constexpr int RPB = 256 / TPR;
    const int lane = threadIdx.x % TPR;
    float dw[MAXV], db[MAXV];
#pragma unroll
    for (int k = 0; k < MAXV; ++k) dw[k] = db[k] = 0.f;
    const float inv_c = 1.f / static_cast<float>(C);
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR; row < rows;
         row += static_cast<int64_t>(gridDim.x) * RPB) {
        const float mu = mean[row], rs = rstd[row];
        float g[MAXV], xh[MAXV];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int k = 0; k < MAXV; ++k) {
            const int c = lane + k * TPR;
            if (c < C) {
                const float d = dy[row * C + c];
                xh[k] = (to_f32(x[row * C + c]) - mu) * rs;
                g[k] = d * w[c];
                dw[k] += d * xh[k];
                db[k] += d;
            } else {
                xh[k] = 0.f;
                g[k] = 0.f;
            }
            s1 += g[k];
            s2 += g[k] * xh[k];
        }
#pragma unroll
        for (int off = TPR / 2; off > 0; off >>= 1) {
            s1 += __shfl_xor(s1, off);
            s2 += __shfl_xor(s2, off);
        }
        s1 *= inv_c;
        s2 *= inv_c;
#pragma unroll
        for (int k = 0; k < MAXV; ++k) {
            const int c = lane + k * TPR;
            if (c < C) dx[row * C + c] = from_f32<T>((g[k] - s1 - xh[k] * s2) * rs);
        }
    }
    // rows of one wave: butterfly over the row bits of the lane index
#pragma unroll
    for (int k = 0; k < MAXV; ++k) {
#pragma unroll
        for (int off = TPR; off < 64; off <<= 1) {
            dw[k] += __shfl_xor(dw[k], off);
            db[k] += __shfl_xor(db[k], off);
        }
    }
    __shared__ float red[4][2][TPR * MAXV];
    const int wave = threadIdx.x / 64;
    if ((threadIdx.x & 63) < TPR) {
#pragma unroll
        for (int k = 0; k < MAXV; ++k) {
            red[wave][0][lane + k * TPR] = dw[k];
            red[wave][1][lane + k * TPR] = db[k];
        }
    }
    __syncthreads();
    float* prow = part + static_cast<int64_t>(blockIdx.x) * 2 * C;
    for (int c = threadIdx.x; c < C; c += 256) {
        prow[c] = ((red[0][0][c] + red[1][0][c]) + red[2][0][c]) + red[3][0][c];
        prow[C + c] = ((red[0][1][c] + red[1][1][c]) + red[2][1][c]) + red[3][1][c];
    }
}

// Vectorised variant for C % 8 == 0 and 16-byte aligned rows: lane l of a row's TPR lanes
// owns channel groups l + k TPR (k < GP) of 8 channels (16-byte x loads, two 16-byte dy
// loads); TPR = the power of two at or above C / 8 / GP.
template <typename T, int TPR, int GP>
__global__ __launch_bounds__(256) void layernorm_backward8_kernel(const float* __restrict__ dy, const T* __restrict__ x,
                                                                  const float* __restrict__ w,
                                                                  const float* __restrict__ mean,
                                                                  const float* __restrict__ rstd, T* __restrict__ dx,
                                                                  float* __restrict__ part, int64_t rows, int C) {
    constexpr int RPB = 256 / TPR;
    const int lane = threadIdx.x % TPR, G = C / 8;
    float dw[GP][8], db[GP][8], wv[GP][8];
#pragma unroll
    for (int k = 0; k < GP; ++k) {
        const int g = lane + k * TPR;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            dw[k][j] = db[k][j] = 0.f;
            wv[k][j] = g < G ? w[g * 8 + j] : 0.f;
        }
    }
    const float inv_c = 1.f / static_cast<float>(C);
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / TPR; row < rows;
         row += static_cast<int64_t>(gridDim.x) * RPB) {
        const float mu = mean[row], rs = rstd[row];
        float g8[GP][8], xh[GP][8];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int k = 0; k < GP; ++k) {
            const int g = lane + k * TPR;
            if (g < G) {
                float d[8], xv[8];
                load8<float>(dy + row * C + g * 8, d);
                load8<T>(x + row * C + g * 8, xv);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    xh[k][j] = (xv[j] - mu) * rs;
                    g8[k][j] = d[j] * wv[k][j];
                    dw[k][j] += d[j] * xh[k][j];
                    db[k][j] += d[j];
                    s1 += g8[k][j];
                    s2 += g8[k][j] * xh[k][j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) xh[k][j] = g8[k][j] = 0.f;
            }
        }
#pragma unroll
        for (int off = TPR / 2; off > 0; off >>= 1) {
            s1 += __shfl_xor(s1, off);
            s2 += __shfl_xor(s2, off);
        }
        s1 *= inv_c;
        s2 *= inv_c;
#pragma unroll
        for (int k = 0; k < GP; ++k) {
            const int g = lane + k * TPR;
            if (g < G) {
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = (g8[k][j] - s1 - xh[k][j] * s2) * rs;
                store8<T>(dx + row * C + g * 8, o);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < GP; ++k)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int off = TPR; off < 64; off <<= 1) {
                dw[k][j] += __shfl_xor(dw[k][j], off);
                db[k][j] += __shfl_xor(db[k][j], off);
            }
    __shared__ float red[4][2][TPR * GP * 8];
    const int wave = threadIdx.x / 64;
    if ((threadIdx.x & 63) < TPR) {
#pragma unroll
        for (int k = 0; k < GP; ++k)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                red[wave][0][(lane + k * TPR) * 8 + j] = dw[k][j];
                red[wave][1][(lane + k * TPR) * 8 + j] = db[k][j];
            }
    }
    __syncthreads();
    float* prow = part + static_cast<int64_t>(blockIdx.x) * 2 * C;
    for (int c = threadIdx.x; c < C; c += 256) {
        prow[c] = ((red[0][0][c] + red[1][0][c]) + red[2][0][c]) + red[3][0][c];
        prow[C + c] = ((red[0][1][c] + red[1][1][c]) + red[2][1][c]) + red[3][1][c];
    }
}

// (TPR, GP) of the vectorised LayerNorm backward for C % 8 == 0, C <= 1024.
void ln8_shape(int64_t C, int* tpr, int* gp) {
    const int64_t G = C / 8;
    *gp = G > 64 ? 2 : 1;
    const int64_t per = (G + *gp - 1) / *gp;
    int t = 2;
    while (t < per) t <<= 1;
    *tpr = t;
}

int64_t ln_backward_blocks(int64_t rows, int tpr) {
    const int64_t rpb = 256 / tpr;
    return std::max<int64_t>(1, std::min<int64_t>((rows + rpb - 1) / rpb, 1024));
}

int ln_tpr(int64_t C) { return C <= 16 ? 4 : C <= 32 ? 8 : C <= 64 ? 16 : C <= 128 ? 32 : 64; }

// ---------------------------------------------------------------------------
// Query normalisation backward (reference query_normalization.cu:78-134):
//   q^ = q inv, inv = 1 / max(|q|, 1e-12);  dq = (g - q^ (g . q^)) inv, or g inv where the
//   epsilon bound (inv = 1e12) holds.  g, q^: [B, R, heads, N, d] fp32; inv [B, R, heads, N];
//   dq: [B, R, N, heads d] in the raw query's dtype.
// ---------------------------------------------------------------------------
template <int D, typename T>
__global__ __launch_bounds__(256) void qnorm_backward_kernel(const float* __restrict__ g, const float* __restrict__ qn,
                                                             const float* __restrict__ inv_norm, T* __restrict__ dq,
                                                             int64_t B, int64_t R, int64_t N, int64_t heads) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= B * R * N * heads) return;
    const int64_t head = idx % heads;
    const int64_t t = (idx / heads) % N;
    const int64_t br = idx / (heads * N);
    const int64_t v = (br * heads + head) * N + t;
    const float* gv = g + v * D;
    const float* qv = qn + v * D;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < D; ++j) dot += gv[j] * qv[j];
    const float inv = inv_norm[v];
    const bool eps_bound = inv > 9.999e11f;
    T* dst = dq + (br * N + t) * heads * D + head * D;
#pragma unroll
    for (int j = 0; j < D; ++j) dst[j] = from_f32<T>((eps_bound ? gv[j] : gv[j] - qv[j] * dot) * inv);
}

// ---------------------------------------------------------------------------
// Residual add backward (reference utils/residual.py:55-101,132-170):
//   out = residual + branch gamma_c mask_b:  dbranch = dout gamma_c mask_b,
//   dgamma_c = sum dout branch mask_b  (dresidual = dout is the caller's).
// Grid over row segments of channels-last [rows = B S, C]; partial rows [segments][C].
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void residual_backward_kernel(const float* __restrict__ dout,
                                                                const T* __restrict__ branch,
                                                                const float* __restrict__ gamma,
                                                                const float* __restrict__ mask, T* __restrict__ dbranch,
                                                                float* __restrict__ part, int64_t rows, int64_t S,
                                                                int C, int64_t seg_len) {
    const int64_t r_begin = static_cast<int64_t>(blockIdx.x) * seg_len;
    const int64_t r_end = std::min<int64_t>(rows, r_begin + seg_len);
    float* prow = part + static_cast<int64_t>(blockIdx.x) * C;
    __shared__ float red[256];
    for (int chunk = 0; chunk < C; chunk += 256) {
        const PixelChannelMap m(C, chunk);
        float acc = 0.f;
        if (m.active) {
            const float g = gamma[m.c0];
            for (int64_t r = r_begin + m.pix; r < r_end; r += m.ppb) {
                const int64_t i = r * C + m.c0;
                const float d = dout[i] * mask[r / S];
                dbranch[i] = from_f32<T>(d * g);
                acc += d * to_f32(branch[i]);
            }
        }
        red[threadIdx.x] = acc;
        __syncthreads();
        if (m.active && m.pix == 0) {
            float a = 0.f;
            for (int j = 0; j < m.ppb; ++j) a += red[(C <= 256) ? j * C + m.c0 : static_cast<int>(threadIdx.x)];
            prow[m.c0] = a;
        }
        __syncthreads();
    }
}

int64_t residual_segment(int64_t rows) { return std::max<int64_t>(16, (rows + 2047) / 2048); }

struct FusionLayout {
    int64_t segments, seg_len, width;
    size_t bytes;
};

FusionLayout fusion_layout(int64_t B, int64_t C, int64_t L, int skip_per_dir) {
    FusionLayout f;
    const int64_t want = std::max<int64_t>(1, 2048 / std::max<int64_t>(B, 1));
    f.segments = std::max<int64_t>(1, std::min<int64_t>(want, (L + 15) / 16));
    f.seg_len = (L + f.segments - 1) / f.segments;
    f.segments = (L + f.seg_len - 1) / f.seg_len;
    f.width = ((skip_per_dir ? 4 : 1) + 4) * C;
    f.bytes = round256(static_cast<size_t>(B * f.segments * f.width) * sizeof(float));
    return f;
}

struct GrnLayout {
    int64_t nslab, slab;
    size_t part, coef, pp, total;
};

GrnLayout grn_layout(int64_t B, int64_t C, int64_t S) {
    GrnLayout g;
    const int64_t want = std::max<int64_t>(1, 2048 / std::max<int64_t>(B, 1));
    g.nslab = std::max<int64_t>(1, std::min<int64_t>(want, (S + 7) / 8));
    g.slab = (S + g.nslab - 1) / g.nslab;
    g.nslab = (S + g.slab - 1) / g.slab;
    g.part = round256(static_cast<size_t>(B * g.nslab * 2 * C) * sizeof(float));
    g.coef = round256(static_cast<size_t>(B * 2 * C) * sizeof(float));
    g.pp = g.coef;
    g.total = g.part + g.coef + g.pp;
    return g;
}

}  // namespace
}  // namespace vh

using namespace vh;

extern "C" {

size_t vh_postprocess_scale_backward_workspace_bytes(int64_t B, int64_t heads, int64_t H, int64_t W,
                                                     int32_t head_dim, int32_t skip_per_dir) {
    if (B <= 0 || heads <= 0 || H <= 0 || W <= 0 || head_dim <= 0) return 0;
    // either kernel's partial rows (the tiled one writes one row per image and band of 4 rows)
    const size_t tiled = round256(static_cast<size_t>(B * ((H + 3) / 4) * ((skip_per_dir ? 4 : 1) + 4) * heads *
                                                      head_dim) * sizeof(float));
    return std::max(tiled, fusion_layout(B, heads * head_dim, H * W, skip_per_dir).bytes);
}

int vh_postprocess_scale_backward(const float* dout, int32_t dout_channels_last, const void* y, const void* x,
                                  int32_t io_dtype, const float* d_skip, int32_t skip_per_dir, const float* scale,
                                  void* dy, void* dx, float* d_dskip, float* d_scale, int64_t B, int64_t heads,
                                  int64_t H, int64_t W, int32_t head_dim, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    VH_REQUIRE(dout && y && x && d_skip && scale && dy && dx && d_dskip && d_scale, VH_ERR_ARG,
               "direction fusion backward pointers must not be null");
    VH_REQUIRE(B > 0 && heads > 0 && H > 0 && W > 0 && head_dim > 0, VH_ERR_SHAPE,
               "direction fusion backward expects nonempty input");
    VH_REQUIRE(B <= 65535, VH_ERR_SHAPE, "direction fusion backward supports batch <= 65535");
    const int64_t C = heads * head_dim;
    VH_REQUIRE(C <= (int64_t(1) << 20), VH_ERR_SHAPE, "too many channels (%lld)", (long long)C);
    const FusionLayout f = fusion_layout(B, C, H * W, skip_per_dir);
    const size_t need = vh_postprocess_scale_backward_workspace_bytes(B, heads, H, W, head_dim, skip_per_dir);
    VH_REQUIRE(workspace && workspace_bytes >= need, VH_ERR_WORKSPACE,
               "direction fusion backward workspace needs %zu bytes, got %zu", need,
               workspace ? workspace_bytes : (size_t)0);
    hipStream_t s = static_cast<hipStream_t>(stream);
    FusionBwdParams p{dout, y, x, d_skip, scale, dy, dx, static_cast<float*>(workspace), heads, H, W, head_dim,
                      f.seg_len, skip_per_dir ? 1 : 0, dout_channels_last ? 1 : 0};
    const uintptr_t align = reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(x) |
                            reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(dx);
    if (head_dim >= 8 && head_dim % 8 == 0 && head_dim <= 64 && align % 16 == 0) {
        // at most 96 channels (12 groups of 8) per workgroup: the kernel's one-pixel-per-thread-row layout
        const int hpb = static_cast<int>(std::min<int64_t>(heads, std::max(1, 96 / head_dim)));
        const int64_t bands = (H + 3) / 4, chunks = (heads + hpb - 1) / hpb;
        const size_t lds = static_cast<size_t>(16 * hpb * head_dim + 256 * 8) * sizeof(float);
        const dim3 grid(static_cast<unsigned>(bands), static_cast<unsigned>(B), static_cast<unsigned>(chunks));
        int ok = 1;
        const int rc = dispatch_io(io_dtype, [&](auto tv) {
            using T = decltype(tv);
            switch (head_dim) {
                case 8: hipLaunchKernelGGL((fusion_backward_tile_kernel<8, T>), grid, dim3(256), lds, s, p, hpb); break;
                case 16: hipLaunchKernelGGL((fusion_backward_tile_kernel<16, T>), grid, dim3(256), lds, s, p, hpb); break;
                case 32: hipLaunchKernelGGL((fusion_backward_tile_kernel<32, T>), grid, dim3(256), lds, s, p, hpb); break;
                case 64: hipLaunchKernelGGL((fusion_backward_tile_kernel<64, T>), grid, dim3(256), lds, s, p, hpb); break;
                default: ok = 0;
            }
        });
        if (rc) return rc;
        if (ok) {
            launch_column_sum(p.part, B * bands, (skip_per_dir ? 4 : 1) * C + 4 * C, (skip_per_dir ? 4 : 1) * C,
                              d_dskip, d_scale, s);
            return check_launch("direction fusion backward (tiled)");
        }
    }
    const int rc = dispatch_io(io_dtype, [&](auto tv) {
        hipLaunchKernelGGL((fusion_backward_kernel<decltype(tv)>), dim3(static_cast<unsigned>(f.segments),
                           static_cast<unsigned>(B)), dim3(256), 0, s, p);
    });
    if (rc) return rc;
    const int64_t nk = skip_per_dir ? 4 : 1;
    launch_column_sum(p.part, B * f.segments, f.width, nk * C, d_dskip, d_scale, s);
    return check_launch("direction fusion backward");
}

size_t vh_grn_backward_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W) {
    if (B <= 0 || C <= 0 || H <= 0 || W <= 0) return 0;
    return grn_layout(B, C, H * W).total;
}

int vh_grn_backward(const float* dout, const void* x, int32_t io_dtype, const float* gamma, const float* gx,
                    const float* inv_den, void* dx, float* dgamma, float* dbeta, int64_t B, int64_t C, int64_t H,
                    int64_t W, void* workspace, size_t workspace_bytes, void* stream) {
    VH_REQUIRE(dout && x && gamma && gx && inv_den && dx && dgamma && dbeta, VH_ERR_ARG,
               "GRN backward pointers must not be null");
    VH_REQUIRE(B > 0 && B <= 65535 && C > 0 && H > 0 && W > 0, VH_ERR_SHAPE,
               "GRN backward expects nonempty input and batch <= 65535");
    VH_REQUIRE(C <= (int64_t(1) << 20), VH_ERR_SHAPE, "too many channels (%lld)", (long long)C);
    const int64_t S = H * W;
    const GrnLayout g = grn_layout(B, C, S);
    VH_REQUIRE(workspace && workspace_bytes >= g.total, VH_ERR_WORKSPACE,
               "GRN backward workspace needs %zu bytes, got %zu", g.total, workspace ? workspace_bytes : (size_t)0);
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    float* part = reinterpret_cast<float*>(ws);
    float* coef = reinterpret_cast<float*>(ws + g.part);
    float* pp = reinterpret_cast<float*>(ws + g.part + g.coef);
    const int c = static_cast<int>(C);
    const int64_t total = B * S * C;
    const unsigned dx_blocks = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 8192));
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dx) |
                            reinterpret_cast<uintptr_t>(dout) | reinterpret_cast<uintptr_t>(workspace) | g.part;
    const bool vec = C % 8 == 0 && C / 8 <= 256 && align % 16 == 0;
    const int rc = dispatch_io(io_dtype, [&](auto tv) {
        using T = decltype(tv);
        if (vec) {
            hipLaunchKernelGGL((grn_backward_partial8_kernel<T>), dim3(static_cast<unsigned>(g.nslab),
                               static_cast<unsigned>(B)), dim3(256), 0, s, dout, static_cast<const T*>(x), part, S, c,
                               g.slab);
            hipLaunchKernelGGL(grn_backward_finalize_kernel, dim3(static_cast<unsigned>(B)), dim3(256), 0, s, part,
                               gamma, gx, inv_den, coef, pp, g.nslab, c);
            const int64_t groups = total / 8;
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((groups + 255) / 256, 8192));
            hipLaunchKernelGGL((grn_backward_dx8_kernel<T>), dim3(blocks), dim3(256), 0, s, dout,
                               static_cast<const T*>(x), coef, static_cast<T*>(dx), groups, S, c);
            return;
        }
        hipLaunchKernelGGL((grn_backward_partial_kernel<T>), dim3(static_cast<unsigned>(g.nslab),
                           static_cast<unsigned>(B)), dim3(256), 0, s, dout, static_cast<const T*>(x), part, S, c,
                           g.slab);
        hipLaunchKernelGGL(grn_backward_finalize_kernel, dim3(static_cast<unsigned>(B)), dim3(256), 0, s, part, gamma,
                           gx, inv_den, coef, pp, g.nslab, c);
        hipLaunchKernelGGL((grn_backward_dx_kernel<T>), dim3(dx_blocks), dim3(256), 0, s, dout,
                           static_cast<const T*>(x), coef, static_cast<T*>(dx), total, S, c);
    });
    if (rc) return rc;
    launch_column_sum(pp, B, 2 * C, C, dgamma, dbeta, s);
    return check_launch("GRN backward");
}

size_t vh_layernorm2d_backward_workspace_bytes(int64_t B, int64_t C, int64_t H, int64_t W) {
    if (B <= 0 || C <= 0 || H <= 0 || W <= 0) return 0;
    return round256(static_cast<size_t>(ln_backward_blocks(B * H * W, ln_tpr(C)) * 2 * C) * sizeof(float));
}

int vh_layernorm2d_backward(const float* dy, const void* x, int32_t io_dtype, const float* weight, const float* mean,
                            const float* rstd, void* dx, float* dweight, float* dbias, int64_t B, int64_t C,
                            int64_t H, int64_t W, void* workspace, size_t workspace_bytes, void* stream) {
    VH_REQUIRE(dy && x && weight && mean && rstd && dx && dweight && dbias, VH_ERR_ARG,
               "LayerNorm2d backward pointers must not be null");
    VH_REQUIRE(B > 0 && C > 0 && H > 0 && W > 0, VH_ERR_SHAPE, "LayerNorm2d backward expects nonempty input");
    VH_REQUIRE(C <= 1024, VH_ERR_SHAPE, "LayerNorm2d backward supports at most 1024 channels, got %lld",
               (long long)C);
    const int64_t rows = B * H * W;
    const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dx) |
                            reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(weight);
    int tpr8 = 0, gp8 = 0;
    ln8_shape(C, &tpr8, &gp8);
    const bool vec = C % 8 == 0 && align % 16 == 0;
    const int tpr = vec ? tpr8 : ln_tpr(C);
    const int64_t blocks = ln_backward_blocks(rows, tpr);
    const size_t need = vh_layernorm2d_backward_workspace_bytes(B, C, H, W);
    VH_REQUIRE(workspace && workspace_bytes >= need, VH_ERR_WORKSPACE,
               "LayerNorm2d backward workspace needs %zu bytes, got %zu", need, workspace ? workspace_bytes : (size_t)0);
    hipStream_t s = static_cast<hipStream_t>(stream);
    float* part = static_cast<float*>(workspace);
    const int c = static_cast<int>(C);
    const dim3 grid(static_cast<unsigned>(blocks));
    const int rc = dispatch_io(io_dtype, [&](auto tv) {
        using T = decltype(tv);
        const T* xp = static_cast<const T*>(x);
        T* dxp = static_cast<T*>(dx);
#define VH_LN_BWD8(TPR, GP) \
    hipLaunchKernelGGL((layernorm_backward8_kernel<T, TPR, GP>), grid, dim3(256), 0, s, dy, xp, weight, mean, rstd, \
                       dxp, part, rows, c)
        if (vec) {
            if (gp8 == 2) VH_LN_BWD8(64, 2);
            else if (tpr8 == 2) VH_LN_BWD8(2, 1);
            else if (tpr8 == 4) VH_LN_BWD8(4, 1);
            else if (tpr8 == 8) VH_LN_BWD8(8, 1);
            else if (tpr8 == 16) VH_LN_BWD8(16, 1);
            else if (tpr8 == 32) VH_LN_BWD8(32, 1);
            else VH_LN_BWD8(64, 1);
            return;
        }
#undef VH_LN_BWD8
#define VH_LN_BWD(TPR, MAXV) \
    hipLaunchKernelGGL((layernorm_backward_kernel<T, TPR, MAXV>), grid, dim3(256), 0, s, dy, xp, weight, mean, rstd, \
                       dxp, part, rows, c)
        if (tpr == 4) VH_LN_BWD(4, 4);
        else if (tpr == 8) VH_LN_BWD(8, 4);
        else if (tpr == 16) VH_LN_BWD(16, 4);
        else if (tpr == 32) VH_LN_BWD(32, 4);
        else if (C <= 256) VH_LN_BWD(64, 4);
        else if (C <= 512) VH_LN_BWD(64, 8);
        else VH_LN_BWD(64, 16);
#undef VH_LN_BWD
    });
    if (rc) return rc;
    launch_column_sum(part, blocks, 2 * C, C, dweight, dbias, s);
    return check_launch("LayerNorm2d backward");
}

size_t vh_residual_add_backward_workspace_bytes(int64_t total, int64_t channels) {
    if (total <= 0 || channels <= 0 || total % channels) return 0;
    const int64_t rows = total / channels, seg = residual_segment(rows);
    return round256(static_cast<size_t>((rows + seg - 1) / seg * channels) * sizeof(float));
}

int vh_residual_add_backward(const float* dout, const void* branch, int32_t branch_dtype, const float* gamma,
                             const float* mask, void* dbranch, float* dgamma, int64_t total, int64_t channels,
                             int64_t spatial, void* workspace, size_t workspace_bytes, void* stream) {
    VH_REQUIRE(dout && branch && gamma && mask && dbranch && dgamma, VH_ERR_ARG,
               "residual add backward pointers must not be null");
    VH_REQUIRE(total > 0 && channels > 0 && spatial > 0 && total % (channels * spatial) == 0, VH_ERR_SHAPE,
               "residual add backward: total must be a positive multiple of channels * spatial");
    VH_REQUIRE(channels <= (int64_t(1) << 20), VH_ERR_SHAPE, "too many channels (%lld)", (long long)channels);
    const size_t need = vh_residual_add_backward_workspace_bytes(total, channels);
    VH_REQUIRE(workspace && workspace_bytes >= need, VH_ERR_WORKSPACE,
               "residual add backward workspace needs %zu bytes, got %zu", need, workspace ? workspace_bytes : (size_t)0);
    const int64_t rows = total / channels, seg = residual_segment(rows), nseg = (rows + seg - 1) / seg;
    hipStream_t s = static_cast<hipStream_t>(stream);
    float* part = static_cast<float*>(workspace);
    const int rc = dispatch_io(branch_dtype, [&](auto tv) {
        using T = decltype(tv);
        hipLaunchKernelGGL((residual_backward_kernel<T>), dim3(static_cast<unsigned>(nseg)), dim3(256), 0, s, dout,
                           static_cast<const T*>(branch), gamma, mask, static_cast<T*>(dbranch), part, rows, spatial,
                           static_cast<int>(channels), seg);
    });
    if (rc) return rc;
    launch_column_sum(part, nseg, channels, channels, dgamma, dgamma, s);
    return check_launch("residual add backward");
}

int vh_qnorm_backward(const float* dq_out, const float* q_out, const float* inv_norm, void* dq_raw, int32_t io_dtype,
                      int64_t B, int64_t R, int64_t N, int64_t heads, int32_t head_dim, void* stream) {
    VH_REQUIRE(dq_out && q_out && inv_norm && dq_raw, VH_ERR_ARG, "qnorm backward pointers must not be null");
    VH_REQUIRE(B > 0 && R > 0 && N > 0 && heads > 0, VH_ERR_SHAPE, "qnorm backward expects nonempty input");
    const int64_t total = B * R * N * heads;
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    hipStream_t s = static_cast<hipStream_t>(stream);
    bool ok_d = true;
    const int rc = dispatch_io(io_dtype, [&](auto tv) {
        using T = decltype(tv);
        T* out = static_cast<T*>(dq_raw);
        switch (head_dim) {
            case 4: hipLaunchKernelGGL((qnorm_backward_kernel<4, T>), grid, dim3(256), 0, s, dq_out, q_out, inv_norm, out, B, R, N, heads); break;
            case 8: hipLaunchKernelGGL((qnorm_backward_kernel<8, T>), grid, dim3(256), 0, s, dq_out, q_out, inv_norm, out, B, R, N, heads); break;
            case 16: hipLaunchKernelGGL((qnorm_backward_kernel<16, T>), grid, dim3(256), 0, s, dq_out, q_out, inv_norm, out, B, R, N, heads); break;
            case 32: hipLaunchKernelGGL((qnorm_backward_kernel<32, T>), grid, dim3(256), 0, s, dq_out, q_out, inv_norm, out, B, R, N, heads); break;
            case 64: hipLaunchKernelGGL((qnorm_backward_kernel<64, T>), grid, dim3(256), 0, s, dq_out, q_out, inv_norm, out, B, R, N, heads); break;
            default: ok_d = false;
        }
    });
    if (rc) return rc;
    VH_REQUIRE(ok_d, VH_ERR_HEAD_DIM, "qnorm backward supports head_dim 4, 8, 16, 32, 64, got %d", head_dim);
    return check_launch("qnorm backward");
}

}  // extern "C"
