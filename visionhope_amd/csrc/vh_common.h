// Shared helpers for the gfx950 kernels of libvisionhope_hip.so: element
// conversions, argument checking and the per-thread error message.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdint>
#include <cstdio>
#include <type_traits>

#include "../../include/visionhope_hip.h"
#include "gelu_table.h"

namespace vh {

// ---------------------------------------------------------------------------
// Host-side error reporting: every entry point returns a status code and
// leaves a message for vh_last_error() on the calling thread.
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// Dispatch overrides (vh_set_dispatch_override): the value forced for `name`, or an empty
// string when none is set.  The kernel choice of every entry point is otherwise a function
// of its arguments alone.
struct Override {
    char value[32];
    explicit Override(const char* name);
    bool set() const { return value[0] != 0; }
    int as_int() const;
    long long as_i64() const;
};

// Range checks of the recurrence's stability constants, shared by the forward and the
// backward entry points (the reference validates the same ranges when it reads them from
// the environment, models/srnl_core/chunk.py:50-58).
int check_srnl_consts(const vh_srnl_consts* k);

// The fused four-direction operator of vh_srnl_spatial_forward on a given workspace
// (srnl.hip), and its shape checks.
int check_spatial_shape(int64_t B, int64_t H, int64_t W, int64_t C, int32_t head_dim);
int srnl_spatial_forward_ws(const void* x, const void* q, int32_t io_dtype, const float* M_m, const float* M_v,
                            const float* M_k, const float* M_eta, const float* M_alpha, const float* d_skip,
                            int32_t skip_per_direction, const float* dir_weight, float* out, int64_t B, int64_t H,
                            int64_t W, int64_t C, int32_t head_dim, const int64_t chunks[4],
                            const vh_srnl_consts* consts, void* workspace, size_t workspace_bytes,
                            hipStream_t stream);

// GRN statistics from per-slab partial sums of squares (elementwise.hip).
int launch_grn_finalize(const float* partial, float* gx, float* inv_den, int64_t B, int64_t C, int64_t nslab,
                        float eps, const float* gamma, float* scale, hipStream_t s);

#define VH_REQUIRE(cond, code, ...)                        \
    do {                                                   \
        if (!(cond)) return ::vh::set_error((code), __VA_ARGS__); \
    } while (0)

inline bool valid_head_dim(int d) { return d == 4 || d == 8 || d == 16 || d == 32 || d == 64; }
inline bool valid_dtype(int t) { return t == VH_DTYPE_F32 || t == VH_DTYPE_BF16 || t == VH_DTYPE_F16; }

// ---------------------------------------------------------------------------
// Element types.  bf16 and fp16 are carried as raw 16-bit patterns.
// ---------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16_t v) {
    _Float16 h;
    __builtin_memcpy(&h, &v.bits, 2);
    return static_cast<float>(h);
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
    // v_cvt_pk_bf16_f32: round to nearest even; NaNs stay NaN (quieted).
    return bf16_t{__builtin_bit_cast(uint16_t, static_cast<__bf16>(v))};
}
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float v) {
    _Float16 h = static_cast<_Float16>(v);
    f16_t r;
    __builtin_memcpy(&r.bits, &h, 2);
    return r;
}

// Eight consecutive elements as fp32 (16-byte load of 16-bit types, two of fp32);
// the address must be 16-byte aligned.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
    if constexpr (sizeof(T) == 4) {
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            v[2 * h] = to_f32(T{static_cast<uint16_t>(w[h] & 0xffffu)});
            v[2 * h + 1] = to_f32(T{static_cast<uint16_t>(w[h] >> 16)});
        }
    }
}

// The same eight elements kept as loaded (16 bytes of a 16-bit type, 32 of fp32) so a
// kernel can issue many loads before it spends registers on the fp32 values.
template <typename T> struct Pack8 { uint4 u; };
template <> struct Pack8<float> { float4 a, b; };

template <typename T>
__device__ __forceinline__ Pack8<T> load_pack8(const T* p) {
    Pack8<T> r;
    if constexpr (sizeof(T) == 4) {
        r.a = *reinterpret_cast<const float4*>(p);
        r.b = *reinterpret_cast<const float4*>(p + 4);
    } else {
        r.u = *reinterpret_cast<const uint4*>(p);
    }
    return r;
}

template <typename T>
__device__ __forceinline__ void pack8_to_f32(const Pack8<T>& r, float (&v)[8]) {
    if constexpr (sizeof(T) == 4) {
        v[0] = r.a.x; v[1] = r.a.y; v[2] = r.a.z; v[3] = r.a.w;
        v[4] = r.b.x; v[5] = r.b.y; v[6] = r.b.z; v[7] = r.b.w;
    } else {
        const uint32_t w[4] = {r.u.x, r.u.y, r.u.z, r.u.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            v[2 * h] = to_f32(T{static_cast<uint16_t>(w[h] & 0xffffu)});
            v[2 * h + 1] = to_f32(T{static_cast<uint16_t>(w[h] >> 16)});
        }
    }
}

typedef __bf16 vh_bf16x2 __attribute__((ext_vector_type(2)));
typedef float vh_f32x2 __attribute__((ext_vector_type(2)));

// Two floats as one packed bf16 pair (one v_cvt_pk_bf16_f32), low half first.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const vh_f32x2 f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, vh_bf16x2));
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&v)[8]) {
    if constexpr (sizeof(T) == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else if constexpr (std::is_same<T, bf16_t>::value) {
        *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                  pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
    } else {
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 4; ++h)
            w[h] = static_cast<uint32_t>(from_f32<T>(v[2 * h]).bits) |
                   (static_cast<uint32_t>(from_f32<T>(v[2 * h + 1]).bits) << 16);
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Element size of an io dtype code.
inline int dtype_bytes(int t) { return t == VH_DTYPE_F32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// Scan-order maps of the four-direction operator (models/operator.py:79-86;
// restoration in models/srnl_core/csrc/parallel_line.cuh:16-23).
//   t0 = h*W + w, t1 = L-1-t0, t2 = w*H + h, t3 = L-1-t2.
// ---------------------------------------------------------------------------
// n / d and n % d for n < 2^24 and d >= 1, with inv_d = 1.0f / d rounded to nearest.
// float(n) is exact and n * inv_d is within 2/d of n/d, so the truncated quotient is off
// by at most one (exact for d = 1); one correction step makes it exact.
__device__ __forceinline__ void divmod24(uint32_t n, uint32_t d, float inv_d, uint32_t& q, uint32_t& rem) {
    uint32_t qq = static_cast<uint32_t>(static_cast<float>(n) * inv_d);
    int32_t rr = static_cast<int32_t>(n - qq * d);
    if (rr < 0) {
        --qq;
        rr += static_cast<int32_t>(d);
    } else if (rr >= static_cast<int32_t>(d)) {
        ++qq;
        rr -= static_cast<int32_t>(d);
    }
    q = qq;
    rem = static_cast<uint32_t>(rr);
}

// Pixel of scan index t of direction r on an H x W image (H*W < 2^24, inv_h = 1.0f / H).
__device__ __forceinline__ int64_t scan_to_pixel(int r, int64_t t, int64_t H, int64_t W, float inv_h) {
    const int64_t L = H * W;
    const int64_t orig = (r & 1) ? L - 1 - t : t;
    if (r < 2) return orig;
    uint32_t w, h;
    divmod24(static_cast<uint32_t>(orig), static_cast<uint32_t>(H), inv_h, w, h);
    return static_cast<int64_t>(h) * W + w;
}
__device__ __forceinline__ int64_t pixel_to_scan(int r, int64_t h, int64_t w, int64_t H, int64_t W) {
    const int64_t L = H * W;
    const int64_t base = r < 2 ? h * W + w : w * H + h;
    return (r & 1) ? L - 1 - base : base;
}

// Workgroups are dispatched round-robin over the 8 XCDs of MI355X.  Remap the
// block index so that each XCD receives one contiguous range of work items
// (neighbouring lines of one image share the XCD's L2).
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t n) {
    if (n % 8 != 0) return bid;
    return (bid % 8) * (n / 8) + bid / 8;
}

// The same for any grid size n: XCD x receives the n/8 (+1 for x < n%8) blocks
// x, x+8, ... and maps them to one contiguous range starting at x*(n/8) + min(x, n%8).
__device__ __forceinline__ uint32_t xcd_remap_any(uint32_t bid, uint32_t n) {
    const uint32_t q = n / 8, r = n % 8, x = bid % 8;
    return x * q + (x < r ? x : r) + bid / 8;
}

// ---------------------------------------------------------------------------
// Division by a launch-invariant divisor d >= 1 for dividends n < 2^31, by one
// multiplication (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994).  With l = ceil(log2 d) and m = ceil(2^(32+l) / d),
// n*m / 2^(32+l) = n/d + n*e/2^(32+l) with 0 <= e < 1, and n*e*d < 2^(32+l), so
// the error never reaches the next integer: floor(n/d) = (n*m) >> (32+l).
// n*m < 2^31 * (2^33 + 1) fits 64 bits.
// ---------------------------------------------------------------------------
struct FastDiv {
    uint64_t m;
    uint32_t d;
    uint32_t shift;
};
inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((uint64_t(1) << l) < d) ++l;
    const unsigned __int128 num = static_cast<unsigned __int128>(1) << (32 + l);
    const uint64_t m = static_cast<uint64_t>((num + d - 1) / d);
    return FastDiv{m, d, 32 + l};
}
__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
    return static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> f.shift);
}

// ---------------------------------------------------------------------------
// Activations on the hardware exp2 / reciprocal (v_exp_f32, v_rcp_f32, about one ulp
// each), branch-free.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sigmoid_fast(float v) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.44269504088896341f * v));
}

// GELU in its exact form x * Phi(x), Phi(x) = erfc(-x/sqrt(2)) / 2.  erfc(z), z >= 0,
// takes the form t * exp(-z^2 + P(t)), t = 1 / (1 + z/2) (Press, Teukolsky, Vetterling
// and Flannery, Numerical Recipes, 2nd ed., section 6.2), with our own degree-5 P: a
// minimax fit of ln(erfc(z) / t) + z^2 over z in [0, 7] (largest relative error of erfc
// 7.6e-6; past z = 7 the exponential is below 1e-21).  The coefficients below are
// log2(e) * P with the factor 1/2 folded into the constant term, so one exp2 gives
// erfc(z) / 2.  Evaluating the tail x < 0 through erfc keeps the small outputs
// relatively accurate; in fp32 the result is within 1e-5 (relative) of x * Phi(x) over
// the whole real line.
__device__ __forceinline__ float gelu_fast(float x) {
    // t = 1 / (1 + z/2) with z = |x| / sqrt(2)
    const float t = __builtin_amdgcn_rcpf(fmaf(fabsf(x), 0.35355339059327376f, 1.f));
    float p = 0.3292495f;
    p = p * t - 1.0203389f;
    p = p * t + 0.68085486f;
    p = p * t + 0.3694219f;
    p = p * t + 1.4679759f;
    p = p * t - 2.8271523f;
    // exponent log2(e) * (P(t) - z^2) - 1, with z^2 = x^2 / 2
    const float half_erfc = t * __builtin_amdgcn_exp2f(p - (0.72134752044448170f * x) * x);
    // x Phi(x) = max(x, 0) - |x| erfc(|x| / sqrt(2)) / 2 on both sides of 0
    return fmaf(-fabsf(x), half_erfc, fmaxf(x, 0.f));
}

// Sum of v over aligned groups of 2^lg consecutive lanes (lg <= 6), every lane of a
// group receiving the group's sum: DPP quad permutes and row mirrors, then the
// 16- and 32-lane row swaps.
template <int CTRL>
__device__ __forceinline__ float ln_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float ln_lane_sum(float v, int lg) {
    if (lg >= 1) v += ln_dpp<0xB1>(v);    // lanes (1, 0, 3, 2)
    if (lg >= 2) v += ln_dpp<0x4E>(v);    // lanes (2, 3, 0, 1)
    if (lg >= 3) v += ln_dpp<0x141>(v);   // i <-> 7 - i within 8 lanes
    if (lg >= 4) v += ln_dpp<0x140>(v);   // i <-> 15 - i within 16 lanes
    if (lg >= 5) {
        const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
    }
    if (lg >= 6) {
        const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
    }
    return v;
}

// v rounded to bf16 (nearest even), as an fp32.
__device__ __forceinline__ float round_bf16(float v) {
    return __uint_as_float(static_cast<uint32_t>(from_f32<bf16_t>(v).bits) << 16);
}

// GELU of a bf16 value v (an fp32 whose low 16 bits are zero) through the table of the
// tail Q(a) = Phi(-a) in gelu_table.h: max(v, 0) - |v| Q(|v|) with |v| clamped to the
// table's range [2^-10, 8) (the form of gelu_fast, Q read instead of evaluated).  Inside
// the range the result is within one float32 rounding of each term of the exact GELU;
// outside it the bf16-rounded result is the exact one's (v/2 below, v or a magnitude
// under 7e-15 above).  tab is the table (GELU_TAB_N floats), normally copied to LDS by
// gelu_tab_fill.
__device__ __forceinline__ float gelu_bf16_tab(float v, const float* tab) {
    const uint32_t m = (__float_as_uint(v) >> 16) & 0x7fffu;
    const uint32_t a = m < GELU_TAB_LO ? GELU_TAB_LO : (m > GELU_TAB_HI ? GELU_TAB_HI : m);
    // max(v, 0) as one instruction: fmaxf would first canonicalize v (v is a bit pattern
    // from a shift or mask, which the compiler cannot prove canonical).
    float pos;
    asm("v_max_f32 %0, 0, %1" : "=v"(pos) : "v"(v));
    return fmaf(-fabsf(v), tab[a - GELU_TAB_LO], pos);
}
__device__ __forceinline__ void gelu_tab_fill(float* tab, int tid, int nthreads) {
    for (int i = tid; i < static_cast<int>(GELU_TAB_N); i += nthreads) tab[i] = gelu_tail_table[i];
}

// GELU of a float32 value through the interpolation table of Q(a) = Phi(-a) in
// gelu_table.h (GELU_QI_N (value, step) pairs on the grid a = i / 128, normally copied to
// LDS by gelu_qi_fill): max(v, 0) - |v| Q(|v|) with Q(|v|) = fma(f, step[i], value[i]),
// s = min(128 |v|, 1024 - 2^-14), i = floor(s), f = s - i (exact).  Within 2.3e-6
// absolute and 2.1e-4 relative (where |GELU| > 1e-6) of x Phi(x).
__device__ __forceinline__ float gelu_qi(float v, const float2* tab) {
    const float a = fabsf(v);
    const float s = fminf(a * GELU_QI_SCALE, 1023.99993896484375f);
    const float2 e = tab[static_cast<int>(s)];
    return fmaf(-a, fmaf(__builtin_amdgcn_fractf(s), e.y, e.x), fmaxf(v, 0.f));
}
__device__ __forceinline__ void gelu_qi_fill(float4* tab, int tid, int nthreads) {
    const float4* src = reinterpret_cast<const float4*>(gelu_interp_table);
    for (int i = tid; i < static_cast<int>(GELU_QI_N / 2); i += nthreads) tab[i] = src[i];
}

}  // namespace vh
