// Device-side definitions shared by the SRNL scan and readout kernels (srnl.hip,
// srnl_wide.hip): launch parameters, the stability constants, wave64 reductions, the
// MFMA operand helpers and the per-token gate arithmetic.
#pragma once

#include <type_traits>

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
    float inv_h;  // 1.0f / H (spatial inputs, H * W < 2^24)
};

// Chunk length of direction r.  Constant indices only: a runtime index into a
// kernel-argument array makes the compiler copy the whole argument block to
// scratch memory (and demotes every pointer in it to flat addressing).
__device__ __forceinline__ int chunk_of(const int (&chunk)[4], int r) {
    return r == 0 ? chunk[0] : r == 1 ? chunk[1] : r == 2 ? chunk[2] : chunk[3];
}

template <typename T>
__device__ __forceinline__ const T* line_ptr(const LineInput& in, int64_t b, int r, int64_t head,
                                             int64_t t) {
    const T* base = static_cast<const T*>(in.ptr);
    if (in.spatial) return base + b * in.sb + scan_to_pixel(r, t, in.H, in.W, in.inv_h) * in.st + head * in.sh;
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
    int x_vec;           // input rows are aligned for vector loads
    int lines_per_wave;  // head_dim 16: lines packed into one wave (1, 2 or 4)
    int tiles_per_wave;  // head_dim 16: 16-slot column tiles per wave (2 or 4, >= lines_per_wave)
    int aligned;         // spatial input with chunks (W, W, H, H): chunk c of scan r is a row/column
    int split_states;    // chunk-start states stored as bf16 hi + lo pairs (see state_split_bf16)
    Consts k;
};

// Butterfly steps inside a quad of lanes, on the VALU (DPP quad_perm).
// Quad permutes read only lanes of the same quad, so bound_ctrl never applies; setting
// it lets the compiler fold the move into the consuming add (v_add_f32_dpp).
__device__ __forceinline__ float quad_swap1(float v) {  // lanes (1,0,3,2)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float quad_swap2(float v) {  // lanes (2,3,0,1)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, true));
}

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// bf16 matrix cores for bf16 activations.  v_mfma_f32_16x16x16_bf16 takes from lane l
// the 4 consecutive k values 4(l/16)..4(l/16)+3 of A row l%16 and of B column l%16 (the
// same operands one lane gives the four 16x16x4 fp32 steps above) and accumulates in
// fp32.  An fp32 operand v enters as hi + lo, hi = bf16(v), lo = bf16(v - hi), which
// leaves |v - hi - lo| <= 2^-16 |v|; bf16 activations enter exactly.
typedef short v4s __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma_bf16(v4s a, v4s b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// a0 b0 + a1 b1 (+ c) in ONE v_mfma_f32_16x16x32_bf16: that instruction takes 8 consecutive
// k from each lane instead of 4, so lane l's 8 values [a0, a1] of A row l%16 meet [b0, b1] of
// B column l%16: the same products as mfma_bf16(a0, b0) + mfma_bf16(a1, b1), one issue.
// Never chain its result as the accumulator of a 16x16x16 product (or the reverse): the
// compiler issues such a pair back to back, and on MI355X the second product then read a
// stale accumulator.  Chains of one product size are safe.
typedef __bf16 v8bf16_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v4f mfma_bf16x2(v4s a0, v4s a1, v4s b0, v4s b1, v4f c) {
    const v8bf16_t a = __builtin_bit_cast(v8bf16_t, __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7));
    const v8bf16_t b = __builtin_bit_cast(v8bf16_t, __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7));
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
typedef float v4fl __attribute__((ext_vector_type(4)));

// Hardware round-to-nearest-even conversions (v_cvt_pk_bf16_f32).
__device__ __forceinline__ void split_bf16(const float (&v)[4], v4s& hi, v4s& lo) {
    const v4fl f = {v[0], v[1], v[2], v[3]};
    const v4bf h = __builtin_convertvector(f, v4bf);
    const v4bf l = __builtin_convertvector(f - __builtin_convertvector(h, v4fl), v4bf);
    hi = __builtin_bit_cast(v4s, h);
    lo = __builtin_bit_cast(v4s, l);
}

__device__ __forceinline__ v4s bf16x4_bits(uint2 r) {
    v4s s;
    s[0] = static_cast<short>(r.x & 0xffffu);
    s[1] = static_cast<short>(r.x >> 16);
    s[2] = static_cast<short>(r.y & 0xffffu);
    s[3] = static_cast<short>(r.y >> 16);
    return s;
}

// Four consecutive elements of a row as fp32 (8- or 16-byte load when `vec`).
template <typename T>
__device__ __forceinline__ void load4(const T* p, bool vec, float (&out)[4]) {
    if (vec) {
        if constexpr (sizeof(T) == 4) {
            const float4 v = *reinterpret_cast<const float4*>(p);
            out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(p);
            out[0] = to_f32(T{static_cast<uint16_t>(v.x & 0xffffu)});
            out[1] = to_f32(T{static_cast<uint16_t>(v.x >> 16)});
            out[2] = to_f32(T{static_cast<uint16_t>(v.y & 0xffffu)});
            out[3] = to_f32(T{static_cast<uint16_t>(v.y >> 16)});
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = to_f32(p[j]);
}

template <int CTRL>
__device__ __forceinline__ float quad_perm(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over lanes l, l^16, l^32, l^48 with the gfx950 row-swap permutes (VALU, no LDS):
// permlane16_swap(v, v) yields rows (r0, r0, r2, r2) and (r1, r1, r3, r3), so their sum
// holds the xor-16 pair sums; permlane32_swap does the same for the two halves.
__device__ __forceinline__ float xor16_32_sum(float v) {
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
}

// Element offset of scan token `tok` of direction r from the start of its line.
template <bool SPATIAL>
__device__ __forceinline__ int64_t token_offset(const LineInput& in, int r, int64_t tok) {
    if constexpr (SPATIAL) return scan_to_pixel(r, tok, in.H, in.W, in.inv_h) * in.st;
    else return tok * in.st;
}

// Gates of one token from its pre-activations pe = x.e and pa = x.a, ||k - v||^2 and
// ||k||^2 (reference chunk.cu:382-393, memory.cuh:219-233):
//   eta = ETA_SCALE softplus(clamp(pe)), alpha = ALPHA_MIN + (1 - ALPHA_MIN) sigmoid(clamp(pa + bias)),
//   cap = STAB_MU (1 - alpha) / (sqrt(||k - v||^2 + 1e-12) + 1e-6), eff = cap (1 - exp(-eta / cap)),
//   eff = min(eff, nextafter(FACTOR alpha / max(||k||^2, 1e-20), 0)) with the spectral clamp.
// On the hardware exp2, log2, reciprocal and square root (about one ulp each), as the
// reference's --use_fast_math build evaluates them with approximate intrinsics of its
// own.  pe <= 10 after the clamp, so the reference's softplus branch for inputs above 20
// never applies.  1 - exp(-r) is its Taylor series below r = 1/4 (relative error under
// 2e-8 there, where 1 - exp2 would cancel) and 1 - exp2(-r log2 e) above.  The bound is
// positive (alpha > 0), so nextafter toward 0 is one less in its bit pattern.
__device__ __forceinline__ void token_gates_fast(const Consts& k, float pe, float pa, float dsq, float ksq,
                                                 float& alpha, float& eff) {
    constexpr float kLog2e = 1.44269504088896341f, kLn2 = 0.69314718055994531f;
    const float ep = fminf(10.f, fmaxf(-10.f, pe));
    const float ap = fminf(10.f, fmaxf(-10.f, pa + k.alpha_bias));
    const float eta = k.eta_scale * (kLn2 * __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(kLog2e * ep)));
    alpha = k.alpha_min + (1.f - k.alpha_min) * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * ap));
    const float dn = __builtin_amdgcn_sqrtf(dsq + 1e-12f);
    const float cap = k.stab_mu * (1.f - alpha) * __builtin_amdgcn_rcpf(dn + 1e-6f);
    const float r = eta * __builtin_amdgcn_rcpf(cap);
    const float series =
        r * (1.f - r * (0.5f - r * (1.f / 6.f - r * (1.f / 24.f - r * (1.f / 120.f - r * (1.f / 720.f))))));
    eff = cap * (r < 0.25f ? series : 1.f - __builtin_amdgcn_exp2f(-kLog2e * r));
    if (k.clamp) {
        const float bound = k.factor * alpha * __builtin_amdgcn_rcpf(fmaxf(ksq, 1e-20f));
        eff = fminf(eff, __uint_as_float(__float_as_uint(bound) - 1u));
    }
}

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v8fl __attribute__((ext_vector_type(8)));

// DPP row shift right by M lanes inside each 16-lane row (lane i reads lane i - M).
template <int M>
__device__ __forceinline__ float row_shr(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x110 + M, 0xF, 0xF, false));
}
// Reversal inside each 8-lane half row / 16-lane row (lane i reads lane 7 - i / 15 - i).
__device__ __forceinline__ float half_mirror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));
}
__device__ __forceinline__ float row_mirror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, true));
}

// Sum over the RL consecutive lanes holding one row of G (RL in {2, 4, 8, 16}).
template <int RL>
__device__ __forceinline__ float row_group_sum(float v) {
    v += quad_swap1(v);
    if constexpr (RL >= 4) v += quad_swap2(v);
    if constexpr (RL >= 8) v += half_mirror(v);
    if constexpr (RL >= 16) v += row_mirror(v);
    return v;
}

// Operand K-range of one lane: D/4 consecutive channels, raw bits as loaded (16-bit
// types: 8 or 16 bytes; fp32: 16 or 32 bytes).
template <int BYTES>
struct RawBytes;
template <>
struct RawBytes<8> { uint2 v; };
template <>
struct RawBytes<16> { uint4 v; };
template <>
struct RawBytes<32> { uint4 v0, v1; };
template <typename T, int D>
using XRaw = RawBytes<static_cast<int>(sizeof(T)) * D / 4>;

template <typename T, int D>
__device__ __forceinline__ XRaw<T, D> load_xraw(const T* p) {
    XRaw<T, D> r;
    if constexpr (sizeof(T) * D / 4 == 8) r.v = *reinterpret_cast<const uint2*>(p);
    else if constexpr (sizeof(T) * D / 4 == 16) r.v = *reinterpret_cast<const uint4*>(p);
    else {
        r.v0 = *reinterpret_cast<const uint4*>(p);
        r.v1 = *reinterpret_cast<const uint4*>(p + 4);
    }
    return r;
}

// bf16 matrix-core operands of one lane: 4 values (16x16x16) at D = 16, 8 (16x16x32) at 32.
template <int D>
struct BfOp;
template <>
struct BfOp<16> {
    using type = v4s;
    static __device__ __forceinline__ v4f mma(v4s a, v4s b, v4f c) { return mfma_bf16(a, b, c); }
    // a0 b0 + a1 b1 + c: one 16x16x32 product
    static __device__ __forceinline__ v4f mma_pair(v4s a0, v4s a1, v4s b0, v4s b1, v4f c) {
        return mfma_bf16x2(a0, a1, b0, b1, c);
    }
    static __device__ __forceinline__ void split(const float (&v)[4], v4s& hi, v4s& lo) { split_bf16(v, hi, lo); }
    static __device__ __forceinline__ v4s exact(const XRaw<bf16_t, 16>& r) { return bf16x4_bits(r.v); }
};
template <>
struct BfOp<32> {
    using type = v8bf;
    static __device__ __forceinline__ v4f mma(v8bf a, v8bf b, v4f c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    // a0 b0 + a1 b1 + c: two 16x16x32 products (K = 32 fills one instruction already)
    static __device__ __forceinline__ v4f mma_pair(v8bf a0, v8bf a1, v8bf b0, v8bf b1, v4f c) {
        return mma(a1, b1, mma(a0, b0, c));
    }
    static __device__ __forceinline__ void split(const float (&v)[8], v8bf& hi, v8bf& lo) {
        v8fl f;
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = v[j];
        hi = __builtin_convertvector(f, v8bf);
        lo = __builtin_convertvector(f - __builtin_convertvector(hi, v8fl), v8bf);
    }
    static __device__ __forceinline__ v8bf exact(const XRaw<bf16_t, 32>& r) { return __builtin_bit_cast(v8bf, r.v); }
};

// The D/4 channels of a raw operand as fp32.
template <typename T, int D>
__device__ __forceinline__ void decode_x(const XRaw<T, D>& r, float (&x)[D / 4]) {
    if constexpr (sizeof(T) == 4 && D == 16) {
        x[0] = __uint_as_float(r.v.x); x[1] = __uint_as_float(r.v.y);
        x[2] = __uint_as_float(r.v.z); x[3] = __uint_as_float(r.v.w);
    } else if constexpr (sizeof(T) == 4) {
        x[0] = __uint_as_float(r.v0.x); x[1] = __uint_as_float(r.v0.y);
        x[2] = __uint_as_float(r.v0.z); x[3] = __uint_as_float(r.v0.w);
        x[4] = __uint_as_float(r.v1.x); x[5] = __uint_as_float(r.v1.y);
        x[6] = __uint_as_float(r.v1.z); x[7] = __uint_as_float(r.v1.w);
    } else {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&r);
#pragma unroll
        for (int j = 0; j < D / 8; ++j) {
            x[2 * j] = to_f32(T{static_cast<uint16_t>(w[j] & 0xffffu)});
            x[2 * j + 1] = to_f32(T{static_cast<uint16_t>(w[j] >> 16)});
        }
    }
}

// KQ consecutive fp32 values from LDS (16-byte aligned).
template <int KQ>
__device__ __forceinline__ void lds_vec(const float* p, float (&v)[KQ]) {
#pragma unroll
    for (int j = 0; j < KQ; j += 4) {
        const float4 f = *reinterpret_cast<const float4*>(p + j);
        v[j] = f.x; v[j + 1] = f.y; v[j + 2] = f.z; v[j + 3] = f.w;
    }
}

struct FuseParams {
    const void* x;
    const void* q;
    int per_direction;  // 1: x, q are serialized stacks [B, 4, L, C]; 0: channels-last [B, L, C]
    const float* states;
    int64_t max_chunks;
    const float* skip;
    int skip_per_dir;
    const float* wgt;
    void* out;          // [B, H, W, C], fp32 or the io dtype (see the kernel's TO)
    const void* aux;    // optional [B, H, W, C] io-dtype addend of the fused result
    // optional 5x5 depthwise convolution of x added to the fused result (the tiled
    // readout only): taps [25, C] FP32 taps-major, bias [C] FP32 or null
    const float* lepe_taps;
    const float* lepe_bias;
    int64_t B, H, W, C, heads;
    int chunk[4];
    int split_states;   // states stored as bf16 hi + lo pairs (see state_split_bf16)
};

// Chunk-start states in the split format: the 16 bytes that hold M[i][4g..4g+3] in FP32
// hold instead bf16 hi[4] then bf16 lo[4] with hi = bf16(v), lo = bf16(v - hi), the
// operand pair the bf16 matrix-core readout multiplies (same size, same addressing).
__device__ __forceinline__ float split_state_at(const float* row, int col) {
    const uint16_t* u = reinterpret_cast<const uint16_t*>(row + 4 * (col >> 2));
    const int j = col & 3;
    return __uint_as_float(static_cast<uint32_t>(u[j]) << 16) + __uint_as_float(static_cast<uint32_t>(u[4 + j]) << 16);
}

// Stores four consecutive entries M[i][4g..4g+3] of a chunk-start state at dst: FP32, or
// when split, the same 16 bytes as bf16 hi[4] then bf16 lo[4] (round to nearest even,
// |v - hi - lo| <= 2^-16 |v|), the format split_state_at reads.
__device__ __forceinline__ void store_state4(float* dst, float4 v, bool split) {
    if (!split) {
        *reinterpret_cast<float4*>(dst) = v;
        return;
    }
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const uint32_t h01 = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{v.x, v.y}, bf2));
    const uint32_t h23 = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{v.z, v.w}, bf2));
    const f2 r01 = {v.x - __uint_as_float(h01 << 16), v.y - __uint_as_float(h01 & 0xffff0000u)};
    const f2 r23 = {v.z - __uint_as_float(h23 << 16), v.w - __uint_as_float(h23 & 0xffff0000u)};
    const uint32_t l01 = __builtin_bit_cast(uint32_t, __builtin_convertvector(r01, bf2));
    const uint32_t l23 = __builtin_bit_cast(uint32_t, __builtin_convertvector(r23, bf2));
    *reinterpret_cast<uint4*>(dst) = make_uint4(h01, h23, l01, l23);
}

// Scan with one line per workgroup of `waves` waves (srnl_wide.hip): head_dim 16 or 32,
// fp32 or bf16 activations, vector-aligned rows.  Returns false (nothing launched) for
// any other case.  scan_wide_waves picks the waves per line for a line count;
// token_blocks > 1 selects the token-block mode (blocks of the chunk composed).
int scan_wide_waves(int64_t lines, int head_dim);
// Scan for head_dim 16 in the block form (srnl_ut.hip), packed as sp.lines_per_wave x
// sp.tiles_per_wave like srnl_scan16_kernel.  T: the activation type (bf16_t, f16_t, float).
template <typename T>
bool launch_scan16_ut(const ScanParams& sp, hipStream_t stream);
// The block form with the blocks of a chunk spread over the waves of one workgroup per line
// (srnl_utw.hip): head_dim 16, chunks of at most 128 tokens.  Returns false (nothing
// launched) when the chunks or the input alignment do not allow it.
template <typename T>
bool launch_scan16_utw(const ScanParams& sp, hipStream_t stream);
// head_dim 32, chunks of at most 64 tokens (srnl_utw32.hip); false when the call does not
// qualify.
template <typename T>
bool launch_scan32_utw(const ScanParams& sp, hipStream_t stream);
bool launch_scan_wide(const ScanParams& sp, int io_dtype, int head_dim, int waves, int token_blocks,
                      hipStream_t stream);

}  // namespace vh
