// Helpers of the block-form (UT) SRNL scans (srnl_ut.hip, srnl_utw.hip, srnl_utw32.hip):
// FP32 values as bf16 hi + lo matrix-core operands, the 16x16 products built from them and
// the token operands of bf16, fp16 and FP32 maps.
#pragma once

#include "srnl_device.h"

namespace vh {
namespace blockform {

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// FP32 values as bf16 hi + lo, |v - hi - lo| <= 2^-16 |v| (round-to-nearest-even
// conversions, two values per conversion).
__device__ __forceinline__ void split4(const float (&v)[4], v4s& hi, v4s& lo) {
    const uint32_t h01 = __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{v[0], v[1]}, v2bf));
    const uint32_t h23 = __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{v[2], v[3]}, v2bf));
    const v2f r01 = {v[0] - __uint_as_float(h01 << 16), v[1] - __uint_as_float(h01 & 0xffff0000u)};
    const v2f r23 = {v[2] - __uint_as_float(h23 << 16), v[3] - __uint_as_float(h23 & 0xffff0000u)};
    const uint32_t l01 = __builtin_bit_cast(uint32_t, __builtin_convertvector(r01, v2bf));
    const uint32_t l23 = __builtin_bit_cast(uint32_t, __builtin_convertvector(r23, v2bf));
    hi = __builtin_bit_cast(v4s, make_uint2(h01, h23));
    lo = __builtin_bit_cast(v4s, make_uint2(l01, l23));
}
__device__ __forceinline__ void split4(const v4f& v, v4s& hi, v4s& lo) {
    const float a[4] = {v[0], v[1], v[2], v[3]};
    split4(a, hi, lo);
}

// A B + C for FP32 A, B given as bf16 hi + lo (the lo x lo term dropped).  Three products of
// one size: an accumulation chain that mixes 16x16x32 and 16x16x16 products on one
// accumulator was issued back to back by the compiler and gave wrong results on MI355X.
__device__ __forceinline__ v4f mma3(v4s ah, v4s al, v4s bh, v4s bl, v4f c) {
    c = mfma_bf16(ah, bh, c);
    c = mfma_bf16(ah, bl, c);
    return mfma_bf16(al, bh, c);
}

// The same over K = 32 held as two 16-wide K tiles (each operand: the lane's quads of tile 0
// and tile 1): three 16x16x32 products, which take tile 0's quad and tile 1's quad of a lane
// as eight consecutive k (the sum over k does not depend on their order).  One product size
// per chain, as for mma3.
__device__ __forceinline__ v4f mma3k2(const v4s (&ah)[2], const v4s (&al)[2], const v4s (&bh)[2], const v4s (&bl)[2],
                                      v4f c) {
    c = mfma_bf16x2(ah[0], ah[1], bh[0], bh[1], c);
    c = mfma_bf16x2(ah[0], ah[1], bl[0], bl[1], c);
    return mfma_bf16x2(al[0], al[1], bh[0], bh[1], c);
}

// x of one lane's four features of a token as bf16 matrix-core operands.  bf16 maps enter
// exactly (hi = the bits, no lo); fp16 and FP32 maps are decoded and split into hi + lo,
// exact for every fp16 value (11 significant bits, exponents inside bf16's range) and within
// 2^-16 |x| for FP32.  Products against x keep the state's hi + lo: two products for exact
// x, three (lo x lo dropped, as in mma3) otherwise.
template <typename T>
struct XQuad {
    static constexpr bool EXACT = std::is_same<T, bf16_t>::value;
    using Raw = XRaw<T, 16>;   // 8 bytes (16-bit types) or 16 bytes (FP32)
    // one vector load; `p` aligned to the raw size
    static __device__ __forceinline__ Raw load(const T* p) { return load_xraw<T, 16>(p); }
    // element by element, for rows that are not aligned
    static __device__ __forceinline__ Raw load_scalar(const T* p) {
        Raw r;
        if constexpr (sizeof(T) == 4)
            r.v = make_uint4(__float_as_uint(p[0]), __float_as_uint(p[1]), __float_as_uint(p[2]), __float_as_uint(p[3]));
        else
            r.v = make_uint2(static_cast<uint32_t>(p[0].bits) | (static_cast<uint32_t>(p[1].bits) << 16),
                             static_cast<uint32_t>(p[2].bits) | (static_cast<uint32_t>(p[3].bits) << 16));
        return r;
    }
    // operands of a token; zero for a slot past the chunk
    static __device__ __forceinline__ void operands(const Raw& r, bool ok, v4s& hi, v4s& lo) {
        if constexpr (EXACT) {
            hi = ok ? bf16x4_bits(r.v) : v4s{0, 0, 0, 0};
            lo = v4s{0, 0, 0, 0};
        } else {
            float x[4];
            decode_x<T, 16>(r, x);
#pragma unroll
            for (int j = 0; j < 4; ++j) x[j] = ok ? x[j] : 0.f;
            split4(x, hi, lo);
        }
    }
    // A X + c, A (state rows) as hi + lo, X the token columns
    static __device__ __forceinline__ v4f mma(v4s ah, v4s al, v4s xh, v4s xl, v4f c) {
        if constexpr (EXACT) return mfma_bf16(al, xh, mfma_bf16(ah, xh, c));
        else return mma3(ah, al, xh, xl, c);
    }
    // the same over K = 32: a lane's quads of the two 16-feature halves
    static __device__ __forceinline__ v4f mma_k2(const v4s (&ah)[2], const v4s (&al)[2], const v4s (&xh)[2],
                                                 const v4s (&xl)[2], v4f c) {
        if constexpr (EXACT)
            return mfma_bf16x2(al[0], al[1], xh[0], xh[1], mfma_bf16x2(ah[0], ah[1], xh[0], xh[1], c));
        else
            return mma3k2(ah, al, xh, xl, c);
    }
};

// d I in the accumulator layout of lane 16 q + i (entries: rows 4q..4q+3 of column i).
__device__ __forceinline__ v4f diag4(float d, int q, int i) {
    v4f o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = (4 * q + j == i) ? d : 0.f;
    return o;
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

}  // namespace blockform
}  // namespace vh
