// Helpers of the block-form (UT) SRNL scans (srnl_ut.hip, srnl_utw.hip): FP32 values as
// bf16 hi + lo matrix-core operands and the 16x16 products built from them.
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
