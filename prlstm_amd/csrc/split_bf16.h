// Exact three-way bf16 split of fp32 values and the six-product form on
// v_mfma_f32_32x32x16_bf16, shared by the split-product GEMM (gemm_x6.hip) and the fused
// products of the persistent recurrent kernels (recurrent.hip).
//
// Each fp32 value v is written as v = v0 + v1 + v2 with bf16 pieces v0 = bf16(v) (round
// to nearest even), v1 = bf16(v - v0), v2 = v - v0 - v1.  The residuals are exact in
// fp32: v - v0 has at most 16 significant bits, so v2 has at most 8 and is itself a bf16
// value; the split loses nothing.  A product a b is then the sum of the nine piece
// products a_i b_j, each exact in fp32 (8-bit by 8-bit significands).  |a1|, |b1| <= 2^-8
// and |a2|, |b2| <= 2^-16 of |a|, |b|, so the three smallest (a1 b2, a2 b1, a2 b2) add up
// to less than 2^-23 |a b| and are dropped; the other six run with fp32 accumulation.
// This is the "bf16x6" product of Henry, Tang and Heinecke ("Leveraging the bfloat16
// Artificial Intelligence Datatype For Higher-Precision Computations", ARITH 2019).
#pragma once

#include "hsl_internal.h"

namespace hsl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ unsigned bf16_pair(float a, float b) {  // round to nearest even
  const bf16x2 h = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(unsigned, h);
}
__device__ __forceinline__ float low_half(unsigned u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float high_half(unsigned u) { return __uint_as_float(u & 0xFFFF0000u); }

// The three bf16 pieces of two values, each piece a packed pair (a in the low half).
__device__ __forceinline__ void split2(float a, float b, unsigned (&p)[3]) {
  p[0] = bf16_pair(a, b);
  const float ra = a - low_half(p[0]), rb = b - high_half(p[0]);
  p[1] = bf16_pair(ra, rb);
  p[2] = bf16_pair(ra - low_half(p[1]), rb - high_half(p[1]));
}

// The three pieces of eight consecutive values as 32x32x16 operands (element 2m in the
// low half of word m).
__device__ __forceinline__ void split8(const float* v, u32x4 (&p)[3]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    unsigned q[3];
    split2(v[2 * m], v[2 * m + 1], q);
#pragma unroll
    for (int i = 0; i < 3; ++i) p[i][m] = q[i];
  }
}

__device__ __forceinline__ f16v mfma_bf16(u32x4 a, u32x4 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

// Pieces (of A, of B) of the six products, largest first.
constexpr int kPa[6] = {0, 0, 1, 0, 1, 2};
constexpr int kPb[6] = {0, 1, 0, 2, 1, 0};

}  // namespace hsl
