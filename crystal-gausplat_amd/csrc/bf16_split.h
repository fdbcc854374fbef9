// Exact three-term bf16 splits of fp32 values, shared by the bf16x6 GEMM and
// attention kernels: x = x0 + x1 + x2 with x0 = bf16(x), x1 = bf16(x - x0),
// x2 = bf16(x - x0 - x1), each rounded to nearest even. Both subtractions are
// exact in fp32 (Sterbenz), so x0 + x1 + x2 matches x to about 2^-24 relative.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gs {

// Two floats to packed bf16, the first in the low half (round to nearest
// even). A vector conversion, which the compiler issues as one
// v_cvt_pk_bf16_f32 and, unlike an inline-asm form of that instruction, also
// schedules: it then inserts the wait states that a matrix-core instruction
// reading the result (and a VALU instruction reading a transcendental's
// result) needs. Inline asm left those to chance.
typedef float gs_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 gs_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  const gs_f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, gs_bf16x2));
}
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// Split of two values: h, m, l hold the packed terms x0, x1, x2.
__device__ __forceinline__ void split3_pk(float a, float b, uint32_t& h, uint32_t& m,
                                          uint32_t& l) {
  h = cvt_pk_bf16(a, b);
  const float ra = a - bf16_lo(h), rb = b - bf16_hi(h);
  m = cvt_pk_bf16(ra, rb);
  l = cvt_pk_bf16(ra - bf16_lo(m), rb - bf16_hi(m));
}

}  // namespace gs
