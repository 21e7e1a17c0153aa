// int4 operands on the int8 matrix cores (gfx950): nibble unpacking and the
// epilogue's output narrowing, shared by the GEMM kernels and the fused
// decode kernel.
//
// A packed dword w holds 8 nibbles; the two dwords
//   lo = (w << 4) & 0xF0F0F0F0   (even k, each byte = 16 * nibble value)
//   hi =  w       & 0xF0F0F0F0   (odd k)
// are 8 int8 values scaled by 16 with the sign in the byte's top bit.  A and
// B go through the same k permutation, so a dot product of unpacked operands
// is 256 times the nibble dot product, removed exactly by an arithmetic >> 8.
#pragma once

#include "common.h"

namespace dscq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i unpack8(uint32_t w0, uint32_t w1) {
  v4i r;
  r[0] = (int)((w0 << 4) & 0xF0F0F0F0u);
  r[1] = (int)(w0 & 0xF0F0F0F0u);
  r[2] = (int)((w1 << 4) & 0xF0F0F0F0u);
  r[3] = (int)(w1 & 0xF0F0F0F0u);
  return r;
}

template <typename OutT>
__device__ __forceinline__ OutT to_out(float v);
// The reference rounds the fp32 result, then narrows it to fp16 (two
// roundings).  Left alone, the compiler folds a preceding fp32 multiply / add
// into the narrowing (v_fma_mixlo_f16: one rounding), which differs on exact
// fp16 ties; the empty asm pins the fp32 value first.
template <>
__device__ __forceinline__ __half to_out<__half>(float v) {
  asm("" : "+v"(v));
  return __float2half_rn(v);
}
template <>
__device__ __forceinline__ float to_out<float>(float v) {
  return v;
}

// Two fp32 results narrowed to fp16 (round to nearest even) and packed, low
// half first: one v_cvt_pk_f16_f32.  The values are pinned first, so no
// preceding multiply or add is folded into the narrowing (one rounding of the
// fp32 result, as to_out<__half>).
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  asm("" : "+v"(lo), "+v"(hi));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, h2));
}

}  // namespace dscq
