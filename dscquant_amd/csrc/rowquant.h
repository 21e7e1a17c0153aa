// Row quantization building blocks for gfx950, shared by the quantize
// kernels and the fused decode kernel: vector loads of a row chunk, the
// 128-point block-Hadamard butterflies, and the per-row scale / code rules.
//
// Exact division at bandwidth.  The reference computes
// code = clamp(round_half_even(fl(fl(x / s) + z))).  Per element we use
// t' = fma(x, y, z) with y = rcp(s) (relative error <= 2^-23) computed once
// per row.  With Q = x / s exact, a = fl(Q) and t = fl(a + z):
//   t  = Q + Q d1 + z + (a + z) d2,         |d1|, |d2| <= 2^-24
//   t' = Q + Q e  + z + (Q(1 + e) + z) d3,  |e| <= 2^-23, |d3| <= 2^-24
// so |t - t'| <= 2^-24 (5 |Q| + 2 z) up to terms of order 2^-47 |Q|.  If
// |t' - rne(t')| < 0.5 - B with B = (5 Qmax + 2 z + 3) 2^-24 (Qmax an upper
// bound of |Q| over the row; the +3 absorbs the roundings of B itself and of
// 0.5 - B), t is on the same side of every half-integer as t' and both round
// to the same integer.  A chunk of 8 elements with any element closer than
// that is recomputed with IEEE division (a few chunks per thousand).
// Clamping commutes with rounding because the bounds are integers.

#pragma once

#include "common.h"

namespace dscq {

enum Mode { kAct = 0, kWgt = 1 };

// ------------------------------------------------------------------ loading
// Loads are unconditional: an out-of-range chunk reads element 0 of its row
// (always valid) and is zeroed afterwards, so every 16-byte load of a lane
// is in flight at once instead of each waiting inside its own branch.
// Zero is a neutral placeholder: it never moves min(x, 0) / max(x, 0) or
// max|w|, and it quantizes to the row's zero-point (activations) or to 0
// (weights) -- exactly the padding the reference writes.

template <typename T>
struct Raw;
template <>
struct Raw<__half> {
  uint4 w;
};
template <>
struct Raw<float> {
  uint4 w0, w1;
};

template <typename T>
__device__ __forceinline__ Raw<T> load_raw(const T* row, int64_t e0, bool ok);

template <>
__device__ __forceinline__ Raw<__half> load_raw<__half>(const __half* row, int64_t e0,
                                                        bool ok) {
  Raw<__half> r;
  r.w = *reinterpret_cast<const uint4*>(row + (ok ? e0 : 0));
  return r;
}

// The same with a 32-bit element offset (rows of at most 2^28 elements): the
// wave-uniform row base and a per-lane byte offset map onto one
// global_load_dwordx4 with scalar base and vector offset, with no 64-bit
// address arithmetic per load.
template <typename T>
__device__ __forceinline__ Raw<T> load_raw32(const T* row, int e0, bool ok) {
  const uint32_t off = (uint32_t)(ok ? e0 : 0) * (uint32_t)sizeof(T);
  const uint8_t* base = reinterpret_cast<const uint8_t*>(row);
  Raw<T> r;
  if constexpr (sizeof(T) == 2) {
    r.w = *reinterpret_cast<const uint4*>(base + off);
  } else {
    r.w0 = *reinterpret_cast<const uint4*>(base + off);
    r.w1 = *reinterpret_cast<const uint4*>(base + off + 16);
  }
  return r;
}

template <>
__device__ __forceinline__ Raw<float> load_raw<float>(const float* row, int64_t e0,
                                                      bool ok) {
  Raw<float> r;
  const float* p = row + (ok ? e0 : 0);
  r.w0 = *reinterpret_cast<const uint4*>(p);
  r.w1 = *reinterpret_cast<const uint4*>(p + 4);
  return r;
}

__device__ __forceinline__ float h2f(uint32_t bits16) {
  return __half2float(__ushort_as_half((unsigned short)bits16));
}

// SiLU-gated MLP activation of two fp16 pairs: h = fp16(fp16(silu(g)) * u),
// the roundings an fp16 model applies to act_fn(gate) and to the product.
// silu(g) = g / (1 + e^-g) is evaluated with the hardware exp2 and reciprocal
// (a few fp32 ulps), far inside the fp16 rounding that follows; exp's last
// bit differs between math libraries anyway.  g -> -inf gives e^-g = inf and
// g * rcp(inf) = -0, the limit.  Used by the requantizing kernel and by the
// GEMM's gated epilogue, so both give the same h.
__device__ __forceinline__ uint32_t silu_mul_f16x2(uint32_t g2, uint32_t u2) {
  uint32_t h2 = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float g = h2f((g2 >> (16 * i)) & 0xFFFFu);
    const float u = h2f((u2 >> (16 * i)) & 0xFFFFu);
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    const float sg = __half2float(__float2half_rn(g * __builtin_amdgcn_rcpf(1.0f + e)));
    const __half h = __float2half_rn(sg * u);
    h2 |= (uint32_t)__half_as_ushort(h) << (16 * i);
  }
  return h2;
}

// Zero the values of a chunk that was loaded from the placeholder address.
template <typename T>
__device__ __forceinline__ void mask_f32(bool ok, float v[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = ok ? v[i] : 0.0f;
}

__device__ __forceinline__ void to_f32(const Raw<__half>& r, float v[8]) {
  const uint32_t w[4] = {r.w.x, r.w.y, r.w.z, r.w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = h2f(w[i] & 0xFFFFu);
    v[2 * i + 1] = h2f(w[i] >> 16);
  }
}

__device__ __forceinline__ void to_f32(const Raw<float>& r, float v[8]) {
  v[0] = __uint_as_float(r.w0.x); v[1] = __uint_as_float(r.w0.y);
  v[2] = __uint_as_float(r.w0.z); v[3] = __uint_as_float(r.w0.w);
  v[4] = __uint_as_float(r.w1.x); v[5] = __uint_as_float(r.w1.y);
  v[6] = __uint_as_float(r.w1.z); v[7] = __uint_as_float(r.w1.w);
}

// Element-wise form for rows that are not 16-byte aligned or whose K is not a
// multiple of 8 (streaming kernel only).
template <typename T>
__device__ __forceinline__ void load_scalar(const T* row, int64_t e0, int64_t K, bool ok,
                                            float v[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const bool in = ok && (e0 + i < K);
    const float f = (float)row[in ? e0 + i : 0];
    v[i] = in ? f : 0.0f;
  }
}

// -------------------------------------------------------- block transform

// Butterfly (u, w) -> (u + w, u - w) on index bit `h` within one chunk.
__device__ __forceinline__ void fwht_chunk(float v[8]) {
#pragma unroll
  for (int h = 1; h < 8; h <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (!(i & h)) {
        const float u = v[i], w = v[i + h];
        v[i] = u + w;
        v[i + h] = u - w;
      }
}

// Stages for index bits 3..6 of one block held as c[4][8] by a quad lane.
// Bits 3-4 pair lanes r^1 and r^2: the lane with the bit clear keeps
// own + partner, the other partner - own, i.e. fma(+-1, own, partner), which
// rounds exactly like the plain add / subtract.
__device__ __forceinline__ void fwht_block_tail(float c[4][8], int r) {
  const float s1 = (r & 1) ? -1.0f : 1.0f;
  const float s2 = (r & 2) ? -1.0f : 1.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) c[j][i] = __builtin_fmaf(s1, c[j][i], dpp_f32<kDppQuadXor1>(c[j][i]));
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) c[j][i] = __builtin_fmaf(s2, c[j][i], dpp_f32<kDppQuadXor2>(c[j][i]));
#pragma unroll
  for (int h = 1; h < 4; h <<= 1)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!(j & h)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float u = c[j][i], w = c[j + h][i];
          c[j][i] = u + w;
          c[j + h][i] = u - w;
        }
      }
}

// ------------------------------------------------------------ quantization

struct RowScale {
  float scale, y, zf, qmax, thr;
};

// Activation chunk -> bytes u = q (evens: elements 0,2,4,6; odds: 1,3,5,7).
// Fast path; returns in *dmax the largest |t - round(t)| seen.
__device__ __forceinline__ void act_chunk_fast(const float v[8], const RowScale& rs,
                                               uint32_t& ev, uint32_t& od,
                                               float& dmax) {
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = __builtin_amdgcn_fmed3f(__builtin_fmaf(v[i], rs.y, rs.zf), 0.0f, rs.qmax);
    q[i] = __builtin_rintf(t);
    dmax = fmaxf(dmax, fabsf(t - q[i]));
  }
  ev = put_u8<0>(q[0], 0u); ev = put_u8<1>(q[2], ev); ev = put_u8<2>(q[4], ev); ev = put_u8<3>(q[6], ev);
  od = put_u8<0>(q[1], 0u); od = put_u8<1>(q[3], od); od = put_u8<2>(q[5], od); od = put_u8<3>(q[7], od);
}

// Activation chunk with correctly rounded division (the reference's exact rule).
// The chunk holds sgn * x; dividing by sgn * s gives fl(x / s) exactly, since
// IEEE division is symmetric under sign changes.
__device__ __forceinline__ void act_chunk_exact(const float v[8], const RowScale& rs,
                                                float sgn, uint32_t& ev, uint32_t& od) {
  const float ss = sgn * rs.scale;
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
    q[i] = __builtin_amdgcn_fmed3f(__builtin_rintf(v[i] / ss + rs.zf), 0.0f, rs.qmax);
  ev = put_u8<0>(q[0], 0u); ev = put_u8<1>(q[2], ev); ev = put_u8<2>(q[4], ev); ev = put_u8<3>(q[6], ev);
  od = put_u8<0>(q[1], 0u); od = put_u8<1>(q[3], od); od = put_u8<2>(q[5], od); od = put_u8<3>(q[7], od);
}

// Weight chunk -> bytes u = c + qmax + 1 (so u ^ 8 is the int4 nibble when
// qmax = 7) and the chunk's code sum.
__device__ __forceinline__ void wgt_chunk(const float v[8], const RowScale& rs,
                                          uint32_t& ev, uint32_t& od, int& sum) {
  float c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    c[i] = __builtin_amdgcn_fmed3f(__builtin_rintf(v[i] / rs.scale), -rs.qmax, rs.qmax);
    sum += (int)c[i];
  }
  const float off = rs.qmax + 1.0f;
  ev = put_u8<0>(c[0] + off, 0u); ev = put_u8<1>(c[2] + off, ev);
  ev = put_u8<2>(c[4] + off, ev); ev = put_u8<3>(c[6] + off, ev);
  od = put_u8<0>(c[1] + off, 0u); od = put_u8<1>(c[3] + off, od);
  od = put_u8<2>(c[5] + off, od); od = put_u8<3>(c[7] + off, od);
}

template <int MODE>
__device__ __forceinline__ RowScale row_scale(float mn, float mx, float clip,
                                              float qmax) {
  RowScale rs;
  rs.qmax = qmax;
  if (MODE == kAct) {
    // core/quantization.py:15-19; kernel/w4a4.cu:42-44.
    const float lo = mn * clip, hi = mx * clip;
    rs.scale = fmaxf((hi - lo) / qmax, 1e-8f);
    rs.zf = __builtin_amdgcn_fmed3f(__builtin_rintf(-lo / rs.scale), 0.0f, qmax);
    // Only the fast path uses y; a 1-ulp reciprocal is inside its margin.
    rs.y = __builtin_amdgcn_rcpf(rs.scale);
    // Upper bound of |x| / scale over the row: |x| <= max(mx, -mn), and the
    // factor covers the reciprocal's and the product's rounding.
    const float qbound = fmaxf(mx, -mn) * rs.y * (1.0f + 0x1p-20f);
    rs.thr = 0.5f - (5.0f * qbound + 2.0f * rs.zf + 3.0f) * 0x1p-24f;
  } else {
    // core/quantization.py:9 (amax * clip / bound, then the 1e-8 floor).
    rs.scale = fmaxf(mx * clip / qmax, 1e-8f);
    rs.zf = 0.0f;
    rs.y = 0.0f;
    rs.thr = 1.0f;
  }
  return rs;
}

// --------------------------------------------------------- register kernel

// First butterfly stage straight from a dword holding two fp16 values:
// y0 = lo + hi, y1 = lo - hi, each a single IEEE fp32 rounding of the exact
// result (v_fma_mix widens the fp16 operands exactly), so the fp16 -> fp32
// conversion costs nothing.
__device__ __forceinline__ void bfly_f16x2(uint32_t w, float& y0, float& y1) {
  asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(y0) : "v"(w));
  asm("v_fma_mix_f32 %0, %1, -1.0, %1 op_sel:[1,0,0] op_sel_hi:[1,0,1]" : "=v"(y1) : "v"(w));
}

// Stages for index bits 1 and 2 of one chunk (bit 0 already applied).
__device__ __forceinline__ void fwht_chunk_tail(float v[8]) {
#pragma unroll
  for (int h = 2; h < 8; h <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (!(i & h)) {
        const float u = v[i], w = v[i + h];
        v[i] = u + w;
        v[i + h] = u - w;
      }
}

// Cross-lane stages of the register kernel, one instruction per element:
// v_fmac_f32_dpp computes own + sgn * partner, partner read across the quad
// by DPP.  For the pair (lo, hi) the lane holding lo (sgn = +1) gets lo + hi,
// the lane holding hi (sgn = -1) gets hi - lo = -(lo - hi): exactly the
// negated butterfly output, since round-to-nearest is symmetric.  Each stage
// thus leaves a known per-lane sign, tracked by the caller (lanes r = 1 and
// r = 2 of a quad end up holding -y).  The leading s_nop covers the
// two-wait-state gap gfx9 requires between a VALU write and a DPP read.
#define DSCQ_FMAC_DPP8(PERM)                                                              \
  asm("s_nop 1\n\t"                                                                       \
      "v_fmac_f32_dpp %0, %0, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf\n\t"       \
      "v_fmac_f32_dpp %1, %1, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf\n\t"       \
      "v_fmac_f32_dpp %2, %2, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf\n\t"       \
      "v_fmac_f32_dpp %3, %3, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf\n\t"       \
      "v_fmac_f32_dpp %4, %4, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf\n\t"       \
      "v_fmac_f32_dpp %5, %5, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf\n\t"       \
      "v_fmac_f32_dpp %6, %6, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf\n\t"       \
      "v_fmac_f32_dpp %7, %7, %8 quad_perm:" PERM " row_mask:0xf bank_mask:0xf"           \
      : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5]), "+v"(c[6]), \
        "+v"(c[7])                                                                        \
      : "v"(sgn))

__device__ __forceinline__ void fmac_dpp_xor1(float (&c)[8], float sgn) {
  DSCQ_FMAC_DPP8("[1,0,3,2]");
}
__device__ __forceinline__ void fmac_dpp_xor2(float (&c)[8], float sgn) {
  DSCQ_FMAC_DPP8("[2,3,0,1]");
}
#undef DSCQ_FMAC_DPP8

// Cross-lane butterfly through the LDS crossbar (ds_swizzle, no memory):
// partner = lane ^ XOR within 32 lanes; the lane whose XOR bit is clear keeps
// own + partner, the other partner - own -- fma(+-1, own, partner), rounded
// exactly like the plain add / subtract.
template <int XOR>
__device__ __forceinline__ void bfly_swizzle(float (&c)[8], float sgn) {
  constexpr int kPattern = 0x1F | (XOR << 10);  // bit mode: and 0x1f, xor XOR
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float p = __builtin_bit_cast(
        float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, c[i]), kPattern));
    c[i] = __builtin_fmaf(sgn, c[i], p);
  }
}

// Index bits 3..6 of one block as c[4][8] in quad lane r; afterwards the lane
// holds sign(r) * y with sign(r) = -1 for r = 1, 2 and +1 for r = 0, 3.
__device__ __forceinline__ void fwht_block_tail_signed(float c[4][8], int r) {
  const float s1 = (r & 1) ? -1.0f : 1.0f;
  const float s2 = (r & 2) ? -1.0f : 1.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) fmac_dpp_xor1(*reinterpret_cast<float(*)[8]>(c[j]), s1);
#pragma unroll
  for (int j = 0; j < 4; ++j) fmac_dpp_xor2(*reinterpret_cast<float(*)[8]>(c[j]), s2);
#pragma unroll
  for (int h = 1; h < 4; h <<= 1)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!(j & h)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float u = c[j][i], w = c[j + h][i];
          c[j][i] = u + w;
          c[j + h][i] = u - w;
        }
      }
}

// Activation chunk -> bytes u = q, clip == 1 form: no clamp.  With clip 1 the
// exact t lies in [-0.5, 15.5] (t = 15 - u + rne(u) at the row maximum and
// -u + rne(u) at the minimum, u = -lo / scale), so a code outside [0, 15]
// needs t within rounding distance of -0.5 or 15.5 -- exactly the near-tie
// case the dmax check sends to the exact path.  cvt_pk_u8 saturates -0 to 0.
__device__ __forceinline__ void act_chunk_fast_noclamp(const float v[8], const RowScale& rs,
                                                       uint32_t& ev, uint32_t& od,
                                                       float& dmax) {
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float t = __builtin_fmaf(v[i], rs.y, rs.zf);
    q[i] = __builtin_rintf(t);
    dmax = fmaxf(dmax, fabsf(t - q[i]));
  }
  ev = put_u8<0>(q[0], 0u); ev = put_u8<1>(q[2], ev); ev = put_u8<2>(q[4], ev); ev = put_u8<3>(q[6], ev);
  od = put_u8<0>(q[1], 0u); od = put_u8<1>(q[3], od); od = put_u8<2>(q[5], od); od = put_u8<3>(q[7], od);
}

}  // namespace dscq
