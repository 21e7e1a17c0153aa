// Shared device helpers and host error plumbing for libdscq (gfx950 only).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace dscq {

// ---------------------------------------------------------------- host side

// Records a printf-style message as this thread's last error and returns
// DSCQ_EINVAL.
int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
// Checks the launch status; records the HIP error string on failure.
int launch_status(const char* what);

inline int64_t ceil_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// -------------------------------------------------------------- device side

// DPP lane permutations (gfx9 encodings).  quad_perm [1,0,3,2] swaps lanes
// xor 1, [2,3,0,1] swaps lanes xor 2; row_ror:n rotates within 16 lanes.
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                      false));
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Min / max over the 64 lanes of a wave; every lane gets the result.
__device__ __forceinline__ float wave_min(float v) {
  v = fminf(v, dpp_f32<kDppQuadXor1>(v));
  v = fminf(v, dpp_f32<kDppQuadXor2>(v));
  v = fminf(v, dpp_f32<kDppRowRor4>(v));
  v = fminf(v, dpp_f32<kDppRowRor8>(v));
  return fminf(fminf(readlane_f32(v, 0), readlane_f32(v, 16)),
               fminf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f32<kDppRowRor4>(v));
  v = fmaxf(v, dpp_f32<kDppRowRor8>(v));
  return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)),
               fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

__device__ __forceinline__ int wave_sum_i32(int v) {
  v += __builtin_amdgcn_mov_dpp(v, kDppQuadXor1, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, kDppQuadXor2, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, kDppRowRor4, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, kDppRowRor8, 0xF, 0xF, false);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

// Byte `sel` of the result = (uint8)v (v must be an integer value 0..255).
template <int SEL>
__device__ __forceinline__ uint32_t put_u8(float v, uint32_t old) {
  return __builtin_amdgcn_cvt_pk_u8_f32(v, SEL, old);
}

}  // namespace dscq
