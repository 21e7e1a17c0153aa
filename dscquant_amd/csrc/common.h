// Shared device helpers and host error plumbing for libdscq (gfx950 only).
#pragma once

#include <hip/hip_ext.h>
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
// Compute units of the current device (cached per device; 256 on MI355X).
int cu_count();

// Events armed by dscq_time_next_kernel for this thread's next kernel launch
// (both null when none is armed); taking them disarms them.
struct KernelEvents {
  hipEvent_t start, stop;
};
KernelEvents take_kernel_events();
// Arms events for the next launch (used to hand the stop event of a call to
// its last kernel).
void arm_kernel_events(KernelEvents ev);

// Placed first in every entry point that may launch: whatever path the call
// leaves by (an argument error, an empty shape, a failed launch), events armed
// for it do not stay armed for a later, unrelated call.
struct DisarmOnExit {
  DisarmOnExit() = default;
  DisarmOnExit(const DisarmOnExit&) = delete;
  DisarmOnExit& operator=(const DisarmOnExit&) = delete;
  ~DisarmOnExit() { take_kernel_events(); }
};

// Every kernel of the library is launched through here.  With events armed the
// launch goes through hipExtLaunchKernel, which stamps the kernel's own start
// and end into them (a kernel trace's duration, without event markers around
// the launch).
template <typename F, typename... Args>
void launch(F kernel, dim3 grid, dim3 block, hipStream_t stream, Args... args) {
  const KernelEvents ev = take_kernel_events();
  if (ev.start || ev.stop)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, ev.start, ev.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
}

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

// Min / max over the 64 lanes of a wave; every lane gets the result.  Each
// 16-lane row is reduced with v_min / v_max taking one operand through DPP
// (one instruction per step; written out because the compiler pairs a DPP
// move with a canonicalizing max before every fminf / fmaxf), then
// row_bcast:15 folds row 0 into row 1 and row 2 into row 3, row_bcast:31 rows
// 0-1 into rows 2-3, leaving the wave's result in lane 63.  The s_nops cover
// the two wait states gfx9 needs between a VALU write and a DPP read of the
// same register.  Inputs are finite.
#define DSCQ_DPP_REDUCE(OP, V)                                                         \
  asm("s_nop 1\n\t"                                                                   \
      "v_" OP "_f32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"  \
      "s_nop 1\n\t"                                                                   \
      "v_" OP "_f32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"  \
      "s_nop 1\n\t"                                                                   \
      "v_" OP "_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf\n\t"            \
      "s_nop 1\n\t"                                                                   \
      "v_" OP "_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"            \
      "s_nop 1\n\t"                                                                   \
      "v_" OP "_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"         \
      "s_nop 1\n\t"                                                                   \
      "v_" OP "_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf"              \
      : "+v"(V))

__device__ __forceinline__ float wave_min(float v) {
  DSCQ_DPP_REDUCE("min", v);
  return readlane_f32(v, 63);
}

__device__ __forceinline__ float wave_max(float v) {
  DSCQ_DPP_REDUCE("max", v);
  return readlane_f32(v, 63);
}
#undef DSCQ_DPP_REDUCE

__device__ __forceinline__ int wave_sum_i32(int v) {
  v += __builtin_amdgcn_mov_dpp(v, kDppQuadXor1, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, kDppQuadXor2, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, kDppRowRor4, 0xF, 0xF, false);
  v += __builtin_amdgcn_mov_dpp(v, kDppRowRor8, 0xF, 0xF, false);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}

// Streaming stores (non-temporal cache policy) for outputs no later work of the
// same kernel reads: the quantize kernel's packed codes and the GEMM's output
// rows.  Measured on the prefill step (M=2048, K=N=4096): quantize ~0.5 us
// and GEMM ~0.5-1 us shorter, identical bytes.
__device__ __forceinline__ void store_stream(uint4 v, void* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4 t;
  t.x = v.x;
  t.y = v.y;
  t.z = v.z;
  t.w = v.w;
  __builtin_nontemporal_store(t, static_cast<u32x4*>(p));
}
__device__ __forceinline__ void store_stream(uint32_t v, void* p) {
  __builtin_nontemporal_store(v, static_cast<uint32_t*>(p));
}

// Byte `sel` of the result = (uint8)v (v must be an integer value 0..255).
template <int SEL>
__device__ __forceinline__ uint32_t put_u8(float v, uint32_t old) {
  return __builtin_amdgcn_cvt_pk_u8_f32(v, SEL, old);
}

}  // namespace dscq
