// Arguments of the GEMM kernels, shared by gemm.hip (the pipelined, skinny-M
// and general kernels, and the dispatch) and gemm_wide.hip (the wide-tile
// kernel for grids of several rounds).
#pragma once

#include "common.h"

namespace dscq {

struct GemmArgs {
  const uint8_t* a;
  const uint8_t* b;
  const float* sx;
  const int32_t* zx;
  const float* sw;
  const int32_t* sums;
  const void* bias;  // null or [N] of the output type
  void* out;         // [M, N] fp16 or fp32
  int32_t* raw;      // null or [M, N]
  int64_t M, N, KP;
  int64_t arows, brows;  // readable rows of a (>= MP) and b (>= NP)
  int tiles_n;
  // K split over workgroups (pipelined kernel only): part p of every tile
  // covers 256-nibble slices [p * kslices, (p + 1) * kslices) and writes its
  // int32 sums to part + p * M * N; a second pass adds the parts and applies
  // the epilogue.
  int32_t* part = nullptr;
  int kslices = 0;
  int tiles = 0;  // tiles per part
};

// The wide-tile kernel (gemm_wide.hip): 256 x bn tiles (bn = 256 or 128),
// one wave per SIMD, fp16 output without raw accumulators.  wide_gemm_fits
// says whether a shape and its buffers meet the kernel's requirements;
// launch_wide_gemm runs it.
bool wide_gemm_fits(const GemmArgs& g);
int launch_wide_gemm(GemmArgs g, int bn, hipStream_t stream);
// The same kernel with 256 x 256 tiles and the SiLU-gated epilogue of
// dscq_matmul_silu_mul (gate and up rows interleaved in blocks of 64, h
// [M, N / 2] fp16 out).
int launch_wide_gemm_gated(GemmArgs g, hipStream_t stream);

// This thread's GEMM kernel preference (dscq_set_gemm_kernel): 0 automatic,
// 1 the wide-tile kernel wherever it applies, 2 never, 3 / 4 the wide-tile
// kernel with 256 x 256 / 256 x 128 tiles wherever it applies.
int gemm_kernel_preference();

}  // namespace dscq
