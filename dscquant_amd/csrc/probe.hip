// Measurement probes (no reference counterpart): the ceilings the W4A4
// kernels are compared against, measured on the same device in the same run.
//
//   stream_probe_kernel  a plain streaming kernel: each thread reads R 16-byte
//                        pieces (consecutive threads read consecutive pieces,
//                        so every load instruction of a wave reads 1 KiB
//                        contiguous) and, when there is an output, writes
//                        their XOR as one 16-byte piece with the same
//                        streaming stores the quantize kernel uses.  With
//                        R = 4 over fp16 activations it moves exactly the
//                        bytes of one activation quantize (read 2 M K, write
//                        M K / 2); without an output it is a bare read (the
//                        decode kernels' weight stream).
//   mfma_probe_kernel    only v_mfma_i32_32x32x32_i8 on register operands, no
//                        memory traffic in the loop: each wave issues the
//                        MFMAs of a 2 x 2 block of 32 x 32 tiles per k-step,
//                        as a wave of the pipelined GEMM does, alternating
//                        two operand sets.  At the prefill GEMM's grid
//                        (256 workgroups of 8 waves, 512 MFMAs per wave) it
//                        is the time the matrix cores alone take for that
//                        GEMM's 2 M N K operations.

#include "../../include/dscq.h"
#include "common.h"
#include "mma_int4.h"

namespace dscq {
namespace {

template <int R, bool WRITE>
__global__ __launch_bounds__(256) void stream_probe_kernel(const uint4* __restrict__ src,
                                                           uint4* __restrict__ dst,
                                                           int64_t threads) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= threads) return;
  uint4 v[R];
#pragma unroll
  for (int j = 0; j < R; ++j) v[j] = src[t + j * threads];
  uint4 acc = v[0];
#pragma unroll
  for (int j = 1; j < R; ++j) {
    acc.x ^= v[j].x;
    acc.y ^= v[j].y;
    acc.z ^= v[j].z;
    acc.w ^= v[j].w;
  }
  if (WRITE) {
    store_stream(acc, dst + t);
  } else if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u && acc.z == 0xF39CC060u &&
             acc.w == 0x5CEDC834u) {
    // Keeps the loads live; a thread writes only if its pieces XOR to this value.
    dst[0] = acc;
  }
}

// Operand byte p (0..15) of lane l in set `seed`: f(l % 32) + g(l / 32, p),
// both multiples of 16 in [-64, 48] (the unpacked operands are nibble * 16),
// so the values vary over lanes and bytes like real operands.  An MFMA
// computing C[i][j] += sum_k X[i][k] Y[k][j] from two such operands (row or
// column index l % 32, k given by (l / 32, p) the same way for both) adds
// sum_k (Fx + 32 gx(k)) (Fy + 32 gy(k)) to the sum of C's elements, F = sum_i f(i),
// whatever the operand layout.
__device__ __forceinline__ int probe_part(uint32_t seed, uint32_t idx) {
  const uint32_t h = (seed * 0x9E3779B1u) ^ (idx * 0x85EBCA77u);
  return (int)(((h >> 13) ^ (h >> 7)) & 7u) * 16 - 64;
}

__device__ __forceinline__ v4i probe_operand(uint32_t seed, int lane) {
  const int f = probe_part(seed, 64u + (uint32_t)(lane & 31));
  v4i r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int v = f + probe_part(seed ^ 0x5bd1e995u, (uint32_t)((lane >> 5) * 16 + 4 * i + b));
      w |= ((uint32_t)v & 0xFFu) << (8 * b);
    }
    r[i] = (int)w;
  }
  return r;
}

__global__ __launch_bounds__(512, 1) void mfma_probe_kernel(int steps, int32_t* out) {
  // Operands built in registers; the asm keeps the compiler from treating
  // them as constants across the loop.
  const int lane = threadIdx.x & 63;
  v4i a0 = probe_operand(1, lane), b0 = probe_operand(2, lane), a1 = probe_operand(3, lane),
      b1 = probe_operand(4, lane);
  asm volatile("" : "+v"(a0), "+v"(b0), "+v"(a1), "+v"(b1));
  v16i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v16i{0};
  for (int s = 0; s < steps; s += 2) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b0, a0, acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b1, a1, acc[i][j], 0, 0, 0);
  }
  int32_t sum = 0;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sum += acc[i][j][e];
  sum = wave_sum_i32(sum);
  if ((threadIdx.x & 63) == 0) out[(int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = sum;
}

}  // namespace
}  // namespace dscq

using namespace dscq;

extern "C" {

int dscq_stream_probe(const void* src, int64_t read_bytes, void* dst, int64_t write_bytes,
                      int pieces, void* stream) {
  DisarmOnExit disarm;
  if (!(pieces == 1 || pieces == 2 || pieces == 4 || pieces == 8 || pieces == 16))
    return fail("stream_probe: pieces must be 1, 2, 4, 8 or 16 (got %d)", pieces);
  if (!(read_bytes > 0 && read_bytes % (16LL * pieces) == 0))
    return fail("stream_probe: read_bytes must be a positive multiple of 16 * pieces");
  const int64_t threads = read_bytes / (16LL * pieces);
  if (write_bytes != 0 && write_bytes != 16 * threads)
    return fail("stream_probe: write_bytes must be 0 or read_bytes / pieces");
  if (!src || !dst) return fail("stream_probe: null buffer");
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15)
    return fail("stream_probe: buffers must be 16-byte aligned");
  if ((threads + 255) / 256 > 0x7FFFFFFFLL) return fail("stream_probe: grid too large");
  const dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint4* in = static_cast<const uint4*>(src);
  uint4* o = static_cast<uint4*>(dst);
#define DSCQ_PROBE(R)                                                                   \
  if (pieces == R) {                                                                    \
    if (write_bytes)                                                                    \
      launch((stream_probe_kernel<R, true>), grid, block, s, in, o, threads);           \
    else                                                                                \
      launch((stream_probe_kernel<R, false>), grid, block, s, in, o, threads);          \
  }
  DSCQ_PROBE(1) DSCQ_PROBE(2) DSCQ_PROBE(4) DSCQ_PROBE(8) DSCQ_PROBE(16)
#undef DSCQ_PROBE
  return launch_status("stream_probe_kernel");
}

int dscq_mfma_probe(int64_t workgroups, int waves, int64_t mfmas_per_wave, int32_t* out,
                    void* stream) {
  DisarmOnExit disarm;
  if (!(workgroups > 0 && workgroups <= 0x7FFFFFFFLL))
    return fail("mfma_probe: workgroups must be in [1, 2^31)");
  if (!(waves >= 1 && waves <= 8)) return fail("mfma_probe: waves must be in [1, 8]");
  if (!(mfmas_per_wave > 0 && mfmas_per_wave % 8 == 0 && mfmas_per_wave / 4 <= 0x7FFFFFFFLL))
    return fail("mfma_probe: mfmas_per_wave must be a positive multiple of 8");
  if (!out) return fail("mfma_probe: null buffer");
  launch(mfma_probe_kernel, dim3((unsigned)workgroups), dim3(64 * waves),
         static_cast<hipStream_t>(stream), (int)(mfmas_per_wave / 4), out);
  return launch_status("mfma_probe_kernel");
}

}  // extern "C"
