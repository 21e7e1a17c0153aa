// Packed-int4 x packed-int4 GEMM for gfx950 with int32 accumulation on the
// int8 matrix cores and the fused dequant epilogue.
//
// Semantics (kernel/w4a4.cu:70-161):
//   raw[m, n] = sum_{k < KP} sa(m, k) * sb(n, k),   s = signed nibble in [-8, 7]
//   out[m, n] = (float)(raw + (8 - zx[m]) * sums[n]) * sx[m] * sw[n] (+ bias[n])
// Both operands are row-major with K contiguous (TN): a [>= MP, KP/2],
// b [>= NP, KP/2].
//
// CDNA4 has no int4 MFMA.  A packed dword w holds 8 nibbles; the two dwords
//   lo = (w << 4) & 0xF0F0F0F0   (even k, each byte = 16 * nibble value)
//   hi =  w       & 0xF0F0F0F0   (odd k)
// are 8 int8 values scaled by 16 with the sign in the byte's top bit, so one
// shift and two ANDs unpack 8 k-values.  A and B go through the same k
// permutation, so the dot product is unchanged and carries a factor 256,
// removed exactly by an arithmetic >> 8 (the accumulator is a multiple of
// 256).  |partial sums| <= 256 * 64 * K stays below 2^31 for K <= 65536;
// longer rows drain the accumulator into an unscaled total every 65536 k.
//
// Tiling.  A workgroup owns a BM x BN output tile; WM x WN waves each own a
// (BM/WM) x (BN/WN) sub-tile made of 32 x 32 v_mfma_i32_32x32x32_i8 tiles.
// The K loop walks 128-nibble (64-byte) slices: each slice of A and B is
// staged in LDS as four 16-byte "planes" (k-bytes 0-15, 16-31, ...), one per
// MFMA k-step, laid out [plane][row][16 B] so a fragment read -- lane l takes
// row l % 32, bytes 8 * (l / 32) .. +7 -- is one conflict-free ds_read_b64.
// Planes are padded by 64 bytes so the 16-byte writes of four consecutive
// lanes (one 64-byte global segment of a row) land in distinct banks.  Two
// LDS stages double-buffer the slices: global loads for slice k+1 are in
// flight while slice k feeds the matrix cores; one barrier per slice.

#include <cstdlib>
#include <cstring>

#include "../../include/dscq.h"
#include "common.h"

namespace dscq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

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
};

constexpr int kSliceBytes = 64;  // 128 nibbles of K per LDS stage
constexpr int kPlanePad = 64;

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
template <>
__device__ __forceinline__ __half to_out<__half>(float v) {
  return __float2half_rn(v);
}
template <>
__device__ __forceinline__ float to_out<float>(float v) {
  return v;
}

template <typename OutT, int BM, int BN, int WM, int WN, bool HUGE>
__global__ __launch_bounds__(64 * WM * WN) void w4a4_gemm_kernel(GemmArgs g) {
  constexpr int THREADS = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int A_PLANE = BM * 16 + kPlanePad;
  constexpr int B_PLANE = BN * 16 + kPlanePad;
  constexpr int STAGE = 4 * A_PLANE + 4 * B_PLANE;
  constexpr int PIECES = (BM + BN) * 4;  // 16-byte pieces per slice
  constexpr int LOADS = (PIECES + THREADS - 1) / THREADS;
  static_assert(FM >= 1 && FN >= 1, "wave tile must hold a 32x32 MFMA tile");

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int tile_m = blockIdx.x / g.tiles_n;
  const int tile_n = blockIdx.x % g.tiles_n;
  const int64_t m0 = (int64_t)tile_m * BM;
  const int64_t n0 = (int64_t)tile_n * BN;
  const int64_t KB = g.KP / 2;  // bytes per packed row
  const int nslices = (int)((KB + kSliceBytes - 1) / kSliceBytes);

  // ---- global -> register staging for one slice
  const uint8_t* src[LOADS];
  int lds_off[LOADS];
  bool row_ok[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int q = tid + i * THREADS;
    const int plane = q & 3;
    if (q >= PIECES) {
      row_ok[i] = false;
      src[i] = g.a;
      lds_off[i] = -1;
    } else if (q < BM * 4) {
      const int r = q >> 2;
      row_ok[i] = m0 + r < g.arows;
      src[i] = g.a + (row_ok[i] ? (m0 + r) : 0) * KB + plane * 16;
      lds_off[i] = plane * A_PLANE + r * 16;
    } else {
      const int r = (q - BM * 4) >> 2;
      row_ok[i] = n0 + r < g.brows;
      src[i] = g.b + (row_ok[i] ? (n0 + r) : 0) * KB + plane * 16;
      lds_off[i] = 4 * A_PLANE + plane * B_PLANE + r * 16;
    }
  }
  uint4 stage[LOADS];
  auto gload = [&](int s) {
    const int64_t kb = (int64_t)s * kSliceBytes;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int plane = (tid + i * THREADS) & 3;
      if (row_ok[i] && kb + plane * 16 < KB) {
        stage[i] = *reinterpret_cast<const uint4*>(src[i] + kb);
      } else {
        stage[i] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i)
      if (PIECES % THREADS == 0 || lds_off[i] >= 0)
        *reinterpret_cast<uint4*>(smem + buf * STAGE + lds_off[i]) = stage[i];
  };

  v16i acc[FM][FN];
  v16i tot[HUGE ? FM : 1][HUGE ? FN : 1];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      acc[i][j] = v16i{0};
      if (HUGE) tot[HUGE ? i : 0][HUGE ? j : 0] = v16i{0};
    }

  // Fragment read offsets within a plane (bytes).
  const int frag_row = lane & 31;
  const int frag_half = (lane >> 5) * 8;

  gload(0);
  lstore(0);
  __syncthreads();
  for (int s = 0; s < nslices; ++s) {
    const int buf = s & 1;
    if (s + 1 < nslices) gload(s + 1);
    const uint8_t* As = smem + buf * STAGE;
    const uint8_t* Bs = As + 4 * A_PLANE;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      v4i af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const uint2 w = *reinterpret_cast<const uint2*>(
            As + p * A_PLANE + (wm * TM + i * 32 + frag_row) * 16 + frag_half);
        af[i] = unpack8(w.x, w.y);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const uint2 w = *reinterpret_cast<const uint2*>(
            Bs + p * B_PLANE + (wn * TN + j * 32 + frag_row) * 16 + frag_half);
        bf[j] = unpack8(w.x, w.y);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (HUGE && ((s + 1) % 512 == 0)) {  // 512 slices = 65536 k: drain
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
          for (int v = 0; v < 16; ++v) tot[HUGE ? i : 0][HUGE ? j : 0][v] += acc[i][j][v] >> 8;
          acc[i][j] = v16i{0};
        }
    }
    if (s + 1 < nslices) lstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: D[i][j] of a 32x32 tile sits in lane (j % 32) + 32 * ((i / 4) % 2),
  // register (i % 4) + 4 * (i / 8).
  OutT* out = static_cast<OutT*>(g.out);
  const OutT* bias = static_cast<const OutT*>(g.bias);
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * TN + j * 32 + (lane & 31);
    const bool col_ok = col < g.N;
    const float swc = col_ok ? g.sw[col] : 0.0f;
    const int32_t sumc = col_ok ? g.sums[col] : 0;
    const float bc = (col_ok && bias) ? (float)bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * TM + i * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
        if (!col_ok || row >= g.M) continue;
        int32_t r = acc[i][j][v] >> 8;
        if (HUGE) r += tot[HUGE ? i : 0][HUGE ? j : 0][v];
        const int32_t corrected = r + (8 - g.zx[row]) * sumc;
        float res = (float)corrected * g.sx[row];
        res = res * swc;
        if (bias) res = res + bc;
        out[row * g.N + col] = to_out<OutT>(res);
        if (g.raw) g.raw[row * g.N + col] = r;
      }
    }
  }
}

template <typename OutT, int BM, int BN, int WM, int WN, bool HUGE>
int launch_cfg(GemmArgs g, hipStream_t stream) {
  g.tiles_n = (int)((g.N + BN - 1) / BN);
  const int64_t tiles_m = (g.M + BM - 1) / BM;
  const int64_t nblocks = tiles_m * g.tiles_n;
  if (nblocks > 0x7FFFFFFF) return fail("matmul: grid too large (M=%lld, N=%lld)",
                                        (long long)g.M, (long long)g.N);
  hipLaunchKernelGGL((w4a4_gemm_kernel<OutT, BM, BN, WM, WN, HUGE>), dim3((unsigned)nblocks),
                     dim3(64 * WM * WN), 0, stream, g);
  return launch_status("w4a4_gemm_kernel");
}

// DSCQ_GEMM_TILE=<BM>x<BN>[w8] pins the tile shape (tuning sweeps only).
template <typename OutT>
int tile_override(const GemmArgs& g, hipStream_t stream, int* handled) {
  static const char* env = getenv("DSCQ_GEMM_TILE");
  *handled = 1;
  if (env && g.KP <= 65536) {
    if (!strcmp(env, "128x256")) return launch_cfg<OutT, 128, 256, 2, 2, false>(g, stream);
    if (!strcmp(env, "128x128")) return launch_cfg<OutT, 128, 128, 2, 2, false>(g, stream);
    if (!strcmp(env, "256x128")) return launch_cfg<OutT, 256, 128, 2, 2, false>(g, stream);
    if (!strcmp(env, "256x256")) return launch_cfg<OutT, 256, 256, 2, 2, false>(g, stream);
    if (!strcmp(env, "128x256w8")) return launch_cfg<OutT, 128, 256, 2, 4, false>(g, stream);
    if (!strcmp(env, "256x128w8")) return launch_cfg<OutT, 256, 128, 4, 2, false>(g, stream);
    if (!strcmp(env, "64x128")) return launch_cfg<OutT, 64, 128, 2, 2, false>(g, stream);
  }
  *handled = 0;
  return 0;
}

template <typename OutT>
int gemm_typed(const GemmArgs& g, bool decode, hipStream_t stream) {
  int handled = 0;
  const int rc = tile_override<OutT>(g, stream, &handled);
  if (handled) return rc;
  if (g.KP > 65536) return launch_cfg<OutT, 64, 64, 2, 2, true>(g, stream);
  if (decode || g.M <= 32) return launch_cfg<OutT, 32, 128, 1, 4, false>(g, stream);
  const int64_t big_tiles = ((g.M + 127) / 128) * ((g.N + 255) / 256);
  if (big_tiles >= 192) return launch_cfg<OutT, 128, 256, 2, 2, false>(g, stream);
  return launch_cfg<OutT, 128, 128, 2, 2, false>(g, stream);
}

}  // namespace

int w4a4_gemm(const uint8_t* a, const uint8_t* b, const float* sx, const int32_t* zx,
              const float* sw, const int32_t* sums, const void* bias, int64_t M,
              int64_t N, int64_t KP, bool decode, bool out_fp32, void* out,
              int32_t* raw, hipStream_t stream) {
  GemmArgs g;
  g.a = a;
  g.b = b;
  g.sx = sx;
  g.zx = zx;
  g.sw = sw;
  g.sums = sums;
  g.bias = bias;
  g.out = out;
  g.raw = raw;
  g.M = M;
  g.N = N;
  g.KP = KP;
  g.arows = ceil_to(M, 8);
  g.brows = ceil_to(N, 8);
  g.tiles_n = 0;
  return out_fp32 ? gemm_typed<float>(g, decode, stream)
                  : gemm_typed<__half>(g, decode, stream);
}

}  // namespace dscq
