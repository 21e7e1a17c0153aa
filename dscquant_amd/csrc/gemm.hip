// Packed-int4 x packed-int4 GEMM for gfx950 with int32 accumulation on the
// int8 matrix cores and the fused dequant epilogue.
//
// Semantics (kernel/w4a4.cu:70-161):
//   raw[m, n] = sum_{k < KP} sa(m, k) * sb(n, k),   s = signed nibble in [-8, 7]
//   out[m, n] = (float)(raw + (8 - zx[m]) * sums[n]) * sx[m] * sw[n] (+ bias[n])
// Both operands are row-major with K contiguous (TN): a [>= MP, KP/2],
// b [>= NP, KP/2].
//
// CDNA4 has no int4 MFMA: both operands are unpacked from nibbles to int8 in
// registers (mma_int4.h), so every dot product carries a factor 256, removed
// exactly by an arithmetic >> 8.  |partial sums| <= 256 * 64 * K stays below
// 2^31 for K <= 65536; longer rows drain the accumulator into an unscaled
// total every 65536 k.
//
// Kernels (dispatch in gemm_typed):
//   w4a4_gemm_pipe_kernel  the main kernel (M >= 64 bar the skinny rule below, or
//                          16 < M < 64 with N > 8064;
//                          N % 8 == 0): 256-nibble slices, swizzled LDS rows,
//                          two slices of global loads in flight, one barrier
//                          per slice (its own comment below);
//   w4a4_gemv_kernel       M < 64 otherwise, ceil(M/16) * N <= 16384 with
//                          4096 <= KP <= 65536, or force_decode: weights streamed
//                          once per 16 rows, K split over the waves of a
//                          workgroup;
//   w4a4_gemm_kernel       everything else (N % 8 != 0, output not 16-byte
//                          aligned, KP > 65536 at M >= 64): a simpler tiled kernel.
//
// w4a4_gemm_kernel tiling.  A workgroup owns a BM x BN output tile; WM x WN
// waves each own a (BM/WM) x (BN/WN) sub-tile made of 32 x 32
// v_mfma_i32_32x32x32_i8 tiles.  The K loop walks 128-nibble (64-byte) slices:
// each slice of A and B is staged in LDS as four 16-byte "planes" (k-bytes
// 0-15, 16-31, ...), one per MFMA k-step, laid out [plane][row][16 B] so a
// fragment read -- lane l takes row l % 32, bytes 8 * (l / 32) .. +7 -- is one
// conflict-free ds_read_b64.  Planes are padded by 64 bytes so the 16-byte
// writes of four consecutive lanes (one 64-byte global segment of a row) land
// in distinct banks.  Two LDS stages double-buffer the slices: global loads
// for slice k+1 are in flight while slice k feeds the matrix cores; one
// barrier per slice.

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "../../include/dscq.h"
#include "common.h"
#include "gemm_args.h"
#include "mma_int4.h"
#include "rowquant.h"

namespace dscq {
namespace {


constexpr int kSliceBytes = 64;  // 128 nibbles of K per LDS stage
constexpr int kPlanePad = 64;

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
  // register (i % 4) + 4 * (i / 8).  All row / column metadata is fetched
  // before any of it is used, so the loads overlap.
  OutT* out = static_cast<OutT*>(g.out);
  const OutT* bias = static_cast<const OutT*>(g.bias);
  float sxr[FM][16];
  int32_t zr[FM][16];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t row = min(m0 + wm * TM + i * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2),
                              g.arows - 1);
      sxr[i][v] = g.sx[row];
      zr[i][v] = 8 - g.zx[row];
    }
  float swc[FN], bc[FN];
  int32_t sumc[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * TN + j * 32 + (lane & 31);
    const int64_t colc = col < g.N ? col : 0;
    swc[j] = g.sw[colc];
    sumc[j] = g.sums[colc];
    bc[j] = bias ? (float)bias[colc] : 0.0f;
  }
  // The raw-accumulator mode is a separate uniform path so that store data
  // registers of one mode are never recycled under the other's stores.
  auto store_all = [&](auto with_raw) {
  constexpr bool WITH_RAW = decltype(with_raw)::value;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t col = n0 + wn * TN + j * 32 + (lane & 31);
    const bool col_ok = col < g.N;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * TM + i * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
        int32_t r = acc[i][j][v] >> 8;
        if (HUGE) r += tot[HUGE ? i : 0][HUGE ? j : 0][v];
        const int32_t corrected = r + zr[i][v] * sumc[j];
        float res = (float)corrected * sxr[i][v];
        res = res * swc[j];
        if (bias) res = res + bc[j];
        if (col_ok && row < g.M) {
          out[row * g.N + col] = to_out<OutT>(res);
          if (WITH_RAW) g.raw[row * g.N + col] = r;
        }
      }
    }
  }
  };
  if (g.raw)
    store_all(std::true_type{});
  else
    store_all(std::false_type{});
}

// ------------------------------------------------------ pipelined kernel
// BM x BN output tile, WM x WN waves, each wave a (BM/WM) x (BN/WN) block of
// 32 x 32 MFMA tiles.  K advances in slices of 256 nibbles: 128 bytes of every
// A and B row of the tile, staged in LDS row-major (A rows, then B rows) as
// eight 16-byte units per row, unit u of row r stored at position
// u ^ ((r >> 1) & 7).  With that swizzle the 16-byte accesses of any 16
// consecutive lanes -- 16 rows x one unit on reads, 2 rows x 8 units on
// writes -- cover all 64 banks once.  Lane l of a fragment read takes row
// l % 32, unit 2q + l / 32 (q = 0..3): the low 8 bytes feed MFMA k-step 2q,
// the high 8 bytes k-step 2q + 1 -- the same assignment for A and B, so every
// product pairs equal k.
//
// Pipeline, one barrier per slice (two slices in flight in LDS), memory
// operations spread over the steps so LDS traffic never comes in one burst:
//   steps 0-2     slice s + 1 (in registers since slice s - 1) written to LDS;
//                 global loads of slice s + 2 issued at step 0
//   steps 1, 3    fragment units q = 2, 3 of slice s read from LDS
//   step 5        barrier; units q = 0 (step 5) and 1 (step 6) of slice s + 1
// The barrier also orders every read of a buffer (slice s - 1's, at or
// before step 1 of slice s - 1) before the next write into it (step 2 of
// slice s).
// Each step interleaves its MFMAs with the nibble unpack of the next step's
// fragments.  The tile's row scales / zero-points are staged in LDS once.
// The epilogue (N % 8 == 0; out and raw 16-byte aligned) writes fp16 output
// through LDS as whole 128-byte row segments; fp32 output and the raw
// accumulators are stored as runs of 4 columns per lane straight from the
// accumulators.  Row and column metadata (sx, zx, sw, sums, bias) are staged
// in LDS with the first slice.

__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <typename OutT, int BM, int BN, int WM, int WN, int MINB, bool KTAIL, bool BIAS,
          bool GATED = false, bool SPLIT = false>
__global__ __launch_bounds__(64 * WM * WN, MINB) void w4a4_gemm_pipe_kernel(GemmArgs g) {
  constexpr int THREADS = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32, NF = FM + FN;
  constexpr int ROWS = BM + BN;
  constexpr int SB = 128;         // bytes of a row per slice
  constexpr int UNITS = SB / 16;  // 16-byte units per row per slice
  constexpr int STAGE = ROWS * SB;
  constexpr int LOADS = ROWS * UNITS / THREADS;  // 16-byte pieces per thread per slice
  static_assert(ROWS * UNITS % THREADS == 0 && THREADS / UNITS % 16 == 0, "load split");
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE + BM * 8 + BN * 12];
  float* const lds_sx = reinterpret_cast<float*>(smem + 2 * STAGE);
  float* const lds_z = reinterpret_cast<float*>(smem + 2 * STAGE + BM * 4);
  float* const lds_sw = reinterpret_cast<float*>(smem + 2 * STAGE + BM * 8);
  float* const lds_sum = reinterpret_cast<float*>(smem + 2 * STAGE + BM * 8 + BN * 4);
  float* const lds_b = reinterpret_cast<float*>(smem + 2 * STAGE + BM * 8 + BN * 8);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int bid = blockIdx.x;
  int s0 = 0;  // first slice of this workgroup's part of K
  int32_t* part = nullptr;
  if constexpr (SPLIT) {
    const int p = bid / g.tiles;
    bid -= p * g.tiles;
    s0 = p * g.kslices;
    part = g.part + (int64_t)p * g.M * g.N;
  }
  int tile_m = bid / g.tiles_n;
  int tile_n = bid % g.tiles_n;
  if constexpr (!SPLIT && BM == 256) {
    // Whole rounds of 256 x 128 tiles with wide N (>= 128 column tiles):
    // workgroup b runs on XCD b % 8, so each XCD's 32 workgroups of a round
    // take a 4 x 8 block of tiles (A read once per round, 2048 B rows instead
    // of up to all of B per XCD).  Measured, row-major order / blocks:
    // 4096 x 28672 x 8192 722 / 708 us, 2048 x 16384 x 4096 112.5 / 111.7 us;
    // at N = 8192 no gain (206.2 / 207.2 us), so narrower N keeps row order.
    const int tiles_m = (int)((g.M + BM - 1) / BM);
    if (g.tiles_n >= 128 && g.tiles_n % 8 == 0 && tiles_m % 4 == 0 &&
        (tiles_m * g.tiles_n) % 256 == 0) {
      const int grp = (bid >> 8) * 8 + (bid & 7), l = (bid & 255) >> 3;
      const int gm = tiles_m / 4;
      tile_m = (grp % gm) * 4 + (l & 3);
      tile_n = (grp / gm) * 8 + (l >> 2);
    }
  }
  const int64_t m0 = (int64_t)tile_m * BM;
  const int64_t n0 = (int64_t)tile_n * BN;
  const int64_t KB = g.KP / 2;
  const int nslices = SPLIT ? min(g.kslices, (int)((KB + SB - 1) / SB) - s0)
                            : (int)((KB + SB - 1) / SB);

  // Global pieces of this thread: unit u = tid % UNITS of rows
  // tid / UNITS + (THREADS / UNITS) i -- rows of A for i < BM / (THREADS / UNITS),
  // of B after.  Rows past MP / NP are clamped (never stored).  Offsets are
  // 32-bit (the launcher checks rows * KB < 2^32), so every load is the
  // scalar-base + 32-bit vector-offset form: no 64-bit address arithmetic per
  // load, measurably cheaper in the K loop.
  static_assert(BM % (THREADS / UNITS) == 0, "a piece index is all-A or all-B");
  constexpr int A_PIECES = BM / (THREADS / UNITS);
  const int u = tid % UNITS;
  uint32_t src_off[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int R = tid / UNITS + (THREADS / UNITS) * i;
    const int64_t row = i < A_PIECES ? min(m0 + R, g.arows - 1) : min(n0 + (R - BM), g.brows - 1);
    src_off[i] = (uint32_t)(row * KB + u * 16);
  }
  // (R >> 1) & 7 depends on tid only: THREADS / UNITS is a multiple of 16.
  const int wr_off = (tid / UNITS) * SB + 16 * (u ^ ((tid / UNITS >> 1) & 7));

  auto gload = [&](uint4 (&st)[LOADS], int slice) {
    const int sl = s0 + min(slice, nslices - 1);
    int64_t kb = (int64_t)sl * SB;
    // Pieces past the row end (only in the last slice when KB % SB != 0) read
    // the row's last in-bounds piece and are zeroed.
    const bool tail = KTAIL && kb + u * 16 >= KB;
    if (KTAIL && tail) kb = KB - 16 - u * 16;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const uint8_t* base = i < A_PIECES ? g.a : g.b;
      uint4 v = *reinterpret_cast<const uint4*>(base + (src_off[i] + (uint32_t)kb));
      if (KTAIL && tail) v = make_uint4(0u, 0u, 0u, 0u);
      st[i] = v;
    }
  };
  // Pieces [I0, I1) of a slice held in registers -> LDS stage `buf`.
  auto lstore = [&](const uint4 (&st)[LOADS], int buf, auto i0, auto i1) {
#pragma unroll
    for (int i = decltype(i0)::value; i < decltype(i1)::value; ++i)
      *reinterpret_cast<uint4*>(smem + buf * STAGE + wr_off + i * (THREADS / UNITS) * SB) = st[i];
  };
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, (LOADS + 2) / 3>;
  using C2 = std::integral_constant<int, (2 * LOADS + 2) / 3>;
  using C3 = std::integral_constant<int, LOADS>;

  // Fragment read offsets (bytes within a stage) for q = 0..3.
  const int fr_row = lane & 31;
  const int fr_sw = (fr_row >> 1) & 7;
  int rd_off[NF][4];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int R = f < FM ? (wm * TM + f * 32 + fr_row) : (BM + wn * TN + (f - FM) * 32 + fr_row);
#pragma unroll
    for (int q = 0; q < 4; ++q) rd_off[f][q] = R * SB + 16 * ((2 * q + (lane >> 5)) ^ fr_sw);
  }
  uint4 P[4][NF];
  auto lread = [&](int buf, int q) {
#pragma unroll
    for (int f = 0; f < NF; ++f)
      P[q][f] = *reinterpret_cast<const uint4*>(smem + buf * STAGE + rd_off[f][q]);
  };

  v16i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v16i{0};

  v4i U0[NF], U1[NF];
  // k-step t of a slice uses P[t / 2] dwords (2 * (t % 2), +1).
  auto unpack_step = [&](v4i (&U)[NF], int t) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint4 w = P[t >> 1][f];
      U[f] = (t & 1) ? unpack8(w.z, w.w) : unpack8(w.x, w.y);
    }
  };
  // B first: acc[i][j] accumulates the transposed tile (see the epilogue).
  auto mfma_step = [&](const v4i (&U)[NF]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(U[FM + j], U[i], acc[i][j], 0, 0, 0);
  };
  // Pins the instruction mix of one step: MFMA, a share of the VALU work,
  // MFMA, ...; the closing sched_barrier keeps every step's memory
  // operations inside it.
  constexpr int VPM = (6 * NF + FM * FN - 1) / (FM * FN);  // unpack VALU per MFMA
  auto interleave = [&]() {
#pragma unroll
    for (int k = 0; k < FM * FN; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Row and column metadata of the tile, once per workgroup, loaded between
  // the two slices: a wave's loads complete in issue order, so storing it to
  // LDS before the first barrier waits for slice 0 but not for slice 1.  Every
  // thread loads (indices clamped) so that no load sits behind a branch.
  uint4 G0[LOADS], G1[LOADS];
  gload(G0, 0);
  const int64_t mrow = min(m0 + min(tid, BM - 1), g.arows - 1);
  const int64_t mcol = min(n0 + min(tid, BN - 1), g.brows - 1);
  const float meta_sx = g.sx[mrow], meta_sw = g.sw[mcol];
  const int32_t meta_z = g.zx[mrow], meta_sum = g.sums[mcol];
  const float meta_b =
      BIAS ? (float)static_cast<const OutT*>(g.bias)[min(n0 + min(tid, BN - 1), g.N - 1)] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);
  gload(G1, 1);
  __builtin_amdgcn_sched_barrier(0);
  if (tid < BM) {
    // Staged pre-scaled for the epilogue: sx / 256 and (8 - zx) * 256 (exact).
    lds_sx[tid] = meta_sx * 0.00390625f;
    lds_z[tid] = (float)((8 - meta_z) * 256);
  }
  if (tid < BN) {
    lds_sw[tid] = meta_sw;
    lds_sum[tid] = (float)meta_sum;
    if (BIAS) lds_b[tid] = meta_b;
  }
  lstore(G0, 0, C0{}, C3{});
  lds_barrier();
  lread(0, 0);
  lread(0, 1);
  unpack_step(U0, 0);

  // st_next holds slice s + 1 (loaded during slice s - 1); st_free held
  // slice s, already in LDS, and now receives slice s + 2.
  // FIRST (slice 0 only): the writes of slice 1 move to steps 2-4, so the
  // loop starts as soon as slice 0 has arrived instead of waiting for both.
  auto slice = [&](int s, uint4 (&st_next)[LOADS], uint4 (&st_free)[LOADS], auto first) {
    constexpr bool FIRST = decltype(first)::value;
    const int cbuf = s & 1, nbuf = cbuf ^ 1;
    mfma_step(U0);
    unpack_step(U1, 1);
    gload(st_free, s + 2);
    if (!FIRST) lstore(st_next, nbuf, C0{}, C1{});
    interleave();
    mfma_step(U1);
    unpack_step(U0, 2);
    lread(cbuf, 2);
    if (!FIRST) lstore(st_next, nbuf, C1{}, C2{});
    interleave();
    mfma_step(U0);
    unpack_step(U1, 3);
    if (FIRST) lstore(st_next, nbuf, C0{}, C1{});
    else lstore(st_next, nbuf, C2{}, C3{});
    interleave();
    mfma_step(U1);
    unpack_step(U0, 4);
    lread(cbuf, 3);
    if (FIRST) lstore(st_next, nbuf, C1{}, C2{});
    interleave();
    mfma_step(U0);
    unpack_step(U1, 5);
    if (FIRST) lstore(st_next, nbuf, C2{}, C3{});
    interleave();
    // Slice s + 1 is complete in LDS once every wave passes here; its first
    // fragments (P[0], P[1]: free since step 2) are read over the next two
    // steps.
    lds_barrier();
    lread(nbuf, 0);
    mfma_step(U1);
    unpack_step(U0, 6);
    interleave();
    mfma_step(U0);
    unpack_step(U1, 7);
    lread(nbuf, 1);
    interleave();
    mfma_step(U1);
    unpack_step(U0, 0);
    interleave();
  };
  // The last slice: its fragments only (units 2, 3 read at steps 1, 3); no
  // next slice to load, store, publish or read.
  auto last_slice = [&](int s) {
    const int cbuf = s & 1;
    mfma_step(U0);
    unpack_step(U1, 1);
    interleave();
    mfma_step(U1);
    unpack_step(U0, 2);
    lread(cbuf, 2);
    interleave();
    mfma_step(U0);
    unpack_step(U1, 3);
    interleave();
    mfma_step(U1);
    unpack_step(U0, 4);
    lread(cbuf, 3);
    interleave();
    mfma_step(U0);
    unpack_step(U1, 5);
    interleave();
    mfma_step(U1);
    unpack_step(U0, 6);
    interleave();
    mfma_step(U0);
    unpack_step(U1, 7);
    interleave();
    mfma_step(U1);
  };
  // Slice s + 1 sits in G1 when s is even, in G0 when s is odd.
  int s = 0;
  if (nslices > 1) {
    slice(0, G1, G0, std::true_type{});
    s = 1;
    for (; s + 2 < nslices; s += 2) {
      slice(s, G0, G1, std::false_type{});
      slice(s + 1, G1, G0, std::false_type{});
    }
    if (s + 1 < nslices) {
      slice(s, G0, G1, std::false_type{});
      ++s;
    }
  }
  last_slice(s);
  // The LDS stage of the last slice's neighbour, (s + 1) & 1, is idle: its
  // slice's fragments were read before the barrier every wave passed in
  // slice s - 1, and nothing was written to it since.
  [[maybe_unused]] const int idle_buf = (s + 1) & 1;

  // ---- epilogue.  The MFMAs took B as their first operand, so acc[i][j] is
  // the transposed 32 x 32 tile: output row m, column n sits in lane
  // (m % 32) + 32 * ((n / 4) % 2), register (n % 4) + 4 * (n / 8).  Every lane
  // therefore holds runs of 4 consecutive columns of one row and writes them
  // straight to memory (8 bytes fp16 / 16 bytes fp32).  Operation order of
  // kernel/w4a4.cu:74-77, with the row factors staged as sx / 256 and
  // (8 - zx) * 256 and the column sums as floats: corrected * 256 =
  // fma((8 - zx) * 256, sums, float(acc)) is exact for K <= 65536 (every term
  // is an integer multiple of 256 below 2^31 with at most 24 significant bits:
  // |acc / 256| <= 2^22, |(8 - zx) * sums| <= 2^22, |corrected| <= 2^23), and
  // float(corrected * 256) * (sx / 256) equals float(corrected) * sx exactly
  // (power-of-two scalings).
  // Row and column metadata were staged in LDS before the first barrier of
  // the K loop.
  const int rl = lane & 31;
  const int cq = 4 * (lane >> 5);
  if constexpr (SPLIT) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int64_t row = m0 + wm * TM + i * 32 + rl;
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t c0 = n0 + wn * TN + j * 32 + 8 * q + cq;
          if (row < g.M && c0 < g.N)
            *reinterpret_cast<int4*>(part + row * g.N + c0) =
                make_int4(acc[i][j][4 * q] >> 8, acc[i][j][4 * q + 1] >> 8,
                          acc[i][j][4 * q + 2] >> 8, acc[i][j][4 * q + 3] >> 8);
        }
    }
    return;
  }
  float sxr[FM];
  float zr[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    sxr[i] = lds_sx[wm * TM + i * 32 + rl];
    zr[i] = lds_z[wm * TM + i * 32 + rl];
  }
  float4 swc[FN][4], bc[FN][4];
  float4 sumc[FN][4];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int cl = wn * TN + j * 32 + 8 * q + cq;
      swc[j][q] = *reinterpret_cast<const float4*>(lds_sw + cl);
      sumc[j][q] = *reinterpret_cast<const float4*>(lds_sum + cl);
      if (BIAS) bc[j][q] = *reinterpret_cast<const float4*>(lds_b + cl);
    }
  auto value = [&](int i, int j, int v, float sw, float sum, float b) {
    float res = fmaf(zr[i], sum, (float)acc[i][j][v]) * sxr[i];
    res = res * sw;
    if (BIAS) res = res + b;
    return res;
  };
  OutT* out = static_cast<OutT*>(g.out);
  // fp16 output without raw accumulators: each wave's TM x 64 tile passes
  // through LDS so that a store instruction writes 8 whole 128-byte row
  // segments instead of 16-byte pieces of 32 rows (M=2048, N=4096: 2.1-2.6 us
  // faster at every K; the 16 MiB of output then take ~3.2 us).  Rows in LDS
  // are 128 bytes, 16-byte chunk c of row r stored at c ^ (r & 7), so 8
  // consecutive lanes -- 8 rows on the writes, one row on the reads -- cover
  // all banks.
  if constexpr (sizeof(OutT) == 2 && TN == 64) {
    static_assert(WM * WN * TM * TN * 2 <= 2 * STAGE, "staged tiles fit the slice buffers");
    static_assert(WM * WN * 32 * 128 <= STAGE, "a 32-row group per wave fits one stage");
    if (!g.raw) {
      // Rows i * 32 .. + 31 of the wave's tile into LDS, row i * 32 + r at
      // dst + r * 128.
      auto stage_rows = [&](int i, uint8_t* dst) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 sw = swc[j][q];
            const float4 sm = sumc[j][q];
            const float4 b = bc[j][q];
            uint2 pk;
            pk.x = pack_h2(value(i, j, 4 * q + 0, sw.x, sm.x, b.x),
                           value(i, j, 4 * q + 1, sw.y, sm.y, b.y));
            pk.y = pack_h2(value(i, j, 4 * q + 2, sw.z, sm.z, b.z),
                           value(i, j, 4 * q + 3, sw.w, sm.w, b.w));
            *reinterpret_cast<uint2*>(dst + rl * 128 + 16 * ((4 * j + q) ^ (rl & 7)) +
                                      8 * (lane >> 5)) = pk;
          }
      };
      if constexpr (GATED) {
        // Whole tiles in the slice buffers, once every wave is past the K loop.
        __syncthreads();
        uint8_t* const tile = smem + wave * (TM * TN * 2);
#pragma unroll
        for (int i = 0; i < FM; ++i) stage_rows(i, tile + i * 32 * 128);
        // SiLU-gated MLP (weights interleaved in 64-row blocks: gate rows then
        // up rows of the same 64 outputs): the gate half of the tile's rows
        // is in the LDS tiles of waves (wm, 0), the up half in (wm, 1).  Wave
        // (wm, wn) combines rows wn * TM/2 .. +TM/2 of its row group into
        // h = silu_mul_f16x2(g, u) -- the requantizing kernel's arithmetic --
        // at h columns n0 / 2 .. +63 of the [M, N/2] output.
        static_assert(WN == 2, "gated epilogue: gate in wave column 0, up in column 1");
        __syncthreads();
        const uint8_t* const gate_t = smem + (wm * WN + 0) * (TM * TN * 2);
        const uint8_t* const up_t = smem + (wm * WN + 1) * (TM * TN * 2);
        const int c8 = lane & 7;
        const int64_t NH = g.N / 2;
        const int64_t hcol = n0 / 2 + 8 * c8;
#pragma unroll
        for (int s = 0; s < TM / 16; ++s) {
          const int lr = wn * (TM / 2) + 8 * s + (lane >> 3);
          const int off = lr * 128 + 16 * (c8 ^ (lr & 7));
          const uint4 gv = *reinterpret_cast<const uint4*>(gate_t + off);
          const uint4 uv = *reinterpret_cast<const uint4*>(up_t + off);
          const uint4 hv = make_uint4(silu_mul_f16x2(gv.x, uv.x), silu_mul_f16x2(gv.y, uv.y),
                                      silu_mul_f16x2(gv.z, uv.z), silu_mul_f16x2(gv.w, uv.w));
          const int64_t row = m0 + wm * TM + lr;
          if (row < g.M && hcol < NH) store_stream(hv, out + row * NH + hcol);
        }
        return;
      }
      // One 32-row group at a time through the wave's own 4 KiB of the idle
      // stage (no workgroup barrier: no other wave touches it): the group's
      // stores go out while the next group is converted.  A wave reads back
      // only what its own lanes wrote; the wave-scope fences keep the LDS
      // writes of a group after the reads of the previous one and before its
      // own reads.
      uint8_t* const tile = smem + idle_buf * STAGE + wave * (32 * 128);
      const int c8 = lane & 7;
      const int64_t col = n0 + wn * TN + 8 * c8;
      // A tile inside the output (every tile of a grid whose M and N are
      // multiples of the tile) stores without per-row tests: a wave-uniform
      // row base plus a 32-bit lane offset, all of a group's LDS reads issued
      // before its stores.
      const int wv = __builtin_amdgcn_readfirstlane(wave);
      const bool whole = m0 + BM <= g.M && n0 + BN <= g.N;
      uint8_t* const obase = reinterpret_cast<uint8_t*>(out) +
                             2 * ((m0 + (wv / WN) * TM) * g.N + n0 + (wv % WN) * TN);
      const uint32_t lane_off = (uint32_t)(2 * ((lane >> 3) * g.N + 8 * c8));
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        if (i > 0) {
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          __builtin_amdgcn_wave_barrier();
        }
        stage_rows(i, tile);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        uint4 v[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int lr = 8 * s + (lane >> 3);
          v[s] = *reinterpret_cast<const uint4*>(tile + lr * 128 + 16 * (c8 ^ (lr & 7)));
        }
        if (whole) {
#pragma unroll
          for (int s = 0; s < 4; ++s)
            store_stream(v[s], obase + 2 * (i * 32 + 8 * s) * g.N + lane_off);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const int64_t row = m0 + wm * TM + i * 32 + 8 * s + (lane >> 3);
            if (row < g.M && col < g.N) store_stream(v[s], out + row * g.N + col);
          }
        }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int64_t row = m0 + wm * TM + i * 32 + rl;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t c0 = n0 + wn * TN + j * 32 + 8 * q + cq;
        const float4 sw = swc[j][q];
        const float4 sm = sumc[j][q];
        const float4 b = bc[j][q];
        const float r0 = value(i, j, 4 * q + 0, sw.x, sm.x, b.x);
        const float r1 = value(i, j, 4 * q + 1, sw.y, sm.y, b.y);
        const float r2 = value(i, j, 4 * q + 2, sw.z, sm.z, b.z);
        const float r3 = value(i, j, 4 * q + 3, sw.w, sm.w, b.w);
        if (row < g.M && c0 < g.N) {
          if (sizeof(OutT) == 2) {
            uint2 pk;
            pk.x = pack_h2(r0, r1);
            pk.y = pack_h2(r2, r3);
            *reinterpret_cast<uint2*>(out + row * g.N + c0) = pk;
          } else {
            *reinterpret_cast<float4*>(out + row * g.N + c0) = make_float4(r0, r1, r2, r3);
          }
          if (g.raw)  // the reference's raw-accumulator mode (fused = false)
            *reinterpret_cast<int4*>(g.raw + row * g.N + c0) =
                make_int4(acc[i][j][4 * q] >> 8, acc[i][j][4 * q + 1] >> 8,
                          acc[i][j][4 * q + 2] >> 8, acc[i][j][4 * q + 3] >> 8);
        }
      }
  }
}

template <typename OutT, int BM, int BN, int WM, int WN, int MINB, bool GATED = false>
int launch_pipe_cfg(GemmArgs g, hipStream_t stream) {
  g.tiles_n = (int)((g.N + BN - 1) / BN);
  const int64_t nblocks = ((g.M + BM - 1) / BM) * g.tiles_n;
  if (nblocks > 0x7FFFFFFF) return fail("matmul: grid too large");
  const bool ktail = (g.KP / 2) % 128 != 0;  // rows end inside a 128-byte slice
  const dim3 grid((unsigned)nblocks), block(64 * WM * WN);
#define DSCQ_PIPE(KT, BI)                                                                  \
  launch((w4a4_gemm_pipe_kernel<OutT, BM, BN, WM, WN, MINB, KT, BI, GATED>), grid, block, \
         stream, g)
  if (g.bias) {
    if (ktail) DSCQ_PIPE(true, true); else DSCQ_PIPE(false, true);
  } else {
    if (ktail) DSCQ_PIPE(true, false); else DSCQ_PIPE(false, false);
  }
#undef DSCQ_PIPE
  return launch_status("w4a4_gemm_pipe_kernel");
}

// Tile choice.  256 x 128 tiles (one workgroup per CU, two waves per SIMD)
// move the least data per MFMA and win whenever their rounds of one tile per
// CU are well filled (a whole number of rounds, a last round more than 60%
// full, or a single round over at least 60% of the CUs) and M wastes at most
// an eighth more padded rows than 128-row tiles would (M=128, N=22016: 27.0 us
// on 256-row tiles, 20.2 us on 128-row tiles; M=512, N=11008: 25.9 us on 172
// CUs against 34 us on 128-row tiles over all of them).  Otherwise 128 x 128
// or 64 x 128 tiles, whichever gives the busiest CU fewer rows (ties to the
// larger tile, which moves less data per MFMA): M=320, N=11008 22.6 us on
// 64-row tiles (two per CU) against 28.0 us on 128-row tiles (three on some
// CUs).  A size whose tiles all fit one per CU runs eight waves per tile (two
// per SIMD: one wave per SIMD leaves its LDS and load waits in series with its
// MFMAs), else four waves and two workgroups per CU.  Measured, eight against
// four waves: 64 x 128 at M=64..256, N=K=4096 11.4-11.7 against 12.7 us;
// 128 x 128 at M=384, N=8192 17.7 against 18.7 us.  The gated epilogue needs
// two wave columns, so gated 64-row tiles keep four waves.
template <typename OutT, bool GATED = false>
int launch_pipe(GemmArgs g, hipStream_t stream) {
  const int64_t cus = cu_count();
  const int64_t tn = (g.N + 127) / 128;
  const int64_t rm256 = (g.M + 255) / 256, rm128 = (g.M + 127) / 128, rm64 = (g.M + 63) / 64;
  const int64_t t256 = rm256 * tn, t128 = rm128 * tn, t64 = rm64 * tn;
  const int64_t last = t256 % cus;
  const bool filled =
      (t256 >= cus && (last == 0 || 10 * last > 6 * cus)) || (t256 < cus && 10 * t256 >= 6 * cus);
  if (filled && 8 * (rm256 * 256) <= 9 * (rm128 * 128))
    return launch_pipe_cfg<OutT, 256, 128, 4, 2, 1, GATED>(g, stream);
  const int64_t busiest128 = (t128 + cus - 1) / cus * 128, busiest64 = (t64 + cus - 1) / cus * 64;
  if (busiest128 <= busiest64) {
    if (t128 <= cus) return launch_pipe_cfg<OutT, 128, 128, 4, 2, 2, GATED>(g, stream);
    return launch_pipe_cfg<OutT, 128, 128, 2, 2, 2, GATED>(g, stream);
  }
  if constexpr (!GATED) {
    if (t64 <= cus) return launch_pipe_cfg<OutT, 64, 128, 2, 4, 2>(g, stream);
  }
  return launch_pipe_cfg<OutT, 64, 128, 2, 2, 2, GATED>(g, stream);
}

// Second pass of a K split: adds the int32 parts of four adjacent outputs
// (exact in any order) and applies the epilogue in the pipelined kernel's
// operation order.  N % 8 == 0, so the four columns share a row.
template <typename OutT, bool BIAS>
__global__ __launch_bounds__(256) void w4a4_split_reduce_kernel(GemmArgs g, int parts) {
  const int64_t total = g.M * g.N;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (idx >= total) return;
  const int64_t row = idx / g.N, col = idx - row * g.N;
  int4 r = *reinterpret_cast<const int4*>(g.part + idx);
  for (int p = 1; p < parts; ++p) {
    const int4 v = *reinterpret_cast<const int4*>(g.part + p * total + idx);
    r.x += v.x;
    r.y += v.y;
    r.z += v.z;
    r.w += v.w;
  }
  const int32_t z = 8 - g.zx[row];
  const float sx = g.sx[row];
  const int32_t rv[4] = {r.x, r.y, r.z, r.w};
  float res[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int32_t corrected = rv[c] + __mul24(z, g.sums[col + c]);
    float v = (float)corrected * sx;
    v = v * g.sw[col + c];
    if (BIAS) v = v + (float)static_cast<const OutT*>(g.bias)[col + c];
    res[c] = v;
  }
  OutT* out = static_cast<OutT*>(g.out);
  if constexpr (sizeof(OutT) == 2) {
    uint2 pk;
    pk.x = (uint32_t)__half_as_ushort(to_out<__half>(res[0])) |
           ((uint32_t)__half_as_ushort(to_out<__half>(res[1])) << 16);
    pk.y = (uint32_t)__half_as_ushort(to_out<__half>(res[2])) |
           ((uint32_t)__half_as_ushort(to_out<__half>(res[3])) << 16);
    *reinterpret_cast<uint2*>(out + idx) = pk;
  } else {
    *reinterpret_cast<float4*>(out + idx) = make_float4(res[0], res[1], res[2], res[3]);
  }
  if (g.raw) *reinterpret_cast<int4*>(g.raw + idx) = r;
}

// K split for the 64 x 128 eight-wave pick when its tiles leave most CUs idle
// and K is long (small-batch down projections): one workgroup per CU, parts of
// at least eight slices, at most eight parts, and at least twelve slices saved
// per workgroup so that the saving outweighs the second pass (~2-5 us).
// Measured: M=128, N=4096, K=11008 25.0 -> 19.0 us; where the tiles already
// fill the CUs or K is short, splitting is slower (M=512, N=4096, K=11008
// 29.6 -> 34.3 us with two workgroups per CU; M=256, K=N=4096 12.3 -> 18.8 us).
// 0 when not split.
int split_parts(const GemmArgs& g) {
  const int64_t cus = cu_count();
  const int64_t tn = (g.N + 127) / 128;
  const int64_t t64 = ((g.M + 63) / 64) * tn, t128 = ((g.M + 127) / 128) * tn;
  const int64_t busiest128 = (t128 + cus - 1) / cus * 128, busiest64 = (t64 + cus - 1) / cus * 64;
  if (t64 > cus || busiest128 <= busiest64) return 0;
  const int64_t nsl = (g.KP / 2 + 127) / 128;
  const int64_t parts = std::min<int64_t>(std::min<int64_t>(cus / t64, nsl / 8), 8);
  if (parts < 2) return 0;
  const int64_t ks = (nsl + parts - 1) / parts;
  if (nsl - ks < 12) return 0;
  return (int)((nsl + ks - 1) / ks);  // every part non-empty
}

template <typename OutT>
int launch_pipe_split(GemmArgs g, int parts, int32_t* ws, hipStream_t stream) {
  g.tiles_n = (int)((g.N + 127) / 128);
  g.tiles = (int)(((g.M + 63) / 64) * g.tiles_n);
  const int64_t nsl = (g.KP / 2 + 127) / 128;
  g.kslices = (int)((nsl + parts - 1) / parts);
  g.part = ws;
  const int64_t quads = g.M * g.N / 4;
  if ((quads + 255) / 256 > 0x7FFFFFFF) return fail("matmul: grid too large");
  const bool ktail = (g.KP / 2) % 128 != 0;
  const dim3 grid((unsigned)(g.tiles * parts)), block(512);
  // Timing events armed for this call: the split kernel stamps the start, the
  // reduce kernel the end.
  const KernelEvents ev = take_kernel_events();
  arm_kernel_events({ev.start, nullptr});
  if (ktail)
    launch((w4a4_gemm_pipe_kernel<OutT, 64, 128, 2, 4, 2, true, false, false, true>),
                       grid, block, stream, g);
  else
    launch((w4a4_gemm_pipe_kernel<OutT, 64, 128, 2, 4, 2, false, false, false, true>),
                       grid, block, stream, g);
  const int rc = launch_status("w4a4_gemm_pipe_kernel");
  if (rc) return rc;
  const dim3 rgrid((unsigned)((quads + 255) / 256)), rblock(256);
  arm_kernel_events({nullptr, ev.stop});
  if (g.bias)
    launch((w4a4_split_reduce_kernel<OutT, true>), rgrid, rblock, stream, g, parts);
  else
    launch((w4a4_split_reduce_kernel<OutT, false>), rgrid, rblock, stream, g, parts);
  return launch_status("w4a4_split_reduce_kernel");
}

int64_t split_workspace_bytes(const GemmArgs& g) {
  const int parts = split_parts(g);
  return parts >= 2 ? (int64_t)parts * g.M * g.N * 4 : 0;
}

// The pipelined kernel, split over K when a workspace (16-byte aligned, large
// enough) was given and the shape asks for it.
template <typename OutT>
int launch_pipe_ws(const GemmArgs& g, int32_t* ws, int64_t ws_bytes, hipStream_t stream) {
  if (ws && (reinterpret_cast<uintptr_t>(ws) & 15) == 0) {
    const int64_t need = split_workspace_bytes(g);
    if (need > 0 && ws_bytes >= need) return launch_pipe_split<OutT>(g, split_parts(g), ws, stream);
  }
  return launch_pipe<OutT>(g, stream);
}

template <typename OutT, int BM, int BN, int WM, int WN, bool HUGE>
int launch_cfg(GemmArgs g, hipStream_t stream) {
  g.tiles_n = (int)((g.N + BN - 1) / BN);
  const int64_t tiles_m = (g.M + BM - 1) / BM;
  const int64_t nblocks = tiles_m * g.tiles_n;
  if (nblocks > 0x7FFFFFFF) return fail("matmul: grid too large (M=%lld, N=%lld)",
                                        (long long)g.M, (long long)g.N);
  launch((w4a4_gemm_kernel<OutT, BM, BN, WM, WN, HUGE>), dim3((unsigned)nblocks),
                     dim3(64 * WM * WN), stream, g);
  return launch_status("w4a4_gemm_kernel");
}

// ------------------------------------------------------ skinny-M kernel
// M <= 16 (decode) or force_decode: the weights are streamed once and the
// work is split over K instead of M.  A workgroup owns 16 output columns
// (B rows) and 16 output rows of A; its 8 waves take consecutive slices of
// K.  Per 64-byte block of a row (128 nibbles) lane l loads 16 bytes of A
// row l % 16 and of B row l % 16 at byte 16 * (l / 16); their low / high
// halves feed two v_mfma_i32_16x16x64_i8 (A and B use the same k order).
// Partial 16 x 16 sums meet in LDS; the epilogue is the reference's.
// Bytes per launch: N * KP / 2 (weights) + the small A, read once per column
// block from L2.
// Where the grid would take two or more rounds over the CUs, a workgroup
// owns two or three tiles of 16 columns and loads its A pieces once for them.
// GATED (dscq_matmul_silu_mul at M <= 16): output column n of h [M, N / 2]
// takes weight row 128 (n / 64) + n % 64 (gate) and that row + 64 (up); both
// are streamed by the same workgroup and combined in the epilogue with the
// gated epilogue's silu_mul_f16x2.
// NT > 1 (not gated): the workgroup owns NT tiles of 16 columns, n0 + 16 t,
// each wave's A pieces loaded once and used for all of them.
template <typename OutT, bool BIAS, bool GATED = false, int NT = 1>
__global__ __launch_bounds__(512) void w4a4_gemv_kernel(GemmArgs g) {
  constexpr int WAVES = 8;
  static_assert(!GATED || NT == 1, "the gated form owns one tile");
  constexpr int NB = GATED ? 2 : NT;  // weight row streams (gate, up / the tiles)
  __shared__ int32_t part[NB][WAVES][16][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 16 * NT, m0 = (int64_t)blockIdx.y * 16;
  const int r = lane & 15, grp = lane >> 4;
  const int64_t KB = g.KP / 2;
  const int64_t nblk = (KB + 63) / 64;
  const int64_t per = (nblk + WAVES - 1) / WAVES;
  const int64_t b0 = wave * per, b1 = min(b0 + per, nblk);
  const int64_t NOUT = GATED ? g.N / 2 : g.N;  // output columns
  // Weight row of stream s for output column n of tile 0 (gated: gate / up
  // row; else the row of tile s, 16 s columns on).
  auto wrow = [&](int64_t n, int s) -> int64_t {
    return GATED ? 128 * (n / 64) + n % 64 + 64 * s : n + 16 * s;
  };
  const uint8_t* arow = g.a + min(m0 + r, g.arows - 1) * KB;
  const uint8_t* brow[NB];
#pragma unroll
  for (int s = 0; s < NB; ++s) brow[s] = g.b + min(wrow(n0 + r, s), g.brows - 1) * KB;
  const int64_t off = grp * 16;

  // Epilogue operands of output (m0 + tid / 16 % 16, n0 + tid % 16), fetched
  // up front by every thread (indices clamped; only threads < 256 use them) so
  // that the epilogue does not wait for a second trip to memory.
  const int ml = (tid >> 4) & 15, nl = tid & 15;
  const int64_t mc = min(m0 + ml, g.arows - 1), nout = min(n0 + nl, NOUT - 1);
  const float e_sx = g.sx[mc];
  const int32_t e_z = 8 - g.zx[mc];
  float e_sw[NB], e_b[NB];
  int32_t e_sum[NB];
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    const int64_t nc = min(GATED ? wrow(nout, s) : n0 + 16 * s + nl, g.brows - 1);
    e_sw[s] = g.sw[nc];
    e_sum[s] = g.sums[nc];
    e_b[s] = BIAS ? (float)static_cast<const OutT*>(
                        g.bias)[min(GATED ? wrow(nout, s) : n0 + 16 * s + nl, g.N - 1)]
                  : 0.0f;
  }

  v4i acc[NB];
  int32_t tot[NB][4];
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    acc[s] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int v = 0; v < 4; ++v) tot[s][v] = 0;
  }
  auto piece = [&](const uint8_t* row, int64_t kb) {
    // The last block of a row with KB % 64 == 32 is half empty: its upper
    // pieces re-read the row's last piece and are zeroed.
    const bool in = kb + off < KB;
    uint4 v = *reinterpret_cast<const uint4*>(row + (in ? kb + off : KB - 16));
    if (!in) v = make_uint4(0u, 0u, 0u, 0u);
    return v;
  };
  auto mfma2 = [&](const uint4& a4, const uint4& b4, v4i& c) {
    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack8(a4.x, a4.y), unpack8(b4.x, b4.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack8(a4.z, a4.w), unpack8(b4.z, b4.w), c, 0, 0, 0);
  };
  constexpr int U = 4;  // blocks in flight per wave
  int64_t blk = b0;
  for (; blk + U <= b1; blk += U) {
    uint4 av[U], bv[NB][U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      av[i] = piece(arow, (blk + i) * 64);
#pragma unroll
      for (int s = 0; s < NB; ++s) bv[s][i] = piece(brow[s], (blk + i) * 64);
    }
#pragma unroll
    for (int i = 0; i < U; ++i)
#pragma unroll
      for (int s = 0; s < NB; ++s) mfma2(av[i], bv[s][i], acc[s]);
    // |partial| <= 2^14 per product: drain every 65536 k (512 blocks).
    if (((blk - b0) / U + 1) % (512 / U) == 0) {
#pragma unroll
      for (int s = 0; s < NB; ++s) {
#pragma unroll
        for (int v = 0; v < 4; ++v) tot[s][v] += acc[s][v] >> 8;
        acc[s] = v4i{0, 0, 0, 0};
      }
    }
  }
  for (; blk < b1; ++blk) {
    const uint4 a4 = piece(arow, blk * 64);
#pragma unroll
    for (int s = 0; s < NB; ++s) mfma2(a4, piece(brow[s], blk * 64), acc[s]);
  }
  // D of a 16 x 16 tile: row (A) 4 * (lane / 16) + v, column (B) lane % 16.
#pragma unroll
  for (int s = 0; s < NB; ++s)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[s][wave][4 * grp + v][r] = tot[s][v] + (acc[s][v] >> 8);
  __syncthreads();
  if (tid >= 256) return;
  int32_t raw[NB];
  float res[NB];
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    raw[s] = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) raw[s] += part[s][w][ml][nl];
    // Operation order of kernel/w4a4.cu:74-77.
    const int32_t corrected = raw[s] + e_z * e_sum[s];
    res[s] = (float)corrected * e_sx;
    res[s] = res[s] * e_sw[s];
    if (BIAS) res[s] = res[s] + e_b[s];
  }
  const int64_t m = m0 + ml, n = n0 + nl;
  if (m >= g.M) return;
  if constexpr (GATED) {
    if (n >= NOUT) return;
    const uint32_t gb = __half_as_ushort(to_out<__half>(res[0]));
    const uint32_t ub = __half_as_ushort(to_out<__half>(res[1]));
    static_cast<uint16_t*>(g.out)[m * NOUT + n] = (uint16_t)(silu_mul_f16x2(gb, ub) & 0xFFFFu);
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t nt = n + 16 * t;
      if (nt >= g.N) break;
      static_cast<OutT*>(g.out)[m * g.N + nt] = to_out<OutT>(res[t]);
      if (g.raw) g.raw[m * g.N + nt] = raw[t];
    }
  }
}

template <typename OutT, bool GATED = false>
int launch_gemv(GemmArgs g, hipStream_t stream) {
  const int64_t tiles = ((GATED ? g.N / 2 : g.N) + 15) / 16, gy = (g.M + 15) / 16;
  // Tiles per workgroup as in the fused decode kernel: up to three tiles per
  // CU in one round, two beyond.  Quantize + this kernel, graph-replayed,
  // weights from HBM, one tile / NT: M = 8, N = 11008 11.07 / 10.81 us (two
  // tiles: 12.25); M = 16, N = 11008 12.56 / 11.25; M = 16, N = 14336 14.93 /
  // 13.37; M = 8, N = 28672 19.3 / 18.8; M = 32, N = 4096 9.92 / 9.21.
  const int64_t cus = cu_count(), per_cu = (tiles * gy + cus - 1) / cus;
  const int nt = GATED ? 1 : per_cu > 3 ? 2 : (int)std::max<int64_t>(1, per_cu);
  const int64_t gx = (tiles + nt - 1) / nt;
  if (gx > 0x7FFFFFFF || gy > 65535) return fail("matmul: grid too large");
  const dim3 grid((unsigned)gx, (unsigned)gy), block(512);
#define DSCQ_GEMV(NTV)                                                            \
  if (g.bias)                                                                     \
    launch((w4a4_gemv_kernel<OutT, true, GATED, NTV>), grid, block, stream, g);   \
  else                                                                            \
    launch((w4a4_gemv_kernel<OutT, false, GATED, NTV>), grid, block, stream, g);
  if constexpr (GATED) {
    DSCQ_GEMV(1)
  } else {
    if (nt == 1) {
      DSCQ_GEMV(1)
    } else if (nt == 2) {
      DSCQ_GEMV(2)
    } else {
      DSCQ_GEMV(3)
    }
  }
#undef DSCQ_GEMV
  return launch_status("w4a4_gemv_kernel");
}

// The pipelined kernel's layout requirements: whole 8-column groups, 16-byte
// aligned output and raw rows, 32-bit row offsets.
bool pipe_layout_ok(const GemmArgs& g) {
  auto al = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; };
  const int64_t KB = g.KP / 2;
  return g.N % 8 == 0 && al(g.out, 16) && al(g.raw, 16) && g.arows * KB <= 0xFFFFFFFFll &&
         g.brows * KB <= 0xFFFFFFFFll;
}
bool pipe_ok(const GemmArgs& g) { return g.M >= 64 && pipe_layout_ok(g); }
// 16 < M < 64 with N / 128 >= 64 tiles: the pipelined kernel over the skinny-M
// one (its eight-wave 64 x 128 tiles; measured at N=11008, K=4096: M=20..32
// 10.8-11.0 against 11.8-12.8 us, M=40..56 11.1-11.4 against 17.0-21.2 us; at
// N <= 4096 the skinny-M kernel stays ahead).  The gated GEMM keeps M > 32: its
// 64-row tiles run four waves.
bool use_pipe_mid_m(const GemmArgs& g, bool gated = false) {
  return g.M > (gated ? 32 : 16) && g.M < 64 && (g.N + 127) / 128 >= 64 && g.KP <= 65536 &&
         pipe_layout_ok(g);
}

// The wide-tile kernel (gemm_wide.hip) for fp16 output without raw
// accumulators: its tile width (256 or 128), or 0 for another kernel.
// 256 x 256 tiles (or as dscq_set_gemm_kernel forces) when they fill at least
// three quarters of a round of one tile per CU and their rounds, each worth 1.8
// rounds of the pipelined kernel's 256 x 128 tiles (the wide kernel does the
// same work ~10% faster), take no longer.  Measured in steps, pipelined /
// wide: 4096 x 4096 x 4096 (256 tiles) 56.4 / 54.6 us; 3584 x 4096 x 4096 (224)
// 51.9 / 48.9; 4096 x 11008 x 4096 (688) 168.8 / 149.6; 1024 x 16384 x 8192
// 104.5 / 92.5; 3072 x 8192 x 8192 (384: three full pipelined rounds) 155.5 /
// 166.6; 2048 x 4096 x 4096 (128) 28.7 / 43.4.
int use_wide(const GemmArgs& g, bool out_half) {
  const int pref = gemm_kernel_preference();
  if (pref == 2 || !out_half || g.M < 64 || !wide_gemm_fits(g)) return 0;
  if (pref == 3) return 256;
  if (pref == 4) return 128;
  const int64_t cus = cu_count();
  const int64_t rows = (g.M + 255) / 256;
  const int64_t t256 = rows * ((g.N + 255) / 256), t128 = rows * ((g.N + 127) / 128);
  const int64_t wide_rounds = (t256 + cus - 1) / cus, pipe_rounds = (t128 + cus - 1) / cus;
  if (g.M >= 256 && 4 * t256 >= 3 * cus && 18 * wide_rounds <= 10 * pipe_rounds) return 256;
  return pref == 1 ? 256 : 0;
}

// The gated GEMM of dscq_matmul_silu_mul on the wide-tile kernel (256 x 256
// tiles; each wave's 128 columns are the gate and up rows of 64 outputs), by
// the rule of use_wide; preferences 1 and 3 take it wherever it applies, 2
// and 4 never.  Gated GEMM alone, graph-replayed, identical h, pipelined /
// wide (M x N/2, K = 4096 unless noted): 512 x 14336 55.4-62.4 / 49.6-53.2
// us; 2048 x 11008 176.5-199.2 / 154.0-160.2; 4096 x 11008 312-331 /
// 294-304; 2048 x 28672, K = 8192 688-714 / 621-631; left to the pipelined
// kernel by the rule: 512 x 11008 49.9-53.6 / 49.1-51.5; 1024 x 11008
// 85.6-97.6 / 98.1-99.6; 256 x 11008 25.9-27.8 / 44.6-46.3.
bool use_wide_gated(const GemmArgs& g) {
  return g.N % 128 == 0 && use_wide(g, true) == 256;
}

template <typename OutT>
int gemm_typed(const GemmArgs& g, bool decode, int32_t* ws, int64_t ws_bytes,
               hipStream_t stream) {
  if (decode || g.M <= 16) return launch_gemv<OutT>(g, stream);
  // 16 < M < 64: the skinny-M kernel streams the weights once per 16 rows but
  // keeps every CU busy; the pipelined kernel's 64-row tiles pay off once N
  // gives 64+ tiles (measured, M = 20..56: N = K = 4096 skinny 6.3-9.0 us vs
  // pipelined 10.7-11.3 us; N = 11008, K = 4096 pipelined 10.8-11.4 us vs
  // skinny 11.8-21.2 us).
  if (g.M < 64) {
    if (use_pipe_mid_m(g)) return launch_pipe_ws<OutT>(g, ws, ws_bytes, stream);
    return launch_gemv<OutT>(g, stream);
  }
  // M >= 64 with few weight rows: the pipelined kernel's single round of tiles
  // takes its serial K loop (~11 us at K = 4096) whatever the size, while the
  // skinny-M kernel streams the weights once per 16 rows over every CU, so it
  // stays ahead while ceil(M/16) * N is small (measured at K = 4096: N = 1024,
  // M = 64..160 6.1-7.5 us against 11.1 us; N = 2048, M = 64..96 6.3-7.5 us
  // against 11.3 us; N = 4096, M = 64 9.3 against 11.4 us, M = 96 13.0 against
  // 11.2 us).  Shorter rows keep the pipelined kernel (not measured there).
  // (The wide-tile kernel's own rule never meets the skinny one; checked
  // first so that a forced choice covers every M >= 64.)
  if (const int bn = use_wide(g, sizeof(OutT) == 2)) return launch_wide_gemm(g, bn, stream);
  if (g.KP >= 4096 && g.KP <= 65536 && (g.M + 15) / 16 * g.N <= 16384)
    return launch_gemv<OutT>(g, stream);
  if (g.KP > 65536) return launch_cfg<OutT, 64, 64, 2, 2, true>(g, stream);
  if (pipe_ok(g)) return launch_pipe_ws<OutT>(g, ws, ws_bytes, stream);
  const int64_t big_tiles = ((g.M + 127) / 128) * ((g.N + 255) / 256);
  if (big_tiles >= 192) return launch_cfg<OutT, 128, 256, 2, 2, false>(g, stream);
  return launch_cfg<OutT, 128, 128, 2, 2, false>(g, stream);
}

// Whether gemm_typed takes the pipelined kernel (the one that may split K).
bool takes_pipe(const GemmArgs& g, bool decode, bool out_half) {
  if (decode || g.M <= 16) return false;
  if (g.M < 64) return use_pipe_mid_m(g);
  if (use_wide(g, out_half)) return false;
  if (g.KP >= 4096 && g.KP <= 65536 && (g.M + 15) / 16 * g.N <= 16384) return false;
  if (g.KP > 65536) return false;
  return pipe_ok(g);
}

}  // namespace

int64_t w4a4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t KP, bool decode) {
  GemmArgs g;
  g.a = g.b = nullptr;
  g.sx = g.sw = nullptr;
  g.zx = g.sums = nullptr;
  g.bias = nullptr;
  g.out = nullptr;
  g.raw = nullptr;
  g.M = M;
  g.N = N;
  g.KP = KP;
  g.arows = ceil_to(M, 8);
  g.brows = ceil_to(N, 8);
  g.tiles_n = 0;
  // The query has no output dtype: shapes the wide-tile kernel takes (fp16)
  // make so many tiles that the pipelined kernel would not split them either.
  return takes_pipe(g, decode, false) ? split_workspace_bytes(g) : 0;
}

int w4a4_gemm(const uint8_t* a, const uint8_t* b, const float* sx, const int32_t* zx,
              const float* sw, const int32_t* sums, const void* bias, int64_t M,
              int64_t N, int64_t KP, bool decode, bool out_fp32, void* out,
              int32_t* raw, hipStream_t stream, int32_t* ws, int64_t ws_bytes) {
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
  return out_fp32 ? gemm_typed<float>(g, decode, ws, ws_bytes, stream)
                  : gemm_typed<__half>(g, decode, ws, ws_bytes, stream);
}

// The gated GEMM's shape requirements (the caller reports them): h columns a
// multiple of 64, KP <= 65536 (the pipelined kernel's accumulator range),
// 32-bit row offsets, 16-byte aligned h.
bool gemm_silu_mul_fits(int64_t M, int64_t NH, int64_t KP, const void* h) {
  const int64_t KB = KP / 2;
  return M >= 1 && NH >= 64 && NH % 64 == 0 && KP >= 64 && KP % 64 == 0 && KP <= 65536 &&
         ceil_to(M, 8) * KB <= 0xFFFFFFFFll && 2 * NH * KB <= 0xFFFFFFFFll &&
         (reinterpret_cast<uintptr_t>(h) & 15) == 0;
}

// h[M, NH] = fp16(fp16(silu(g)) * u) of the gate and up projections of one
// SiLU-gated MLP, from one GEMM against b_gu: 2 * NH packed weight rows
// interleaved in 64-row blocks (block t: gate rows 64t..64t+63, then up rows
// 64t..64t+63), with sw, sums (and bias, fp16, when given) in the same order.
int w4a4_gemm_silu_mul(const uint8_t* a, const uint8_t* b_gu, const float* sx,
                       const int32_t* zx, const float* sw, const int32_t* sums,
                       const void* bias, int64_t M, int64_t NH, int64_t KP, void* h,
                       hipStream_t stream) {
  GemmArgs g;
  g.a = a;
  g.b = b_gu;
  g.sx = sx;
  g.zx = zx;
  g.sw = sw;
  g.sums = sums;
  g.bias = bias;
  g.out = h;
  g.raw = nullptr;
  g.M = M;
  g.N = 2 * NH;
  g.KP = KP;
  g.arows = ceil_to(M, 8);
  g.brows = 2 * NH;
  g.tiles_n = 0;
  // Few tokens: the skinny-M kernel streams each weight row once; up to 64
  // rows it keeps doing so unless the pipelined kernel has 64+ tiles (as for
  // dscq_matmul).
  if (M <= 16 || (M < 64 && !use_pipe_mid_m(g, true))) return launch_gemv<__half, true>(g, stream);
  if (use_wide_gated(g)) return launch_wide_gemm_gated(g, stream);
  return launch_pipe<__half, true>(g, stream);
}

}  // namespace dscq
