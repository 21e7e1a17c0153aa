// Row quantization kernels for gfx950: per-token asymmetric activation codes
// and per-channel symmetric weight codes, optionally preceded by the online
// block-Hadamard rotation, with int4 nibble packing.
//
// Rules restated (reference paths):
//   activations  core/quantization.py:13-21, kernel/w4a4.cu:20-54
//   weights      core/quantization.py:7-11, pack_int4 :31-40
//   rotation     the fold rule of core/linear.py:34-37 with R = H_128/sqrt(128)
//                split as (W H/128)(H x): activations get the unnormalised
//                Sylvester transform, weights the exact 1/128 scale.
//
// Work layout.  A row of K elements is cut into 128-element blocks.  Four
// lanes (a "quad") own a block: lane r of the quad holds four 8-element
// chunks j = 0..3 at block offsets j*32 + r*8, each chunk fetched with one
// 16-byte load (fp16).  Block index bits 0-2 are therefore in-chunk, bits 3-4
// are the lane within the quad and bits 5-6 are the chunk: the transform's
// seven butterfly stages run as 3 in-register + 2 DPP quad_perm + 2
// in-register stages, and a load instruction of the wave reads 16 quads x 64
// contiguous bytes.  A row is spread over WPR waves (16*WPR quads), each quad
// taking blocks quad, quad + 16*WPR, ... up to ITERS of them; the whole row
// stays in VGPRs, so x is read from HBM exactly once.  The packed codes of a
// wave's 16 blocks pass through LDS on the way out, so that each lane stores
// 16 contiguous bytes.  Rows longer than the register capacity use the
// two-pass streaming kernel at the end; up to 512 activation rows of at most
// 96 blocks (decode and small batches) take the few-row kernel, a block over
// 16 lanes instead of 4.
//
// The per-element rules and the exactness argument of the fast division are
// in rowquant.h.

#include <cstdio>
#include <cstdlib>

#include "../../include/dscq.h"
#include "common.h"
#include "rowquant.h"

namespace dscq {
namespace {

constexpr int kThreads = 256;
// Rows up to which activations of at most 96 blocks take the few-row kernel.
// Graph-replayed, K = 4096 with rotation, identical codes, register kernel /
// few-row kernel: 1 row 2.63 / 2.28 us, 16 rows 3.05 / 2.50, 64 3.57 / 2.96,
// 256 3.84 / 3.29, 512 4.30 / 4.08, 1024 5.77 / 5.80.
// Up to three passes of 32 blocks (K <= 12288): 16 x 11008 4.17 -> 3.55 us,
// 128 x 12288 4.78 -> 4.30, 512 x 11008 7.28 -> 6.87, 64 x 8192 3.72 -> 3.44;
// 512 x 8192 equal (5.74 / 5.76).
constexpr int64_t kSpreadMaxRows = 512;
constexpr int kSpreadMaxPasses = 3;
// Rows from which the few-row kernel computes each row's scale in one wave and
// shares it (RowArgs::share_scale).  Graph-replayed, rotation 128, identical
// codes, every wave / one wave: 512 x 4096 3.84-4.03 / 3.68-3.90 us, 512 x
// 11008 6.63-6.70 / 6.46-6.51; 8-256 rows equal within 0.05 us (the decode
// step at 8 rows measured 2% slower with the extra barrier, so fewer rows
// keep the per-wave form).
constexpr int64_t kShareScaleRows = 128;

struct RowArgs {
  const void* x;       // [M, K] T
  int64_t M, K, KP, MP;
  int nblk;            // ceil(KP / 128)
  float clip;
  float qmax;          // act: 2^bits - 1;  weight: 2^(bits-1) - 1
  uint8_t* packed;     // [MP, KP/2] or null
  uint8_t* codes;      // [MP, KP] or null (u8 act codes / int8 weight codes)
  float* scales;       // [MP]
  int32_t* zeros;      // [MP] act zero-points or null
  int32_t* sums;       // [MP] weight code sums or null
  int vec;             // rows 16-byte aligned and K % 8 == 0
  int share_scale = 0; // few-row kernel: one wave computes the row scale for all
  int64_t ldx;         // elements between consecutive rows of x (and up)
  const void* up;      // gated input: up [M, ldx] fp16, or null
  __half* hout;        // gated input: the activation h [M, K] fp16, or null
};


// Outputs of one chunk: packed nibbles and / or codes.  Byte i of ev / od is
// u = q (activations) or u = c + qmax + 1 (weights) for element 2i / 2i + 1.
template <int MODE>
__device__ __forceinline__ void store_codes(const RowArgs& a, int64_t row, int64_t e0,
                                            uint32_t ev, uint32_t od);

// Packed nibbles of 8 codes: act: (q - 8) & 15 == q ^ 8;  weight: c & 15 == (c + 8) ^ 8.
__device__ __forceinline__ uint32_t packed_nibbles(uint32_t ev, uint32_t od) {
  return (ev | (od << 4)) ^ 0x88888888u;
}

template <int MODE>
__device__ __forceinline__ void store_chunk(const RowArgs& a, int64_t row,
                                            int64_t e0, uint32_t ev, uint32_t od) {
  if (e0 >= a.KP) return;
  if (a.packed)
    *reinterpret_cast<uint32_t*>(a.packed + row * (a.KP / 2) + e0 / 2) = packed_nibbles(ev, od);
  if (a.codes) store_codes<MODE>(a, row, e0, ev, od);
}

// The 8 codes unpacked, one byte each (the reference's two-step mode).
template <int MODE>
__device__ __forceinline__ void store_codes(const RowArgs& a, int64_t row, int64_t e0,
                                            uint32_t ev, uint32_t od) {
  uint32_t lo = __builtin_amdgcn_perm(od, ev, 0x05010400u);
  uint32_t hi = __builtin_amdgcn_perm(od, ev, 0x07030602u);
  if (MODE == kWgt) {
    // Per byte (no borrow between bytes): int8 code = u - (qmax + 1).
    const uint32_t off = (uint32_t)(a.qmax + 1.0f);
    uint32_t l2 = 0, h2 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      l2 |= ((((lo >> (8 * i)) & 0xFFu) - off) & 0xFFu) << (8 * i);
      h2 |= ((((hi >> (8 * i)) & 0xFFu) - off) & 0xFFu) << (8 * i);
    }
    lo = l2;
    hi = h2;
  }
  uint2 w;
  w.x = lo;
  w.y = hi;
  *reinterpret_cast<uint2*>(a.codes + row * a.KP + e0) = w;
}

template <int MODE>
__device__ __forceinline__ void write_row_meta(const RowArgs& a, int64_t row, bool real,
                                               const RowScale& rs, int sum) {
  if (MODE == kAct) {
    a.scales[row] = rs.scale;
    if (a.zeros) a.zeros[row] = (int32_t)rs.zf;
  } else {
    // Padded weight rows carry scale 0 and sum 0.
    a.scales[row] = real ? rs.scale : 0.0f;
    if (a.sums) a.sums[row] = real ? sum : 0;
  }
}

// FIT describes how the row fills the blocks the quads walk:
//   kFull   every quad has a whole block in every iteration (K == nblk * 128
//           == 16 * WPR * ITERS * 128): no masking and no per-iteration tests;
//   kWhole  K == nblk * 128, so every 128-block is complete, but the quads
//           walk past the row's last block.  Those blocks are handled per
//           iteration at wave granularity: an iteration none of whose quads
//           has a block skips its arithmetic and stores (a uniform branch);
//           one whose quads are partly past the row zeroes those quads' chunks;
//   kPart   the last block is partial as well: every iteration is masked.
// CLAMP (activations): 0 when clip == 1 and qmax == 15, whose codes need no
// clamp (act_chunk_fast_noclamp), else 1.
// Gated input (the SiLU-gated MLP between its up and down projections): the
// row is h = silu_mul_f16x2(g, u) (rowquant.h) of two fp16 rows g (x) and u (up).
// TPB: threads per workgroup, (TPB / 64) / WPR rows per workgroup.

enum Fit { kPart = 0, kWhole = 1, kFull = 2 };

template <typename T, bool ROT, int MODE, int WPR, int ITERS, int FIT, int CLAMP,
          bool GATED = false, int TPB = kThreads>
__global__ __launch_bounds__(TPB) void row_quant_kernel(RowArgs a) {
  constexpr bool WHOLE = FIT != kPart, FULL = FIT == kFull;
  constexpr int ROWS = (TPB / 64) / WPR;
  constexpr int NQ = 16 * WPR;
  const int lane = threadIdx.x & 63;
  // Wave-uniform values in scalar registers: the row's base address is then
  // the scalar base of every load and store of the wave.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row_in_wg = wave / WPR;
  const int wave_in_row = wave % WPR;
  const int64_t row = (int64_t)blockIdx.x * ROWS + row_in_wg;
  const bool live = row < a.MP;
  const bool real = row < a.M;
  const int quad = wave_in_row * 16 + (lane >> 2);
  const int r = lane & 3;
  const T* xrow = static_cast<const T*>(a.x) + (real ? row : 0) * a.ldx;

  // Per iteration, uniform over the wave: does any quad have a block (wlive),
  // and are some quads past the row (wmix)?  Padded rows compute nothing.
  bool wlive[ITERS], wmix[ITERS];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int first = wave_in_row * 16 + it * NQ;
    wlive[it] = real && (FULL || first < a.nblk);
    wmix[it] = !FULL && first + 15 >= a.nblk;
  }
  auto quad_ok = [&](int it, int j) {
    const int b = quad + it * NQ;
    const int64_t e0 = (int64_t)b * 128 + j * 32 + r * 8;
    return FULL || (b < a.nblk && (WHOLE || e0 < a.K));
  };

  // Rows of this kernel are 16-byte aligned with K % 8 == 0 (see row_quant).
  // Loads are unconditional (out-of-range chunks read element 0 of the row),
  // so every load of a lane is in flight at once.
  Raw<T> raw[ITERS][4];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    const int b = quad + it * NQ;
#pragma unroll
    for (int j = 0; j < 4; ++j) raw[it][j] = load_raw32<T>(xrow, b * 128 + j * 32 + r * 8, quad_ok(it, j));
  }
  if (GATED) {
    static_assert(!GATED || sizeof(T) == 2, "gated rows are fp16");
    const T* urow = static_cast<const T*>(a.up) + (real ? row : 0) * a.ldx;
    Raw<T> rup[ITERS][4];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int b = quad + it * NQ;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        rup[it][j] = load_raw32<T>(urow, b * 128 + j * 32 + r * 8, quad_ok(it, j));
    }
#pragma unroll
    for (int it = 0; it < ITERS; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t* w = reinterpret_cast<uint32_t*>(&raw[it][j]);
        const uint32_t* wu = reinterpret_cast<const uint32_t*>(&rup[it][j]);
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = silu_mul_f16x2(w[k], wu[k]);
      }
  }

  float v[ITERS][4][8];
  float mn = 0.0f, mx = 0.0f;
  // Lane sign after the signed transform (values held are lsign * y).
  const float lsign = (ROT && (r == 1 || r == 2)) ? -1.0f : 1.0f;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    if (!wlive[it]) continue;
    // Zero the chunks loaded from the placeholder address.
    if (!WHOLE || wmix[it]) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool ok = quad_ok(it, j);
        uint32_t* w = reinterpret_cast<uint32_t*>(&raw[it][j]);
#pragma unroll
        for (int k = 0; k < (int)(sizeof(Raw<T>) / 4); ++k) w[k] = ok ? w[k] : 0u;
      }
    }
    if (GATED && a.hout) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t e0 = (int64_t)(quad + it * NQ) * 128 + j * 32 + r * 8;
        if (quad_ok(it, j))
          *reinterpret_cast<uint4*>(a.hout + row * a.K + e0) =
              *reinterpret_cast<const uint4*>(&raw[it][j]);
      }
    }
    if (ROT && sizeof(T) == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&raw[it][j]);
#pragma unroll
        for (int k = 0; k < 4; ++k) bfly_f16x2(w[k], v[it][j][2 * k], v[it][j][2 * k + 1]);
        fwht_chunk_tail(v[it][j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        to_f32(raw[it][j], v[it][j]);
        if (ROT) fwht_chunk(v[it][j]);
      }
    }
    if (ROT) {
      fwht_block_tail_signed(v[it], r);
      if (MODE == kWgt) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i) v[it][j][i] *= 0.0078125f;  // 1/128, exact
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (MODE == kAct) {
          mn = fminf(mn, v[it][j][i]);
          mx = fmaxf(mx, v[it][j][i]);
        } else {
          mx = fmaxf(mx, fabsf(v[it][j][i]));
        }
      }
  }
  if (MODE == kAct && ROT) {
    // Undo the lane sign: min / max of -y are -max / -min of y.
    const float mn_l = mn, mx_l = mx;
    mn = lsign > 0.0f ? mn_l : -mx_l;
    mx = lsign > 0.0f ? mx_l : -mn_l;
  }
  if (MODE == kAct) mn = wave_min(mn);
  mx = wave_max(mx);
  RowScale rs;
  if (WPR > 1) {
    __shared__ float red[2][TPB / 64];
    if (lane == 0) {
      red[0][wave] = mn;
      red[1][wave] = mx;
    }
    __syncthreads();
    auto fold = [&]() {
      mn = red[0][row_in_wg * WPR];
      mx = red[1][row_in_wg * WPR];
#pragma unroll
      for (int w = 1; w < WPR; ++w) {
        mn = fminf(mn, red[0][row_in_wg * WPR + w]);
        mx = fmaxf(mx, red[1][row_in_wg * WPR + w]);
      }
    };
    if constexpr (MODE == kAct) {
      // The row's first wave folds the statistics and computes the scale,
      // zero point, reciprocal and guard (two IEEE divisions, ~50 VALU
      // instructions) once for the row; the other waves read them, leaving
      // their SIMDs to other rows' waves meanwhile.  Same values as every
      // wave computing them: the same inputs in the same order.
      __shared__ float rsh[ROWS][4];
      if (wave_in_row == 0) {
        fold();
        rs = row_scale<MODE>(mn, mx, a.clip, a.qmax);
        if (lane == 0) {
          rsh[row_in_wg][0] = rs.scale;
          rsh[row_in_wg][1] = rs.y;
          rsh[row_in_wg][2] = rs.zf;
          rsh[row_in_wg][3] = rs.thr;
        }
      }
      __syncthreads();
      rs.scale = rsh[row_in_wg][0];
      rs.y = rsh[row_in_wg][1];
      rs.zf = rsh[row_in_wg][2];
      rs.thr = rsh[row_in_wg][3];
      rs.qmax = a.qmax;
    } else {
      fold();
      rs = row_scale<MODE>(mn, mx, a.clip, a.qmax);
    }
  } else {
    rs = row_scale<MODE>(mn, mx, a.clip, a.qmax);
  }
  // The zero point and the guard threshold are uniform over the wave: keep
  // them in scalar registers (operands of every chunk's fma and compare).
  rs.zf = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, rs.zf)));
  rs.thr = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, rs.thr)));
  // Lanes holding -y: the fast path folds the sign into the reciprocal
  // ((-y) * (-1/s) == y * (1/s) exactly); the exact path and the weight path
  // negate the values back first.
  RowScale rs_l = rs;
  rs_l.y = lsign * rs.y;

  uint32_t ev[ITERS][4], od[ITERS][4];
  int sum = 0;
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    if (!wlive[it]) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (MODE == kAct) {
        float dmax = 0.0f;
        if (CLAMP)
          act_chunk_fast(v[it][j], rs_l, ev[it][j], od[it][j], dmax);
        else
          act_chunk_fast_noclamp(v[it][j], rs_l, ev[it][j], od[it][j], dmax);
        if (dmax >= rs.thr) act_chunk_exact(v[it][j], rs, lsign, ev[it][j], od[it][j]);
      } else {
        if (ROT && lsign < 0.0f) {
#pragma unroll
          for (int i = 0; i < 8; ++i) v[it][j][i] = -v[it][j][i];
        }
        wgt_chunk(v[it][j], rs, ev[it][j], od[it][j], sum);
      }
    }
  }
  if (MODE == kWgt && a.sums) {
    sum = wave_sum_i32(sum);
    if (WPR > 1) {
      // Reached by every wave of the workgroup (no early exits above).
      __shared__ int sred[TPB / 64];
      if (lane == 0) sred[wave] = sum;
      __syncthreads();
      sum = 0;
#pragma unroll
      for (int w = 0; w < WPR; ++w) sum += sred[row_in_wg * WPR + w];
    }
  }
  if (!live) return;

  // Padded rows (real == false) computed nothing: every code is the zero
  // point 0 (activations) or 0 (weights), stored as u = 0 / qmax + 1.
  if (!real) {
    const uint32_t u = MODE == kAct ? 0u : 0x01010101u * (uint32_t)(a.qmax + 1.0f);
#pragma unroll
    for (int it = 0; it < ITERS; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ev[it][j] = u;
        od[it][j] = u;
      }
  }
  // Row base computed once (uniform); e0 < KP <= 2^20 fits 32 bits.  Stores
  // are checked per chunk only in iterations whose quads run past the row.
  // The unpacked codes (two-step mode) in their own uniform branch, so the
  // packed stores are straight-line.
  auto checked = [&](int it, int j) {
    const int b = quad + it * NQ;
    const int e0 = b * 128 + j * 32 + r * 8;
    return b < a.nblk && (WHOLE || e0 < a.KP);
  };
  auto store_iters = [&](auto&& store_one) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if (!(wlive[it] || !real)) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e0 = (quad + it * NQ) * 128 + j * 32 + r * 8;
        if (FULL || (WHOLE && !wmix[it]) || checked(it, j)) store_one(it, j, e0);
      }
    }
  };
  if (a.packed) {
    uint8_t* const prow = a.packed + row * (a.KP / 2);
    // A wave's packed blocks of an iteration (16 x 64 bytes, contiguous in the
    // row) pass through LDS so that each lane stores 16 contiguous bytes (32
    // elements; KP is a multiple of 64, so a piece is wholly inside or past
    // it): one store instruction per iteration instead of four 4-byte pieces
    // per lane, and whole 64-byte segments leave the CU.  Measured: M = 2048,
    // K = 4096 5.52 -> 4.33 MB written, 7.57 -> 7.45 us; 4096 x 28672 59.5 ->
    // 55.4 us.  A wave reads back only what its own lanes wrote; the
    // wave-scope release/acquire fence orders the other lanes' writes before
    // the reads in the memory model (the wave's LDS accesses complete in
    // order, so it costs at most a wait for them).
    __shared__ uint32_t pstage[TPB / 64][ITERS][256];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if (!FULL && !(wlive[it] || !real)) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        pstage[wave][it][(lane >> 2) * 16 + j * 4 + r] = packed_nibbles(ev[it][j], od[it][j]);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if (!FULL && !(wlive[it] || !real)) continue;
      const int b = wave_in_row * 16 + it * NQ + (lane >> 2);
      const int pe0 = b * 128 + (lane & 3) * 32;
      const uint4 v = *reinterpret_cast<const uint4*>(&pstage[wave][it][lane * 4]);
      if (FULL || (b < a.nblk && (WHOLE || pe0 < a.KP))) store_stream(v, prow + (uint32_t)pe0 / 2u);
    }
  }
  if (a.codes)
    store_iters([&](int it, int j, int e0) { store_codes<MODE>(a, row, e0, ev[it][j], od[it][j]); });
  if (wave_in_row == 0 && lane == 0) write_row_meta<MODE>(a, row, real, rs, sum);
}

// ------------------------------------------------------ streaming kernel
// For rows longer than the register kernel holds (K > 32768): one row per
// workgroup, 64 quads walk the row's blocks twice -- once for min / max, once
// to quantize -- re-reading x (the second pass mostly hits L2).

template <typename T, bool ROT, int MODE>
__device__ __forceinline__ void load_block(const RowArgs& a, const T* xrow, bool real,
                                           int b, int r, float c[4][8]) {
  if (a.vec) {
    Raw<T> raw[4];
    bool ok[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t e0 = (int64_t)b * 128 + j * 32 + r * 8;
      ok[j] = real && b < a.nblk && e0 < a.K;
      raw[j] = load_raw<T>(xrow, e0, ok[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      to_f32(raw[j], c[j]);
      mask_f32<T>(ok[j], c[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      load_scalar<T>(xrow, (int64_t)b * 128 + j * 32 + r * 8, a.K, real && b < a.nblk, c[j]);
  }
  if (ROT) {
#pragma unroll
    for (int j = 0; j < 4; ++j) fwht_chunk(c[j]);
    fwht_block_tail(c, r);
    if (MODE == kWgt) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) c[j][i] *= 0.0078125f;
    }
  }
}

template <typename T, bool ROT, int MODE>
__global__ __launch_bounds__(kThreads) void row_quant_stream_kernel(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const bool real = row < a.M;
  const int quad = wave * 16 + (lane >> 2);
  const int r = lane & 3;
  const T* xrow = static_cast<const T*>(a.x) + (real ? row : 0) * a.ldx;
  constexpr int NQ = 64;
  // The loop bound is uniform across the workgroup, so every lane runs the
  // same number of iterations and the DPP partners are always live.
  const int rounds = (a.nblk + NQ - 1) / NQ;

  float mn = 0.0f, mx = 0.0f;
  for (int it = 0; it < rounds; ++it) {
    float c[4][8];
    load_block<T, ROT, MODE>(a, xrow, real, quad + it * NQ, r, c);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (MODE == kAct) {
          mn = fminf(mn, c[j][i]);
          mx = fmaxf(mx, c[j][i]);
        } else {
          mx = fmaxf(mx, fabsf(c[j][i]));
        }
      }
  }
  if (MODE == kAct) mn = wave_min(mn);
  mx = wave_max(mx);
  __shared__ float red[2][kThreads / 64];
  if (lane == 0) {
    red[0][wave] = mn;
    red[1][wave] = mx;
  }
  __syncthreads();
  mn = fminf(fminf(red[0][0], red[0][1]), fminf(red[0][2], red[0][3]));
  mx = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
  const RowScale rs = row_scale<MODE>(mn, mx, a.clip, a.qmax);

  int sum = 0;
  for (int it = 0; it < rounds; ++it) {
    const int b = quad + it * NQ;
    float c[4][8];
    load_block<T, ROT, MODE>(a, xrow, real, b, r, c);
    uint32_t ev[4], od[4];
    if (MODE == kAct) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float dmax = 0.0f;
        act_chunk_fast(c[j], rs, ev[j], od[j], dmax);
        if (dmax >= rs.thr) act_chunk_exact(c[j], rs, 1.0f, ev[j], od[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) wgt_chunk(c[j], rs, ev[j], od[j], sum);
    }
    if (b < a.nblk) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        store_chunk<MODE>(a, row, (int64_t)b * 128 + j * 32 + r * 8, ev[j], od[j]);
    }
  }
  if (MODE == kWgt && a.sums) {
    sum = wave_sum_i32(sum);
    __shared__ int sred[kThreads / 64];
    if (lane == 0) sred[wave] = sum;
    __syncthreads();
    sum = sred[0] + sred[1] + sred[2] + sred[3];
  }
  if (wave == 0 && lane == 0) write_row_meta<MODE>(a, row, real, rs, sum);
}

// ------------------------------------------------------- few-row kernel
// Activation rows of at most 32 * PASSES blocks (K <= 4096 * PASSES) when
// there are few of them (decode, small batches): one row per 512-thread
// workgroup, a 128-element block over 16 consecutive lanes, lane 4j + r
// holding elements j*32 + r*8 .. +7 (one 16-byte load) of blocks slot,
// slot + 32, ... (slot = thread / 16) -- 8 elements per lane and pass instead
// of the register kernel's 32 per block, so each wave's chain of arithmetic
// is shorter.  The transform runs index bits 0-2 in the lane, bits 3-4 across
// the quad by DPP (sign-folded as in the register kernel) and bits 5-6
// across quads by ds_swizzle xor 4 / xor 8, the same butterflies in the same
// order, so every value, code, scale and zero-point is the register kernel's.
template <typename T, bool ROT, int CLAMP, int PASSES>
__global__ __launch_bounds__(512) void row_quant_spread_kernel(RowArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const bool real = row < a.M;
  const int qr = lane & 3;
  const T* xrow = static_cast<const T*>(a.x) + (real ? row : 0) * a.ldx;
  int e0[PASSES];
  bool ok[PASSES];
  Raw<T> raw[PASSES];
#pragma unroll
  for (int c = 0; c < PASSES; ++c) {
    const int blk = c * 32 + (tid >> 4);
    e0[c] = blk * 128 + ((lane >> 2) & 3) * 32 + qr * 8;
    ok[c] = real && blk < a.nblk && e0[c] < a.K;
    raw[c] = load_raw32<T>(xrow, e0[c], ok[c]);
  }
  const float s1 = (qr & 1) ? -1.0f : 1.0f, s2 = (qr & 2) ? -1.0f : 1.0f;
  const float s4 = (lane & 4) ? -1.0f : 1.0f, s8 = (lane & 8) ? -1.0f : 1.0f;
  // Lanes r = 1, 2 hold -y after the DPP stages.
  const float lsign = (ROT && (qr == 1 || qr == 2)) ? -1.0f : 1.0f;
  float v[PASSES][8];
  float mn = 0.0f, mx = 0.0f;
#pragma unroll
  for (int c = 0; c < PASSES; ++c) {
    // Chunks past the row (and padded rows) hold zeros: their codes are the
    // zero-point's and they leave the row's min / max (which start at 0) alone.
    uint32_t* w = reinterpret_cast<uint32_t*>(&raw[c]);
#pragma unroll
    for (int k = 0; k < (int)(sizeof(Raw<T>) / 4); ++k) w[k] = ok[c] ? w[k] : 0u;
    if (ROT && sizeof(T) == 2) {
#pragma unroll
      for (int k = 0; k < 4; ++k) bfly_f16x2(w[k], v[c][2 * k], v[c][2 * k + 1]);
      fwht_chunk_tail(v[c]);
    } else {
      to_f32(raw[c], v[c]);
      if (ROT) fwht_chunk(v[c]);
    }
    if (ROT) {
      fmac_dpp_xor1(v[c], s1);
      fmac_dpp_xor2(v[c], s2);
      bfly_swizzle<4>(v[c], s4);
      bfly_swizzle<8>(v[c], s8);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      mn = fminf(mn, v[c][i]);
      mx = fmaxf(mx, v[c][i]);
    }
  }
  if (lsign < 0.0f) {
    const float t = mn;
    mn = -mx;
    mx = -t;
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  __shared__ float red[2][8];
  if (lane == 0) {
    red[0][wave] = mn;
    red[1][wave] = mx;
  }
  __syncthreads();
  auto fold = [&]() {
    mn = red[0][0];
    mx = red[1][0];
#pragma unroll
    for (int k = 1; k < 8; ++k) {
      mn = fminf(mn, red[0][k]);
      mx = fmaxf(mx, red[1][k]);
    }
  };
  RowScale rs;
  if (a.share_scale) {
    // Many rows (the SIMDs hold several workgroups): wave 0 folds the
    // statistics and computes the row's scale, zero point, reciprocal and
    // guard once (~50 VALU instructions) and the other waves read them,
    // leaving their SIMDs to other rows.  With few rows every wave computes
    // them itself, which spares the latency of a second barrier.  Same values
    // either way: the same inputs in the same order.
    __shared__ float rsh[4];
    if (wave == 0) {
      fold();
      const RowScale r0 = row_scale<kAct>(mn, mx, a.clip, a.qmax);
      if (lane == 0) {
        rsh[0] = r0.scale;
        rsh[1] = r0.y;
        rsh[2] = r0.zf;
        rsh[3] = r0.thr;
      }
    }
    __syncthreads();
    rs.scale = rsh[0];
    rs.y = rsh[1];
    rs.zf = rsh[2];
    rs.thr = rsh[3];
    rs.qmax = a.qmax;
  } else {
    fold();
    rs = row_scale<kAct>(mn, mx, a.clip, a.qmax);
  }
  RowScale rs_l = rs;
  rs_l.y = lsign * rs.y;
#pragma unroll
  for (int c = 0; c < PASSES; ++c) {
    uint32_t ev, od;
    float dmax = 0.0f;
    if (CLAMP)
      act_chunk_fast(v[c], rs_l, ev, od, dmax);
    else
      act_chunk_fast_noclamp(v[c], rs_l, ev, od, dmax);
    if (dmax >= rs.thr) {
      // Keeps the IEEE divisions behind the branch (near-ties are rare); the
      // compiler would otherwise compute them for every chunk and select.
      asm volatile("" ::: "memory");
      act_chunk_exact(v[c], rs, lsign, ev, od);
    }
    // A block's 16 lanes store its 64 packed bytes; chunks in [K, KP) hold
    // the zero-point's code.
    if (c * 32 + (tid >> 4) < a.nblk && e0[c] < a.KP) {
      if (a.packed)
        *reinterpret_cast<uint32_t*>(a.packed + row * (a.KP / 2) + e0[c] / 2) =
            packed_nibbles(ev, od);
      if (a.codes) store_codes<kAct>(a, row, e0[c], ev, od);
    }
  }
  if (tid == 0) write_row_meta<kAct>(a, row, real, rs, 0);
}

// ------------------------------------------------------- small kernels

// codes u8 [MP, KP] (0..15) -> packed [MP, KP/2]; kernel/w4a4.cu:65-68.
// Each thread packs 16 codes (one 16-byte load) into 8 bytes.
__global__ __launch_bounds__(kThreads) void pack_codes_kernel(const uint8_t* codes,
                                                              uint8_t* packed,
                                                              int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n16) return;
  const uint4 c = reinterpret_cast<const uint4*>(codes)[i];
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  uint32_t outw[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // bytes [q0 q1 q2 q3] [q4 q5 q6 q7] -> evens / odds, then nibbles.
    const uint32_t ev = __builtin_amdgcn_perm(w[2 * h + 1], w[2 * h], 0x06040200u);
    const uint32_t od = __builtin_amdgcn_perm(w[2 * h + 1], w[2 * h], 0x07050301u);
    outw[h] = ((ev & 0x0F0F0F0Fu) | ((od & 0x0F0F0F0Fu) << 4)) ^ 0x88888888u;
  }
  uint2 o;
  o.x = outw[0];
  o.y = outw[1];
  reinterpret_cast<uint2*>(packed)[i] = o;
}

// pack_int4, core/quantization.py:31-40: int8 [R, C] -> u8 [R, ceil(C/2)].
__global__ __launch_bounds__(kThreads) void pack_int4_kernel(const int8_t* codes,
                                                             int64_t R, int64_t C,
                                                             uint8_t* packed) {
  const int64_t CB = (C + 1) / 2;
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= R * CB) return;
  const int64_t r = i / CB, j = i % CB;
  const int lo = codes[r * C + 2 * j] & 15;
  const int hi = (2 * j + 1 < C) ? (codes[r * C + 2 * j + 1] & 15) : 0;
  packed[i] = (uint8_t)(lo | (hi << 4));
}

// unpack_int4, core/quantization.py:42-45: u8 [R, CB] -> int8 [R, width].
__global__ __launch_bounds__(kThreads) void unpack_int4_kernel(const uint8_t* packed,
                                                               int64_t R, int64_t CB,
                                                               int64_t width,
                                                               int8_t* codes) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= R * width) return;
  const int64_t r = i / width, c = i % width;
  const int nib = (packed[r * CB + c / 2] >> ((c & 1) * 4)) & 15;
  codes[i] = (int8_t)(nib >= 8 ? nib - 16 : nib);
}

}  // namespace
}  // namespace dscq

// ================================================================ host side

namespace dscq {
namespace {

template <typename T, bool ROT, int MODE>
int launch_rows_typed(const RowArgs& a, int wpr, int iters, hipStream_t stream) {
  if (wpr == 0) {
    launch((row_quant_stream_kernel<T, ROT, MODE>), dim3((unsigned)a.MP),
                       dim3(kThreads), stream, a);
    return launch_status("row_quant_stream_kernel");
  }
  // Activations with two waves per row over many rows (K in (2048, 4096],
  // MP >= 2048) run one row per workgroup: the barrier between the two halves
  // of a row then waits for those two waves only, not for a second row's.
  // Measured at M = 2048, K = 4096: 7.62 -> 7.34 us (fp32 input 9.39 -> 8.83);
  // at M <= 1200 the 4-wave workgroups stay faster (M = 512: 4.28 against 4.62).
  const bool one_row = MODE == kAct && wpr == 2 && iters == 1 && a.MP >= 2048;
  const int rows_per_wg = one_row ? 1 : (kThreads / 64) / wpr;
  const dim3 grid((unsigned)((a.MP + rows_per_wg - 1) / rows_per_wg));
  // How the row fills the quads' blocks; clip 1 at 4 bits needs no clamp.
  const bool whole = a.K == (int64_t)a.nblk * 128;
  const bool full = whole && a.nblk == 16 * wpr * iters;
  const bool noclamp = MODE == kAct && a.clip == 1.0f && a.qmax == 15.0f;
  if constexpr (MODE == kAct) {
    if (one_row) {
      if (full && noclamp)
        launch((row_quant_kernel<T, ROT, MODE, 2, 1, kFull, 0, false, 128>), grid, dim3(128),
               stream, a);
      else if (full)
        launch((row_quant_kernel<T, ROT, MODE, 2, 1, kFull, 1, false, 128>), grid, dim3(128),
               stream, a);
      else if (whole && noclamp)
        launch((row_quant_kernel<T, ROT, MODE, 2, 1, kWhole, 0, false, 128>), grid, dim3(128),
               stream, a);
      else if (whole)
        launch((row_quant_kernel<T, ROT, MODE, 2, 1, kWhole, 1, false, 128>), grid, dim3(128),
               stream, a);
      else
        launch((row_quant_kernel<T, ROT, MODE, 2, 1, kPart, 1, false, 128>), grid, dim3(128),
               stream, a);
      return launch_status("row_quant_kernel");
    }
  }
#define DSCQ_ROWS(W, I)                                                                   \
  if (wpr == W && iters == I) {                                                           \
    if (MODE == kAct && full && noclamp)                                                  \
      launch((row_quant_kernel<T, ROT, MODE, W, I, kFull, 0>), grid, dim3(kThreads), stream, a); \
    else if (MODE == kAct && full)                                                        \
      launch((row_quant_kernel<T, ROT, MODE, W, I, kFull, 1>), grid, dim3(kThreads), stream, a); \
    else if (MODE == kAct && whole && noclamp)                                            \
      launch((row_quant_kernel<T, ROT, MODE, W, I, kWhole, 0>), grid, dim3(kThreads), stream, a); \
    else if (whole)                                                                       \
      launch((row_quant_kernel<T, ROT, MODE, W, I, kWhole, 1>), grid, dim3(kThreads), stream, a); \
    else                                                                                  \
      launch((row_quant_kernel<T, ROT, MODE, W, I, kPart, 1>), grid, dim3(kThreads), stream, a); \
    return launch_status("row_quant_kernel");                                            \
  }
  DSCQ_ROWS(1, 1) DSCQ_ROWS(1, 2) DSCQ_ROWS(1, 4)
  DSCQ_ROWS(2, 1) DSCQ_ROWS(2, 2) DSCQ_ROWS(2, 4)
  DSCQ_ROWS(4, 1) DSCQ_ROWS(4, 2) DSCQ_ROWS(4, 4)
#undef DSCQ_ROWS
  return fail("internal: no row kernel for wpr=%d iters=%d", wpr, iters);
}

// Register-kernel shape for a row of nblk 128-blocks: waves per row (wpr)
// and blocks per quad (iters).  Few blocks per lane keeps each wave's
// arithmetic short, so waves whose rows arrive late finish soon after; one
// block per quad (32 elements per lane) is preferred, spreading the row over
// up to four waves.  wpr = 0 selects the streaming kernel.
void pick_shape(int64_t MP, int nblk, int* wpr, int* iters) {
  (void)MP;
  for (int i : {1, 2, 4})
    for (int w : {1, 2, 4})
      if (16 * w * i >= nblk) {
        *wpr = w;
        *iters = i;
        return;
      }
  *wpr = 0;
  *iters = 0;
}

}  // namespace

// Launches one row-quantization pass.  mode 0: activations (qmax = 2^bits-1),
// 1: weights (qmax = 2^(bits-1)-1).  Rows M..MP-1 are written as padding.
int row_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t MP, float clip,
              int mode, float qmax, int rotate_block, uint8_t* packed, uint8_t* codes,
              float* scales, int32_t* zeros, int32_t* sums, hipStream_t stream) {
  RowArgs a;
  a.x = x;
  a.M = M;
  a.K = K;
  a.KP = ceil_to(K, 64);
  a.MP = MP;
  a.nblk = (int)((a.KP + 127) / 128);
  a.clip = clip;
  a.qmax = qmax;
  a.packed = packed;
  a.codes = codes;
  a.scales = scales;
  a.zeros = zeros;
  a.sums = sums;
  a.ldx = K;
  a.up = nullptr;
  a.hout = nullptr;
  const int esize = dtype == DSCQ_F16 ? 2 : 4;
  a.vec = (K % 8 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
          ((K * esize) % 16 == 0);
  const bool rot = rotate_block != 0;
  // Few activation rows of at most 32 * kSpreadMaxPasses blocks: the few-row kernel.
  if (mode == kAct && a.vec && a.nblk <= 32 * kSpreadMaxPasses && MP <= kSpreadMaxRows) {
    const bool noclamp = clip == 1.0f && qmax == 15.0f;
    const int passes = (a.nblk + 31) / 32;
    a.share_scale = MP >= kShareScaleRows;
#define DSCQ_SPREAD_P(T, R, C)                                                                  \
  if (passes == 1)                                                                              \
    launch((row_quant_spread_kernel<T, R, C, 1>), dim3((unsigned)MP), dim3(512), stream, a);    \
  else if (passes == 2)                                                                         \
    launch((row_quant_spread_kernel<T, R, C, 2>), dim3((unsigned)MP), dim3(512), stream, a);    \
  else                                                                                          \
    launch((row_quant_spread_kernel<T, R, C, 3>), dim3((unsigned)MP), dim3(512), stream, a);
#define DSCQ_SPREAD(T, R)  \
  if (noclamp) {           \
    DSCQ_SPREAD_P(T, R, 0) \
  } else {                 \
    DSCQ_SPREAD_P(T, R, 1) \
  }
    if (dtype == DSCQ_F16) {
      if (rot) { DSCQ_SPREAD(__half, true) } else { DSCQ_SPREAD(__half, false) }
    } else {
      if (rot) { DSCQ_SPREAD(float, true) } else { DSCQ_SPREAD(float, false) }
    }
#undef DSCQ_SPREAD
#undef DSCQ_SPREAD_P
    return launch_status("row_quant_spread_kernel");
  }
  int wpr, iters;
  pick_shape(MP, a.nblk, &wpr, &iters);
  if (!a.vec) wpr = iters = 0;  // element-wise loads: streaming kernel only
#define DSCQ_T(T)                                                                    \
  if (rot)                                                                           \
    return mode == kAct ? launch_rows_typed<T, true, kAct>(a, wpr, iters, stream)    \
                        : launch_rows_typed<T, true, kWgt>(a, wpr, iters, stream);   \
  return mode == kAct ? launch_rows_typed<T, false, kAct>(a, wpr, iters, stream)     \
                      : launch_rows_typed<T, false, kWgt>(a, wpr, iters, stream);
  if (dtype == DSCQ_F16) {
    DSCQ_T(__half)
  }
  DSCQ_T(float)
#undef DSCQ_T
}

// SiLU-gated activation quantization: rows h = silu(g) * u (fp16 roundings as
// in silu_mul_f16x2) of g = gate[m, 0..N), u = up[m, 0..N), row stride ld
// elements; the register kernel only (N <= 32768, 16-byte aligned rows).
int silu_mul_quant(const void* gate, const void* up, int64_t ld, int64_t M, int64_t N,
                   int64_t MP, float clip, int rotate_block, uint8_t* packed, float* scales,
                   int32_t* zeros, void* hout, hipStream_t stream) {
  RowArgs a;
  a.x = gate;
  a.up = up;
  a.hout = static_cast<__half*>(hout);
  a.ldx = ld;
  a.M = M;
  a.K = N;
  a.KP = ceil_to(N, 64);
  a.MP = MP;
  a.nblk = (int)((a.KP + 127) / 128);
  a.clip = clip;
  a.qmax = 15.0f;
  a.packed = packed;
  a.codes = nullptr;
  a.scales = scales;
  a.zeros = zeros;
  a.sums = nullptr;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  a.vec = N % 8 == 0 && ld % 8 == 0 && al16(gate) && al16(up) && al16(hout);
  int wpr, iters;
  pick_shape(MP, a.nblk, &wpr, &iters);
  if (!a.vec || wpr == 0)
    return fail("silu_mul_quantize: need N %% 8 == 0, N <= 32768 and 16-byte aligned rows");
  const int rows_per_wg = (kThreads / 64) / wpr;
  const dim3 grid((unsigned)((a.MP + rows_per_wg - 1) / rows_per_wg));
  const bool whole = a.K == (int64_t)a.nblk * 128;
  const bool full = whole && a.nblk == 16 * wpr * iters;
  const int fit = full ? kFull : whole ? kWhole : kPart;
  const bool noclamp = a.clip == 1.0f;
#define DSCQ_GROWS(ROT, W, I)                                                                   \
  if (wpr == W && iters == I) {                                                                 \
    if (fit == kFull && noclamp)                                                                \
      launch((row_quant_kernel<__half, ROT, kAct, W, I, kFull, 0, true>), grid, dim3(kThreads), \
             stream, a);                                                                        \
    else if (fit == kWhole && noclamp)                                                          \
      launch((row_quant_kernel<__half, ROT, kAct, W, I, kWhole, 0, true>), grid, dim3(kThreads),\
             stream, a);                                                                        \
    else                                                                                        \
      launch((row_quant_kernel<__half, ROT, kAct, W, I, kPart, 1, true>), grid, dim3(kThreads), \
             stream, a);                                                                        \
    return launch_status("row_quant_kernel");                                                  \
  }
#define DSCQ_GSHAPES(ROT)                                                                       \
  DSCQ_GROWS(ROT, 1, 1) DSCQ_GROWS(ROT, 1, 2) DSCQ_GROWS(ROT, 1, 4)                             \
  DSCQ_GROWS(ROT, 2, 1) DSCQ_GROWS(ROT, 2, 2) DSCQ_GROWS(ROT, 2, 4)                             \
  DSCQ_GROWS(ROT, 4, 1) DSCQ_GROWS(ROT, 4, 2) DSCQ_GROWS(ROT, 4, 4)
  if (rotate_block) {
    DSCQ_GSHAPES(true)
  } else {
    DSCQ_GSHAPES(false)
  }
#undef DSCQ_GSHAPES
#undef DSCQ_GROWS
  return fail("internal: no row kernel for wpr=%d iters=%d", wpr, iters);
}

int pack_codes(const uint8_t* codes, uint8_t* packed, int64_t MP, int64_t KP,
               hipStream_t stream) {
  const int64_t n16 = MP * KP / 16;
  launch(pack_codes_kernel, dim3((unsigned)((n16 + kThreads - 1) / kThreads)),
                     dim3(kThreads), stream, codes, packed, n16);
  return launch_status("pack_codes_kernel");
}

int pack_int4(const int8_t* codes, int64_t R, int64_t C, uint8_t* packed,
              hipStream_t stream) {
  const int64_t n = R * ((C + 1) / 2);
  if (n == 0) return DSCQ_OK;
  launch(pack_int4_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), stream, codes, R, C, packed);
  return launch_status("pack_int4_kernel");
}

int unpack_int4(const uint8_t* packed, int64_t R, int64_t CB, int64_t width,
                int8_t* codes, hipStream_t stream) {
  const int64_t n = R * width;
  if (n == 0) return DSCQ_OK;
  launch(unpack_int4_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), stream, packed, R, CB, width, codes);
  return launch_status("unpack_int4_kernel");
}

}  // namespace dscq
