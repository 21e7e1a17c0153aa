// Fused decode linear for gfx950: activation quantize (+ online rotation) and
// the skinny-M W4A4 product in one launch.
//
// For a handful of tokens the two-launch path (quantize, then the skinny-M
// GEMM) is latency-bound: each kernel is a few microseconds of launch and
// first-byte latency around well under a microsecond of work.  Here every
// workgroup owns 16 output columns, as in the skinny-M GEMM, and
//   1. issues the loads of its activation blocks and, right behind them, of
//      its whole weight stripe (16 rows of b, all of K), so the HBM stream
//      starts at once;
//   2. quantizes all M activation rows itself -- the same per-element
//      arithmetic as the quantize kernel (rowquant.h), so codes, scales and
//      zero-points are bit-identical -- into LDS, while the weights arrive;
//   3. runs the dot products and applies the reference's epilogue
//      (kernel/w4a4.cu:70-78, 156-161).  Two forms:
//        MFMA (M >= 3): int8 MFMAs over the unpacked nibbles, the 16 columns
//          as one 16 x 16 tile, each wave on a K range, sums meeting in LDS;
//        DOT (M <= 2): v_dot8_i32_i4 (eight signed-nibble products per
//          instruction, straight on the packed bytes: both operands already
//          hold two's-complement nibbles, (q - 8) & 15 and c & 15), each wave
//          on two of the 16 columns over all of K, so no sums cross waves.
//      Where the grid would take two or more rounds over the CUs, a workgroup
//      owns two or three such 16-column tiles (the activation fragment read
//      and unpacked once for all of them), so it quantizes once for them all.
//          Measured against MFMA (graph-replayed, weights from HBM, identical
//          outputs): M = 1, K = N = 4096 4.70 / 4.72 us; M = 1, N = 11008
//          6.87 / 7.50 us; M = 1, K = 11008 7.36 / 9.20 us; M = 2 5.58 /
//          5.76 us; M = 4 6.20 / 5.74 us (there the MFMA's 16 rows win).
// The quantization is repeated by every workgroup; it is cheap only while
// M * ceil(K / 128) <= 128 (one 128-element block per quad of lanes), which
// is the limit this kernel accepts (decode: M <= 4 at K = 4096, M = 1 up to
// K = 12288).  Larger inputs take the two-launch path.
//
// Result: out == matmul(quantize(x, clip, fused, rotate_block), b, ...) of
// the reference extension (kernel/w4a4.cu:164-225), bit for bit.

#include <algorithm>
#include <cstdlib>

#include "../../include/dscq.h"
#include "common.h"
#include "mma_int4.h"
#include "rowquant.h"

namespace dscq {
namespace {

constexpr int kWaves = 8;                 // workgroup = 8 waves = 32 blocks of 16 lanes
constexpr int kMaxBlocks = 128;           // activation blocks (M * nblk)
constexpr int kMaxBlocksPerWave = 12;     // MFMA form: 64-byte k blocks of b per wave (max)
constexpr int kMaxPieces = 12;            // DOT form: 16-byte pieces of a weight row per lane
constexpr int kDotMaxRows = 2;            // DOT form for M <= 2
constexpr int kMaxABytes = 16384;         // LDS for the packed activations

struct DecodeArgs {
  const void* x;          // [M, K] fp16 / fp32, rows 16-byte aligned
  int64_t M, K, KP, KB;   // KB = KP / 2 bytes per packed row
  int nblk;               // ceil(KP / 128)
  float clip;
  const uint8_t* b;       // [>= NP, KB]
  int64_t brows;          // NP
  const float* sw;
  const int32_t* sums;
  const void* bias;       // [N] of the output type, or null
  int64_t N;
  void* out;              // [M, N]
};

// PER: weight pieces held per lane -- MFMA form: 64-byte blocks per wave (4,
// 8 or 12 >= the blocks a wave owns); DOT form: 16-byte pieces of the lane's
// weight row (4, 8 or 12 >= ceil(KB / 512)) -- a compile-time count so the
// loads are unconditional: a load behind a branch makes the wait for an
// earlier load conservative.  NT: tiles of 16 output columns per workgroup
// (1-3; the v_dot8 form only with PER = 4), each with its own weight pieces.
//
// Activation layouts (both run the quantize kernel's butterflies in the same
// order, so every value is rounded identically; rowquant.h):
//   SPREAD (ITERS = 1 or 2 passes of 32 blocks, M * nblk <= 64): a 128-element
//     block over 16 consecutive lanes, lane 4j + r holding elements
//     j*32 + r*8 .. +7 (one 16-byte load).  Index bits 0-2 in the lane, bits
//     3-4 (r) across the quad by DPP (sign-folded: lanes r = 1, 2 end up
//     holding -y), bits 5-6 (j) across quads by ds_swizzle xor 4 / xor 8
//     (pairs share r, hence the sign).  8 elements per lane per pass.
//   QUAD (ITERS = 0, M * nblk <= 128): the quantize kernel's layout, a block
//     per quad of lanes, 32 elements per lane, bits 5-6 in the lane.
template <typename T, typename OutT, bool ROT, bool BIAS, int PER, int ITERS, bool DOT, int NT>
__global__ __launch_bounds__(kWaves * 64) void w4a4_decode_kernel(DecodeArgs d) {
  constexpr bool QUAD = ITERS == 0;
  constexpr int NCH = QUAD ? 4 : ITERS;  // 8-element chunks per lane
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[kMaxABytes];
  __shared__ int32_t part[DOT ? 1 : kWaves][NT][16][16];
  __shared__ float bmin[kMaxBlocks], bmax[kMaxBlocks];
  __shared__ float rmin[kWaves], rmax[kWaves];
  __shared__ float rsx[kWaves];
  __shared__ int32_t rzx[kWaves];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 16 * NT;
  const int r = lane & 15, grp = lane >> 4;

  // ---- 1a. activations.  Chunk c of this lane: block slot g[c] (row
  // g / nblk, block g % nblk), 32-element group jj[c], quad lane qr.
  const int qr = lane & 3;
  int g[NCH], jj[NCH];
  bool ok[NCH];
  Raw<T> raw[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    g[c] = QUAD ? (tid >> 2) : c * 32 + (tid >> 4);
    jj[c] = QUAD ? c : (lane >> 2) & 3;
    const int row = g[c] / d.nblk, blk = g[c] % d.nblk;
    const bool live = row < d.M;
    const int64_t e0 = (int64_t)blk * 128 + jj[c] * 32 + qr * 8;
    ok[c] = live && e0 < d.K;
    const T* xrow = static_cast<const T*>(d.x) + (live ? row : 0) * d.K;
    raw[c] = load_raw<T>(xrow, e0, ok[c]);
  }

  // ---- 1b. the weight stripe, issued right after the activation loads (a
  // wave's loads complete in issue order, so the activations are not queued
  // behind the weights).  MFMA form: lane (r, grp) holds 16 bytes of row
  // n0 + r at byte 16 * grp of each of the wave's 64-byte blocks.  DOT form:
  // wave w owns columns n0 + 2w and n0 + 2w + 1, lanes 0-31 the first, 32-63
  // the second; lane s of a half holds the 16-byte pieces at bytes
  // 512 i + 16 s, so each load instruction reads two 512-byte runs.
  const int64_t nkb = (d.KB + 63) / 64;
  const int64_t per = (nkb + kWaves - 1) / kWaves;
  const int64_t b0 = wave * per;
  const int64_t off = grp * 16;
  const int half = lane >> 5, s16 = (lane & 31) * 16;
  // DOT form: the lane's column of tile t.
  auto dcol = [&](int t) { return n0 + 16 * t + 2 * wave + half; };
  // Pieces past the wave's blocks or the row end (the last block of a row
  // with KB % 64 == 32 is half empty) re-read the row's last piece and are
  // zeroed where they are used: overwriting a load's destination here would
  // wait for the load.  MFMA form: NT tiles of 16 columns, n0 + 16 t + r.
  uint4 bv[NT][PER];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint8_t* brow = d.b + min(DOT ? dcol(t) : n0 + 16 * t + r, d.brows - 1) * d.KB;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if constexpr (DOT) {
        const int64_t kb = (int64_t)i * 512 + s16;
        bv[t][i] = *reinterpret_cast<const uint4*>(brow + (kb < d.KB ? kb : d.KB - 16));
      } else {
        const int64_t kb = (b0 + i) * 64;
        const bool in = i < per && kb + off < d.KB;
        bv[t][i] = *reinterpret_cast<const uint4*>(brow + (in ? kb + off : d.KB - 16));
      }
    }
  }
  // Epilogue operands of this thread's columns (MFMA form: n0 + 16 t + tid %
  // 16, used by threads < 256; DOT form: the lane's column), fetched now
  // (index clamped) instead of after the dot products.
  float e_sw[NT], e_b[NT];
  int32_t e_sum[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t nc = min(DOT ? dcol(t) : n0 + 16 * t + (tid & 15), d.N - 1);
    e_sw[t] = d.sw[nc];
    e_sum[t] = d.sums[nc];
    e_b[t] = BIAS ? (float)static_cast<const OutT*>(d.bias)[nc] : 0.0f;
  }
  // Keep every load above the arithmetic (the scheduler would otherwise sink
  // the weight loads below the transform to save registers).
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. rotate + quantize the activations into LDS.  Blocks past the M
  // rows work on row 0's data and their results are never read.  Elements
  // past K (only without rotation: it needs K % 128 == 0) are zeroed after
  // the conversion; masking the raw load results instead turns the loads
  // into branches issued behind the weight stripe.
  float v[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (ROT && sizeof(T) == 2) {
      const uint32_t* w = reinterpret_cast<const uint32_t*>(&raw[c]);
#pragma unroll
      for (int k = 0; k < 4; ++k) bfly_f16x2(w[k], v[c][2 * k], v[c][2 * k + 1]);
      fwht_chunk_tail(v[c]);
    } else {
      to_f32(raw[c], v[c]);
      if (ROT) fwht_chunk(v[c]);
      else mask_f32<T>(ok[c], v[c]);
    }
  }
  if (ROT) {
    if constexpr (QUAD) {
      fwht_block_tail_signed(v, qr);
    } else {
      const float s1 = (qr & 1) ? -1.0f : 1.0f, s2 = (qr & 2) ? -1.0f : 1.0f;
      const float s4 = (lane & 4) ? -1.0f : 1.0f, s8 = (lane & 8) ? -1.0f : 1.0f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        fmac_dpp_xor1(v[c], s1);
        fmac_dpp_xor2(v[c], s2);
        bfly_swizzle<4>(v[c], s4);
        bfly_swizzle<8>(v[c], s8);
      }
    }
  }
  const float lsign = (ROT && (qr == 1 || qr == 2)) ? -1.0f : 1.0f;
  // Block min / max (with 0, as lo = min(x, 0), hi = max(x, 0)), sign undone,
  // then over the block's lanes (a quad, or 16 lanes).
  auto block_minmax = [&](float mn, float mx, int slot, bool writer) {
    if (ROT && lsign < 0.0f) {
      const float t = mn;
      mn = -mx;
      mx = -t;
    }
    mn = fminf(mn, dpp_f32<kDppQuadXor1>(mn));
    mx = fmaxf(mx, dpp_f32<kDppQuadXor1>(mx));
    mn = fminf(mn, dpp_f32<kDppQuadXor2>(mn));
    mx = fmaxf(mx, dpp_f32<kDppQuadXor2>(mx));
    if (!QUAD) {
      mn = fminf(mn, dpp_f32<kDppRowRor4>(mn));
      mx = fmaxf(mx, dpp_f32<kDppRowRor4>(mx));
      mn = fminf(mn, dpp_f32<kDppRowRor8>(mn));
      mx = fmaxf(mx, dpp_f32<kDppRowRor8>(mx));
    }
    if (writer) {
      bmin[slot] = mn;
      bmax[slot] = mx;
    }
  };
  if constexpr (QUAD) {
    float mn = 0.0f, mx = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        mn = fminf(mn, v[c][i]);
        mx = fmaxf(mx, v[c][i]);
      }
    block_minmax(mn, mx, g[0], qr == 0);
  } else {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      float mn = 0.0f, mx = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        mn = fminf(mn, v[c][i]);
        mx = fmaxf(mx, v[c][i]);
      }
      block_minmax(mn, mx, g[c], r == 0);
    }
  }
  __syncthreads();
  // Row statistics: wave w < M reduces row w's nblk (<= 128) block entries.
  if (wave < d.M) {
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = lane + 64 * h;
      if (e < d.nblk) {
        a0 = fminf(a0, bmin[wave * d.nblk + e]);
        a1 = fmaxf(a1, bmax[wave * d.nblk + e]);
      }
    }
    a0 = wave_min(a0);
    a1 = wave_max(a1);
    if (lane == 0) {
      rmin[wave] = a0;
      rmax[wave] = a1;
    }
  }
  __syncthreads();
  const bool noclamp = d.clip == 1.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int row = g[c] / d.nblk, blk = g[c] % d.nblk;
    if (row < d.M) {
      const RowScale rs = row_scale<kAct>(rmin[row], rmax[row], d.clip, 15.0f);
      RowScale rs_l = rs;
      rs_l.y = lsign * rs.y;
      uint32_t ev, od;
      float dmax = 0.0f;
      if (noclamp)
        act_chunk_fast_noclamp(v[c], rs_l, ev, od, dmax);
      else
        act_chunk_fast(v[c], rs_l, ev, od, dmax);
      if (dmax >= rs.thr) act_chunk_exact(v[c], rs, lsign, ev, od);
      const int64_t e0 = (int64_t)blk * 128 + jj[c] * 32 + qr * 8;
      // (q - 8) & 15 == q ^ 8; elements in [K, KP) hold the zero-point's code.
      if (e0 < d.KP)
        *reinterpret_cast<uint32_t*>(a_lds + row * d.KB + e0 / 2) =
            (ev | (od << 4)) ^ 0x88888888u;
      if (blk == 0 && jj[c] == 0 && qr == 0) {
        rsx[row] = rs.scale;
        rzx[row] = (int32_t)rs.zf;
      }
    }
  }
  __syncthreads();

  if constexpr (DOT) {
    // ---- 3 (DOT). per 16-byte piece and row m < M, four v_dot8_i32_i4 of the
    // activation codes (LDS) with the weight piece; the sums over each 32-lane
    // half (DPP within 16-lane rows, two readlanes); the epilogue of output
    // (m, column) by lane 32 half + m.  The sums are the reference's raw
    // values: the nibbles are multiplied as they are.
    int32_t mine[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) mine[t] = 0;
#pragma unroll
    for (int m = 0; m < kDotMaxRows; ++m) {
      if (m < d.M) {
        int32_t acc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[t] = 0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int64_t kb = (int64_t)i * 512 + s16;
          if (kb < d.KB) {
            const uint4 av = *reinterpret_cast<const uint4*>(a_lds + m * d.KB + kb);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              const uint4 bw = bv[t][i];
              acc[t] = __builtin_amdgcn_sdot8((int)av.x, (int)bw.x, acc[t], false);
              acc[t] = __builtin_amdgcn_sdot8((int)av.y, (int)bw.y, acc[t], false);
              acc[t] = __builtin_amdgcn_sdot8((int)av.z, (int)bw.z, acc[t], false);
              acc[t] = __builtin_amdgcn_sdot8((int)av.w, (int)bw.w, acc[t], false);
            }
          }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          int32_t a = acc[t];
          a += __builtin_amdgcn_mov_dpp(a, kDppQuadXor1, 0xF, 0xF, false);
          a += __builtin_amdgcn_mov_dpp(a, kDppQuadXor2, 0xF, 0xF, false);
          a += __builtin_amdgcn_mov_dpp(a, kDppRowRor4, 0xF, 0xF, false);
          a += __builtin_amdgcn_mov_dpp(a, kDppRowRor8, 0xF, 0xF, false);
          const int32_t s0 = __builtin_amdgcn_readlane(a, 0) + __builtin_amdgcn_readlane(a, 16);
          const int32_t s1 = __builtin_amdgcn_readlane(a, 32) + __builtin_amdgcn_readlane(a, 48);
          if ((lane & 31) == m) mine[t] = half ? s1 : s0;
        }
      }
    }
    const int ml = lane & 31;
    if (ml >= d.M) return;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t n = dcol(t);
      if (n >= d.N) break;
      // Operation order of kernel/w4a4.cu:74-77.
      const int32_t corrected = mine[t] + (8 - rzx[ml]) * e_sum[t];
      float res = (float)corrected * rsx[ml];
      res = res * e_sw[t];
      if (BIAS) res = res + e_b[t];
      static_cast<OutT*>(d.out)[ml * d.N + n] = to_out<OutT>(res);
    }
    return;
  }

  // ---- 3 (MFMA). per 64-byte block two v_mfma_i32_16x16x64_i8 per column
  // tile (A row lane % 16 from LDS, zero past M, shared by the tiles; B from
  // registers), as the skinny-M GEMM.
  v4i acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = v4i{0, 0, 0, 0};
  const bool arow_live = r < d.M;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (i < per) {
      const int64_t kb = (b0 + i) * 64;
      const bool in = kb + off < d.KB;
      uint4 av = make_uint4(0u, 0u, 0u, 0u);
      if (arow_live && in) av = *reinterpret_cast<const uint4*>(a_lds + r * d.KB + kb + off);
      const v4i a_lo = unpack8(av.x, av.y), a_hi = unpack8(av.z, av.w);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        uint4 bw = bv[t][i];
        bw.x = in ? bw.x : 0u;
        bw.y = in ? bw.y : 0u;
        bw.z = in ? bw.z : 0u;
        bw.w = in ? bw.w : 0u;
        acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_lo, unpack8(bw.x, bw.y), acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_hi, unpack8(bw.z, bw.w), acc[t], 0, 0, 0);
      }
    }
  }
  // D of a 16 x 16 tile: row (A) 4 * (lane / 16) + v, column (B) lane % 16.
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) part[wave][t][4 * grp + v][r] = acc[t][v] >> 8;
  __syncthreads();
  if (tid >= 256) return;
  const int ml = tid >> 4, nl = tid & 15;
  if (ml >= d.M) return;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n0 + 16 * t + nl;
    if (n >= d.N) break;
    int32_t rawv = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) rawv += part[w][t][ml][nl];
    // Operation order of kernel/w4a4.cu:74-77.
    const int32_t corrected = rawv + (8 - rzx[ml]) * e_sum[t];
    float res = (float)corrected * rsx[ml];
    res = res * e_sw[t];
    if (BIAS) res = res + e_b[t];
    static_cast<OutT*>(d.out)[ml * d.N + n] = to_out<OutT>(res);
  }
}

}  // namespace

// One launch of the chosen form and tile count.  The MFMA form needs M >= 3,
// so M * ceil(K / 128) <= 128 keeps its K at most 5376 and its weight pieces
// at most 8; the v_dot8 form takes several tiles only with four pieces.
template <typename T, typename O, bool R, bool B, int P, int I>
bool launch_decode(bool dot, int nt, dim3 grid, dim3 block, hipStream_t stream,
                   const DecodeArgs& d) {
  if (dot) {
    if constexpr (P <= 4) {
      if (nt == 2) {
        launch((w4a4_decode_kernel<T, O, R, B, P, I, true, 2>), grid, block, stream, d);
        return true;
      }
      if (nt == 3) {
        launch((w4a4_decode_kernel<T, O, R, B, P, I, true, 3>), grid, block, stream, d);
        return true;
      }
    }
    if (nt != 1) return false;
    launch((w4a4_decode_kernel<T, O, R, B, P, I, true, 1>), grid, block, stream, d);
    return true;
  }
  if constexpr (P <= 8) {
    if (nt == 1)
      launch((w4a4_decode_kernel<T, O, R, B, P, I, false, 1>), grid, block, stream, d);
    else if (nt == 2)
      launch((w4a4_decode_kernel<T, O, R, B, P, I, false, 2>), grid, block, stream, d);
    else if (nt == 3)
      launch((w4a4_decode_kernel<T, O, R, B, P, I, false, 3>), grid, block, stream, d);
    else
      return false;
    return true;
  }
  return false;
}

// The limits the fused kernel accepts (see the file comment); callers check
// them with linear_decode_fits and otherwise quantize and multiply separately.
bool linear_decode_fits(int64_t M, int64_t K) {
  const int64_t KP = ceil_to(K, 64), KB = KP / 2;
  const int64_t nblk = (KP + 127) / 128;
  return M >= 1 && M <= kWaves && K % 8 == 0 && M * nblk <= kMaxBlocks && M * KB <= kMaxABytes &&
         (KB + 63) / 64 <= (int64_t)kWaves * kMaxBlocksPerWave && (KB + 511) / 512 <= kMaxPieces;
}

int linear_decode(const void* x, int dtype, int64_t M, int64_t K, float clip, int rotate_block,
                  const uint8_t* b, const float* sw, const int32_t* sums, const void* bias,
                  int64_t N, bool out_fp32, void* out, hipStream_t stream) {
  DecodeArgs d;
  d.x = x;
  d.M = M;
  d.K = K;
  d.KP = ceil_to(K, 64);
  d.KB = d.KP / 2;
  d.nblk = (int)((d.KP + 127) / 128);
  d.clip = clip;
  d.b = b;
  d.brows = ceil_to(N, 8);
  d.sw = sw;
  d.sums = sums;
  d.bias = bias;
  d.N = N;
  d.out = out;
  const bool rot = rotate_block != 0;
  const bool dot = M <= kDotMaxRows;
  // A workgroup takes NT tiles of 16 columns, since every workgroup
  // re-quantizes all M rows.  Up to three tiles per CU, NT spreads them in
  // one round; past that, two tiles per workgroup (three would leave a short
  // second round).  Graph-replayed, weights from HBM, one tile / NT:
  //   MFMA form, M = 4, K = 4096: N = 8192 8.2 / 7.3 us, N = 11008 10.3 /
  //   8.5, N = 12288 10.5 / 8.8, N = 14336 12.5 / 10.2 (three tiles 14.4),
  //   N = 28672 21.2 / 16.6 (three 21.0);
  //   v_dot8 form, K = 4096 (four weight pieces per lane): M = 1, N = 8192
  //   5.91 / 5.56, N = 11008 6.85 / 6.62 (two tiles 6.94), N = 14336 8.25 /
  //   7.41, N = 28672 12.6 / 12.2; M = 2, N = 11008 8.67 / 7.93.  With eight
  //   pieces (K = 8192) the extra registers cost more (M = 1, N = 8192 8.8 /
  //   9.2; M = 2, N = 28672 25.0 / 30.3): one tile.
  const int64_t tiles = (N + 15) / 16, cus = cu_count();
  const int64_t per_cu = (tiles + cus - 1) / cus;
  const int64_t per = dot ? (d.KB + 511) / 512 : ((d.KB + 63) / 64 + kWaves - 1) / kWaves;
  const int nt = (dot && per > 4) ? 1 : per_cu > 3 ? 2 : (int)std::max<int64_t>(1, per_cu);
  const dim3 grid((unsigned)((tiles + nt - 1) / nt)), block(kWaves * 64);
  // 16-lane blocks for up to two passes of 32 blocks, quads beyond.
  const int64_t iters = (M * d.nblk + 31) / 32;
  bool launched = false;
#define DSCQ_DEC_D(T, O, R, B, P, I) \
  launched = launch_decode<T, O, R, B, P, I>(dot, nt, grid, block, stream, d);
#define DSCQ_DEC_I(T, O, R, B, P)                                                              \
  if (iters <= 1) {                                                                            \
    DSCQ_DEC_D(T, O, R, B, P, 1)                                                               \
  } else if (iters <= 2) {                                                                     \
    DSCQ_DEC_D(T, O, R, B, P, 2)                                                               \
  } else {                                                                                     \
    DSCQ_DEC_D(T, O, R, B, P, 0)                                                               \
  }
#define DSCQ_DEC(T, O, R, B)                                                                   \
  if (per <= 4) {                                                                              \
    DSCQ_DEC_I(T, O, R, B, 4)                                                                  \
  } else if (per <= 8) {                                                                       \
    DSCQ_DEC_I(T, O, R, B, 8)                                                                  \
  } else {                                                                                     \
    DSCQ_DEC_I(T, O, R, B, 12)                                                                 \
  }
#define DSCQ_DEC_B(T, O, R) \
  if (bias) { DSCQ_DEC(T, O, R, true); } else { DSCQ_DEC(T, O, R, false); }
#define DSCQ_DEC_R(T, O) \
  if (rot) { DSCQ_DEC_B(T, O, true) } else { DSCQ_DEC_B(T, O, false) }
#define DSCQ_DEC_O(T) \
  if (out_fp32) { DSCQ_DEC_R(T, float) } else { DSCQ_DEC_R(T, __half) }
  if (dtype == DSCQ_F16) {
    DSCQ_DEC_O(__half)
  } else {
    DSCQ_DEC_O(float)
  }
#undef DSCQ_DEC_O
#undef DSCQ_DEC_R
#undef DSCQ_DEC_B
#undef DSCQ_DEC
#undef DSCQ_DEC_I
#undef DSCQ_DEC_D
  if (!launched) return fail("internal: no decode kernel for M=%lld K=%lld tiles=%d", (long long)M, (long long)K, nt);
  return launch_status("w4a4_decode_kernel");
}

}  // namespace dscq
