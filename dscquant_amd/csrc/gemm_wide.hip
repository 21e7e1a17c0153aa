// Wide-tile W4A4 GEMM for gfx950: 256 x BN output tiles (BN = 256, or 128),
// one workgroup of four waves per CU (one wave per SIMD), 2 x 2 waves each a
// 128 x BN/2 block of 4 x BN/64 v_mfma_i32_32x32x32_i8 tiles whose
// accumulators (256 or 128 registers) live in AGPRs.
//
// Semantics as gemm.hip (kernel/w4a4.cu:70-161): both operands are packed
// int4, K-contiguous; nibbles are unpacked to int8 (x16) in registers
// (mma_int4.h), so the int32 sums carry a factor 256.
//
// Data moved per multiply-accumulate at BN = 256, against the pipelined
// kernel's 256 x 128 tile of eight 64 x 64 waves: per MFMA a wave reads half a
// 16-byte fragment from LDS (8 fragments feed 16 MFMAs per k-step) instead of
// one, and spends 3 VALU instructions on unpacking instead of 6; the tile loads
// (256 + 256) rows per 65536 outputs instead of (256 + 128) per 32768, a third
// fewer bytes.  BN = 128: 6 fragments per 8 MFMAs, 4.5 unpack instructions.
//
// K advances in 256-nibble slices: 128 bytes of every A and B row of the tile,
// 32 KiB + BN * 128 bytes per slice, double-buffered in LDS.  Global memory
// reaches LDS by DMA (global_load_lds_dwordx4, 16 bytes per lane written
// straight to LDS, no register staging): each wave issues (256 + BN) / 32 such
// instructions per slice; instruction j of wave w fills 8 rows, 8d .. 8d + 7 of
// the tile's 256 + BN (d = (256 + BN) / 32 * w + j: A rows first, then B
// rows); lane l writes position l % 8 of row 8d + l / 8, so it loads the row's
// 16-byte unit (l % 8) ^ ((row >> 1) & 7): the pipelined kernel's swizzle,
// applied on the global side, which keeps the fragment reads conflict-free.
//
// Schedule of slice s (LDS stage c = s & 1), k-steps 0..7 of 4 * BN / 64 MFMAs;
// every step interleaves its MFMAs with the unpack of the next step:
//   steps 1, 3   fragment units q = 2, 3 of slice s read from stage c
//   before 5     this wave's DMA of slice s + 1 waited for (vmcnt), then a
//                barrier: slice s + 1 is in stage c ^ 1 for every wave, and
//                every wave's reads of stage c for slice s are complete
//   step 5       unit q = 0 of slice s + 1 read; the DMA of slice s + 2 into
//                stage c issued, a whole slice before the barrier that needs it
//   step 7       unit q = 1 of slice s + 1 read
// Each unit is read two steps before the first unpack that uses it, so no more
// than two units' fragments (64 registers) are held at once.
// Lane l of a fragment read takes row l % 32, unit 2q + l / 32 (stored at
// (2q + l / 32) ^ ((row >> 1) & 7)): its low 8 bytes feed k-step 2q, the high
// 8 bytes k-step 2q + 1, the same for A and B, so every product pairs equal k.
//
// Epilogue: the scale and zero-point factors are staged pre-multiplied, sx / 256
// and (8 - zx) * 256, and the column sums as floats, so corrected * 256 =
// fma((8 - zx) * 256, sums, float(acc)) is exact (integers below 2^31 with at
// most 24 significant bits: |acc / 256| <= 2^22 and |corrected| <= 2^23 for
// K <= 65536) and float(corrected * 256) * (sx / 256) equals
// float(corrected) * sx exactly (power-of-two scalings); then * sw (+ bias)
// and one fp16 rounding (v_cvt_pk_f16_f32), the reference's operation order.
// Each wave's 128 x BN/2 fp16 tile goes through LDS (the idle slice stages)
// so that every store instruction writes whole row segments (four of 256
// bytes at BN = 256).

#include <type_traits>

#include "../../include/dscq.h"
#include "common.h"
#include "gemm_args.h"
#include "mma_int4.h"
#include "rowquant.h"

namespace dscq {
namespace {

constexpr int kTileM = 256;                   // rows of A per tile
constexpr int kSlice = 128;                   // bytes of a packed row per slice
constexpr int kHalfA = kTileM * kSlice;       // 32 KiB: A's rows of one slice
// LDS: A of stage 0, A of stage 1, then B of stage 0 and B of stage 1, so that
// every fragment of either stage is within a ds_read immediate offset
// (< 64 KiB) of one A base and one B base per unit.
constexpr int kBRegion = 2 * kHalfA;
constexpr int kWaves = 4;

__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land
// at LDS byte address lds + 16 l (lds wave-uniform, through M0).  Inline
// assembly, so that the compiler's wait-count pass does not treat LDS reads
// as waiting on it; the kernel waits for these loads itself (vmcnt) before the
// barrier that publishes their data.  M0 is a reserved register, which clang
// warns about on a clobber list: nothing else in this kernel uses it on gfx950
// (its LDS instructions take no M0), as its assembly shows.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

template <int BN, bool BIAS, bool GATED = false>
__global__ __launch_bounds__(64 * kWaves, 1) void w4a4_gemm_wide_kernel(GemmArgs g) {
  // 2 x 2 waves, each 128 x (BN / 2): 4 x FN MFMA tiles.
  constexpr int FM = 4, FN = BN / 64, NF = FM + FN, TN = BN / 2, MF = FM * FN;
  constexpr int kHalfB = BN * kSlice;           // B's rows of one slice
  constexpr int kStages = kBRegion + 2 * kHalfB;
  constexpr int kDma = (kTileM + BN) / 8 / kWaves;  // DMA instructions per wave per slice
  static_assert(BN == 256 || BN == 128, "tile width");
  static_assert(!GATED || BN == 256, "gated tiles pair gate and up rows within a wave's 128 columns");
  static_assert(kDma % 2 == 0, "the per-lane DMA offset pairs with the parity of j");
  __shared__ __attribute__((aligned(16))) uint8_t smem[kStages + kTileM * 8 + BN * 12];
  float* const lds_sx = reinterpret_cast<float*>(smem + kStages);             // sx / 256
  float* const lds_z = reinterpret_cast<float*>(smem + kStages + kTileM * 4);  // (8 - zx) * 256
  float* const lds_sw = reinterpret_cast<float*>(smem + kStages + kTileM * 8);
  float* const lds_sum = reinterpret_cast<float*>(smem + kStages + kTileM * 8 + BN * 4);
  float* const lds_b = reinterpret_cast<float*>(smem + kStages + kTileM * 8 + BN * 8);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tile_m = (int)(blockIdx.x / (unsigned)g.tiles_n);
  const int tile_n = (int)(blockIdx.x % (unsigned)g.tiles_n);
  const int64_t m0 = (int64_t)tile_m * kTileM, n0 = (int64_t)tile_n * BN;
  const int64_t KB = g.KP / 2;
  const int nslices = (int)(KB / kSlice);

  // ---- DMA sources.  Instruction j of this wave covers the 8 tile rows
  // 8d .. 8d + 7, d = kDma * wave + j, of the tile's 256 A rows followed by its
  // BN B rows.  The tile origin and MP / NP are multiples of 8, so a group is
  // wholly inside the operand's rows or wholly past them, and groups past them
  // are clamped to its last 8 rows (their sums are never stored): a
  // wave-uniform base per instruction.  Lane l reads row 8d + l / 8 at unit
  // (l % 8) ^ ((row >> 1) & 7); (row >> 1) & 7 = (4 (d % 2) + l / 16) % 8 and
  // kDma is even, so the per-lane offset depends on the parity of j only.
  const uint32_t lds0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem);
  const uint8_t* gbase[kDma];  // wave-uniform: scalar registers
  uint32_t ldsj[kDma];         // LDS byte address of the group in stage 0
#pragma unroll
  for (int j = 0; j < kDma; ++j) {
    const int R = 8 * (kDma * wave + j);
    if (R < kTileM) {
      gbase[j] = g.a + min(m0 + R, g.arows - 8) * KB;
      ldsj[j] = lds0 + (uint32_t)(R * kSlice);
    } else {
      gbase[j] = g.b + min(n0 + (R - kTileM), g.brows - 8) * KB;
      ldsj[j] = lds0 + (uint32_t)(kBRegion + (R - kTileM) * kSlice);
    }
  }
  uint32_t lane_off[2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
    lane_off[p] = (uint32_t)((lane >> 3) * KB + 16 * ((lane & 7) ^ ((4 * p + (lane >> 4)) & 7)));
  // Instruction j of a slice into `stage`: the slice offset rides on the
  // per-lane offsets (off[p] = lane_off[p] + slice * 128), the bases stay put.
  auto dma_one = [&](int j, const uint32_t (&off)[2], int stage) {
    const int R = 8 * (kDma * wave + j);
    dma16(gbase[j], off[j & 1], ldsj[j] + (uint32_t)stage * (R < kTileM ? kHalfA : kHalfB));
  };
  auto dma = [&](int slice, int stage) {
    const uint32_t off[2] = {lane_off[0] + (uint32_t)slice * kSlice,
                             lane_off[1] + (uint32_t)slice * kSlice};
#pragma unroll
    for (int j = 0; j < kDma; ++j) dma_one(j, off, stage);
  };

  // ---- fragment reads: per unit q one A base and one B base (stage 0,
  // fragment 0); the stage and the fragment are immediate offsets.
  const int fr = lane & 31;
  const int fsw = (fr >> 1) & 7;
  uint32_t abase[4], bbase[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t qo = 16 * ((2 * q + (lane >> 5)) ^ fsw);
    abase[q] = (uint32_t)((wm * 128 + fr) * kSlice) + qo;
    bbase[q] = (uint32_t)(kBRegion + (wn * TN + fr) * kSlice) + qo;
  }
  uint4 P[4][NF];
  auto lread = [&](int stage, int q) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint32_t off = f < FM ? abase[q] + (uint32_t)(stage * kHalfA + f * 32 * kSlice)
                                  : bbase[q] + (uint32_t)(stage * kHalfB + (f - FM) * 32 * kSlice);
      P[q][f] = *reinterpret_cast<const uint4*>(smem + off);
    }
  };

  // Accumulators: the first MFMA of each takes a literal zero as its C operand
  // (slice 0's first step, peeled), so no registers are ever zero-filled --
  // a zero-filled accumulator array takes VGPRs that only then move to AGPRs.
  v16i acc[FM][FN];
  v4i U0[NF], U1[NF];
  // k-step t of a slice uses P[t / 2] dwords (2 * (t % 2), +1).
  auto unpack_step = [&](v4i (&U)[NF], int t) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const uint4 w = P[t >> 1][f];
      U[f] = (t & 1) ? unpack8(w.z, w.w) : unpack8(w.x, w.y);
    }
  };
  // B first: acc[i][j] accumulates the transposed 32 x 32 tile.
  auto mfma_step = [&](const v4i (&U)[NF]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(U[FM + j], U[i], acc[i][j], 0, 0, 0);
  };
  auto mfma_first = [&](const v4i (&U)[NF]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(U[FM + j], U[i], v16i{0}, 0, 0, 0);
  };
  // Half h of fragment f of k-step t (3 VALU: two unpacked dwords).
  auto unpack_half = [&](v4i (&U)[NF], int t, int f, int h) {
    const uint4 w = P[t >> 1][f];
    const uint32_t x = (t & 1) ? (h ? w.w : w.z) : (h ? w.y : w.x);
    U[f][2 * h] = (int)((x << 4) & 0xF0F0F0F0u);
    U[f][2 * h + 1] = (int)(x & 0xF0F0F0F0u);
  };
  // One MFMA, then a share of the step's unpack VALU instructions, and so on.
  constexpr int VPM = (6 * NF + MF - 1) / MF;
  auto interleave = [&]() {
#pragma unroll
    for (int k = 0; k < MF; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- prologue: slice 0 and the tile's row / column metadata, then slice 1.
  dma(0, 0);
  const int64_t mrow = min(m0 + tid, g.arows - 1), ncol = min(n0 + tid, g.brows - 1);
  const float meta_sx = g.sx[mrow];
  const int32_t meta_z = g.zx[mrow];
  const float meta_sw = g.sw[ncol];
  const int32_t meta_sum = g.sums[ncol];
  const float meta_b =
      BIAS ? __half2float(static_cast<const __half*>(g.bias)[min(n0 + tid, g.N - 1)]) : 0.0f;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // slice 0 and the metadata
  lds_sx[tid] = meta_sx * 0.00390625f;                // exact: a power-of-two scaling
  lds_z[tid] = (float)((8 - meta_z) * 256);
  if (tid < BN) {
    lds_sw[tid] = meta_sw;
    lds_sum[tid] = (float)meta_sum;
    if (BIAS) lds_b[tid] = meta_b;
  }
  if (nslices > 1) dma(1, 1);
  barrier_lds();
  lread(0, 0);
  lread(0, 1);
  unpack_step(U0, 0);

  // The barrier and the reads of the next slice's first units run after the
  // last slice too (they read a stage nothing uses any more, and the unpack
  // result is dropped), so one body serves every slice.
  auto slice = [&](int s, auto stage, auto first) {
    constexpr int C = decltype(stage)::value, NX = C ^ 1;
    if constexpr (decltype(first)::value)
      mfma_first(U0);
    else
      mfma_step(U0);
    unpack_step(U1, 1);
    interleave();
    mfma_step(U1);
    unpack_step(U0, 2);
    lread(C, 2);
    interleave();
    mfma_step(U0);
    unpack_step(U1, 3);
    interleave();
    mfma_step(U1);
    unpack_step(U0, 4);
    lread(C, 3);
    interleave();
    mfma_step(U0);
    unpack_step(U1, 5);
    interleave();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA of slice s + 1
    barrier_lds();
    lread(NX, 0);
    // Step 5 by hand: MF groups of one MFMA, a share of the unpack of step 6
    // and a share of the DMA of slice s + 2, so the loads issue in the MFMAs'
    // shadow instead of in a burst before them.  The DMA is unconditional (no
    // branch around MFMA code, whose accumulators would be copied at the
    // join): in the last two slices it reloads the last slice into stage c,
    // whose reads all completed before the barrier above; the epilogue waits
    // for it before it reuses the stages.
    {
      const uint32_t sl = (uint32_t)min(s + 2, nslices - 1) * kSlice;
      const uint32_t off[2] = {lane_off[0] + sl, lane_off[1] + sl};
#pragma unroll
      for (int k = 0; k < MF; ++k) {
        acc[k / FN][k % FN] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
            U1[FM + k % FN], U1[k / FN], acc[k / FN][k % FN], 0, 0, 0);
#pragma unroll
        for (int pc = k * 2 * NF / MF; pc < (k + 1) * 2 * NF / MF; ++pc)
          unpack_half(U0, 6, pc / 2, pc % 2);
#pragma unroll
        for (int j = k * kDma / MF; j < (k + 1) * kDma / MF; ++j) dma_one(j, off, C);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    mfma_step(U0);
    unpack_step(U1, 7);
    interleave();
    mfma_step(U1);
    unpack_step(U0, 0);
    lread(NX, 1);
    interleave();
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  slice(0, S0{}, std::true_type{});
  for (int s = 1; s < nslices; s += 2) {
    slice(s, S1{}, std::false_type{});
    if (s + 1 < nslices) slice(s + 1, S0{}, std::false_type{});
  }

  // ---- epilogue.  acc[i][j] is the transposed tile: output row m, column n of
  // the 32 x 32 tile sits in lane (m % 32) + 32 * ((n / 4) % 2), register
  // (n % 4) + 4 * (n / 8): runs of 4 columns of one row per lane.
  // The stages are free once every wave is past its last fragment read and
  // its last (redundant) DMA has landed.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // The epilogue's lane-derived indices are computed here from the lane's own
  // position (mbcnt over all lanes), not kept live across the K loop, which
  // holds 256 VGPRs and would spill them.
  const int el = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int rl = el & 31;
  float sxr[FM];
  float zr[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    sxr[i] = lds_sx[wm * 128 + i * 32 + rl];
    zr[i] = lds_z[wm * 128 + i * 32 + rl];
  }
  if constexpr (GATED) {
    // SiLU-gated MLP (dscq_matmul_silu_mul): the weight rows are interleaved in
    // blocks of 64 -- gate rows of 64 outputs, then the up rows of the same
    // outputs -- so a wave's 128 columns hold gate (MFMA tiles j = 0, 1) and up
    // (j = 2, 3) of 64 outputs, element for element in the same lane and
    // register.  Each pair is narrowed to fp16 as the GEMM output would be and
    // combined into h = silu_mul_f16x2(g, u) (rowquant.h, the arithmetic of
    // the pipelined kernel's gated epilogue and of the requantizing kernel);
    // the wave's 128 x 64 h tile goes through LDS (rows of 128 bytes, the
    // 128-column layout of the plain epilogue) and out to h [M, N / 2].
    constexpr int HRB = 128, HCPR = 8, HRPI = 8;
    uint8_t* const tile = smem + wave * (128 * HRB);
    const int half = ((el >> 5) ^ (rl >> 3)) & 1;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cg = wn * TN + j * 32 + 8 * q + 4 * (el >> 5), cu = cg + 64;
        const float4 swg = *reinterpret_cast<const float4*>(lds_sw + cg);
        const float4 smg = *reinterpret_cast<const float4*>(lds_sum + cg);
        const float4 swu = *reinterpret_cast<const float4*>(lds_sw + cu);
        const float4 smu = *reinterpret_cast<const float4*>(lds_sum + cu);
        float4 bg = make_float4(0.0f, 0.0f, 0.0f, 0.0f), bu = bg;
        if (BIAS) {
          bg = *reinterpret_cast<const float4*>(lds_b + cg);
          bu = *reinterpret_cast<const float4*>(lds_b + cu);
        }
        const float swg_[4] = {swg.x, swg.y, swg.z, swg.w}, smg_[4] = {smg.x, smg.y, smg.z, smg.w};
        const float swu_[4] = {swu.x, swu.y, swu.z, swu.w}, smu_[4] = {smu.x, smu.y, smu.z, smu.w};
        const float bg_[4] = {bg.x, bg.y, bg.z, bg.w}, bu_[4] = {bu.x, bu.y, bu.z, bu.w};
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          float gv[4], uv[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            // Operation order of kernel/w4a4.cu:74-77, as in the plain epilogue.
            gv[v] = fmaf(zr[i], smg_[v], (float)acc[i][j][4 * q + v]) * sxr[i];
            gv[v] = gv[v] * swg_[v];
            uv[v] = fmaf(zr[i], smu_[v], (float)acc[i][j + 2][4 * q + v]) * sxr[i];
            uv[v] = uv[v] * swu_[v];
            if (BIAS) {
              gv[v] = gv[v] + bg_[v];
              uv[v] = uv[v] + bu_[v];
            }
          }
          uint2 pk;
          pk.x = silu_mul_f16x2(pack_h2(gv[0], gv[1]), pack_h2(uv[0], uv[1]));
          pk.y = silu_mul_f16x2(pack_h2(gv[2], gv[3]), pack_h2(uv[2], uv[3]));
          const int r = i * 32 + rl;
          *reinterpret_cast<uint2*>(tile + r * HRB + 16 * ((4 * j + q) ^ (r & 7)) + 8 * half) = pk;
        }
      }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __half* const hout = static_cast<__half*>(g.out);
    const int64_t NH = g.N / 2;
    const int c = el % HCPR;
    const int64_t hcol = n0 / 2 + wn * 64 + 8 * c;
    const bool whole = m0 + kTileM <= g.M && n0 + BN <= g.N;
    uint8_t* const obase =
        reinterpret_cast<uint8_t*>(hout) + 2 * ((m0 + wm * 128) * NH + n0 / 2 + wn * 64);
    const uint32_t out_off = (uint32_t)(2 * ((el / HCPR) * NH + 8 * c));
    constexpr int kBatch = 8;
#pragma unroll
    for (int sb = 0; sb < 128 / HRPI; sb += kBatch) {
      uint4 v[kBatch];
#pragma unroll
      for (int t = 0; t < kBatch; ++t) {
        const int sr = sb + t;
        const int r = HRPI * sr + el / HCPR;
        v[t] = *reinterpret_cast<const uint4*>(tile + r * HRB + 16 * (c ^ (r & 7)));
        if (sr & 1) {  // bit 3 of r: halves stored swapped
          const uint32_t x = v[t].x, y = v[t].y;
          v[t].x = v[t].z;
          v[t].y = v[t].w;
          v[t].z = x;
          v[t].w = y;
        }
      }
      if (whole) {
#pragma unroll
        for (int t = 0; t < kBatch; ++t)
          store_stream(v[t], obase + 2 * (int64_t)(HRPI * (sb + t)) * NH + out_off);
      } else {
#pragma unroll
        for (int t = 0; t < kBatch; ++t) {
          const int64_t row = m0 + wm * 128 + HRPI * (sb + t) + el / HCPR;
          if (row < g.M && hcol < NH) store_stream(v[t], hout + row * NH + hcol);
        }
      }
    }
    return;
  }
  // The wave's 128 x TN fp16 tile in LDS: row r (RB = 2 TN bytes, CPR 16-byte
  // chunks) holds chunk c at position c ^ (r % CPR), the two 8-byte halves of a
  // chunk swapped in rows with bit log2(CPR) set, so that a half-wave's 8-byte
  // writes (rows r .. r + 31) spread over the banks and every row's 16-byte
  // reads cover them.
  constexpr int RB = 2 * TN, CPR = TN / 8, LCPR = CPR == 16 ? 4 : 3, RPI = 64 / CPR;
  uint8_t* const tile = smem + wave * (128 * RB);
  const int half = ((el >> 5) ^ (rl >> LCPR)) & 1;
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int cl = wn * TN + j * 32 + 8 * q + 4 * (el >> 5);
      const float4 sw = *reinterpret_cast<const float4*>(lds_sw + cl);
      const float4 sm = *reinterpret_cast<const float4*>(lds_sum + cl);
      float4 bv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (BIAS) bv = *reinterpret_cast<const float4*>(lds_b + cl);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const v16i& a = acc[i][j];
        float r0 = fmaf(zr[i], sm.x, (float)a[4 * q + 0]) * sxr[i];
        float r1 = fmaf(zr[i], sm.y, (float)a[4 * q + 1]) * sxr[i];
        float r2 = fmaf(zr[i], sm.z, (float)a[4 * q + 2]) * sxr[i];
        float r3 = fmaf(zr[i], sm.w, (float)a[4 * q + 3]) * sxr[i];
        r0 = r0 * sw.x;
        r1 = r1 * sw.y;
        r2 = r2 * sw.z;
        r3 = r3 * sw.w;
        if (BIAS) {
          r0 = r0 + bv.x;
          r1 = r1 + bv.y;
          r2 = r2 + bv.z;
          r3 = r3 + bv.w;
        }
        uint2 pk;
        pk.x = pack_h2(r0, r1);
        pk.y = pack_h2(r2, r3);
        const int r = i * 32 + rl;
        *reinterpret_cast<uint2*>(tile + r * RB + 16 * ((4 * j + q) ^ (r & (CPR - 1))) +
                                  8 * half) = pk;
      }
    }
  // A wave reads back only what its own lanes wrote.
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __half* const out = static_cast<__half*>(g.out);
  const int c = el % CPR;
  const int64_t col = n0 + wn * TN + 8 * c;
  // A tile inside the output stores without per-row tests: a wave-uniform row
  // base plus a 32-bit lane offset, the LDS reads of eight store instructions
  // issued before their stores.
  const bool whole = m0 + kTileM <= g.M && n0 + BN <= g.N;
  uint8_t* const obase =
      reinterpret_cast<uint8_t*>(out) + 2 * ((m0 + wm * 128) * g.N + n0 + wn * TN);
  const uint32_t out_off = (uint32_t)(2 * ((el / CPR) * g.N + 8 * c));
  constexpr int kBatch = 8;
#pragma unroll
  for (int sb = 0; sb < 128 / RPI; sb += kBatch) {
    uint4 v[kBatch];
#pragma unroll
    for (int t = 0; t < kBatch; ++t) {
      const int sr = sb + t;
      const int r = RPI * sr + el / CPR;
      v[t] = *reinterpret_cast<const uint4*>(tile + r * RB + 16 * (c ^ (r & (CPR - 1))));
      if ((sr >> (2 * LCPR - 6)) & 1) {  // bit log2(CPR) of r: halves stored swapped
        const uint32_t x = v[t].x, y = v[t].y;
        v[t].x = v[t].z;
        v[t].y = v[t].w;
        v[t].z = x;
        v[t].w = y;
      }
    }
    if (whole) {
#pragma unroll
      for (int t = 0; t < kBatch; ++t)
        store_stream(v[t], obase + 2 * (int64_t)(RPI * (sb + t)) * g.N + out_off);
    } else {
#pragma unroll
      for (int t = 0; t < kBatch; ++t) {
        const int64_t row = m0 + wm * 128 + RPI * (sb + t) + el / CPR;
        if (row < g.M && col < g.N) store_stream(v[t], out + row * g.N + col);
      }
    }
  }
}

}  // namespace

bool wide_gemm_fits(const GemmArgs& g) {
  const int64_t KB = g.KP / 2;
  return g.raw == nullptr && g.M >= 1 && g.N % 8 == 0 && KB % kSlice == 0 && KB > 0 &&
         g.KP <= 65536 && (reinterpret_cast<uintptr_t>(g.out) & 15) == 0 &&
         g.arows * KB <= 0xFFFFFFFFll && g.brows * KB <= 0xFFFFFFFFll;
}

int launch_wide_gemm(GemmArgs g, int bn, hipStream_t stream) {
  if (!wide_gemm_fits(g) || (bn != 256 && bn != 128))
    return fail("internal: shape outside the wide-tile GEMM");
  g.tiles_n = (int)((g.N + bn - 1) / bn);
  const int64_t nblocks = ((g.M + kTileM - 1) / kTileM) * g.tiles_n;
  if (nblocks > 0x7FFFFFFF) return fail("matmul: grid too large");
  const dim3 grid((unsigned)nblocks), block(64 * kWaves);
#define DSCQ_WIDE(BNV)                                                   \
  if (g.bias)                                                            \
    launch(w4a4_gemm_wide_kernel<BNV, true>, grid, block, stream, g);    \
  else                                                                   \
    launch(w4a4_gemm_wide_kernel<BNV, false>, grid, block, stream, g);
  if (bn == 256) {
    DSCQ_WIDE(256)
  } else {
    DSCQ_WIDE(128)
  }
#undef DSCQ_WIDE
  return launch_status("w4a4_gemm_wide_kernel");
}

int launch_wide_gemm_gated(GemmArgs g, hipStream_t stream) {
  if (!wide_gemm_fits(g) || g.N % 128 != 0)
    return fail("internal: shape outside the gated wide-tile GEMM");
  g.tiles_n = (int)((g.N + 255) / 256);
  const int64_t nblocks = ((g.M + kTileM - 1) / kTileM) * g.tiles_n;
  if (nblocks > 0x7FFFFFFF) return fail("matmul_silu_mul: grid too large");
  const dim3 grid((unsigned)nblocks), block(64 * kWaves);
  if (g.bias)
    launch((w4a4_gemm_wide_kernel<256, true, true>), grid, block, stream, g);
  else
    launch((w4a4_gemm_wide_kernel<256, false, true>), grid, block, stream, g);
  return launch_status("w4a4_gemm_wide_kernel");
}

}  // namespace dscq
