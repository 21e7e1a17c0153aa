/*
 * dscq.h — C ABI of the MI355X (gfx950) W4A4 linear-layer library
 * (libdscq.so, built from dscquant_amd/csrc/).
 *
 * Plain pointers and sizes only.  Every device pointer is HIP device memory
 * on the current device; `stream` is a hipStream_t (NULL = the default
 * stream).  Calls are asynchronous on `stream` and never synchronize.
 *
 * Return value: DSCQ_OK (0) on success; DSCQ_EINVAL (-1) when an argument
 * check fails (nothing was launched; the message is in dscq_last_error());
 * otherwise the positive hipError_t returned by the launch.
 *
 * Padded layout (the reference extension's, kernel/w4a4.cu:170,196):
 *   MP = ceil(M / 8) * 8,  NP = ceil(N / 8) * 8,  KP = ceil(K / 64) * 64.
 * Packed int4 matrices are row-major u8 [rows, KP/2]; byte j of a row holds
 * element 2j in its low nibble and 2j+1 in its high nibble.
 */
#ifndef DSCQ_H
#define DSCQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSCQ_OK 0
#define DSCQ_EINVAL (-1)

/* Element types of floating-point tensors. */
#define DSCQ_F16 0
#define DSCQ_F32 1

/*
 * Per-token activation quantization + int4 packing, optionally preceded by
 * an online block rotation.
 * Replaces the reference extension's `quantize(x, clip, fused)`
 * (kernel/w4a4.cu:164-187, kernels :20-68) and follows the rule of
 * activation_codes (core/quantization.py:13-21).
 *
 *   x        [M, K] fp16 or fp32 (x_dtype), row-major, contiguous.
 *   clip     activation clip ratio, 0.5 <= clip <= 1 (w4a4.cu:168).
 *   fused    1: one kernel writes `packed` directly (w4a4.cu:177);
 *            0: a codes kernel writes `codes` [MP, KP] u8 (values 0..15),
 *               then a pack kernel writes `packed` (w4a4.cu:178-185).
 *   rotate_block  0 = no rotation; 128 = unnormalised Sylvester Hadamard
 *            H_128 applied to every 128-wide block of each row before
 *            quantization (K must be a multiple of 128).  Pair it with
 *            weights packed by dscq_pack_weight(..., rotate_block = 128).
 *   packed   out u8 [MP, KP/2]; nibble = (q - 8) & 15.
 *   scales   out f32 [MP]; zeros out i32 [MP] (padded rows: 1e-8, 0).
 *   codes    scratch/out u8 [MP, KP] when fused == 0, else ignored (may be NULL).
 * Limits (w4a4.cu:166): 1 <= M <= 65535, 1 <= K <= 1048576.
 */
int dscq_quantize(const void* x, int x_dtype, int64_t M, int64_t K, float clip,
                  int fused, int rotate_block, uint8_t* packed, float* scales,
                  int32_t* zeros, uint8_t* codes, void* stream);

/*
 * Quantize + pack of the SiLU-gated activation between the up and down
 * projections of a gated MLP (the caller of two QuantLinear layers in a
 * Llama MLP: down(act_fn(gate(x)) * up(x)); core/model_ops.py drives such
 * models, core/linear.py:48-52 quantizes the down projection's input).  The
 * rows quantized are h = fp16(fp16(silu(g)) * u) with silu(g) = g / (1 + e^-g)
 * in fp32 -- the two roundings an fp16 model applies -- then exactly as
 * dscq_quantize(h, F16, M, N, clip, fused = 1, rotate_block).  No reference
 * counterpart exists: the reference runs these ops unquantized in torch.
 *   gate, up  fp16 rows [M, >= N] with row stride ld elements (e.g. the two
 *             halves of one [M, 2N] gate|up GEMM output: up = gate + N,
 *             ld = 2N); 16-byte aligned, N % 8 == 0 and ld % 8 == 0.
 *   packed, scales, zeros  as dscq_quantize (MP = ceil(M/8)*8, KP = ceil(N/64)*64).
 *   h         optional out fp16 [M, N]: the activation quantized (may be NULL).
 * Limits: 1 <= M <= 65535, 1 <= N <= 32768.
 */
int dscq_silu_mul_quantize(const void* gate, const void* up, int64_t ld, int64_t M,
                           int64_t N, float clip, int rotate_block, uint8_t* packed,
                           float* scales, int32_t* zeros, void* h, void* stream);

/*
 * The gate and up projections of a SiLU-gated MLP and the activation between
 * them in one GEMM: h = fp16(fp16(silu(g)) * u) with g, u the fp16 outputs
 * dscq_matmul(a, gate / up weights, ..., fused = 1) would give, and silu as
 * in dscq_silu_mul_quantize (bit-identical h).  dscq_quantize(h, ...) then
 * gives the down projection's input, as dscq_silu_mul_quantize does, without
 * the [M, 2N] gate|up output going through HBM.  No reference counterpart
 * exists: it replaces the gate and up QuantLinear calls of core/linear.py:48-52
 * and the unquantized torch activation between them.
 *   a, sx, zx  as dscq_matmul (the quantized MLP input, KP = ceil(K/64)*64).
 *   b_gu       u8 [2N, KP/2]: gate and up weights packed as dscq_pack_weight
 *              does, rows interleaved in 64-row blocks: rows 128t .. 128t+63
 *              are gate rows 64t .. 64t+63, rows 128t+64 .. 128t+127 the up
 *              rows 64t .. 64t+63.
 *   sw, sums   f32 / i32 [2N] in the same row order; bias NULL or fp16 [2N]
 *              in the same order (added to g and u before the activation).
 *   h          out fp16 [M, N], 16-byte aligned.
 * Limits: 1 <= M <= 65535, N % 64 == 0, KP <= 65536.
 */
int dscq_matmul_silu_mul(const uint8_t* a, const uint8_t* b_gu, const float* sx,
                         const int32_t* zx, const float* sw, const int32_t* sums,
                         const void* bias, int64_t M, int64_t N, int64_t KP, void* h,
                         void* stream);

/*
 * Activation codes with any bit width 2..8 (no packing), the GPU form of
 * activation_codes (core/quantization.py:13-21) on the padded layout.
 *   codes  out u8 [MP, KP] in [0, 2^bits - 1] (padded k / rows: the row's zero)
 *   scales out f32 [MP], zeros out i32 [MP].
 * clip may be any value in (0, 1].  rotate_block as in dscq_quantize.
 */
int dscq_activation_codes(const void* x, int x_dtype, int64_t M, int64_t K,
                          float clip, int bits, int rotate_block,
                          uint8_t* codes, float* scales, int32_t* zeros,
                          void* stream);

/*
 * Weight-side glue of the W4A4 GEMM: per-output-channel symmetric int4 codes
 * (weight_codes, core/quantization.py:7-11, bits = 4), packed as pack_int4
 * (core/quantization.py:31-40) into the padded operand `b` of dscq_matmul,
 * plus the per-channel scale `sw` and code sums `sums` the epilogue needs
 * (kernel/w4a4.cu:74-75, shape contract :195-200).  The reference leaves
 * this glue unwritten; its layout is pinned by matmul's checks.
 *   w       [N, K] fp16 or fp32 (w_dtype), row-major.
 *   clip    weight clip ratio in (0, 1].
 *   rotate_block 0, or 128: quantize W' = W H_128 / 128 (blockwise, exact
 *           power-of-two scale), the fold that pairs with the rotated
 *           activations of dscq_quantize (rule of core/linear.py:34-37).
 *   packed  out u8 [NP, KP/2] (padding: code 0); sw out f32 [NP];
 *   sums    out i32 [NP] (padded rows: sw 0, sums 0).
 *   codes   optional out int8 [NP, KP] (the signed codes), may be NULL.
 * Limits: 1 <= N <= 1048576, 1 <= K <= 1048576.
 */
int dscq_pack_weight(const void* w, int w_dtype, int64_t N, int64_t K,
                     float clip, int rotate_block, uint8_t* packed, float* sw,
                     int32_t* sums, int8_t* codes, void* stream);

/*
 * Weight codes with any bit width 2..8 (no packing): codes int8 [NP, KP] in
 * [-(2^(bits-1)-1), 2^(bits-1)-1], scales f32 [NP].  The GPU form of
 * weight_codes (core/quantization.py:7-11).  rotate_block as in
 * dscq_pack_weight.
 */
int dscq_weight_codes(const void* w, int w_dtype, int64_t N, int64_t K,
                      float clip, int bits, int rotate_block, int8_t* codes,
                      float* scales, void* stream);

/*
 * Packed-int4 x packed-int4 GEMM with int32 accumulation and the fused
 * zero-point / scale / bias epilogue.  Replaces the reference extension's
 * `matmul(a, b, sx, zx, sw, sums, bias, M, N, fused, force_decode, fp32)`
 * (kernel/w4a4.cu:189-225, kernels :70-161):
 *   raw[m, n] = sum_{k < KP} (a nibble - 16*(a nibble >= 8)) * (b nibble ...)
 *   out[m, n] = (float)(raw + (8 - zx[m]) * sums[n]) * sx[m] * sw[n] (+ bias[n])
 *   a     u8 [>= MP, KP/2] activations (dscq_quantize's `packed`).
 *   b     u8 [>= NP, KP/2] weights (dscq_pack_weight's `packed`).
 *   sx    f32 [>= MP], zx i32 [>= MP], sw f32 [>= NP], sums i32 [>= NP].
 *   bias  NULL or [N] of the output type.
 *   KP    packed width * 2; a multiple of 64, 64 <= KP <= 1048576.
 *   fused 1: out only (raw may be NULL); 0: out and raw [M, N] int32
 *         (the reference's raw-accumulator mode).
 *   force_decode  selects the skinny-M kernel (the reference's decode_gemm,
 *         dispatched there for M < 8) regardless of M; it is also chosen for
 *         M <= 16, and for M < 64 unless N > 8064 (64+ column tiles of 128).
 *         Results are identical either way.
 *   out_fp32  0: out is fp16 [M, N]; 1: fp32.
 * Limits (w4a4.cu:197): 1 <= M <= 65535, N >= 1.
 */
int dscq_matmul(const uint8_t* a, const uint8_t* b, const float* sx,
                const int32_t* zx, const float* sw, const int32_t* sums,
                const void* bias, int64_t M, int64_t N, int64_t KP, int fused,
                int force_decode, int out_fp32, void* out, int32_t* raw,
                void* stream);

/* dscq_matmul with a caller-provided device workspace (no counterpart in the
 * reference, whose matmul, kernel/w4a4.cu:189-225, allocates only its
 * outputs; the Python matmul allocates the workspace the same way, from
 * torch's allocator).  Shapes for which one round of 64 x 128 tiles leaves the
 * K loop's latency exposed (small M with few output tiles, long K) then split
 * K over workgroups: int32 partial sums per part go to the workspace and a
 * second kernel adds them and applies the epilogue.  Integer partial sums add
 * exactly, so the results are bit-identical to dscq_matmul's.
 *   workspace        NULL, or 16-byte aligned device memory of
 *                    workspace_bytes; too small, misaligned or NULL: no split.
 * Every other argument and error is as for dscq_matmul.  The workspace is
 * scratch for this call only; calls that may overlap need their own. */
int dscq_matmul_ws(const uint8_t* a, const uint8_t* b, const float* sx,
                   const int32_t* zx, const float* sw, const int32_t* sums,
                   const void* bias, int64_t M, int64_t N, int64_t KP, int fused,
                   int force_decode, int out_fp32, void* out, int32_t* raw,
                   void* workspace, int64_t workspace_bytes, void* stream);

/* dscq_matmul that allocates nothing: no counterpart in the reference; it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture that forbids allocation, tight serving loops, harnesses that forbid
 * hipMalloc).  Arguments, errors and results are dscq_matmul's (bit-identical
 * to dscq_matmul_ws with a workspace).  The K split's int32 partial sums go
 * to a fixed device array of the library, DSCQ_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends; a shape whose split would need more returns
 * DSCQ_EINVAL (on a 256-CU MI355X no shape does).  Calls on one GPU share
 * that array, so calls that may overlap on one GPU race: serialize them on
 * one stream.  Nothing in it needs clearing between calls. */
#define DSCQ_NOALLOC_SCRATCH_BYTES (8LL << 20)
int dscq_matmul_noalloc(const uint8_t* a, const uint8_t* b, const float* sx,
                        const int32_t* zx, const float* sw, const int32_t* sums,
                        const void* bias, int64_t M, int64_t N, int64_t KP, int fused,
                        int force_decode, int out_fp32, void* out, int32_t* raw,
                        void* stream);

/* Bytes of workspace dscq_matmul_ws uses for this shape (0: it does not split;
 * the workspace may then be NULL), or a negative value for invalid dimensions
 * (as dscq_matmul reports them).  Host-only: launches nothing. */
int64_t dscq_matmul_workspace_bytes(int64_t M, int64_t N, int64_t KP, int force_decode);

/*
 * Standalone int4 packer for signed codes already in [-8, 7]: the GPU form
 * of pack_int4 (core/quantization.py:31-40; range checking is the caller's,
 * see dscquant_amd.core.quantization.pack_int4).
 *   codes int8 [R, C] -> packed u8 [R, ceil(C/2)] (odd width padded with 0).
 */
int dscq_pack_int4(const int8_t* codes, int64_t R, int64_t C, uint8_t* packed,
                   void* stream);

/* The GPU form of unpack_int4 (core/quantization.py:42-45):
 * packed u8 [R, CB] -> codes int8 [R, width], width <= 2*CB. */
int dscq_unpack_int4(const uint8_t* packed, int64_t R, int64_t CB,
                     int64_t width, int8_t* codes, void* stream);

/*
 * Fused decode linear: the quantize and matmul steps of a W4A4 linear layer
 * in one launch, for a few tokens.  Equal, bit for bit, to
 *   dscq_quantize(x, x_dtype, M, K, clip, fused = 1, rotate_block, a, sx, zx)
 *   dscq_matmul(a, b, sx, zx, sw, sums, bias, M, N, KP, fused = 1, ...)
 * (kernel/w4a4.cu:164-225 called back to back, as QuantLinear's forward
 * does, core/linear.py:48-52), without the intermediate buffers.  Each
 * workgroup re-quantizes the M rows it needs while its weight stripe streams
 * in, so the launch costs what the weight stream costs.
 *   x      fp16 / fp32 [M, K], 16-byte aligned, K % 8 == 0.
 *   b, sw, sums, bias, out_fp32, out  as dscq_matmul (b: [>= NP, KP/2]).
 * Limits: dscq_linear_decode_supported(M, K) must hold (M <= 4 at K = 4096,
 * M = 1 up to K = 12288); otherwise DSCQ_EINVAL, and the caller runs
 * dscq_quantize + dscq_matmul.  No reference counterpart: it replaces the
 * pair above on the decode path.
 */
int dscq_linear_decode(const void* x, int x_dtype, int64_t M, int64_t K, float clip,
                       int rotate_block, const uint8_t* b, const float* sw,
                       const int32_t* sums, const void* bias, int64_t N, int out_fp32,
                       void* out, void* stream);

/* 1 if dscq_linear_decode accepts an [M, K] input, else 0. */
int dscq_linear_decode_supported(int64_t M, int64_t K);

/*
 * 1 if the current HIP device is a gfx950 (MI355X-class) GPU the kernels
 * were built for, 0 if not, negative hipError_t if no device is usable.
 * Replaces the SM75-89 capability check of kernel/w4a4.cu:204-206.
 */
int dscq_device_supported(void);

/*
 * Kernel timing without a profiler (no reference counterpart): the next call
 * the calling thread makes into this library stamps the device start and end
 * times of its kernel into the HIP events `start` and `stop` (hipEvent_t created
 * with timing enabled; either may be NULL).  The launch goes through
 * hipExtLaunchKernel, so hipEventElapsedTime(start, stop) is the kernel's
 * duration as a kernel trace reports it, without the event markers and
 * dispatch gaps of events recorded around the call.  An entry point that
 * launches two kernels (a K-split matmul: partial sums, then their reduction)
 * stamps the start of the first and the end of the second.  Not for use under
 * graph capture.
 */
int dscq_time_next_kernel(void* start, void* stop);

/*
 * GEMM kernel choice for this thread's later dscq_matmul / dscq_matmul_ws /
 * dscq_matmul_noalloc / dscq_matmul_silu_mul calls (no reference counterpart;
 * the analogue of the reference's force_decode for the dense kernels, for
 * tests and measurement):
 *   0  automatic (the default): for fp16 output without raw accumulators the
 *      wide-tile kernel (256 x 256 tiles, one wave per SIMD) when its tiles
 *      fill at least three quarters of a round of one tile per compute unit
 *      and its rounds take no longer than the pipelined kernel's, else the
 *      pipelined kernel;
 *   1  the wide-tile kernel wherever it applies (fp16 output, no raw
 *      accumulators, N % 8 == 0, K a multiple of 256, KP <= 65536, M >= 64),
 *      with the tile width the automatic rule would take (256 by default);
 *   2  never the wide-tile kernel;
 *   3, 4  the wide-tile kernel wherever it applies, with 256 x 256 / 256 x 128
 *      tiles.
 * dscq_matmul_silu_mul (M > 16) follows the same choices with 256 x 256 tiles
 * only: settings 1 and 3 and the automatic rule may take the wide-tile kernel,
 * 4 takes the pipelined kernel.
 * Every kernel gives the same results.  Returns the previous setting, or
 * DSCQ_EINVAL for another value.
 */
int dscq_set_gemm_kernel(int which);

/*
 * Measurement probes (no reference counterpart): the ceilings the kernels
 * above are compared against, timed on the same device in the same run (with
 * dscq_time_next_kernel like any other call).
 *
 * dscq_stream_probe: a plain streaming kernel.  Each thread reads `pieces`
 * (1, 2, 4, 8 or 16) 16-byte pieces of `src`, thread t the pieces t + j * T
 * (T = read_bytes / (16 * pieces) threads, so each load instruction of a wave
 * reads 1 KiB contiguous), and
 *   write_bytes == read_bytes / pieces: writes their XOR to dst piece t
 *     (with pieces = 4 over fp16 input: exactly the bytes of an activation
 *     quantize, read 2 M K and write M K / 2);
 *   write_bytes == 0: writes nothing (a bare read; dst, 16 bytes, receives a
 *     piece only if some thread's pieces XOR to a fixed 128-bit constant).
 * src and dst 16-byte aligned; read_bytes a positive multiple of 16 * pieces.
 */
int dscq_stream_probe(const void* src, int64_t read_bytes, void* dst, int64_t write_bytes,
                      int pieces, void* stream);

/*
 * dscq_mfma_probe: the matrix cores alone.  `workgroups` workgroups of `waves`
 * (1..8) waves; each wave issues `mfmas_per_wave` (a multiple of 8)
 * v_mfma_i32_32x32x32_i8 on register operands, four per step over a 2 x 2
 * block of accumulators (a pipelined-GEMM wave's step), with no memory
 * traffic in the loop, alternating two operand sets.  Operand bytes vary over
 * lanes and bytes (multiples of 16 in [-128, 96], as unpacked int4 operands);
 * out[workgroup * waves + wave] (int32) receives the wave's wrapping sum of all
 * its accumulator elements, a closed form of the operand values that does not
 * depend on the operand layout (the checksum the GPU tests recompute).  256 workgroups of 8 waves and 512 MFMAs per
 * wave are the 2 M N K operations of a 2048 x 4096 x 4096 GEMM.
 */
int dscq_mfma_probe(int64_t workgroups, int waves, int64_t mfmas_per_wave, int32_t* out,
                    void* stream);

/* Message of the last DSCQ_EINVAL / launch failure on this thread. */
const char* dscq_last_error(void);

/* Library version string. */
const char* dscq_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DSCQ_H */
