/*
 * CPU oracle for the DSCQuant W4A4 linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the reference the HIP kernels are
 * compared against; nothing in the product (dscquant_amd/) links, loads or
 * calls it.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may use it.
 *
 * It restates, in plain C with IEEE fp32 arithmetic (correctly rounded
 * + - * /, round-half-even, no contraction: build with -ffp-contract=off),
 * the reference's quantization rules and the W4A4 extension's padding,
 * packing, integer GEMM and dequant epilogue.  Every function cites the
 * reference lines it follows (paths relative to the reference repository).
 *
 * Pinning (tests/test_oracle.py): closed-form special cases, exact .5 ties,
 * range invariants, the exhaustive 16x16 nibble table, brute-force int64 GEMM
 * against numpy's integer matmul, FWHT against the dense Sylvester matrix,
 * and the fake-quant identity F.linear(x_hat, W_hat) = sx*sw*sum((q-z)*c).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

static inline float clampf(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

/* fp32 round-half-even (torch.round, __float2int_rn); default FE mode is RNE. */
static inline float rne(float v) { return rintf(v); }

/*
 * Per-token asymmetric activation codes.
 * core/quantization.py:13-21 (activation_codes):
 *   lo    = min(amin(x), 0) * clip                       (:15)
 *   hi    = max(amax(x), 0) * clip                       (:16)
 *   scale = max((hi - lo) / (2^bits - 1), 1e-8)           (:17-18)
 *   zero  = clamp(round(-lo / scale), 0, 2^bits - 1)      (:19)
 *   code  = clamp(round(x / scale + zero), 0, 2^bits - 1) (:20)
 * x is [M, K] fp32 (fp16 inputs are widened exactly by the caller).
 * codes: [M, K] u8; scales, zeros: [M] fp32 (zero is integer-valued).
 */
ORACLE_API void oracle_activation_codes(const float* x, int64_t M, int64_t K,
                                        float clip, int bits, uint8_t* codes,
                                        float* scales, float* zeros) {
  const float qmax = (float)((1 << bits) - 1);
  for (int64_t m = 0; m < M; ++m) {
    const float* row = x + m * K;
    float mn = row[0], mx = row[0];
    for (int64_t k = 1; k < K; ++k) {
      if (row[k] < mn) mn = row[k];
      if (row[k] > mx) mx = row[k];
    }
    float lo = (mn < 0.0f ? mn : 0.0f) * clip;
    float hi = (mx > 0.0f ? mx : 0.0f) * clip;
    float scale = (hi - lo) / qmax;
    if (scale < 1e-8f) scale = 1e-8f;
    float zero = clampf(rne(-lo / scale), 0.0f, qmax);
    for (int64_t k = 0; k < K; ++k) {
      float t = row[k] / scale + zero;
      codes[m * K + k] = (uint8_t)clampf(rne(t), 0.0f, qmax);
    }
    scales[m] = scale;
    zeros[m] = zero;
  }
}

/*
 * Per-output-channel symmetric weight codes.
 * core/quantization.py:7-11 (weight_codes):
 *   bound = 2^(bits-1) - 1                                  (:8)
 *   scale = max(amax(|w|) * clip / bound, 1e-8)             (:9)
 *   code  = clamp(round(w / scale), -bound, bound)          (:10)
 * w is [N, K] fp32; codes [N, K] int8; scales [N].
 */
ORACLE_API void oracle_weight_codes(const float* w, int64_t N, int64_t K,
                                    float clip, int bits, int8_t* codes,
                                    float* scales) {
  const float bound = (float)((1 << (bits - 1)) - 1);
  for (int64_t n = 0; n < N; ++n) {
    const float* row = w + n * K;
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float a = fabsf(row[k]);
      if (a > amax) amax = a;
    }
    float scale = amax * clip / bound;
    if (scale < 1e-8f) scale = 1e-8f;
    for (int64_t k = 0; k < K; ++k)
      codes[n * K + k] = (int8_t)clampf(rne(row[k] / scale), -bound, bound);
    scales[n] = scale;
  }
}

/*
 * Unnormalised Sylvester fast Walsh-Hadamard transform over consecutive
 * blocks of `block` elements (block a power of two) of every row, in place.
 * Butterfly order is fixed: index bit 0 first, then bit 1, ... so rounding is
 * reproducible; for the pair (i, i + 2^b) with bit b of i clear:
 *   x[i] <- x[i] + x[i+2^b],   x[i+2^b] <- x[i] - x[i+2^b].
 * This is the online activation rotation; the weight side is folded with
 * W * H / block (power-of-two, exact), so (W H / block)(H x) = W x.
 * The fold rule follows core/linear.py:34-37 (W' = W R for an orthogonal R,
 * here R = H/sqrt(block), symmetric) with the sqrt(block) factor moved from
 * the activation to the weight.
 */
ORACLE_API void oracle_fwht_rows(float* x, int64_t M, int64_t K, int block) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t b0 = 0; b0 + block <= K; b0 += block) {
      float* v = x + m * K + b0;
      for (int h = 1; h < block; h <<= 1) {
        for (int i = 0; i < block; ++i) {
          if (i & h) continue;
          float u = v[i], w = v[i + h];
          v[i] = u + w;
          v[i + h] = u - w;
        }
      }
    }
  }
}

/*
 * The W4A4 extension's quantize (kernel/w4a4.cu:20-54 fused, :55-68 unfused +
 * pack_rows): padded layout MP = ceil8(M), KP = ceil64(K).
 *   - real rows use the activation rule above (w4a4.cu:42-44, 50-52);
 *   - padded k (K <= k < KP) take q = zero (w4a4.cu:48);
 *   - padded rows (M <= m < MP) see lo = hi = 0: scale 1e-8, zero 0,
 *     every q = 0, so every byte is 0x88 (w4a4.cu:26-27, 42-44);
 *   - the stored nibble is (q - 8) & 15, low nibble = even k (w4a4.cu:53).
 * packed [MP, KP/2] u8, scales [MP], zeros [MP] int32, codes [MP, KP] u8
 * (codes may be NULL).
 */
ORACLE_API void oracle_quantize_rows(const float* x, int64_t M, int64_t K,
                                     float clip, uint8_t* packed, float* scales,
                                     int32_t* zeros, uint8_t* codes) {
  const int64_t MP = (M + 7) / 8 * 8, KP = (K + 63) / 64 * 64;
  for (int64_t m = 0; m < MP; ++m) {
    float mn = 0.0f, mx = 0.0f; /* fminf(0, .) / fmaxf(0, .) seeds */
    if (m < M)
      for (int64_t k = 0; k < K; ++k) {
        float v = x[m * K + k];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
      }
    float lo = mn * clip, hi = mx * clip;
    float scale = (hi - lo) / 15.0f;
    if (scale < 1e-8f) scale = 1e-8f;
    int zero = (int)clampf(rne(-lo / scale), 0.0f, 15.0f);
    scales[m] = scale;
    zeros[m] = zero;
    for (int64_t k = 0; k < KP; ++k) {
      int q = zero;
      if (m < M && k < K)
        q = (int)clampf(rne(x[m * K + k] / scale + (float)zero), 0.0f, 15.0f);
      if (codes) codes[m * KP + k] = (uint8_t)q;
      uint8_t nib = (uint8_t)((q - 8) & 15);
      uint8_t* byte = packed + m * (KP / 2) + k / 2;
      if (k & 1) *byte = (uint8_t)(*byte | (nib << 4));
      else *byte = nib;
    }
  }
}

/*
 * core/quantization.py:31-40 (pack_int4): signed [-8, 7] codes -> bytes,
 * byte j = (c[2j] & 15) | (c[2j+1] & 15) << 4, odd width padded with 0.
 * Range checking is the caller's (the Python wrapper raises ValueError).
 */
ORACLE_API void oracle_pack_int4(const int8_t* codes, int64_t R, int64_t C,
                                 uint8_t* packed) {
  const int64_t CB = (C + 1) / 2;
  for (int64_t r = 0; r < R; ++r)
    for (int64_t j = 0; j < CB; ++j) {
      int lo = codes[r * C + 2 * j] & 15;
      int hi = (2 * j + 1 < C) ? (codes[r * C + 2 * j + 1] & 15) : 0;
      packed[r * CB + j] = (uint8_t)(lo | (hi << 4));
    }
}

/* core/quantization.py:42-45 (unpack_int4): nibble >= 8 -> nibble - 16. */
ORACLE_API void oracle_unpack_int4(const uint8_t* packed, int64_t R, int64_t CB,
                                   int64_t width, int8_t* codes) {
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < width; ++c) {
      int nib = (packed[r * CB + c / 2] >> ((c & 1) * 4)) & 15;
      codes[r * width + c] = (int8_t)(nib >= 8 ? nib - 16 : nib);
    }
}

/*
 * Weight-side glue the GEMM consumes (shape contract kernel/w4a4.cu:195-200):
 * optional block rotation W' = W H / block (see oracle_fwht_rows), then
 * weight_codes (quantization.py:7-11), pack_int4 (:31-40) into [NP, KP/2]
 * with zero padding, sw [NP] and sums[n] = sum_k code[n, k] (the zero-point
 * correction term of kernel/w4a4.cu:74).  Padded rows N <= n < NP get
 * code 0, sw 0 and sums 0.
 * w is [N, K] fp32 (fp16 widened exactly).  scratch must hold N*K floats.
 */
ORACLE_API void oracle_pack_weight(const float* w, int64_t N, int64_t K,
                                   float clip, int block, float* scratch,
                                   int8_t* codes_scratch, uint8_t* packed,
                                   float* sw, int32_t* sums) {
  const int64_t NP = (N + 7) / 8 * 8, KP = (K + 63) / 64 * 64;
  memcpy(scratch, w, sizeof(float) * (size_t)(N * K));
  if (block > 0) {
    oracle_fwht_rows(scratch, N, K, block);
    const float inv = 1.0f / (float)block; /* power of two: exact */
    for (int64_t i = 0; i < N * K; ++i) scratch[i] *= inv;
  }
  oracle_weight_codes(scratch, N, K, clip, 4, codes_scratch, sw);
  memset(packed, 0, (size_t)(NP * (KP / 2)));
  for (int64_t n = 0; n < N; ++n) {
    int32_t s = 0;
    for (int64_t k = 0; k < K; ++k) {
      int c = codes_scratch[n * K + k];
      s += c;
      uint8_t nib = (uint8_t)(c & 15);
      uint8_t* byte = packed + n * (KP / 2) + k / 2;
      *byte = (uint8_t)(*byte | ((k & 1) ? (nib << 4) : nib));
    }
    sums[n] = s;
  }
  for (int64_t n = N; n < NP; ++n) {
    sw[n] = 0.0f;
    sums[n] = 0;
  }
}

static inline int sign4(int nib) { return nib >= 8 ? nib - 16 : nib; }

/*
 * Raw int32 accumulators of the W4A4 GEMM, kernel/w4a4.cu:80-121 (tensor
 * path) and :123-154 (decode path), which agree exactly:
 *   raw[m, n] = sum_{k < KP} sign4(a nibble[m, k]) * sign4(b nibble[n, k])
 * a [>=M, KP/2], b [>=N, KP/2] u8 (row-major, K contiguous).  Accumulates in
 * int64; returns 0, or -1 if any result leaves the int32 range.
 */
ORACLE_API int oracle_gemm_raw(const uint8_t* a, const uint8_t* b, int64_t M,
                               int64_t N, int64_t KP, int32_t* raw) {
  const int64_t KB = KP / 2;
  int bad = 0;
  for (int64_t m = 0; m < M; ++m) {
    const uint8_t* ar = a + m * KB;
    for (int64_t n = 0; n < N; ++n) {
      const uint8_t* br = b + n * KB;
      int64_t acc = 0;
      for (int64_t j = 0; j < KB; ++j) {
        acc += (int64_t)sign4(ar[j] & 15) * sign4(br[j] & 15);
        acc += (int64_t)sign4(ar[j] >> 4) * sign4(br[j] >> 4);
      }
      if (acc > INT32_MAX || acc < INT32_MIN) bad = 1;
      raw[m * N + n] = (int32_t)acc;
    }
  }
  return bad ? -1 : 0;
}

/*
 * Dequant epilogue, kernel/w4a4.cu:70-78 (restore_value):
 *   corrected = raw + (8 - zx[m]) * sums[n]      (= sum (q - z) * c)
 *   out = float(corrected) * sx[m] * sw[n] (+ bias[n])
 * evaluated left to right in fp32 with separate roundings (no fma).
 * bias may be NULL.  out is fp32 [M, N]; narrowing to fp16 (round to nearest
 * even) is the caller's.
 */
ORACLE_API void oracle_restore(const int32_t* raw, const float* sx,
                               const int32_t* zx, const float* sw,
                               const int32_t* sums, const float* bias,
                               int64_t M, int64_t N, float* out) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      int32_t corrected = raw[m * N + n] + (8 - zx[m]) * sums[n];
      float r = (float)corrected * sx[m];
      r = r * sw[n];
      if (bias) r = r + bias[n];
      out[m * N + n] = r;
    }
}
