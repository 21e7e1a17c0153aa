// extern "C" entry points of libdscq (declared in include/dscq.h): argument
// checks with the reference extension's messages (kernel/w4a4.cu:164-225),
// then asynchronous launches on the caller's stream.

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/dscq.h"
#include "common.h"
#include "gemm_args.h"

namespace dscq {

int row_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t MP, float clip,
              int mode, float qmax, int rotate_block, uint8_t* packed, uint8_t* codes,
              float* scales, int32_t* zeros, int32_t* sums, hipStream_t stream);
int pack_codes(const uint8_t* codes, uint8_t* packed, int64_t MP, int64_t KP,
               hipStream_t stream);
int silu_mul_quant(const void* gate, const void* up, int64_t ld, int64_t M, int64_t N,
                   int64_t MP, float clip, int rotate_block, uint8_t* packed, float* scales,
                   int32_t* zeros, void* hout, hipStream_t stream);
int pack_int4(const int8_t* codes, int64_t R, int64_t C, uint8_t* packed,
              hipStream_t stream);
int unpack_int4(const uint8_t* packed, int64_t R, int64_t CB, int64_t width,
                int8_t* codes, hipStream_t stream);
int w4a4_gemm(const uint8_t* a, const uint8_t* b, const float* sx, const int32_t* zx,
              const float* sw, const int32_t* sums, const void* bias, int64_t M,
              int64_t N, int64_t KP, bool decode, bool out_fp32, void* out,
              int32_t* raw, hipStream_t stream, int32_t* ws = nullptr, int64_t ws_bytes = 0);
int64_t w4a4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t KP, bool decode);
bool gemm_silu_mul_fits(int64_t M, int64_t NH, int64_t KP, const void* h);
int w4a4_gemm_silu_mul(const uint8_t* a, const uint8_t* b_gu, const float* sx,
                       const int32_t* zx, const float* sw, const int32_t* sums,
                       const void* bias, int64_t M, int64_t NH, int64_t KP, void* h,
                       hipStream_t stream);
bool linear_decode_fits(int64_t M, int64_t K);
int linear_decode(const void* x, int dtype, int64_t M, int64_t K, float clip, int rotate_block,
                  const uint8_t* b, const float* sw, const int32_t* sums, const void* bias,
                  int64_t N, bool out_fp32, void* out, hipStream_t stream);

namespace {
thread_local char g_last_error[512] = "";
thread_local KernelEvents g_kernel_events = {nullptr, nullptr};
thread_local int g_gemm_kernel = 0;
}  // namespace

int gemm_kernel_preference() { return g_gemm_kernel; }

KernelEvents take_kernel_events() {
  const KernelEvents ev = g_kernel_events;
  g_kernel_events = {nullptr, nullptr};
  return ev;
}

void arm_kernel_events(KernelEvents ev) { g_kernel_events = ev; }

int cu_count() {
  // Per device, filled on first use; concurrent first calls store the same value.
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return DSCQ_EINVAL;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return DSCQ_OK;
  snprintf(g_last_error, sizeof(g_last_error), "%s launch failed: %s", what,
           hipGetErrorString(e));
  return (int)e;
}

namespace {

bool valid_dtype(int t) { return t == DSCQ_F16 || t == DSCQ_F32; }

int check_rotation(int rotate_block, int64_t K) {
  if (rotate_block != 0 && rotate_block != 128)
    return fail("rotate_block must be 0 or 128 (got %d)", rotate_block);
  if (rotate_block && K % rotate_block != 0)
    return fail("Rotation needs K to be a multiple of %d (got K=%lld)", rotate_block,
                (long long)K);
  return DSCQ_OK;
}

}  // namespace
}  // namespace dscq

using namespace dscq;

extern "C" {

const char* dscq_last_error(void) { return g_last_error; }

const char* dscq_version(void) { return "dscq 0.2.0 (gfx950)"; }

int dscq_time_next_kernel(void* start, void* stop) {
  g_kernel_events = {static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)};
  return DSCQ_OK;
}

int dscq_set_gemm_kernel(int which) {
  if (which < 0 || which > 4) return fail("set_gemm_kernel: 0 to 4 (got %d)", which);
  const int prev = g_gemm_kernel;
  g_gemm_kernel = which;
  return prev;
}

int dscq_device_supported(void) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return -(int)e;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int dscq_quantize(const void* x, int x_dtype, int64_t M, int64_t K, float clip, int fused,
                  int rotate_block, uint8_t* packed, float* scales, int32_t* zeros,
                  uint8_t* codes, void* stream) {
  DisarmOnExit disarm;
  // kernel/w4a4.cu:165-168
  if (!valid_dtype(x_dtype)) return fail("Only FP16 and FP32 inputs are supported");
  if (!(M > 0 && M <= 65535 && K > 0 && K <= 1048576))
    return fail("Require 1<=M<=65535 and 1<=K<=1048576");
  if (!(clip >= 0.5f && clip <= 1.0f)) return fail("Activation clip must be in [0.5,1]");
  if (int rc = check_rotation(rotate_block, K)) return rc;
  if (!x || !packed || !scales || !zeros) return fail("quantize: null buffer");
  if (!fused && !codes) return fail("quantize: the unfused path needs a codes buffer");
  const int64_t MP = ceil_to(M, 8), KP = ceil_to(K, 64);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fused)
    return row_quant(x, x_dtype, M, K, MP, clip, 0, 15.0f, rotate_block, packed, nullptr,
                     scales, zeros, nullptr, s);
  // Two kernels: timing events, if armed, span both.
  const KernelEvents ev = take_kernel_events();
  arm_kernel_events({ev.start, nullptr});
  if (int rc = row_quant(x, x_dtype, M, K, MP, clip, 0, 15.0f, rotate_block, nullptr,
                         codes, scales, zeros, nullptr, s))
    return rc;
  arm_kernel_events({nullptr, ev.stop});
  return pack_codes(codes, packed, MP, KP, s);
}

int dscq_linear_decode(const void* x, int x_dtype, int64_t M, int64_t K, float clip,
                       int rotate_block, const uint8_t* b, const float* sw,
                       const int32_t* sums, const void* bias, int64_t N, int out_fp32,
                       void* out, void* stream) {
  DisarmOnExit disarm;
  if (!valid_dtype(x_dtype)) return fail("Only FP16 and FP32 inputs are supported");
  if (!linear_decode_fits(M, K))
    return fail("linear_decode: M=%lld, K=%lld exceed the fused decode kernel (quantize + "
                "matmul instead)", (long long)M, (long long)K);
  if (!(N > 0 && N <= 0x7FFFFFFFLL)) return fail("Invalid dimensions");
  if (!(clip >= 0.5f && clip <= 1.0f)) return fail("Activation clip must be in [0.5,1]");
  if (int rc = check_rotation(rotate_block, K)) return rc;
  if (!x || !b || !sw || !sums || !out) return fail("linear_decode: null buffer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0)
    return fail("linear_decode: x must be 16-byte aligned");
  return linear_decode(x, x_dtype, M, K, clip, rotate_block, b, sw, sums, bias, N,
                       out_fp32 != 0, out, static_cast<hipStream_t>(stream));
}

int dscq_linear_decode_supported(int64_t M, int64_t K) { return linear_decode_fits(M, K) ? 1 : 0; }

int dscq_silu_mul_quantize(const void* gate, const void* up, int64_t ld, int64_t M,
                           int64_t N, float clip, int rotate_block, uint8_t* packed,
                           float* scales, int32_t* zeros, void* h, void* stream) {
  DisarmOnExit disarm;
  if (!(M > 0 && M <= 65535 && N > 0 && N <= 32768))
    return fail("silu_mul_quantize: require 1<=M<=65535 and 1<=N<=32768");
  if (ld < N) return fail("silu_mul_quantize: row stride %lld is below N=%lld", (long long)ld,
                          (long long)N);
  if (!(clip >= 0.5f && clip <= 1.0f)) return fail("Activation clip must be in [0.5,1]");
  if (int rc = check_rotation(rotate_block, N)) return rc;
  if (!gate || !up || !packed || !scales || !zeros) return fail("silu_mul_quantize: null buffer");
  return silu_mul_quant(gate, up, ld, M, N, ceil_to(M, 8), clip, rotate_block, packed, scales,
                        zeros, h, static_cast<hipStream_t>(stream));
}

int dscq_matmul_silu_mul(const uint8_t* a, const uint8_t* b_gu, const float* sx,
                         const int32_t* zx, const float* sw, const int32_t* sums,
                         const void* bias, int64_t M, int64_t N, int64_t KP, void* h,
                         void* stream) {
  DisarmOnExit disarm;
  if (!(M > 0 && M <= 65535)) return fail("matmul_silu_mul: require 1<=M<=65535");
  if (!a || !b_gu || !sx || !zx || !sw || !sums || !h) return fail("matmul_silu_mul: null buffer");
  if (!gemm_silu_mul_fits(M, N, KP, h))
    return fail("matmul_silu_mul: need N %% 64 == 0, KP %% 64 == 0, KP <= 65536, 16-byte "
                "aligned h (M=%lld, N=%lld, KP=%lld)", (long long)M, (long long)N,
                (long long)KP);
  return w4a4_gemm_silu_mul(a, b_gu, sx, zx, sw, sums, bias, M, N, KP, h,
                            static_cast<hipStream_t>(stream));
}

int dscq_activation_codes(const void* x, int x_dtype, int64_t M, int64_t K, float clip,
                          int bits, int rotate_block, uint8_t* codes, float* scales,
                          int32_t* zeros, void* stream) {
  DisarmOnExit disarm;
  if (!valid_dtype(x_dtype)) return fail("Only FP16 and FP32 inputs are supported");
  if (!(M > 0 && M <= 65535 && K > 0 && K <= 1048576))
    return fail("Require 1<=M<=65535 and 1<=K<=1048576");
  if (!(clip > 0.0f && clip <= 1.0f)) return fail("Activation clip must be in (0,1]");
  if (bits < 2 || bits > 8) return fail("bits must be in [2,8] (got %d)", bits);
  if (int rc = check_rotation(rotate_block, K)) return rc;
  if (!x || !codes || !scales || !zeros) return fail("activation_codes: null buffer");
  const int64_t MP = ceil_to(M, 8);
  return row_quant(x, x_dtype, M, K, MP, clip, 0, (float)((1 << bits) - 1), rotate_block,
                   nullptr, codes, scales, zeros, nullptr, static_cast<hipStream_t>(stream));
}

int dscq_pack_weight(const void* w, int w_dtype, int64_t N, int64_t K, float clip,
                     int rotate_block, uint8_t* packed, float* sw, int32_t* sums,
                     int8_t* codes, void* stream) {
  DisarmOnExit disarm;
  if (!valid_dtype(w_dtype)) return fail("Only FP16 and FP32 inputs are supported");
  if (!(N > 0 && N <= 1048576 && K > 0 && K <= 1048576))
    return fail("Require 1<=N<=1048576 and 1<=K<=1048576");
  if (!(clip > 0.0f && clip <= 1.0f)) return fail("Weight clip must be in (0,1]");
  if (int rc = check_rotation(rotate_block, K)) return rc;
  if (!w || !packed || !sw || !sums) return fail("pack_weight: null buffer");
  return row_quant(w, w_dtype, N, K, ceil_to(N, 8), clip, 1, 7.0f, rotate_block, packed,
                   reinterpret_cast<uint8_t*>(codes), sw, nullptr, sums,
                   static_cast<hipStream_t>(stream));
}

int dscq_weight_codes(const void* w, int w_dtype, int64_t N, int64_t K, float clip,
                      int bits, int rotate_block, int8_t* codes, float* scales,
                      void* stream) {
  DisarmOnExit disarm;
  if (!valid_dtype(w_dtype)) return fail("Only FP16 and FP32 inputs are supported");
  if (!(N > 0 && N <= 1048576 && K > 0 && K <= 1048576))
    return fail("Require 1<=N<=1048576 and 1<=K<=1048576");
  if (!(clip > 0.0f && clip <= 1.0f)) return fail("Weight clip must be in (0,1]");
  if (bits < 2 || bits > 8) return fail("bits must be in [2,8] (got %d)", bits);
  if (int rc = check_rotation(rotate_block, K)) return rc;
  if (!w || !codes || !scales) return fail("weight_codes: null buffer");
  return row_quant(w, w_dtype, N, K, ceil_to(N, 8), clip, 1,
                   (float)((1 << (bits - 1)) - 1), rotate_block, nullptr,
                   reinterpret_cast<uint8_t*>(codes), scales, nullptr, nullptr,
                   static_cast<hipStream_t>(stream));
}

int dscq_matmul(const uint8_t* a, const uint8_t* b, const float* sx, const int32_t* zx,
                const float* sw, const int32_t* sums, const void* bias, int64_t M,
                int64_t N, int64_t KP, int fused, int force_decode, int out_fp32,
                void* out, int32_t* raw, void* stream) {
  DisarmOnExit disarm;
  // kernel/w4a4.cu:197
  if (!(M > 0 && M <= 65535 && N > 0 && KP > 0 && KP <= 1048576 && KP % 64 == 0))
    return fail("Invalid dimensions");
  if (N > 0x7FFFFFFFLL) return fail("Invalid dimensions");
  if (!a || !b || !sx || !zx || !sw || !sums || !out) return fail("matmul: null buffer");
  if (!fused && !raw) return fail("matmul: the unfused path needs a raw buffer");
  // kernel/w4a4.cu:209: the skinny kernel for M < 8 or on request.
  const bool decode = force_decode != 0 || M < 8;
  return w4a4_gemm(a, b, sx, zx, sw, sums, bias, M, N, KP, decode, out_fp32 != 0, out,
                   fused ? nullptr : raw, static_cast<hipStream_t>(stream));
}

int64_t dscq_matmul_workspace_bytes(int64_t M, int64_t N, int64_t KP, int force_decode) {
  if (!(M > 0 && M <= 65535 && N > 0 && N <= 0x7FFFFFFFLL && KP > 0 && KP <= 1048576 &&
        KP % 64 == 0))
    return fail("Invalid dimensions");
  return w4a4_gemm_workspace_bytes(M, N, KP, force_decode != 0 || M < 8);
}

int dscq_matmul_ws(const uint8_t* a, const uint8_t* b, const float* sx, const int32_t* zx,
                   const float* sw, const int32_t* sums, const void* bias, int64_t M,
                   int64_t N, int64_t KP, int fused, int force_decode, int out_fp32,
                   void* out, int32_t* raw, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  DisarmOnExit disarm;
  if (!(M > 0 && M <= 65535 && N > 0 && KP > 0 && KP <= 1048576 && KP % 64 == 0))
    return fail("Invalid dimensions");
  if (N > 0x7FFFFFFFLL) return fail("Invalid dimensions");
  if (!a || !b || !sx || !zx || !sw || !sums || !out) return fail("matmul: null buffer");
  if (!fused && !raw) return fail("matmul: the unfused path needs a raw buffer");
  if (workspace_bytes < 0) return fail("matmul: negative workspace size");
  const bool decode = force_decode != 0 || M < 8;
  return w4a4_gemm(a, b, sx, zx, sw, sums, bias, M, N, KP, decode, out_fp32 != 0, out,
                   fused ? nullptr : raw, static_cast<hipStream_t>(stream),
                   static_cast<int32_t*>(workspace), workspace_bytes);
}

int dscq_pack_int4(const int8_t* codes, int64_t R, int64_t C, uint8_t* packed,
                   void* stream) {
  DisarmOnExit disarm;
  if (R < 0 || C < 0) return fail("pack_int4: negative shape");
  if ((R && C) && (!codes || !packed)) return fail("pack_int4: null buffer");
  return pack_int4(codes, R, C, packed, static_cast<hipStream_t>(stream));
}

int dscq_unpack_int4(const uint8_t* packed, int64_t R, int64_t CB, int64_t width,
                     int8_t* codes, void* stream) {
  DisarmOnExit disarm;
  if (R < 0 || CB < 0 || width < 0 || width > 2 * CB)
    return fail("unpack_int4: width must be in [0, 2 * packed columns]");
  if ((R && width) && (!codes || !packed)) return fail("unpack_int4: null buffer");
  return unpack_int4(packed, R, CB, width, codes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
