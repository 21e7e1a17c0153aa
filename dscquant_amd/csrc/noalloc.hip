// dscq_matmul_noalloc: dscq_matmul for callers that cannot allocate device
// memory (code under HIP graph capture that forbids it, tight serving loops,
// harnesses that forbid hipMalloc).  The one scratch buffer the GEMM can use
// -- the int32 partial sums of a K split -- lives in a fixed device array of
// this library instead of a caller-provided workspace.
//
// The array, `scratch`, is a file-scope __device__ variable: every GPU the
// library runs on holds its own copy for the life of the process.  Its name is
// a host-side stand-in, not a device address, so host code never passes it to
// a kernel or copy: on the first call on a device, with that device current,
// hipGetSymbolAddress gives that device's address, kept per device and used
// from then on.
//
// Nothing in the scratch needs clearing: each part of a split writes every
// partial sum it covers before the reduce kernel reads it.  Calls on one GPU
// share the array, so calls that may overlap on one GPU (different streams,
// or different host threads) race; serialize them on one stream.

#include <mutex>

#include "../../include/dscq.h"
#include "common.h"

namespace dscq {

int w4a4_gemm(const uint8_t* a, const uint8_t* b, const float* sx, const int32_t* zx,
              const float* sw, const int32_t* sums, const void* bias, int64_t M,
              int64_t N, int64_t KP, bool decode, bool out_fp32, void* out,
              int32_t* raw, hipStream_t stream, int32_t* ws, int64_t ws_bytes);
int64_t w4a4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t KP, bool decode);

// 8 MiB: a K split runs at most one 64 x 128 tile part per compute unit, so on
// a 256-CU MI355X its partial sums never exceed 256 * 64 * 128 * 4 bytes.
constexpr int64_t kScratchBytes = DSCQ_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up once per device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail("matmul_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return (int)e;
  }
  if (dev < 0 || dev >= kMaxDevices) return fail("matmul_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail("matmul_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
           hipGetErrorString(e));
      return e != hipSuccess ? (int)e : DSCQ_EINVAL;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DSCQ_OK;
}

}  // namespace
}  // namespace dscq

using namespace dscq;

extern "C" {

int dscq_matmul_noalloc(const uint8_t* a, const uint8_t* b, const float* sx,
                        const int32_t* zx, const float* sw, const int32_t* sums,
                        const void* bias, int64_t M, int64_t N, int64_t KP, int fused,
                        int force_decode, int out_fp32, void* out, int32_t* raw,
                        void* stream) {
  DisarmOnExit disarm;
  // The argument checks of dscq_matmul (kernel/w4a4.cu:197).
  if (!(M > 0 && M <= 65535 && N > 0 && KP > 0 && KP <= 1048576 && KP % 64 == 0))
    return fail("Invalid dimensions");
  if (N > 0x7FFFFFFFLL) return fail("Invalid dimensions");
  if (!a || !b || !sx || !zx || !sw || !sums || !out) return fail("matmul: null buffer");
  if (!fused && !raw) return fail("matmul: the unfused path needs a raw buffer");
  const bool decode = force_decode != 0 || M < 8;
  const int64_t need = w4a4_gemm_workspace_bytes(M, N, KP, decode);
  if (need > kScratchBytes)
    return fail("matmul_noalloc: this shape's K split needs %lld bytes of scratch, above the "
                "library's fixed %lld; use dscq_matmul_ws with a workspace",
                (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_address(&ws)) return rc;
  }
  return w4a4_gemm(a, b, sx, zx, sw, sums, bias, M, N, KP, decode, out_fp32 != 0, out,
                   fused ? nullptr : raw, static_cast<hipStream_t>(stream),
                   static_cast<int32_t*>(ws), need);
}

}  // extern "C"
