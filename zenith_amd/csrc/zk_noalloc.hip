// Allocation-free fp16 GEMM: zk_gemm_f16 for callers that cannot allocate
// device memory (code under HIP-graph capture, tight serving loops, hosts
// that forbid allocation). The split-K partial sums that zk_gemm_f16_ws keeps
// in a caller workspace live here in a file-scope device array instead.
//
// Size: the split plan only splits products whose 64 x 64 tiles number
// t64 < 128, into at most 512 / t64 splits, and M * N <= t64 * 64 * 64, so
// the partials (splits * M * N fp32) never exceed 512 * 4096 * 4 bytes =
// 8 MiB: the array holds exactly that. Each GPU the library runs on holds its
// own copy until the process ends.
//
// The array's host-side name is not a device address: its address on each
// device is looked up once, with that device current, through
// hipGetSymbolAddress, and only that address is handed to kernels.
//
// Every call on one GPU shares that GPU's array, which keeps the last call's
// partials. Each split writes its whole partial tile before the reduction
// reads it, so nothing needs clearing; two calls that overlap in time on one
// GPU (different streams, or concurrent host threads) race on the array.
#include <mutex>

#include "zk_common.hpp"

namespace zk {

constexpr int64_t kScratchBytes = 8ll << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void *g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up on the first
// call made with that device current.
static int scratch_on_current_device(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(ZK_ERR_HIP, "zk_gemm_f16_noalloc: hipGetDevice: %s",
                                   hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ZK_ERR_UNSUPPORTED, "zk_gemm_f16_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(ZK_ERR_HIP, "zk_gemm_f16_noalloc: hipGetSymbolAddress(scratch): %s",
                  hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return ZK_OK;
}

}  // namespace zk

using namespace zk;

extern "C" int zk_gemm_f16_noalloc(const void *A, const void *B, void *C, int64_t M, int64_t N,
                                   int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int trans_b,
                                   int out_dtype, const void *bias, const void *residual,
                                   int64_t ldr, int epilogue, void *stream) {
  const int64_t need = zk_gemm_workspace_size(M, N, K, ZK_F16);
  if (need > kScratchBytes)
    return fail(ZK_ERR_UNSUPPORTED,
                "zk_gemm_f16_noalloc: split partials need %lld bytes, the static scratch holds %lld",
                (long long)need, (long long)kScratchBytes);
  void *ws = nullptr;
  if (need > 0) {
    const int st = scratch_on_current_device(&ws);
    if (st) return st;
  }
  return gemm_f16_impl(A, B, C, M, N, K, lda, ldb, ldc, trans_b, out_dtype, bias, residual, ldr,
                       epilogue, ws, need, stream);
}
