// Error reporting and version entry points of libzenith_hip.so.
#include <stdarg.h>
#include <stdio.h>

#include "zk_common.hpp"

namespace zk {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(ZK_ERR_HIP, "%s: kernel launch failed: %s", what,
                hipGetErrorString(e));
  return ZK_OK;
}

}  // namespace zk

// Sustained shader clock under matrix-core load. Every wavefront keeps four
// independent chains of 32x32x16 fp16 MFMAs going (the matrix pipe never
// waits on a result) for n_mfma steps; the first lane of each workgroup
// records the shader-clock cycles and the constant-rate wall-clock ticks its
// loop took. Cycles / (ticks / wall rate) is the clock the MFMAs ran at.
__global__ __launch_bounds__(512) void clock_probe_kernel(int n, int64_t *out) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  typedef float f16v __attribute__((ext_vector_type(16)));
  const int lane = threadIdx.x & 63;
  h8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (_Float16)(1e-3f * (lane + e));
    b[e] = (_Float16)(1e-3f * (lane - e));
  }
  f16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
  __syncthreads();
  const int64_t t0 = clock64(), w0 = wall_clock64();
  for (int i = 0; i < n; ++i) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
  }
  const float sink = c0[0] + c1[1] + c2[2] + c3[3];
  const int64_t t1 = clock64(), w1 = wall_clock64();
  if (threadIdx.x == 0) {
    out[2 * blockIdx.x] = t1 - t0;
    out[2 * blockIdx.x + 1] = sink == 123456.f ? 0 : w1 - w0;
  }
}

extern "C" const char *zk_last_error(void) { return zk::g_last_error; }

extern "C" int zk_clock_probe(int grid, int n_mfma, int64_t *out, int64_t *khz, void *stream) {
  if (grid <= 0 || n_mfma <= 0 || !out || !khz)
    return zk::fail(ZK_ERR_INVALID, "zk_clock_probe: grid, n_mfma > 0 and out, khz needed");
  int dev = 0, wall = 0, sclk = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&wall, hipDeviceAttributeWallClockRate, dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&sclk, hipDeviceAttributeClockRate, dev);
  if (e != hipSuccess)
    return zk::fail(ZK_ERR_HIP, "zk_clock_probe: clock rates: %s", hipGetErrorString(e));
  khz[0] = wall;
  khz[1] = sclk;
  clock_probe_kernel<<<grid, 512, 0, (hipStream_t)stream>>>(n_mfma, out);
  return zk::check_launch("zk_clock_probe");
}

// Major * 10000 + minor * 100 + patch.
extern "C" int zk_version(void) { return 100; }
