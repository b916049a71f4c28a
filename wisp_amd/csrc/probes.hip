// Bandwidth probes: pinned host -> HBM copies (the page-in link) and a
// streaming device copy kernel (HBM read + write, used to calibrate the
// byte counters of the profiler).
//
// wisp_probe_h2d replaces the reference's torch copy_ probe
// (scripts/m3_11_anvil_bandwidth_probe.py:42-82) with hipMemcpyAsync, the
// same call the page-in path issues.
#include <vector>

#include "common.h"

namespace {

__global__ __launch_bounds__(256) void copy16_kernel(uint4* __restrict__ dst,
                                                      const uint4* __restrict__ src, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = src[i];
}

}  // namespace

extern "C" int wisp_probe_hbm_copy(void* dst, const void* src, size_t bytes,
                                   wisp_stream_t stream) {
  if (!dst || !src || bytes % 16 || ((uintptr_t)dst) % 16 || ((uintptr_t)src) % 16)
    return WISP_ERR_INVALID;
  const size_t n = bytes / 16;
  if (n == 0) return WISP_OK;
  size_t blocks = (n + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;  // 64 workgroups per CU, grid-stride beyond
  hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (uint4*)dst, (const uint4*)src, n);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

extern "C" int wisp_probe_h2d(void* dst, const void* src_host, size_t bytes, int iters,
                              int streams, float* ms_per_iter) {
  if (!dst || !src_host || iters < 1 || streams < 1 || streams > 8 || !ms_per_iter)
    return WISP_ERR_INVALID;
  std::vector<hipStream_t> ss(streams, nullptr);
  std::vector<hipEvent_t> done(streams, nullptr);
  hipEvent_t t0 = nullptr, t1 = nullptr;
  int rc = WISP_OK;
  auto fail = [&](hipError_t e, const char* where) {
    wisp_set_last_error(hipGetErrorString(e), where);
    rc = WISP_ERR_HIP;
  };
  hipError_t e = hipSuccess;
  for (int i = 0; i < streams && e == hipSuccess; ++i) {
    e = hipStreamCreateWithFlags(&ss[i], hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
  }
  if (e == hipSuccess) e = hipEventCreate(&t0);
  if (e == hipSuccess) e = hipEventCreate(&t1);
  if (e != hipSuccess) fail(e, "wisp_probe_h2d setup");
  const size_t chunk = ((bytes / streams) + 255) & ~(size_t)255;
  for (int it = 0; it < iters && rc == WISP_OK; ++it) {
    e = hipEventRecord(t0, ss[0]);
    for (int i = 1; i < streams && e == hipSuccess; ++i) e = hipStreamWaitEvent(ss[i], t0, 0);
    for (int i = 0; i < streams && e == hipSuccess; ++i) {
      const size_t off = (size_t)i * chunk;
      if (off >= bytes) break;
      const size_t n = off + chunk > bytes ? bytes - off : chunk;
      e = hipMemcpyAsync((char*)dst + off, (const char*)src_host + off, n,
                         hipMemcpyHostToDevice, ss[i]);
      if (e == hipSuccess) e = hipEventRecord(done[i], ss[i]);
    }
    for (int i = 1; i < streams && e == hipSuccess; ++i) e = hipStreamWaitEvent(ss[0], done[i], 0);
    if (e == hipSuccess) e = hipEventRecord(t1, ss[0]);
    if (e == hipSuccess) e = hipEventSynchronize(t1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms_per_iter[it], t0, t1);
    if (e != hipSuccess) fail(e, "wisp_probe_h2d");
  }
  for (int i = 0; i < streams; ++i) {
    if (ss[i]) (void)hipStreamSynchronize(ss[i]);
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (ss[i]) (void)hipStreamDestroy(ss[i]);
  }
  if (t0) (void)hipEventDestroy(t0);
  if (t1) (void)hipEventDestroy(t1);
  return rc;
}
