// Device-driven page-in: a kernel copies the experts the pager chose to load
// from the pinned host masters (read over the host link through their device
// mapping) into their HBM scratch slots.
//
// Replaces the per-miss copies of ensure_resident
// (src/wisp/integrations/vllm/fused_moe.py:338-354: scratch_w13[slot].copy_,
// scratch_w2[slot].copy_ on the copy stream; for block-FP8 experts also the
// two scale tensors, fused_moe_fp8.py:135-141).  The load list comes from the
// pager kernel in device memory, so a decode call needs no host round trip
// between the decision and the copy: the layer enqueues pager, page-in, w13
// and w2 back to back on one stream.  64 blocks of 16-byte loads keep about
// 1 MiB of reads in flight, which saturates a PCIe 5.0 x16 link (54.7 GB/s for
// one 9 MiB expert, against 52.6 GB/s for hipMemcpyAsync of the same bytes).
#include "common.h"
#include "pagein.h"

namespace wisp {
namespace {

__global__ __launch_bounds__(256) void pagein_kernel(PageInArgs a) {
  const int n = a.count ? *a.count : a.n;
  if (a.hist && blockIdx.x == 0 && threadIdx.x == 0) {
    *a.hist = n;
    __threadfence_system();
  }
  for (int j = 0; j < n; ++j) {
    const int e = a.loads[2 * j], s = a.loads[2 * j + 1];
    if (e < 0 || e >= a.num_experts || s < 0 || s >= a.cap) continue;
    if (a.pk.m) {
      unpack_expert(a.pk, e, s, blockIdx.x, gridDim.x);
      continue;
    }
    for (int q = 0; q < a.nplanes; ++q) {
      const PageInPlane& pl = a.p[q];
      copy_range(pl.m + (size_t)e * pl.m_stride, pl.d + (size_t)s * pl.d_stride, pl.bytes,
                 blockIdx.x, gridDim.x);
    }
  }
}

}  // namespace

int launch_pagein(const PageInArgs& a, hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
  // packed masters: twice the blocks, since a chunk's loads move fewer bytes
  launch_timed(pagein_kernel, dim3(a.pk.m ? 2 * kPageInBlocks : kPageInBlocks), dim3(256), st,
               ev_start, ev_stop, a);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

const char* mapped_host_range(const void* base, size_t bytes) {
  unsigned int type = 0;
  void* dptr = nullptr;
  void* start = nullptr;
  size_t size = 0;
  const hipDeviceptr_t p = (hipDeviceptr_t)base;
  if (!base || hipPointerGetAttribute(&type, HIP_POINTER_ATTRIBUTE_MEMORY_TYPE, p) != hipSuccess ||
      type != hipMemoryTypeHost ||
      hipPointerGetAttribute(&dptr, HIP_POINTER_ATTRIBUTE_DEVICE_POINTER, p) != hipSuccess ||
      hipPointerGetAttribute(&start, HIP_POINTER_ATTRIBUTE_RANGE_START_ADDR, p) != hipSuccess ||
      hipPointerGetAttribute(&size, HIP_POINTER_ATTRIBUTE_RANGE_SIZE, p) != hipSuccess || !dptr) {
    (void)hipGetLastError();
    return nullptr;
  }
  const char* b = (const char*)base;
  const char* lo = (const char*)start;
  if (b < lo || bytes == 0) return nullptr;
  if (bytes <= size && (size_t)(b - lo) <= size - bytes) return (const char*)dptr;
  // The range-size attribute of a pinned host allocation of 4 GiB or more
  // reads modulo 2^32 on this runtime (torch rounds a 2.1 GiB pinned request
  // up to 4 GiB, which reads 0).  Then the last byte of the range must lie
  // in the same allocation and map to the device at the same offset.
  const hipDeviceptr_t last = (hipDeviceptr_t)(b + (bytes - 1));
  unsigned int type_last = 0;
  void* start_last = nullptr;
  void* dptr_last = nullptr;
  if (hipPointerGetAttribute(&type_last, HIP_POINTER_ATTRIBUTE_MEMORY_TYPE, last) != hipSuccess ||
      type_last != hipMemoryTypeHost ||
      hipPointerGetAttribute(&start_last, HIP_POINTER_ATTRIBUTE_RANGE_START_ADDR, last) !=
          hipSuccess ||
      hipPointerGetAttribute(&dptr_last, HIP_POINTER_ATTRIBUTE_DEVICE_POINTER, last) !=
          hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (start_last != start || (const char*)dptr_last != (const char*)dptr + (bytes - 1))
    return nullptr;
  return (const char*)dptr;
}

}  // namespace wisp
