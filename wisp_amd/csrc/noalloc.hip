// wisp_moe_experts without a caller-provided workspace, for callers that
// cannot allocate device memory (work captured into a HIP graph, serving
// loops or harnesses that forbid hipMalloc).
//
// The expert kernels need two buffers besides their inputs and outputs: the
// act intermediate [T*K, I] (both algorithms) and, for the MFMA grouped GEMM,
// its work buffer (per-slot pair lists and counts, fp32 per-pair outputs).
// Here both live in `scratch`, a static device array of this file: every GPU
// the library runs on holds its own copy of WISP_NOALLOC_SCRATCH_BYTES from
// the moment the code object is loaded there until the process ends.
//
// Nothing in it has to start at zero: the act rows and the per-pair outputs
// are written for every pair before they are read (a pair with an absent
// slot gets zero act rows from the GEMV kernel and is skipped by the combine
// of the MFMA path), and the gather kernel writes every slot's count.
//
// In host code `scratch` names a host-side stand-in, not device memory, so
// its device address is looked up once per device with hipGetSymbolAddress
// (the device current at the lookup) and kept; only that address reaches the
// kernels.  No hipMalloc, hipFree or allocating library call happens here.
#include <atomic>
#include <mutex>

#include "common.h"

static __device__ __align__(256) unsigned char scratch[WISP_NOALLOC_SCRATCH_BYTES];

namespace wisp {

int experts_gemv(const void* x, int dtype, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                 const void* w2, size_t w2_stride, void* act, void* out, hipStream_t st,
                 const StageEvents* ev);
int experts_mfma(const void* x, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                 const void* w2, size_t w2_stride, void* act, void* out, void* work,
                 size_t work_bytes, hipStream_t st, const StageEvents* ev);
size_t mfma_work_bytes(int T, int K, int H, int nslots);
bool mfma_supported(int H, int I);
bool gemv_supported(int dtype, int H, int K);
int auto_algo(int dtype, int H, int I, int T, int K);

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up once per
// device).
int scratch_address(void** out) {
  int dev = 0;
  WISP_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    wisp_set_last_error("device index beyond the library's table", "wisp_moe_experts_noalloc");
    return WISP_ERR_INVALID;
  }
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
      WISP_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      if (!p) {
        wisp_set_last_error("no device address for the scratch array",
                            "wisp_moe_experts_noalloc");
        return WISP_ERR_HIP;
      }
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return WISP_OK;
}

size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace
}  // namespace wisp

extern "C" int wisp_moe_experts_noalloc(const void* x, int dtype, int T, int H, int I, int K,
                                        const float* topk_w, const int32_t* slots, int nslots,
                                        const void* w13, size_t w13_stride, const void* w2,
                                        size_t w2_stride, void* out, int algo,
                                        wisp_stream_t stream) {
  using namespace wisp;
  const char* where = "wisp_moe_experts_noalloc";
  if (T < 0 || H < 1 || I < 1 || K < 1 || nslots < 1 ||
      (dtype != WISP_F32 && dtype != WISP_BF16) ||
      (T > 0 && (!x || !topk_w || !slots || !w13 || !w2 || !out)))
    return WISP_ERR_INVALID;
  const size_t es = dtype == WISP_F32 ? 4 : 2;
  if ((H * es) % 16 || (I * es) % 16 || (w13_stride * es) % 16 || (w2_stride * es) % 16 ||
      ((uintptr_t)w13) % 16 || ((uintptr_t)w2) % 16 ||
      (T > 0 && (((uintptr_t)x) % 16 || ((uintptr_t)out) % 16))) {
    wisp_set_last_error("H, I and buffers must be 16-byte aligned", where);
    return WISP_ERR_UNSUPPORTED;
  }
  const int a = algo == WISP_ALGO_AUTO ? auto_algo(dtype, H, I, T, K) : algo;
  if (a < 0 || (a == WISP_ALGO_GEMV && !gemv_supported(dtype, H, K)) ||
      (a == WISP_ALGO_MFMA && (dtype != WISP_BF16 || !mfma_supported(H, I))) ||
      (a != WISP_ALGO_GEMV && a != WISP_ALGO_MFMA)) {
    wisp_set_last_error("no expert kernel covers this shape, dtype and top_k", where);
    return WISP_ERR_UNSUPPORTED;
  }
  if (T == 0) return WISP_OK;
  // scratch = [act (T*K*I elements) | MFMA work buffer], each 256-byte aligned
  const size_t act_bytes = up256((size_t)T * K * I * es);
  const size_t work_bytes = a == WISP_ALGO_MFMA ? mfma_work_bytes(T, K, H, nslots) : 0;
  if (act_bytes + work_bytes > (size_t)WISP_NOALLOC_SCRATCH_BYTES) {
    wisp_set_last_error("call needs more scratch than WISP_NOALLOC_SCRATCH_BYTES "
                        "(act T*K*I elements plus, on the MFMA path, the work buffer)", where);
    return WISP_ERR_INVALID;
  }
  void* base = nullptr;
  int rc = scratch_address(&base);
  if (rc != WISP_OK) return rc;
  char* act = (char*)base;
  hipStream_t st = (hipStream_t)stream;
  if (a == WISP_ALGO_MFMA)
    return experts_mfma(x, T, H, I, K, topk_w, slots, nslots, w13, w13_stride, w2, w2_stride, act,
                        out, act + act_bytes, work_bytes, st, nullptr);
  return experts_gemv(x, dtype, T, H, I, K, topk_w, slots, nslots, w13, w13_stride, w2,
                      w2_stride, act, out, st, nullptr);
}

extern "C" size_t wisp_noalloc_scratch_bytes(void) { return (size_t)WISP_NOALLOC_SCRATCH_BYTES; }
