// Batched/prefill expert kernels on the bf16 MFMA units (grouped GEMM).
#include "common.h"

namespace wisp {

int experts_mfma(const void* x, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, const void* w13, size_t w13_stride, const void* w2,
                 size_t w2_stride, void* act, void* out, hipStream_t st, const StageEvents* ev) {
  (void)x; (void)T; (void)H; (void)I; (void)K; (void)topk_w; (void)slots; (void)w13;
  (void)w13_stride; (void)w2; (void)w2_stride; (void)act; (void)out; (void)st; (void)ev;
  wisp_set_last_error("MFMA expert path not built yet", "wisp_moe_experts");
  return WISP_ERR_UNSUPPORTED;
}

}  // namespace wisp
