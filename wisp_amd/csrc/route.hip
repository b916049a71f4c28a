// Router kernel: softmax over E logits -> top-k -> optional renormalisation.
//
// Replaces the vLLM routing the reference calls through
// layer.select_experts(..., scoring_func="softmax", renormalize=...)
// (src/wisp/integrations/vllm/fused_moe.py:1054-1076).  One wavefront per
// token, four tokens per block; the per-token work is route_token_wave.
// Experts are ranked by logit, descending, ties to the lower id; weights are
// p = exp(l - max) / sum_e exp(l_e - max) and, with renormalisation,
// w = p / sum_topk p.
#include "common.h"
#include "route_core.h"

namespace wisp {
namespace {

template <typename TL, int VALS>
__global__ __launch_bounds__(256) void route_kernel(const TL* __restrict__ logits, int T, int E,
                                                     int K, int renorm, float* __restrict__ w_out,
                                                     int32_t* __restrict__ id_out,
                                                     int64_t* __restrict__ forward_counter) {
  __shared__ RoutePos pos[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (forward_counter && blockIdx.x == 0 && threadIdx.x == 0) forward_counter[0] += 1;
  // a zero-token call launches this block for the counter only: its logits
  // buffer may be empty (null), and the waves below load row 0 even for an
  // inactive token
  if (T <= 0) return;
  const int t = blockIdx.x * 4 + wave;
  const bool active = t < T;
  float w;
  int id;
  route_token_wave<TL, VALS>(logits + (size_t)(active ? t : 0) * E, E, K, renorm, lane, active,
                             &w, &id, pos[wave]);
  if (active && lane < K) {
    w_out[(size_t)t * K + lane] = w;
    id_out[(size_t)t * K + lane] = id;
  }
}

}  // namespace
}  // namespace wisp

extern "C" int wisp_route_topk_softmax(const void* logits, int logits_dtype, int T, int E, int K,
                                       int renormalize, float* topk_w, int32_t* topk_ids,
                                       int64_t* forward_counter, wisp_stream_t stream) {
  using namespace wisp;
  if (T < 0 || E < 1 || E > kMaxExperts || K < 1 || K > E || K > 64 ||
      (T > 0 && (!logits || !topk_w || !topk_ids)) ||
      (logits_dtype != WISP_F32 && logits_dtype != WISP_BF16)) {
    wisp_set_last_error("invalid routing arguments", "wisp_route_topk_softmax");
    return WISP_ERR_INVALID;
  }
  const int blocks = T > 0 ? (T + 3) / 4 : (forward_counter ? 1 : 0);
  if (blocks == 0) return WISP_OK;
  with_route_vals(E, [&](auto vals) {
    constexpr int V = decltype(vals)::value;
    if (logits_dtype == WISP_F32)
      hipLaunchKernelGGL((route_kernel<float, V>), dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                         (const float*)logits, T, E, K, renormalize, topk_w, topk_ids,
                         forward_counter);
    else
      hipLaunchKernelGGL((route_kernel<uint16_t, V>), dim3(blocks), dim3(256), 0,
                         (hipStream_t)stream, (const uint16_t*)logits, T, E, K, renormalize,
                         topk_w, topk_ids, forward_counter);
  });
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}
