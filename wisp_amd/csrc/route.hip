// Router: softmax over E logits -> top-k -> optional renormalisation.
//
// Replaces the vLLM routing the reference calls through
// layer.select_experts(..., scoring_func="softmax", renormalize=...)
// (src/wisp/integrations/vllm/fused_moe.py:1054-1076).  One wavefront per
// token; each lane holds logits j*64 + lane (coalesced), so E <= 512.
// Experts are ranked by logit, descending, ties to the lower id; weights are
// p = exp(l - max) / sum_e exp(l_e - max) and, with renormalisation,
// w = p / sum_topk p.  All sums use a fixed butterfly order.
#include <math.h>

#include "common.h"

namespace wisp {
namespace {

constexpr int kVals = kMaxExperts / 64;

template <typename TL>
__device__ inline float load_logit(const TL* p);
template <>
__device__ inline float load_logit<float>(const float* p) { return *p; }
template <>
__device__ inline float load_logit<uint16_t>(const uint16_t* p) {
  return __uint_as_float((uint32_t)(*p) << 16);
}

template <typename TL>
__global__ __launch_bounds__(256) void route_kernel(const TL* __restrict__ logits, int T, int E,
                                                     int K, int renorm, float* __restrict__ w_out,
                                                     int32_t* __restrict__ id_out,
                                                     int64_t* __restrict__ forward_counter) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (forward_counter && blockIdx.x == 0 && threadIdx.x == 0) forward_counter[0] += 1;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  const TL* row = logits + (size_t)t * E;

  float v[kVals];
#pragma unroll
  for (int j = 0; j < kVals; ++j) {
    const int e = j * 64 + lane;
    v[j] = e < E ? load_logit(row + e) : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kVals; ++j) m = fmaxf(m, v[j]);
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kVals; ++j)
    if (j * 64 + lane < E) s += expf(v[j] - m);
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);

  uint32_t taken = 0;
  int my_id = -1;
  float my_val = -INFINITY;
  for (int r = 0; r < K; ++r) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kVals; ++j) {
      const int e = j * 64 + lane;
      if (e < E && !(taken & (1u << j)) && (v[j] > bv || bi == 0x7fffffff)) {
        bv = v[j];
        bi = e;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    if (lane == r) {
      my_id = bi;
      my_val = bv;
    }
  }
  float p = lane < K ? expf(my_val - m) / s : 0.f;
  if (renorm) {
    float tot = p;
    for (int off = 32; off > 0; off >>= 1) tot += __shfl_xor(tot, off);
    p = p / tot;
  }
  if (lane < K) {
    w_out[(size_t)t * K + lane] = p;
    id_out[(size_t)t * K + lane] = my_id;
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
  if (logits_dtype == WISP_F32)
    hipLaunchKernelGGL(route_kernel<float>, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       (const float*)logits, T, E, K, renormalize, topk_w, topk_ids,
                       forward_counter);
  else
    hipLaunchKernelGGL(route_kernel<uint16_t>, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)logits, T, E, K, renormalize, topk_w, topk_ids,
                       forward_counter);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}
