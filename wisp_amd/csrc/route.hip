// Router: softmax over E logits -> top-k -> optional renormalisation.
//
// Replaces the vLLM routing the reference calls through
// layer.select_experts(..., scoring_func="softmax", renormalize=...)
// (src/wisp/integrations/vllm/fused_moe.py:1054-1076).  One wavefront per
// token; each lane holds logits j*64 + lane (coalesced), so E <= 512.
// Top-k by rank counting: no k rounds of cross-lane argmax.
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

// One wave per token (4 tokens per block).  Each logit's rank is the number
// of logits ahead of it in (value desc, id asc) order, counted against an LDS
// copy of the row; ranks 0..K-1 are the routed experts in routing order.
template <typename TL>
__global__ __launch_bounds__(256) void route_kernel(const TL* __restrict__ logits, int T, int E,
                                                     int K, int renorm, float* __restrict__ w_out,
                                                     int32_t* __restrict__ id_out,
                                                     int64_t* __restrict__ forward_counter) {
  __shared__ __align__(16) float s_row[4][kMaxExperts];
  __shared__ float s_val[4][64];
  __shared__ int s_id[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (forward_counter && blockIdx.x == 0 && threadIdx.x == 0) forward_counter[0] += 1;
  const int t = blockIdx.x * 4 + wave;
  const bool active = t < T;
  const int per = (E + 63) >> 6;
  float v[kVals];
#pragma unroll
  for (int j = 0; j < kVals; ++j) {
    const int e = j * 64 + lane;
    v[j] = (active && j < per && e < E) ? load_logit(logits + (size_t)t * E + e) : -INFINITY;
    if (j < per && e < E) s_row[wave][e] = v[j];
  }
  __syncthreads();
  if (active) {
    const float* row = s_row[wave];
#pragma unroll
    for (int j = 0; j < kVals; ++j) {
      const int e = j * 64 + lane;
      if (j < per && e < E) {
        const float x = v[j];
        int r = 0;
        int q = 0;
        for (; q + 4 <= E; q += 4) {
          const float4 c = *reinterpret_cast<const float4*>(row + q);
          r += (c.x > x) | ((c.x == x) & (q + 0 < e));
          r += (c.y > x) | ((c.y == x) & (q + 1 < e));
          r += (c.z > x) | ((c.z == x) & (q + 2 < e));
          r += (c.w > x) | ((c.w == x) & (q + 3 < e));
        }
        for (; q < E; ++q) r += (row[q] > x) | ((row[q] == x) & (q < e));
        if (r < K) {
          s_val[wave][r] = x;
          s_id[wave][r] = e;
        }
      }
    }
  }
  __syncthreads();
  if (!active) return;
  const float m = s_val[wave][0];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kVals; ++j)
    if (j < per && j * 64 + lane < E) s += expf(v[j] - m);
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  float p = lane < K ? expf(s_val[wave][lane] - m) / s : 0.f;
  if (renorm) {
    float tot = p;
    for (int off = 32; off > 0; off >>= 1) tot += __shfl_xor(tot, off);
    p = p / tot;
  }
  if (lane < K) {
    w_out[(size_t)t * K + lane] = p;
    id_out[(size_t)t * K + lane] = s_id[wave][lane];
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
