// Wave-level router used by the routing kernel and by the fused
// route + pager kernel.
//
// One wavefront routes one token: softmax over E <= 512 logits (lane holds
// logits j*64 + lane), top-k by logit (descending, ties to the lower id),
// optional renormalisation over the k selected.  NaN logits rank as -inf.
//
// Reductions stay in registers: four DPP steps inside each 16-lane row
// (xor 1, xor 2, half-mirror, mirror - after each step both partners hold
// the same bits, since IEEE add and max are commutative), then the four row
// results are combined with readlane in a fixed order.  The result is
// deterministic and identical in every lane.  The argmax of each top-k
// round is the wave max followed by a ballot for the lowest id holding it.
#pragma once

#include <math.h>

#include "common.h"

namespace wisp {

constexpr int kRouteVals = kMaxExperts / 64;

template <typename TL>
__device__ inline float load_logit(const TL* p);
template <>
__device__ inline float load_logit<float>(const float* p) { return *p; }
template <>
__device__ inline float load_logit<uint16_t>(const uint16_t* p) {
  return __uint_as_float((uint32_t)(*p) << 16);
}

template <int kCtrl>
__device__ inline float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, false));
}

__device__ inline float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum over the 64 lanes, same bits in every lane.
__device__ inline float wave_sum_f32(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  return ((readlane_f32(v, 0) + readlane_f32(v, 16)) + readlane_f32(v, 32)) +
         readlane_f32(v, 48);
}

// Max over the 64 lanes, same bits in every lane.
__device__ inline float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)),
               fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

// Routes one token.  Lanes < K return (weight, id) of routing position
// `lane`; other lanes return (0, -1).  Needs no shared memory; all lanes of
// the wave must call it.
template <typename TL>
__device__ inline void route_token_wave(const TL* __restrict__ logits_row, int E, int K,
                                        int renorm, int lane, bool active, float* w_out,
                                        int* id_out) {
  const int per = (E + 63) >> 6;
  float v[kRouteVals];
  uint32_t taken = 0;  // bit j: entry j of this lane is not eligible
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j) {
    const int e = j * 64 + lane;
    float x = -INFINITY;
    if (active && j < per && e < E) {
      x = load_logit(logits_row + e);
      if (x != x) x = -INFINITY;
    } else {
      taken |= 1u << j;
    }
    v[j] = x;
  }
  *w_out = 0.f;
  *id_out = -1;
  if (!active) return;

  float lmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j)
    if (!(taken & (1u << j))) lmax = fmaxf(lmax, v[j]);
  const float m = wave_max_f32(lmax);
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < kRouteVals; ++j)
    if (!(taken & (1u << j))) ls += expf(v[j] - m);
  const float s = wave_sum_f32(ls);

  int my_id = -1;
  float my_v = 0.f;
  for (int r = 0; r < K; ++r) {
    float best = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRouteVals; ++j)
      if (!(taken & (1u << j))) best = fmaxf(best, v[j]);
    const float bm = wave_max_f32(best);
    int e = -1;
#pragma unroll
    for (int j = 0; j < kRouteVals; ++j) {
      if (j >= per || e >= 0) continue;
      const uint64_t b = __ballot(!(taken & (1u << j)) && v[j] == bm);
      if (b) e = j * 64 + __builtin_ctzll(b);
    }
    if (e >= 0 && (e & 63) == lane) taken |= 1u << (e >> 6);
    if (lane == r) {
      my_id = e;
      my_v = bm;
    }
  }
  float p = lane < K ? expf(my_v - m) / s : 0.f;
  if (renorm) p = p / wave_sum_f32(p);
  if (lane < K) {
    *w_out = p;
    *id_out = my_id;
  }
}

}  // namespace wisp
