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
// deterministic and identical in every lane.  The softmax maximum is the
// first top-k value, so the denominator pass follows the top-k rounds.
#pragma once

#include <math.h>

#include <type_traits>

#include "common.h"

namespace wisp {

// Logits per lane a router instance holds: 2 (E <= 128), 4 (E <= 256) or 8
// (E <= 512).  The top-k rescans and the softmax sum are unrolled over them,
// so the smallest instance that covers E keeps the serial path short.
template <int VALS>
struct RouteVals {
  static_assert(VALS == 2 || VALS == 4 || VALS == 8, "2, 4 or 8 logits per lane");
};

// Calls f(std::integral_constant<int, VALS>) with the smallest VALS covering E.
template <typename F>
__host__ inline void with_route_vals(int E, F&& f) {
  if (E <= 128)
    f(std::integral_constant<int, 2>());
  else if (E <= 256)
    f(std::integral_constant<int, 4>());
  else
    f(std::integral_constant<int, 8>());
}

template <typename TL>
__device__ inline float load_logit(const TL* p);
template <>
__device__ inline float load_logit<float>(const float* p) { return *p; }
template <>
__device__ inline float load_logit<uint16_t>(const uint16_t* p) {
  return __uint_as_float((uint32_t)(*p) << 16);
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

// Minimum over the 64 lanes (same value in every lane).
__device__ inline int wave_min_i32(int v) {
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false));
  v = min(v, __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Routes one token.  Lanes < K return (weight, id) of routing position
// `lane`; other lanes return (0, -1).  Needs no shared memory; all lanes of
// the wave must call it.
//
// Top-k: each lane keeps the best of its own not-yet-taken entries (value
// and the lowest position j holding it).  A round takes the wave max of the
// lane bests; the winner is the lowest id e = 64 j + lane among the lanes
// holding that value, and only the winning lane rescans its entries.
// This lane's logits of one row, at clamped positions (the row is valid
// even for an inactive token), with no branch around the loads: a load under
// a branch waited for everything before it, one logit at a time.
template <typename TL, int VALS>
__device__ inline void route_load_logits(const TL* __restrict__ logits_row, int E, int lane,
                                         float (&raw)[VALS]) {
#pragma unroll
  for (int j = 0; j < VALS; ++j) raw[j] = load_logit(logits_row + min(j * 64 + lane, E - 1));
}

// route_token_wave on logits already loaded by route_load_logits.
template <int VALS>
__device__ inline void route_token_loaded(const float (&raw)[VALS], int E, int K, int renorm,
                                          int lane, bool active, float* w_out, int* id_out) {
  (void)RouteVals<VALS>();
  const int per = min((E + 63) >> 6, VALS);
  float v[VALS];
  uint32_t taken = 0;  // bit j: entry j of this lane is not eligible
#pragma unroll
  for (int j = 0; j < VALS; ++j) {
    const bool ok = active && j < per && j * 64 + lane < E;
    const float x = raw[j];
    v[j] = ok && x == x ? x : -INFINITY;
    if (!ok) taken |= 1u << j;
  }
  *w_out = 0.f;
  *id_out = -1;
  if (!active) return;

  // best eligible entry of this lane: value lb at position lbj (-1: none)
  float lb = -INFINITY;
  int lbj = -1;
  auto rescan = [&]() {
    lb = -INFINITY;
    lbj = -1;
#pragma unroll
    for (int j = VALS - 1; j >= 0; --j)
      if (!(taken & (1u << j)) && (lbj < 0 || v[j] >= lb)) {
        lb = v[j];
        lbj = j;
      }
  };
  rescan();

  float m = 0.f;
  int my_id = -1;
  float my_v = 0.f;
  for (int r = 0; r < K; ++r) {
    const float bm = wave_max_f32(lbj >= 0 ? lb : -INFINITY);
    if (r == 0) m = bm;
    const bool cand = lbj >= 0 && lb == bm;
    const uint64_t cb = __ballot(cand);
    int e;
    if (__popcll(cb) == 1) {
      const int wl = __builtin_ctzll(cb);
      e = __builtin_amdgcn_readlane(lbj, wl) * 64 + wl;
    } else {
      e = wave_min_i32(cand ? lbj * 64 + lane : 0x7fffffff);
    }
    if (lane == (e & 63)) {
      taken |= 1u << (e >> 6);
      rescan();
    }
    if (lane == r) {
      my_id = e;
      my_v = bm;
    }
  }
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < VALS; ++j)
    if (j < per && j * 64 + lane < E) ls += expf(v[j] - m);
  const float s = wave_sum_f32(ls);
  float p = lane < K ? expf(my_v - m) / s : 0.f;
  if (renorm) p = p / wave_sum_f32(p);
  if (lane < K) {
    *w_out = p;
    *id_out = my_id;
  }
}

template <typename TL, int VALS>
__device__ inline void route_token_wave(const TL* __restrict__ logits_row, int E, int K,
                                        int renorm, int lane, bool active, float* w_out,
                                        int* id_out) {
  float raw[VALS];
  route_load_logits<TL, VALS>(logits_row, E, lane, raw);
  route_token_loaded<VALS>(raw, E, K, renorm, lane, active, w_out, id_out);
}

}  // namespace wisp
