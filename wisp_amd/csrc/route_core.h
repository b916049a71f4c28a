// Wave-level router used by the routing kernel and by the fused
// route + pager kernel.
//
// One wavefront routes one token: softmax over E <= 512 logits (lane holds
// logits j*64 + lane), top-k by logit (descending, ties to the lower id),
// optional renormalisation over the k selected.  NaN logits rank as -inf.
//
// Top-k ranks 64-bit keys: an order-preserving image of the logit above the
// complement of the expert id, so keys are distinct and the largest key is
// the largest logit with the lowest id among equals.  A round takes the wave
// maximum of the lanes' best images with the result in every lane (DPP
// inside each 16-lane row, then the gfx950 row-pair and half-wave swaps,
// v_permlane16_swap / v_permlane32_swap); the one lane holding it takes its
// best entry.  Only when several lanes hold that image (equal logits) does a
// second maximum, over their keys' low words, pick the lowest id.  Each lane
// notes the round of the entries it gave, and writes them by routing
// position to LDS once at the end.  The softmax sums combine row totals
// with readlane in a fixed order, so the weights are deterministic.
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

// Order-preserving image of a non-NaN float: unsigned comparison of images
// is float comparison, with -0 ranked as +0.  Every image is above 0, which
// marks an entry that cannot be chosen.
__device__ inline uint32_t rank_bits(float x) {
  const uint32_t u = __float_as_uint(x == 0.f ? 0.f : x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The float whose image rank_bits is r (r != 0).
__device__ inline float unrank_bits(uint32_t r) {
  return __uint_as_float((r & 0x80000000u) ? (r & 0x7fffffffu) : ~r);
}

// One wave's chosen entries by routing position.
struct RoutePos {
  int32_t id[kMaxTopK];
  float v[kMaxTopK];
};

// Unsigned max over the 64 lanes, in every lane: xor 1, xor 2, half-row
// mirror and row mirror by DPP, then the row pairs and the two halves
// exchanged by the gfx950 lane swaps.  All 64 lanes must be active.
__device__ inline uint32_t wave_max_u32_all(uint32_t v) {
  // (0 is max's identity, so each step folds into one v_max_u32 with DPP)
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
  // lane i of rows 0/1 (and 2/3) meet: row 2r of the first result and row
  // 2r + 1 of the second hold this lane's partner, the others itself
  const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((uint32_t)r16[0], (uint32_t)r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((uint32_t)r32[0], (uint32_t)r32[1]);
}

// This lane's logits of one row, at clamped positions (the row is valid
// even for an inactive token), with no branch around the loads: a load under
// a branch waited for everything before it, one logit at a time.
template <typename TL, int VALS>
__device__ inline void route_load_logits(const TL* __restrict__ logits_row, int E, int lane,
                                         float (&raw)[VALS]) {
#pragma unroll
  for (int j = 0; j < VALS; ++j) raw[j] = load_logit(logits_row + min(j * 64 + lane, E - 1));
}

// route_token_wave on logits already loaded by route_load_logits.  Lanes < K
// return (weight, id) of routing position `lane`; other lanes return
// (0, -1).  `picked` (optional): bit j is set in lane l when expert 64 j + l
// was chosen.  `pos`: this wave's LDS.  All lanes of the wave must call it,
// with K <= E (every round then chooses an eligible entry).
template <int VALS>
__device__ inline void route_token_loaded(const float (&raw)[VALS], int E, int K, int renorm,
                                          int lane, bool active, float* w_out, int* id_out,
                                          RoutePos& pos, uint32_t* picked = nullptr) {
  (void)RouteVals<VALS>();
  const int per = min((E + 63) >> 6, VALS);
  float v[VALS];
  uint64_t key[VALS];  // 0: not eligible
#pragma unroll
  for (int j = 0; j < VALS; ++j) {
    const bool ok = active && j < per && j * 64 + lane < E;
    const float x = raw[j];
    v[j] = ok && x == x ? x : -INFINITY;
    key[j] = ok ? ((uint64_t)rank_bits(v[j]) << 32) | (uint32_t)~(uint32_t)(j * 64 + lane) : 0ull;
  }
  *w_out = 0.f;
  *id_out = -1;
  if (picked) *picked = 0u;
  if (!active) return;

  uint64_t lb = key[0];  // this lane's best remaining key
#pragma unroll
  for (int j = 1; j < VALS; ++j) lb = key[j] > lb ? key[j] : lb;
  uint32_t first = 0, sel = 0;
  int rnd[VALS];  // the round entry j was chosen in (bit j of sel set)
#pragma unroll
  for (int j = 0; j < VALS; ++j) rnd[j] = 0;
  for (int r = 0; r < K; ++r) {
    const uint32_t bh = (uint32_t)(lb >> 32);
    const uint32_t mh = wave_max_u32_all(bh);
    if (r == 0) first = mh;
    bool mine = bh == mh;  // this lane's best entry is the round's choice
    if (__popcll(__ballot(mine)) != 1) {
      // equal logits in several lanes: the lowest id (largest low word)
      const uint32_t ml = wave_max_u32_all(mine ? (uint32_t)lb : 0u);
      mine = mine && (uint32_t)lb == ml;
    }
    // (in the choosing lane the low words tell its entries apart, and an
    // entry leaves by losing its high word: it then ranks below every
    // eligible key)
    const uint32_t taken = (uint32_t)lb;
    lb = 0ull;
#pragma unroll
    for (int j = 0; j < VALS; ++j) {
      const bool hit = mine && (uint32_t)key[j] == taken;
      key[j] = hit ? (uint64_t)(uint32_t)key[j] : key[j];
      sel |= hit ? 1u << j : 0u;
      rnd[j] = hit ? r : rnd[j];
      lb = key[j] > lb ? key[j] : lb;
    }
  }
#pragma unroll
  for (int j = 0; j < VALS; ++j)
    if ((sel >> j) & 1u) {
      pos.id[rnd[j]] = j * 64 + lane;
      pos.v[rnd[j]] = v[j];
    }
  wave_lds_sync();
  const float m = unrank_bits(first);
  const int my_id = lane < K ? pos.id[lane] : -1;
  const float my_v = lane < K ? pos.v[lane] : 0.f;
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
  if (picked) *picked = sel;
}

template <typename TL, int VALS>
__device__ inline void route_token_wave(const TL* __restrict__ logits_row, int E, int K,
                                        int renorm, int lane, bool active, float* w_out,
                                        int* id_out, RoutePos& pos,
                                        uint32_t* picked = nullptr) {
  float raw[VALS];
  route_load_logits<TL, VALS>(logits_row, E, lane, raw);
  route_token_loaded<VALS>(raw, E, K, renorm, lane, active, w_out, id_out, pos, picked);
}

}  // namespace wisp
