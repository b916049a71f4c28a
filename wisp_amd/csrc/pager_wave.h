// The pager's device implementation: one wavefront makes a layer call's
// routing (up to kFusedRouteTokens tokens), group planning and LRU paging
// decisions.  Shared by the pager kernel (pager.hip) and the fused one-token
// decode launches, whose first block runs the pager in its first wave.
#pragma once

#include "common.h"
#include "pager_core.h"
#include "route_core.h"
#include "wave_set.h"

namespace wisp {
namespace {

// The wave's LDS for layers of at most MAXE experts (a CPython set of n <=
// MAXE keys never needs a table above 8 * MAXE slots).
template <int MAXE>
struct PagerSmemT {
  int32_t lru[MAXE];    // occupied slots in (tick, slot) order
  int32_t lru_pos[64];  // slot -> its place in lru (register path)
  int32_t map[MAXE];
  int32_t s2e[MAXE];
  int64_t tick[MAXE];
  uint32_t need[MAXE / 32];
  uint32_t loaded[MAXE / 32];
  int32_t keys[MAXE];
  int32_t order[MAXE];
  int32_t table[8 * MAXE];
  int32_t missing[MAXE];
  int32_t freel[MAXE];
  int32_t cand[MAXE];
  int32_t sorted[MAXE];
};

// Four 32-bit words stored by one 16-byte store at a dword-aligned address
// (gfx950's global stores need only dword alignment).
struct __attribute__((aligned(4))) Words4 {
  int32_t w0, w1, w2, w3;
};

// Routed ids of calls up to this many (token, k) pairs are staged in LDS
// once, so the serial parts of the kernel never wait on a global load (a
// 512-token x top-8 chunk fits); larger calls read them from global memory.
constexpr int kStagedPairs = 4096;

// Routed ids of a call of at most MAXP pairs, and the routing weights of a
// call routed in the wave.
template <int MAXP>
struct FusedRouteSmemT {
  alignas(16) int32_t ids[MAXP];
  float w[kFusedRouteTokens * kMaxTopK];  // routing weights of a routed call
  RoutePos pos;                           // the router's positions, per token
};

// Size of the table of a CPython set of n small ints built by insertion: 8
// slots, then the smallest power of two above 4 * fill at each resize (at 5,
// 19, 77 and 307 keys).  When every key is below it, each key sits in its own
// slot (hash(i) == i, so slot i & mask == i) and the iteration order is
// ascending: no probing decides anything.
__device__ inline int set_table_size(int n) {
  return n <= 4 ? 8 : n <= 18 ? 32 : n <= 76 ? 128 : n <= 306 ? 512 : 2048;
}

// One wavefront.  With `logits` non-null it first routes the T <= 8 tokens
// (writing topk_w / topk_ids) and takes the ids from LDS; otherwise it reads
// `ids_in` (staged in LDS when the call has at most kStagedPairs pairs).
// Outputs: device state, slots[p] (slot of pair p, -1 for pairs of a group
// that was not completed), flags (optional): flags[0] = experts loaded by
// this call, flags[1 + p] = pair_word(slot, loaded expert) (pager_core.h);
// loads (optional): the (expert, slot) pairs loaded, in the record's order;
// and the decision record.
//
// The kernel is one wavefront, so its time is the length of its chain of
// dependent steps (each LDS round trip, each hand-off between the scalar and
// the vector unit); it is built to keep that chain short per token group:
//   * group planning (greedy first-fit in token order) on per-token expert
//     bitmasks: lane l holds the mask of token b + l of a 64-token window,
//     and one scan per window finds, for every lane at once, where a group
//     starting at its token ends and that group's union, so a group costs a
//     few readlanes;
//   * for E <= 128 and cap <= 64, the layer state in registers (a lane per
//     slot and per expert) and each group's decisions as lane arithmetic,
//     ballots and lane permutes; otherwise staged in LDS, with the needed
//     and the missing experts of a group in one pass over E;
//   * eviction candidates from an LRU list kept in (tick, slot) order across
//     the groups of a call instead of a sort per group;
//   * the CPython set order only where collisions can reorder it;
//   * no global loads after the start when the ids are staged in LDS
//     (STAGED, decided at launch): on CDNA a wait for a global load also
//     waits for every global store before it (one counter covers both), so
//     a load that could read LDS or global memory (a flat load) would hold
//     every group behind the previous group's record and slot stores.
//
// pager_wave is the kernel's body: wave 0 of its block runs it (the pager
// kernel, or the pager wave of a fused one-token decode launch), with its
// LDS given by the caller for at most MAXE experts and, staged, MAXP pairs.
// ONE (decided at launch): a one-token call routed here, on the register
// path (E <= 128, cap <= 64) - the decode step's case, compiled without the
// other paths, whose set-up and register pressure it would otherwise carry.
// REGS (decided at launch): a call whose ids were routed before the launch,
// on the register path - batched decode and prefill chunks - compiled
// without the routing and the LDS path.
template <typename TL, int VALS, bool STAGED, int MAXE, int MAXP, bool ONE = false,
          bool REGS = false>
__device__ __attribute__((always_inline)) inline void pager_wave(
    const int32_t* __restrict__ ids_in, const TL* __restrict__ logits, int renorm,
    float* __restrict__ w_out, int32_t* __restrict__ id_out, int T, int K, int E, int cap,
    int single_group, int32_t* __restrict__ map_g, int32_t* __restrict__ s2e_g,
    int64_t* __restrict__ tick_g, int64_t* __restrict__ ctr_g, int32_t* __restrict__ slots_g,
    int32_t* __restrict__ flags_g, int32_t* __restrict__ loads_g, int32_t* __restrict__ rec,
    int32_t* __restrict__ rec_host, PagerSmemT<MAXE>& sm, FusedRouteSmemT<MAXP>& fr) {
  static_assert(!ONE || (VALS == 2 && STAGED), "a routed one-token call on the register path");
  static_assert(!REGS || (VALS == 2 && !ONE), "ids given, on the register path");
  if constexpr (ONE) T = 1;
  const bool routed = ONE || (!REGS && logits != nullptr);
  constexpr int W = 2 * VALS;  // 32-bit mask words per token: E <= 32 * W
  const int lane = threadIdx.x & 63;
  const int nwords = (E + 31) >> 5;
  const RecordLayout L(T, K);
  const int P = T * K;

  // The register path (E <= 128, cap <= 64): the layer state lives in
  // registers for the whole call, one lane per slot (expert, tick, place in
  // the LRU list) and per expert (slot), and a group's needed experts in
  // scalar registers, so a group's decisions are lane arithmetic, ballots and
  // lane permutes instead of chains of LDS round trips.
  constexpr bool kRegsPath = VALS <= 2;
  const bool regs = ONE || REGS || (kRegsPath && cap <= 64);
  // Otherwise, with the router fused (the launcher picks VALS * 64 >= E) and
  // cap within the same bound, the layer state is read into registers first
  // and reaches LDS after routing, so its loads travel while the router loads
  // and ranks the logits instead of before them.
  const bool state_in_regs = regs || (routed && cap <= VALS * 64);
  // The state's pointers are read with the first kernel arguments (an empty
  // asm statement that takes them), not in a second round trip after the
  // first branch.  The first token's logits go out before the layer state's
  // loads, so both arrive in one memory round trip (the routing loop below
  // otherwise waited for the state before loading them).
  asm volatile("" ::"s"(map_g), "s"(s2e_g), "s"(tick_g), "s"(ctr_g));
  float raw0[VALS] = {};
  if (routed && T > 0) route_load_logits<TL, VALS>(logits, E, lane, raw0);
  int map_r[VALS] = {}, s2e_r[VALS] = {};
  int64_t tick_r[VALS] = {};
  // Register path: loads at clamped positions, with no branch around them,
  // masked (mask_state) only after the router has issued its logit loads, so
  // that both travel together.
  auto mask_state = [&]() {
#pragma unroll
    for (int v = 0; v < VALS; ++v) {
      const int i = v * 64 + lane;
      if (i >= E) map_r[v] = -1;
      if (i >= cap) {
        s2e_r[v] = -1;
        tick_r[v] = 0;
      }
    }
  };
  if (state_in_regs) {
#pragma unroll
    for (int v = 0; v < VALS; ++v) {
      const int i = v * 64 + lane;
      map_r[v] = map_g[min(i, E - 1)];
      s2e_r[v] = s2e_g[min(i, cap - 1)];
      tick_r[v] = tick_g[min(i, cap - 1)];
    }
  } else {
    for (int e = lane; e < E; e += 64) sm.map[e] = map_g[e];
    for (int s = lane; s < cap; s += 64) {
      sm.s2e[s] = s2e_g[s];
      sm.tick[s] = tick_g[s];
    }
  }
  int64_t clock = ctr_g[kClock];
  int64_t n_forward = ctr_g[kForward], n_miss = ctr_g[kMiss], n_evict = ctr_g[kEvict],
          n_hits = ctr_g[kHits];
  // Takes every value loaded above, on each path before the first global
  // store.  The compiler tracks pending loads per path without knowing which
  // paths run together, and one memory counter covers loads and stores: a
  // load it still counts as pending at a later join (the logits of a call
  // with no tokens, the state of a call that keeps it in LDS) would make it
  // wait there for the whole counter, this call's output stores included.
  auto take_loads = [&]() {
#pragma unroll
    for (int v = 0; v < VALS; ++v)
      asm volatile("" ::"v"(raw0[v]), "v"(map_r[v]), "v"(s2e_r[v]), "v"(tick_r[v]));
    asm volatile("" ::"v"(clock), "v"(n_forward), "v"(n_miss), "v"(n_evict), "v"(n_hits));
  };
  // Routed ids: staged in LDS when the call has at most kStagedPairs pairs
  // or was routed here (STAGED), else read from global memory.
  auto id_at = [&](int p) -> int {
    if constexpr (STAGED) return fr.ids[p];
    else return ids_in[p];
  };
  // A routed call: the union of the chosen experts (bit v: expert
  // 64 v + lane), and token 0's (weight, id) of routing position `lane`.
  uint32_t picked_all = 0u;
  float w0 = 0.f;
  int id0 = -1;
  // an id outside [0, E) (a routed call's ids are in range: K <= E); staged
  // ids are checked in the registers they arrive in, except by REGS (whose
  // main loop measured slower when it did: 18.1 -> 18.5 us a bs=32 call)
  bool bad = false;
  constexpr bool kCheckStaged = STAGED && !REGS;
  auto out_of_range = [&](int e) { return (unsigned)e >= (unsigned)E; };
  if (routed) {
    for (int t = 0; t < T; ++t) {
      float w;
      int id;
      uint32_t pk;
      if (t == 0)
        route_token_loaded<VALS>(raw0, E, K, renorm, lane, true, &w, &id, fr.pos, &pk);
      else
        route_token_wave<TL, VALS>(logits + (size_t)t * E, E, K, renorm, lane, true, &w, &id,
                                   fr.pos, &pk);
      picked_all |= pk;
      if (t == 0) {
        w0 = w;
        id0 = id;
      }
      if (lane < K) {
        fr.w[t * K + lane] = w;
        fr.ids[t * K + lane] = id;
      }
    }
    if (state_in_regs) mask_state();
    take_loads();
    if (state_in_regs && !regs) {
#pragma unroll
      for (int v = 0; v < VALS; ++v) {
        const int i = v * 64 + lane;
        if (i < E) sm.map[i] = map_r[v];
        if (i < cap) {
          sm.s2e[i] = s2e_r[v];
          sm.tick[i] = tick_r[v];
        }
      }
    }
    // The first global stores come only now: a wait for the state's loads
    // above would otherwise also wait for them.  Token 0's from registers.
    if (lane < K) {
      w_out[lane] = w0;
      id_out[lane] = id0;
    }
    wave_lds_sync();
    for (int p = K + lane; p < P; p += 64) {
      w_out[p] = fr.w[p];
      id_out[p] = fr.ids[p];
    }
  } else if (STAGED && (reinterpret_cast<uintptr_t>(ids_in) & 15) == 0) {
    // 16-byte loads, every one in flight before the LDS stores: a 4096-pair
    // call waits for one global round trip (four ids a lane and load).
    constexpr int kQ = (MAXP + 255) / 256;  // loads per lane for MAXP pairs
    const int nq = P >> 2;                  // whole quads of ids
    uint4 q[kQ];
#pragma unroll
    for (int i = 0; i < kQ; ++i) {
      const int j = i * 64 + lane;
      q[i] = j < nq ? reinterpret_cast<const uint4*>(ids_in)[j] : make_uint4(0u, 0u, 0u, 0u);
    }
    for (int p = 4 * nq + lane; p < P; p += 64) {  // the last P % 4
      const int e = ids_in[p];
      fr.ids[p] = e;
      if constexpr (kCheckStaged) bad |= out_of_range(e);
    }
#pragma unroll
    for (int i = 0; i < kQ; ++i) {
      const int j = i * 64 + lane;
      if (j < nq) {
        reinterpret_cast<uint4*>(fr.ids)[j] = q[i];
        // as unsigned, a negative id is above every valid one
        if constexpr (kCheckStaged)
          bad |= out_of_range((int)max(max(q[i].x, q[i].y), max(q[i].z, q[i].w)));
      }
    }
    wave_lds_sync();
  } else if (STAGED) {
    // 16 loads in flight per lane before their LDS stores: a 4096-pair call
    // waits for 4 global round trips instead of 64.
    constexpr int kBatch = 16;
    for (int p0 = 0; p0 < P; p0 += 64 * kBatch) {
      int v[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int p = p0 + i * 64 + lane;
        v[i] = p < P ? ids_in[p] : 0;
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int p = p0 + i * 64 + lane;
        if (p < P) {
          fr.ids[p] = v[i];
          if constexpr (kCheckStaged) bad |= out_of_range(v[i]);
        }
      }
    }
    wave_lds_sync();
  }
  if (!routed) {
    if (state_in_regs) mask_state();
    take_loads();
  }
  // Each completed group writes its pairs' slot and flag words; the pairs
  // from done_p on (groups not completed) are written "not computed" (slot
  // -1, not loaded) at the end, so every word is stored once (a wave's
  // stores are limited by its memory counter: a 4096-pair call spent ~3 us
  // on stores it later overwrote).
  int done_p = 0;

  // Validate the ids not checked above, four a lane at a time.
  if (!routed && !kCheckStaged)
    for (int p0 = 0; p0 < P; p0 += 256) {
      int e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int p = p0 + i * 64 + lane;
        e[i] = p < P ? id_at(p) : 0;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) bad |= out_of_range(e[i]);
    }
  const bool any_bad = ballot(bad) != 0;
  // the planner's masks hold E <= 32 * W experts
  const bool masks_ok = E <= 32 * W;

  int status = WISP_OK, groups_done = 0, groups_planned = 0, fail_group = -1, fail_u = 0;
  int ev_total = 0, ld_total = 0;
  // The LRU list (sm.lru), built from the state the first time a group must
  // evict, then kept up to date after every group: a group gives the slots
  // of its needed experts the new clock, larger than every other tick, so
  // they move to the list's end in slot order and the rest keep their order.
  // Eviction candidates are then the list filtered, with no sort per group.
  int nlru = -1;
  int lru_r = 0, lru_pos_r = 0;  // register path: entry `lane` of the list, slot `lane`'s place
  // The planner's window: lane l holds the expert mask of token wb + l.
  uint32_t wm[W];
#pragma unroll
  for (int w = 0; w < W; ++w) wm[w] = 0u;
  int wb = -1;
  auto load_window = [&](int b) {
    wb = b;
#pragma unroll
    for (int w = 0; w < W; ++w) wm[w] = 0u;
    const int tw = wb + lane;
    if (tw < T) {
      for (int j0 = 0; j0 < K; j0 += 8) {
        int e8[8];
        if (STAGED && (K & 3) == 0) {
          // the token's ids are 16-byte aligned in LDS: two reads, where
          // eight 4-byte reads with lanes 4 * K bytes apart conflicted in
          // banks
          const uint4 a = *reinterpret_cast<const uint4*>(&fr.ids[tw * K + j0]);
          const uint4 c = j0 + 4 < K ? *reinterpret_cast<const uint4*>(&fr.ids[tw * K + j0 + 4])
                                     : make_uint4(~0u, ~0u, ~0u, ~0u);
          e8[0] = (int)a.x; e8[1] = (int)a.y; e8[2] = (int)a.z; e8[3] = (int)a.w;
          e8[4] = (int)c.x; e8[5] = (int)c.y; e8[6] = (int)c.z; e8[7] = (int)c.w;
        } else {
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) e8[jj] = j0 + jj < K ? id_at(tw * K + j0 + jj) : -1;
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int e = e8[jj];
#pragma unroll
          for (int w = 0; w < W; ++w) wm[w] |= (e >= 0 && (e >> 5) == w) ? 1u << (e & 31) : 0u;
        }
      }
    }
  };
  // The window's scan: lane l finds where a group that starts at token
  // wb + l ends (the first later token whose union with the group exceeds
  // cap; gend = offset from wb, kOpenEnd when that lies past the window) and
  // that group's union gu, reading the next tokens' masks by lane permute.
  // Each group of a call then costs a few readlanes.
  constexpr int kOpenEnd = 65;
  int gend = kOpenEnd;
  uint32_t gu[W];
#pragma unroll
  for (int w = 0; w < W; ++w) gu[w] = 0u;
  int sw = -1;  // the window the scan describes (-1: none)
  auto scan_window = [&](int b) {
    if (wb != b) load_window(b);
    const int lim = min(64, T - wb);  // tokens in the window
    const int closed = wb + lim == T ? lim : kOpenEnd;  // a group running to the window's end
#pragma unroll
    for (int w = 0; w < W; ++w) gu[w] = wm[w];
    bool done = lane >= lim;
    int endl = lim;
    for (int d = 1; d < 64; ++d) {
      if (ballot(!done) == 0) break;
      uint32_t nx[W];
#pragma unroll
      for (int w = 0; w < W; ++w)  // every lane joins the permute
        nx[w] = (uint32_t)__shfl((int)wm[w], (lane + d) & 63);
      if (!done) {
        if (lane + d >= lim) {
          done = true;
          endl = closed;
        } else {
          uint32_t na[W];
          int c = 0;
#pragma unroll
          for (int w = 0; w < W; ++w) {
            na[w] = gu[w] | nx[w];
            c += __popc(na[w]);
          }
          if (c > cap) {
            done = true;
            endl = lane + d;
          } else {
#pragma unroll
            for (int w = 0; w < W; ++w) gu[w] = na[w];
          }
        }
      }
    }
    if (!done) endl = closed;
    gend = endl;
    sw = wb;
  };

  if (any_bad || (!single_group && !masks_ok)) {
    status = WISP_ERR_INVALID;
  } else {
    if (!single_group) n_forward += 1;
    int start = 0;
    bool first = true;
    while (first || start < T) {
      first = false;
      // ---- plan one group: tokens [start, end) -----------------------
      int end = start;
      uint32_t u[W];  // the group's needed experts (wave-uniform)
      if (routed && (single_group || T == 1)) {
        // a routed call's one group: the router's choices, by ballot
#pragma unroll
        for (int v = 0; v < VALS; ++v) {
          const uint64_t b = ballot((picked_all >> v) & 1u);
          u[2 * v] = (uint32_t)b;
          u[2 * v + 1] = (uint32_t)(b >> 32);
        }
        end = T;
        if (!regs && lane == 0) {
          // (from one lane at constant places: a word picked by lane index
          // made the words a private-memory array)
#pragma unroll
          for (int w = 0; w < W; ++w)
            if (w < nwords) {
              sm.need[w] = u[w];
              sm.loaded[w] = 0u;
            }
        }
      } else if (regs && (single_group || T == 1) && P <= 64) {
        // one pair per lane: the needed set by wave ORs of the pairs' bits
        const int e = lane < P ? id_at(lane) : -1;
#pragma unroll
        for (int w = 0; w < W; ++w)
          u[w] = wave_or(e >= 0 && (e >> 5) == w ? 1u << (e & 31) : 0u);
        end = T;
      } else if (single_group || T == 1) {
        for (int w = lane; w < nwords; w += 64) {
          sm.need[w] = 0u;
          sm.loaded[w] = 0u;
        }
        wave_lds_sync();
        for (int p = lane; p < P; p += 64) {
          const int e = id_at(p);
          atomicOr(&sm.need[e >> 5], 1u << (e & 31));
        }
        end = T;
        wave_lds_sync();
#pragma unroll
        for (int w = 0; w < W; ++w)
          u[w] = w < nwords ? (uint32_t)__builtin_amdgcn_readfirstlane((int)sm.need[w]) : 0u;
      } else {
        // The reference's working-set check (fused_moe.py:1102): a call
        // whose distinct experts fit in cap is one group.  The union of all
        // the tokens' masks decides it before any window scan (which would
        // otherwise run every lane to the window's end).
        bool whole = false;
        if (start == 0) {
          uint32_t all[W];
#pragma unroll
          for (int w = 0; w < W; ++w) all[w] = 0u;
          if (STAGED && (P & 3) == 0) {
            // a presence word per expert (sm.cand, free until the evictions
            // fill it), set by every pair's id (validated above), four
            // consecutive ids a lane by one 16-byte LDS read (a lane past
            // the pairs re-reads the first four, whose experts are set
            // anyway), then read back by ballot: straight-line code, where a
            // token window's per-lane reads conflicted in banks and its mask
            // set-up took ~18 instructions per id
            int32_t* pres = sm.cand;
            for (int e = lane; e < E; e += 64) pres[e] = 0;
            wave_lds_sync();
            for (int q0 = 0; q0 < P; q0 += 512) {
              uint4 a[2];
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                const int p = q0 + 256 * h + 4 * lane;
                a[h] = *reinterpret_cast<const uint4*>(&fr.ids[p < P ? p : 0]);
              }
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                pres[a[h].x] = 1;
                pres[a[h].y] = 1;
                pres[a[h].z] = 1;
                pres[a[h].w] = 1;
              }
            }
            wave_lds_sync();
#pragma unroll
            for (int v = 0; v < VALS; ++v) {
              const int e = v * 64 + lane;
              const uint64_t b = ballot(e < E && pres[e] != 0);
              all[2 * v] = (uint32_t)b;
              all[2 * v + 1] = (uint32_t)(b >> 32);
            }
          } else {
            for (int b = 0; b < T; b += 64) {
              load_window(b);
#pragma unroll
              for (int w = 0; w < W; ++w) all[w] |= wm[w];
            }
            // the lanes' words to every lane
#pragma unroll
            for (int w = 0; w < W; ++w) all[w] = wave_or(all[w]);
          }
          int c = 0;
#pragma unroll
          for (int w = 0; w < W; ++w) c += __popc(all[w]);
          if (c <= cap) {
            whole = true;
            end = T;
#pragma unroll
            for (int w = 0; w < W; ++w) u[w] = all[w];
          }
        }
        if (!whole) {
          // Greedy first-fit in token order: the group that starts at `start`
          // from the window scan (scanning a window that starts there when the
          // current one does not cover it).
          int l = start - sw;
          const bool covered = sw >= 0 && l >= 0 && l < 64;
          int eo = covered ? __builtin_amdgcn_readlane(gend, l) : kOpenEnd;
          if (eo == kOpenEnd && !(covered && l == 0)) {
            scan_window(start);
            l = 0;
            eo = __builtin_amdgcn_readlane(gend, 0);
          }
#pragma unroll
          for (int w = 0; w < W; ++w) u[w] = (uint32_t)__builtin_amdgcn_readlane((int)gu[w], l);
          end = eo == kOpenEnd ? -1 : sw + eo;
          // A group longer than the window (it starts the window): extend it
          // window by window with a prefix OR across the lanes (tokens before
          // `b` masked out), up to the first token whose union exceeds cap.
          for (int b = sw + 64; b < T && end < 0;) {
            if (b >= wb + 64) load_window(b);
            sw = -1;  // wm no longer holds the scanned window
            const int tl = wb + lane;
            const bool live = tl >= b && tl < T;
            uint32_t m[W];
            int c = 0;
#pragma unroll
            for (int w = 0; w < W; ++w) {
              m[w] = wave_prefix_or(live ? wm[w] : 0u, lane) | u[w];
              c += __popc(m[w]);
            }
            const uint64_t over = ballot(live && c > cap);
            const int last = over ? __builtin_ctzll(over) - 1 : min(63, T - 1 - wb);
            if (last >= 0) {
#pragma unroll
              for (int w = 0; w < W; ++w)
                u[w] = (uint32_t)__builtin_amdgcn_readlane((int)m[w], last);
            }
            if (over) end = wb + __builtin_ctzll(over);
            b = wb + 64;
          }
          if (end < 0) end = T;
        }
        // (the register path keeps the needed set in u and the loaded
        // experts in ballots)
        if (!regs && lane == 0) {
#pragma unroll
          for (int w = 0; w < W; ++w)
            if (w < nwords) {
              sm.need[w] = u[w];
              sm.loaded[w] = 0u;
            }
        }
      }
      if (!regs) wave_lds_sync();
      const int g = groups_planned++;
      const int t0 = start, t1 = end;
      start = end;

      if (regs) {
        // need bit of expert e (0 <= e < E) from the scalar mask words
        // (E <= 128 here, so the mask is words 0-3; two 64-bit halves and
        // one select, where a select over the words by index became a
        // private-memory array and a load)
        auto need_of = [&](int e) -> bool {
          const uint64_t lo = ((uint64_t)u[1] << 32) | u[0];
          const uint64_t hi = ((uint64_t)u[3] << 32) | u[2];
          return (((e >> 6) ? hi : lo) >> (e & 63)) & 1ull;
        };
        // ---- needed and missing experts, ascending ----------------------
        uint64_t mb[VALS];
        int U = 0, nmiss = 0, kmax = -1;
#pragma unroll
        for (int v = 0; v < VALS; ++v) {
          const int e = v * 64 + lane;
          const uint64_t needw = ((uint64_t)u[2 * v + 1] << 32) | u[2 * v];
          const bool in = e < E && ((needw >> lane) & 1ull);
          const bool miss = in && map_r[v] < 0;
          const uint64_t bb = ballot(in);
          mb[v] = ballot(miss);
          if (in) sm.keys[U + popc_below(bb)] = e;
          if (miss) sm.missing[nmiss + popc_below(mb[v])] = e;
          U += __popcll(bb);
          nmiss += __popcll(mb[v]);
          if (bb) kmax = v * 64 + 63 - __builtin_clzll(bb);
        }
        auto missed = [&](int e) -> bool {
          const uint64_t m = (VALS > 1 && (e >> 6) == 1) ? mb[VALS - 1] : mb[0];
          return (m >> (e & 63)) & 1ull;
        };
        wave_lds_sync();
        // ---- the missing experts in CPython set order -------------------
        // (a group with more needed experts than cap fails below, and its
        // order decides nothing)
        if (nmiss >= 2 && U <= cap && kmax >= set_table_size(U)) {
          const int key = lane < U ? sm.keys[lane] : -1;
          const int pos = U <= 18 ? set_positions_small(key, U, lane)
                                  : set_positions_wave(key, U, lane);
          if (lane < U) sm.order[pos] = key;
          wave_lds_sync();
          const int e = lane < U ? sm.order[lane] : 0;
          const bool m = lane < U && missed(e);
          const uint64_t b = ballot(m);
          if (m) sm.missing[popc_below(b)] = e;
          wave_lds_sync();
        }
        const int hits = U - nmiss;
        n_hits += hits;
        const int gb = L.group_base(g);
        if (lane == 0) {
          rec[gb + 0] = t0; rec[gb + 1] = t1; rec[gb + 2] = U; rec[gb + 3] = hits;
          rec[gb + 4] = ev_total; rec[gb + 5] = 0; rec[gb + 6] = ld_total; rec[gb + 7] = 0;
        }
        if (nmiss > 0) {
          // ---- slot lanes: free slots and eviction candidates -----------
          const int cs = s2e_r[0];  // -1 on lanes >= cap
          const bool occ = cs >= 0;
          const bool cand = occ && !need_of(occ ? cs : 0);
          const uint64_t fbits = ballot(lane < cap && !occ), cbits = ballot(cand);
          const int nfree = __popcll(fbits), ncand = __popcll(cbits);
          const int shortfall = nmiss - nfree;
          if (shortfall > ncand) {
            status = WISP_ERR_SUBBATCH;
            fail_group = g;
            fail_u = U;
            break;
          }
          uint64_t evb = 0;  // evicted slots
          int q = 0;         // this slot's place among the victims
          if (shortfall > 0) {
            if (nlru < 0) {
              // occupied slots ranked by (tick, slot), the other slots' keys
              // by readlane: as one 32-bit key (2^25 - 1 - age) << 6 | slot
              // when every occupied tick lies within 2^25 ticks below the
              // clock, else as 64-bit ticks
              const int64_t ti = occ ? tick_r[0] : 0;
              const uint64_t occ_bits = ballot(occ);
              const int64_t age = clock - ti;
              const bool near = !occ || (age >= 0 && age < (1 << 25));
              int r = 0;
              if (ballot(!near) == 0) {
                const uint32_t key = ((uint32_t)((1 << 25) - 1 - (int)age) << 6) | (uint32_t)lane;
                for (uint64_t b = occ_bits; b; b &= b - 1ull)
                  r += (uint32_t)__builtin_amdgcn_readlane((int)key, __builtin_ctzll(b)) < key;
              } else {
                const uint32_t tlo = (uint32_t)ti, thi = (uint32_t)((uint64_t)ti >> 32);
                for (uint64_t b = occ_bits; b; b &= b - 1ull) {
                  const int j = __builtin_ctzll(b);
                  const uint64_t tj =
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)thi, j) << 32) |
                      (uint32_t)__builtin_amdgcn_readlane((int)tlo, j);
                  r += ((int64_t)tj < ti) || ((int64_t)tj == ti && j < lane);
                }
              }
              if (occ) sm.lru[r] = lane;
              lru_pos_r = r;
              nlru = __popcll(occ_bits);
              wave_lds_sync();
              lru_r = lane < nlru ? sm.lru[lane] : 0;
            }
            // candidates in LRU order: entry j's slot is a candidate; a
            // candidate slot's place among them is the candidates ahead of
            // its entry; the first `shortfall` are evicted
            const uint64_t cb = ballot(lane < nlru && ((cbits >> lru_r) & 1ull));
            q = cand ? __popcll(cb & ((1ull << lru_pos_r) - 1ull)) : 0;
            const bool ev = cand && q < shortfall;
            evb = ballot(ev);
            if (ev) {
              const int o = L.evicted_base() + 2 * (ev_total + q);
              rec[o] = cs;
              rec[o + 1] = lane;
            }
            n_evict += shortfall;
            ev_total += shortfall;
            if (lane == 0) rec[gb + 5] = shortfall;
          }
          // evicted experts leave the map
#pragma unroll
          for (int v = 0; v < VALS; ++v)
            if (map_r[v] >= 0 && ((evb >> map_r[v]) & 1ull)) map_r[v] = -1;
          clock += 1;
          // The free list is the free slots ascending, then the evicted ones
          // in victim order; missing expert j takes entry nfree_all - 1 - j.
          const int sf = shortfall > 0 ? shortfall : 0;
          const int nfree_all = nfree + sf;
          int j = -1;
          if (lane < cap && !occ)
            j = nfree_all - 1 - __popcll(fbits & ((1ull << lane) - 1ull));
          else if ((evb >> lane) & 1ull)
            j = sf - 1 - q;
          const bool takes = j >= 0 && j < nmiss;
          if (takes) {
            const int e = sm.missing[j];
            s2e_r[0] = e;
            tick_r[0] = clock;
            sm.map[e] = lane;  // for the expert lanes below
            const int o = L.loaded_base() + 2 * (ld_total + j);
            rec[o] = e;
            rec[o + 1] = lane;
            if (loads_g) {
              loads_g[2 * (ld_total + j)] = e;
              loads_g[2 * (ld_total + j) + 1] = lane;
            }
          } else if ((evb >> lane) & 1ull) {
            s2e_r[0] = -1;  // (every victim's slot is taken)
          }
          wave_lds_sync();
#pragma unroll
          for (int v = 0; v < VALS; ++v)
            if ((mb[v] >> lane) & 1ull) map_r[v] = sm.map[v * 64 + lane];
          n_miss += nmiss;
          ld_total += nmiss;
          if (lane == 0) rec[gb + 7] = nmiss;
        } else {
          clock += 1;
        }
        // ---- slot lanes: ticks of the needed experts, the LRU list ------
        const int cs2 = s2e_r[0];
        const bool ins = cs2 >= 0 && need_of(cs2 >= 0 ? cs2 : 0);
        if (ins) tick_r[0] = clock;
        if (nlru >= 0) {
          // entries still occupied by an expert the group did not need, in
          // list order, then the needed experts' slots ascending
          const int state = (cs2 >= 0 ? 1 : 0) | (ins ? 2 : 0);
          const int st_entry = __shfl(state, lru_r);  // every lane joins the permute
          const bool keep = lane < nlru && st_entry == 1;
          const uint64_t kb = ballot(keep), ib = ballot(ins);
          const int nk = __popcll(kb);
          if (keep) {
            sm.lru[popc_below(kb)] = lru_r;
            sm.lru_pos[lru_r] = popc_below(kb);
          }
          if (ins) {
            sm.lru[nk + popc_below(ib)] = lane;
            sm.lru_pos[lane] = nk + popc_below(ib);
          }
          nlru = nk + __popcll(ib);
          wave_lds_sync();
          lru_r = lane < nlru ? sm.lru[lane] : 0;
          lru_pos_r = lane < cap ? sm.lru_pos[lane] : 0;
        }
        // ---- the group's pairs: slot and loaded flag --------------------
        for (int base = t0 * K; base < t1 * K; base += 64) {
          const int p = base + lane;
          const bool valid = p < t1 * K;
          // (a routed one-token call's ids are token 0's, in registers)
          const int e = !valid ? 0 : routed && T == 1 ? id0 : id_at(p);
          const int src = e & 63;
          int sl = __shfl(map_r[0], src);
          if (VALS > 1) {
            const int s1 = __shfl(map_r[VALS - 1], src);
            if ((e >> 6) == 1) sl = s1;
          }
          if (valid) {
            if (slots_g) slots_g[p] = sl;
            if (flags_g) flags_g[1 + p] = pair_word(sl, missed(e) ? e : -1);
          }
        }
        groups_done = g + 1;
        done_p = t1 * K;
        wave_lds_sync();
        continue;
      }

      // ---- needed experts (ascending) and the missing ones, one pass ----
      int U = 0, nmiss = 0, kmax = -1;
      for (int base = 0; base < E; base += 64) {
        const int e = base + lane;
        const uint32_t needw = e < E ? sm.need[e >> 5] : 0u;
        const int mp = e < E ? sm.map[e] : 0;
        const bool in = (needw >> (e & 31)) & 1u;
        const bool miss = in && mp < 0;
        const uint64_t bb = ballot(in), mb = ballot(miss);
        if (in) sm.keys[U + popc_below(bb)] = e;
        if (miss) sm.missing[nmiss + popc_below(mb)] = e;
        U += __popcll(bb);
        nmiss += __popcll(mb);
        if (bb) kmax = base + 63 - __builtin_clzll(bb);
      }
      wave_lds_sync();
      // ---- the missing experts in CPython set order -------------------
      // The order only decides which free slot each missing expert takes,
      // so it matters when two or more are missing.  When every key is below
      // the set's table size it is ascending, the order found above.
      if (nmiss >= 2 && kmax >= set_table_size(U)) {
        if (U <= 64) {
          const int key = lane < U ? sm.keys[lane] : -1;
          const int pos = U <= 18 ? set_positions_small(key, U, lane)
                                  : set_positions_wave(key, U, lane);
          if (lane < U) sm.order[pos] = key;
        } else if (lane == 0) {
          cpython_set_order(sm.keys, U, sm.order, sm.table, 8 * MAXE);
        }
        wave_lds_sync();
        int nm = 0;
        for (int base = 0; base < U; base += 64) {
          const int j = base + lane;
          const int e = j < U ? sm.order[j] : 0;
          const bool m = j < U && sm.map[e] < 0;
          const uint64_t mb = ballot(m);
          if (m) sm.missing[nm + popc_below(mb)] = e;
          nm += __popcll(mb);
        }
        wave_lds_sync();
      }
      const int hits = U - nmiss;
      n_hits += hits;
      const int gb = L.group_base(g);
      if (lane == 0) {
        rec[gb + 0] = t0; rec[gb + 1] = t1; rec[gb + 2] = U; rec[gb + 3] = hits;
        rec[gb + 4] = ev_total; rec[gb + 5] = 0; rec[gb + 6] = ld_total; rec[gb + 7] = 0;
      }
      wave_lds_sync();

      if (nmiss > 0) {
        // ---- free slots and eviction candidates, ascending slot --------
        int nfree = 0, ncand = 0;
        uint64_t cand_bits = 0;  // the candidate slots when cap <= 64
        for (int base = 0; base < cap; base += 64) {
          const int s = base + lane;
          bool f = false, c = false;
          if (s < cap) {
            const int cur = sm.s2e[s];
            f = cur < 0;
            c = cur >= 0 && !(sm.need[cur >> 5] & (1u << (cur & 31)));
          }
          const uint64_t fbits = ballot(f), cbits = ballot(c);
          if (f) sm.freel[nfree + popc_below(fbits)] = s;
          if (c) sm.cand[ncand + popc_below(cbits)] = s;
          nfree += __popcll(fbits);
          ncand += __popcll(cbits);
          cand_bits = cbits;
        }
        wave_lds_sync();
        const int shortfall = nmiss - nfree;
        if (shortfall > ncand) {
          status = WISP_ERR_SUBBATCH;
          fail_group = g;
          fail_u = U;
          break;
        }
        if (shortfall > 0) {
          if (nlru < 0) {
            // occupied slots ranked by (tick, slot): up to 64 slots each
            // lane holds one tick and the others come by readlane; beyond
            // that, from LDS
            nlru = 0;
            if (cap <= 64) {
              const bool occ = lane < cap && sm.s2e[lane] >= 0;
              const int64_t ti = occ ? sm.tick[lane] : 0;
              const uint32_t tlo = (uint32_t)ti, thi = (uint32_t)((uint64_t)ti >> 32);
              const uint64_t occ_bits = ballot(occ);
              int r = 0;
              for (int j = 0; j < cap; ++j) {
                if (!((occ_bits >> j) & 1ull)) continue;
                const uint64_t tj =
                    ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)thi, j) << 32) |
                    (uint32_t)__builtin_amdgcn_readlane((int)tlo, j);
                r += ((int64_t)tj < ti) || ((int64_t)tj == ti && j < lane);
              }
              if (occ) sm.lru[r] = lane;
              nlru = __popcll(occ_bits);
            } else {
              for (int s0 = lane; s0 < cap; s0 += 64) {
                if (sm.s2e[s0] < 0) continue;
                const int64_t ti = sm.tick[s0];
                int r = 0;
                for (int j = 0; j < cap; ++j) {
                  if (sm.s2e[j] < 0) continue;
                  const int64_t tj = sm.tick[j];
                  r += (tj < ti) || (tj == ti && j < s0);
                }
                sm.lru[r] = s0;
              }
              for (int base = 0; base < cap; base += 64)
                nlru += __popcll(ballot(base + lane < cap && sm.s2e[base + lane] >= 0));
            }
            wave_lds_sync();
          }
          // candidates in LRU order: the list without the needed experts
          if (cap <= 64) {
            const int sl = lane < nlru ? sm.lru[lane] : 0;
            const bool c = lane < nlru && ((cand_bits >> sl) & 1ull);
            const uint64_t cb = ballot(c);
            if (c) sm.sorted[popc_below(cb)] = sl;
          } else {
            int nc = 0;
            for (int base = 0; base < nlru; base += 64) {
              const int j = base + lane;
              const int sl = j < nlru ? sm.lru[j] : 0;
              const int cur = j < nlru ? sm.s2e[sl] : 0;
              const bool c = j < nlru && !(sm.need[cur >> 5] & (1u << (cur & 31)));
              const uint64_t cb = ballot(c);
              if (c) sm.sorted[nc + popc_below(cb)] = sl;
              nc += __popcll(cb);
            }
          }
          wave_lds_sync();
          for (int r = lane; r < shortfall; r += 64) {
            const int s = sm.sorted[r];
            const int victim = sm.s2e[s];
            sm.map[victim] = -1;
            sm.s2e[s] = -1;
            sm.freel[nfree + r] = s;
            const int o = L.evicted_base() + 2 * (ev_total + r);
            rec[o] = victim;
            rec[o + 1] = s;
          }
          n_evict += shortfall;
          ev_total += shortfall;
          nfree += shortfall;
          if (lane == 0) rec[gb + 5] = shortfall;
          wave_lds_sync();
        }
        clock += 1;
        for (int j = lane; j < nmiss; j += 64) {
          const int s = sm.freel[nfree - 1 - j];
          const int e = sm.missing[j];
          sm.s2e[s] = e;
          sm.map[e] = s;
          sm.tick[s] = clock;
          atomicOr(&sm.loaded[e >> 5], 1u << (e & 31));
          const int o = L.loaded_base() + 2 * (ld_total + j);
          rec[o] = e;
          rec[o + 1] = s;
          if (loads_g) {
            loads_g[2 * (ld_total + j)] = e;
            loads_g[2 * (ld_total + j) + 1] = s;
          }
        }
        n_miss += nmiss;
        ld_total += nmiss;
        if (lane == 0) rec[gb + 7] = nmiss;
        wave_lds_sync();
      } else {
        clock += 1;
      }
      for (int j = lane; j < U; j += 64) sm.tick[sm.map[sm.keys[j]]] = clock;
      wave_lds_sync();
      if (nlru >= 0 && cap <= 64) {
        // The same update with one lane per slot: each lane reads its slot's
        // expert and need bit, and entry j learns its slot's from lane
        // lru[j] by a lane permute instead of two more LDS round trips.
        const int sl = lane < nlru ? sm.lru[lane] : 0;
        const int cs = lane < cap ? sm.s2e[lane] : -1;
        const bool ins = cs >= 0 && ((sm.need[cs >> 5] >> (cs & 31)) & 1u);
        const int state = (cs >= 0 ? 1 : 0) | (ins ? 2 : 0);
        // every lane joins the permute: a lane a permute reads must be active
        const int st_sl = __shfl(state, sl);
        const bool keep = lane < nlru && st_sl == 1;  // occupied, not needed
        const uint64_t kb = ballot(keep), ib = ballot(ins);
        const int nk = __popcll(kb);
        if (keep) sm.lru[popc_below(kb)] = sl;
        if (ins) sm.lru[nk + popc_below(ib)] = lane;
        nlru = nk + __popcll(ib);
        wave_lds_sync();
      } else if (nlru >= 0) {
        // In place: the list's entries still occupied by an expert the
        // group did not need, in list order (an entry moves only towards
        // the front, after every lane has read its own), then the needed
        // experts' slots ascending.
        int n2 = 0;
        for (int base = 0; base < nlru; base += 64) {
          const int j = base + lane;
          const int sl = j < nlru ? sm.lru[j] : 0;
          const int cur = j < nlru ? sm.s2e[sl] : -1;
          const bool keep = cur >= 0 && !(sm.need[cur >> 5] & (1u << (cur & 31)));
          const uint64_t kb = ballot(keep);
          if (keep) sm.lru[n2 + popc_below(kb)] = sl;
          n2 += __popcll(kb);
        }
        for (int base = 0; base < cap; base += 64) {
          const int sl = base + lane;
          const int cur = sl < cap ? sm.s2e[sl] : -1;
          const bool in = cur >= 0 && (sm.need[cur >> 5] & (1u << (cur & 31)));
          const uint64_t ib = ballot(in);
          if (in) sm.lru[n2 + popc_below(ib)] = sl;
          n2 += __popcll(ib);
        }
        nlru = n2;
        wave_lds_sync();
      }
      // four consecutive pairs a lane, two quads at a time: their id
      // reads, then their state reads, then one 16-byte store of each
      // quad's slots and one of its flag words (dword-aligned), so the LDS
      // round trips overlap and a 4096-pair group makes 32 + 32 stores where
      // it made 128 + 128 (a wave's stores are limited by its memory
      // counter)
      const int p1 = t1 * K;
      // with K a multiple of 4 a quad never straddles the group's end; a
      // lane past it re-reads the group's first quad and stores nothing
      const bool quads = STAGED && (K & 3) == 0;
      for (int p0 = t0 * K; p0 < p1; p0 += 512) {
        int e[8], m[8], f[8];
        uint32_t ld[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int p = p0 + 256 * h + 4 * lane;
          if (quads) {
            const uint4 a = *reinterpret_cast<const uint4*>(&fr.ids[p < p1 ? p : t0 * K]);
            e[4 * h] = (int)a.x; e[4 * h + 1] = (int)a.y;
            e[4 * h + 2] = (int)a.z; e[4 * h + 3] = (int)a.w;
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) e[4 * h + i] = p + i < p1 ? id_at(p + i) : 0;
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          m[i] = sm.map[e[i]];
          ld[i] = sm.loaded[e[i] >> 5];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = pair_word(m[i], (ld[i] >> (e[i] & 31)) & 1u ? e[i] : -1);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int p = p0 + 256 * h + 4 * lane;
          const int* mh = m + 4 * h;
          const int* fh = f + 4 * h;
          if (p + 3 < p1) {
            if (slots_g) *reinterpret_cast<Words4*>(slots_g + p) = Words4{mh[0], mh[1], mh[2], mh[3]};
            if (flags_g)
              *reinterpret_cast<Words4*>(flags_g + 1 + p) = Words4{fh[0], fh[1], fh[2], fh[3]};
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (p + i < p1) {
                if (slots_g) slots_g[p + i] = mh[i];
                if (flags_g) flags_g[1 + p + i] = fh[i];
              }
          }
        }
      }
      groups_done = g + 1;
      done_p = t1 * K;
      wave_lds_sync();
    }
  }

  for (int p = done_p + lane; p < P; p += 64) {
    if (slots_g) slots_g[p] = -1;
    if (flags_g) flags_g[1 + p] = pair_word(-1, -1);
  }
  if (regs) {
#pragma unroll
    for (int v = 0; v < VALS; ++v)
      if (v * 64 + lane < E) map_g[v * 64 + lane] = map_r[v];
    if (lane < cap) {
      s2e_g[lane] = s2e_r[0];
      tick_g[lane] = tick_r[0];
    }
  } else {
    for (int e = lane; e < E; e += 64) map_g[e] = sm.map[e];
    for (int s = lane; s < cap; s += 64) {
      s2e_g[s] = sm.s2e[s];
      tick_g[s] = sm.tick[s];
    }
  }
  if (lane == 0) {
    ctr_g[kClock] = clock;
    ctr_g[kForward] = n_forward;
    ctr_g[kMiss] = n_miss;
    ctr_g[kEvict] = n_evict;
    ctr_g[kHits] = n_hits;
    if (flags_g) flags_g[0] = ld_total;
    rec[kRecGroupsDone] = groups_done;
    rec[kRecGroupsPlanned] = groups_planned;
    rec[kRecFailGroup] = fail_group;
    rec[kRecFailUnique] = fail_u;
    rec[kRecEvicted] = ev_total;
    rec[kRecLoaded] = ld_total;
    rec[7] = 0;
    rec[kRecStatus] = status;
  }
  if (rec_host) {
    // Mirror the words the call wrote into the host's record in a few
    // coalesced passes, instead of one host-link write per decision.
    __threadfence();
    const int nhead = 8 + 8 * groups_planned;
    for (int w = lane; w < nhead; w += 64) rec_host[w] = rec[w];
    for (int w = lane; w < 2 * ev_total; w += 64)
      rec_host[L.evicted_base() + w] = rec[L.evicted_base() + w];
    for (int w = lane; w < 2 * ld_total; w += 64)
      rec_host[L.loaded_base() + w] = rec[L.loaded_base() + w];
  }
}

}  // namespace
}  // namespace wisp
