// Expert pager: host (sequential) and device (one wavefront) implementations.
//
// Semantics follow the reference pager, src/wisp/integrations/vllm/fused_moe.py:
//   * grouping: greedy first-fit over tokens in index order, a token joins
//     the open group iff the union of routed experts stays <= cap or the
//     group is empty (1119-1140; when the whole batch fits this is the single
//     fast-path call at 1102-1118);
//   * per group (ensure_resident, 264-358): needed = sorted unique ids; the
//     missing experts in CPython set order; hits += |needed| - |missing|;
//     all-hit -> clock += 1 and touch; else free slots ascending, eviction
//     candidates = occupied slots whose expert is not needed, stable-sorted by
//     tick; evict the first (missing - free) of them, appending each freed
//     slot; clock += 1; each missing expert takes free.pop() (from the end);
//     finally every needed expert's slot gets tick = clock;
//   * a group needing more slots than cap -> WISP_ERR_SUBBATCH (the
//     reference's "sub-batch" RuntimeError, 315-327), after hits were counted;
//   * forward counter += 1 per layer call (1017), not per group.
#include <algorithm>
#include <vector>

#include "common.h"
#include "pager_core.h"
#include "pager_wave.h"

namespace wisp {

// ---------------------------------------------------------------------------
// Host implementation (the specification the device kernel is checked against)
// ---------------------------------------------------------------------------

namespace {

struct HostRecord {
  int32_t* w;
  RecordLayout L;
  int ev = 0, ld = 0;
};

// One ensure_resident call on `needed` (ascending unique ids).
int ensure_group_host(PagerView& st, const std::vector<int32_t>& needed, HostRecord& R,
                      int g, int t0, int t1) {
  const int U = (int)needed.size();
  std::vector<int32_t> order(U > 0 ? U : 1), table(kMaxSetTable);
  if (cpython_set_order(needed.data(), U, order.data(), table.data(), kMaxSetTable) != U)
    return WISP_ERR_INVALID;
  std::vector<char> is_needed(st.E, 0);
  for (int e : needed) is_needed[e] = 1;

  std::vector<int32_t> missing;
  for (int j = 0; j < U; ++j)
    if (st.map[order[j]] < 0) missing.push_back(order[j]);
  const int hits = U - (int)missing.size();
  st.ctr[kHits] += hits;

  int32_t* G = R.w + R.L.group_base(g);
  G[0] = t0; G[1] = t1; G[2] = U; G[3] = hits;
  G[4] = R.ev; G[5] = 0; G[6] = R.ld; G[7] = 0;

  if (missing.empty()) {
    st.ctr[kClock] += 1;
    for (int e : needed) st.tick[st.map[e]] = st.ctr[kClock];
    return WISP_OK;
  }

  std::vector<int32_t> free_slots;
  std::vector<std::pair<int64_t, int32_t>> cand;
  for (int s = 0; s < st.cap; ++s) {
    if (st.s2e[s] < 0) free_slots.push_back(s);
    else if (!is_needed[st.s2e[s]]) cand.emplace_back(st.tick[s], s);
  }
  std::stable_sort(cand.begin(), cand.end(),
                   [](const std::pair<int64_t, int32_t>& a, const std::pair<int64_t, int32_t>& b) {
                     return a.first < b.first;
                   });
  const int shortfall = (int)missing.size() - (int)free_slots.size();
  if (shortfall > 0) {
    if (shortfall > (int)cand.size()) {
      R.w[kRecFailGroup] = g;
      R.w[kRecFailUnique] = U;
      return WISP_ERR_SUBBATCH;
    }
    for (int r = 0; r < shortfall; ++r) {
      const int s = cand[r].second;
      const int victim = st.s2e[s];
      st.map[victim] = -1;
      st.s2e[s] = -1;
      free_slots.push_back(s);
      st.ctr[kEvict] += 1;
      R.w[R.L.evicted_base() + 2 * R.ev] = victim;
      R.w[R.L.evicted_base() + 2 * R.ev + 1] = s;
      ++R.ev;
      ++G[5];
    }
  }
  st.ctr[kClock] += 1;
  const int64_t clock = st.ctr[kClock];
  for (int e : missing) {
    const int s = free_slots.back();
    free_slots.pop_back();
    st.s2e[s] = e;
    st.map[e] = s;
    st.tick[s] = clock;
    st.ctr[kMiss] += 1;
    R.w[R.L.loaded_base() + 2 * R.ld] = e;
    R.w[R.L.loaded_base() + 2 * R.ld + 1] = s;
    ++R.ld;
    ++G[7];
  }
  for (int e : needed) st.tick[st.map[e]] = clock;
  return WISP_OK;
}

}  // namespace

int pager_decide_host(PagerView st, const int32_t* ids, int T, int K, int single_group,
                      int32_t* slots, int32_t* rec, int rec_words) {
  RecordLayout L(T, K);
  if (T < 0 || K < 1 || st.E < 1 || st.E > kMaxExperts || st.cap < 1 || st.cap > kMaxExperts ||
      rec_words < L.words())
    return WISP_ERR_INVALID;
  for (int w = 0; w < 8; ++w) rec[w] = 0;
  rec[kRecFailGroup] = -1;
  const int P = T * K;
  for (int p = 0; p < P; ++p) {
    if (ids[p] < 0 || ids[p] >= st.E) {
      rec[kRecStatus] = WISP_ERR_INVALID;
      return WISP_ERR_INVALID;
    }
  }
  if (!single_group) st.ctr[kForward] += 1;

  // Plan the groups (contiguous token ranges).
  std::vector<int> ends;
  if (single_group) {
    ends.push_back(T);
  } else {
    std::vector<char> cur(st.E, 0);
    int cnt = 0, start = 0;
    for (int t = 0; t < T; ++t) {
      int nnew = 0;
      std::vector<int> fresh;
      for (int j = 0; j < K; ++j) {
        const int e = ids[t * K + j];
        if (!cur[e] && std::find(fresh.begin(), fresh.end(), e) == fresh.end()) {
          fresh.push_back(e);
          ++nnew;
        }
      }
      if (cnt + nnew <= st.cap || t == start) {
        for (int e : fresh) cur[e] = 1;
        cnt += nnew;
      } else {
        ends.push_back(t);
        std::fill(cur.begin(), cur.end(), 0);
        start = t;
        cnt = 0;
        for (int j = 0; j < K; ++j) {
          const int e = ids[t * K + j];
          if (!cur[e]) { cur[e] = 1; ++cnt; }
        }
      }
    }
    ends.push_back(T);
  }
  rec[kRecGroupsPlanned] = (int)ends.size();

  HostRecord R{rec, L};
  int t0 = 0, status = WISP_OK;
  for (int g = 0; g < (int)ends.size(); ++g) {
    const int t1 = ends[g];
    std::vector<char> mark(st.E, 0);
    for (int p = t0 * K; p < t1 * K; ++p) mark[ids[p]] = 1;
    std::vector<int32_t> needed;
    for (int e = 0; e < st.E; ++e)
      if (mark[e]) needed.push_back(e);
    status = ensure_group_host(st, needed, R, g, t0, t1);
    if (status != WISP_OK) break;
    if (slots)
      for (int p = t0 * K; p < t1 * K; ++p) slots[p] = st.map[ids[p]];
    rec[kRecGroupsDone] = g + 1;
    t0 = t1;
  }
  rec[kRecEvicted] = R.ev;
  rec[kRecLoaded] = R.ld;
  rec[kRecStatus] = status;
  return status;
}

namespace {

template <typename TL, int VALS, bool STAGED, bool ONE, bool REGS = false>
__global__ __launch_bounds__(64) void pager_kernel(
    const int32_t* __restrict__ ids_in, const TL* __restrict__ logits, int renorm,
    float* __restrict__ w_out, int32_t* __restrict__ id_out, int T, int K, int E, int cap,
    int single_group, int32_t* __restrict__ map_g, int32_t* __restrict__ s2e_g,
    int64_t* __restrict__ tick_g, int64_t* __restrict__ ctr_g, int32_t* __restrict__ slots_g,
    int32_t* __restrict__ flags_g, int32_t* __restrict__ loads_g, int32_t* __restrict__ rec,
    int32_t* __restrict__ rec_host) {
  __shared__ PagerSmemT<kMaxExperts> sm;
  __shared__ FusedRouteSmemT<kStagedPairs> fr;
  pager_wave<TL, VALS, STAGED, kMaxExperts, kStagedPairs, ONE, REGS>(
      ids_in, logits, renorm, w_out, id_out, T, K, E, cap, single_group, map_g, s2e_g, tick_g,
      ctr_g, slots_g, flags_g, loads_g, rec, rec_host, sm, fr);
}

}  // namespace

int launch_pager(const int32_t* ids, const void* logits, int logits_dtype, int renorm,
                 float* topk_w, int32_t* topk_ids, int T, int K, int E, int cap,
                 int single_group, int32_t* map, int32_t* s2e, int64_t* tick, int64_t* ctr,
                 int32_t* slots, int32_t* flags, int32_t* loads, int32_t* rec, int rec_words,
                 hipStream_t stream, int32_t* rec_host) {
  RecordLayout L(T, K);
  if (T < 0 || K < 1 || K > kMaxTopK || E < 1 || E > kMaxExperts || cap < 1 || cap > kMaxExperts ||
      rec_words < L.words() || !map || !s2e || !tick || !ctr || !rec ||
      (T > 0 && !ids && !logits) ||
      (logits && (T > kFusedRouteTokens || K > E || !topk_w || !topk_ids ||
                  (logits_dtype != WISP_F32 && logits_dtype != WISP_BF16)))) {
    wisp_set_last_error("invalid pager arguments", "wisp_pager_decide");
    return WISP_ERR_INVALID;
  }
  const bool staged = logits != nullptr || (int64_t)T * K <= kStagedPairs;
  // A call with its ids in LDS issues no global load after its start, so
  // nothing in it waits for its record stores: it writes the host record
  // directly.  Otherwise it writes the device record and copies it to the
  // host record at its end (a read of device memory there would wait for
  // every host store before it).
  if (staged && rec_host) {
    rec = rec_host;
    rec_host = nullptr;
  }
  // A one-token call routed here on the register path (E <= 128, cap <= 64)
  // runs the instance compiled for exactly that case; a call with its ids
  // given, on the register path and staged, runs the one compiled without
  // routing and without the LDS path.
  const bool one = logits && T == 1 && E <= 128 && cap <= 64;
  const bool regs_only = !logits && staged && E <= 128 && cap <= 64;
  with_route_vals(E, [&](auto vals) {
    constexpr int V = decltype(vals)::value;
    if constexpr (V == 2) {
      if (one && logits_dtype == WISP_BF16) {
        hipLaunchKernelGGL((pager_kernel<uint16_t, 2, true, true>), dim3(1), dim3(64), 0, stream,
                           ids, (const uint16_t*)logits, renorm, topk_w, topk_ids, T, K, E, cap,
                           single_group, map, s2e, tick, ctr, slots, flags, loads, rec,
                           rec_host);
        return;
      }
      if (one) {
        hipLaunchKernelGGL((pager_kernel<float, 2, true, true>), dim3(1), dim3(64), 0, stream,
                           ids, (const float*)logits, renorm, topk_w, topk_ids, T, K, E, cap,
                           single_group, map, s2e, tick, ctr, slots, flags, loads, rec,
                           rec_host);
        return;
      }
      if (regs_only) {
        hipLaunchKernelGGL((pager_kernel<float, 2, true, false, true>), dim3(1), dim3(64), 0,
                           stream, ids, nullptr, renorm, topk_w, topk_ids, T, K, E, cap,
                           single_group, map, s2e, tick, ctr, slots, flags, loads, rec,
                           rec_host);
        return;
      }
    }
    if (logits && logits_dtype == WISP_BF16)
      hipLaunchKernelGGL((pager_kernel<uint16_t, V, true, false>), dim3(1), dim3(64), 0, stream,
                         ids, (const uint16_t*)logits, renorm, topk_w, topk_ids, T, K, E, cap,
                         single_group, map, s2e, tick, ctr, slots, flags, loads, rec,
                         rec_host);
    else if (staged)
      hipLaunchKernelGGL((pager_kernel<float, V, true, false>), dim3(1), dim3(64), 0, stream,
                         ids, (const float*)logits, renorm, topk_w, topk_ids, T, K, E, cap,
                         single_group, map, s2e, tick, ctr, slots, flags, loads, rec,
                         rec_host);
    else
      hipLaunchKernelGGL((pager_kernel<float, V, false, false>), dim3(1), dim3(64), 0, stream,
                         ids, nullptr, renorm, topk_w, topk_ids, T, K, E, cap, single_group, map,
                         s2e, tick, ctr, slots, flags, loads, rec, rec_host);
  });
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

}  // namespace wisp

extern "C" int wisp_pager_decide(const int32_t* topk_ids, int T, int K, int E, int cap,
                                 int single_group, int32_t* expert_map,
                                 int32_t* slot_to_expert, int64_t* lru_tick,
                                 int64_t* counters, int32_t* slots, int32_t* record,
                                 int record_words, wisp_stream_t stream) {
  return wisp::launch_pager(topk_ids, nullptr, WISP_F32, 0, nullptr, nullptr, T, K, E, cap,
                            single_group, expert_map, slot_to_expert, lru_tick, counters, slots,
                            nullptr, nullptr, record, record_words, (hipStream_t)stream,
                            nullptr);
}

extern "C" int wisp_pager_decide_host(const int32_t* topk_ids, int T, int K, int E, int cap,
                                      int single_group, int32_t* expert_map,
                                      int32_t* slot_to_expert, int64_t* lru_tick,
                                      int64_t* counters, int32_t* slots, int32_t* record,
                                      int record_words) {
  wisp::PagerView st{E, cap, expert_map, slot_to_expert, lru_tick, counters};
  return wisp::pager_decide_host(st, topk_ids, T, K, single_group, slots, record,
                                 record_words);
}

extern "C" int wisp_cpython_set_order(const int32_t* keys, int n, int32_t* order) {
  if (n < 0 || n > wisp::kMaxExperts) return -1;
  std::vector<int32_t> table(wisp::kMaxSetTable);
  return wisp::cpython_set_order(keys, n, order, table.data(), wisp::kMaxSetTable);
}

extern "C" int wisp_subbatch_plan(const int32_t* topk_ids, int T, int K, int cap,
                                  int32_t* group_end) {
  if (T < 0 || K < 1 || cap < 1) return -1;
  int ng = 0, cnt = 0, start = 0;
  std::vector<int32_t> cur;  // current group's distinct experts
  for (int t = 0; t < T; ++t) {
    std::vector<int32_t> fresh;
    for (int j = 0; j < K; ++j) {
      const int32_t e = topk_ids[t * K + j];
      if (std::find(cur.begin(), cur.end(), e) == cur.end() &&
          std::find(fresh.begin(), fresh.end(), e) == fresh.end())
        fresh.push_back(e);
    }
    if (cnt + (int)fresh.size() <= cap || t == start) {
      cur.insert(cur.end(), fresh.begin(), fresh.end());
      cnt += (int)fresh.size();
    } else {
      group_end[ng++] = t;
      start = t;
      cur.clear();
      for (int j = 0; j < K; ++j) {
        const int32_t e = topk_ids[t * K + j];
        if (std::find(cur.begin(), cur.end(), e) == cur.end()) cur.push_back(e);
      }
      cnt = (int)cur.size();
    }
  }
  group_end[ng++] = T;
  return ng;
}

extern "C" int wisp_record_words(int T, int K) { return wisp::RecordLayout(T, K).words(); }
