// Cross-layer speculative prefetch: the co-occurrence predictor and the
// prefetch decisions, on the GPU.
//
// Replaces, from the reference:
//   * CooccurTable.observe_step (src/wisp/oracle/cooccur.py:79-104) and the
//     per-step observation dict of the paged forward
//     (src/wisp/integrations/vllm/fused_moe.py:1199, 1224-1233);
//   * predict_layer (cooccur.py:233-287) as called by _cooccur_predict_top_k
//     (fused_moe.py:634-650);
//   * WispMoEState.prefetch_async (fused_moe.py:360-433): the eviction and
//     slot decisions (the copies run in layer.hip on the layer's side stream).
//
// The table is dense in HBM: count[L_src][e_src][L_dst][e_dst] int32 (151 MB
// for 48 layers x 128 experts) and total[L][e].  A step's observations are
// the set-ordered experts of each layer seen so far in the step, so the
// predictor never waits for the host.
//
// Scores are IEEE doubles accumulated in the reference's order: source
// layers in the order the step saw them, each layer's experts in the
// iteration order of the CPython set the forward built, term (w * c) / denom
// with w = weights[target - L_src - 1] (decay powers computed by the host in
// Python floats).  A destination with no positive count is not a candidate;
// candidates rank by (score desc, id asc).  Zero-count pairs in a loaded
// table are treated as absent.
#include "common.h"
#include "pager_core.h"
#include "wave_set.h"

namespace wisp {
namespace {

constexpr int kMaxLayers = 256;

__device__ inline size_t count_index(int L, int E, int Ls, int es, int Ld, int ed) {
  return (((size_t)Ls * E + es) * L + Ld) * E + ed;
}

struct ObsSmem {
  uint32_t bits[kMaxExperts / 32];
  int32_t keys[kMaxExperts];
  int32_t order[kMaxExperts];
  int32_t table[kMaxSetTable];
};

// Sorted unique of ids[0..n) (ids outside [0, E) skipped) into s.keys; returns U.
__device__ inline int unique_sorted_wave(ObsSmem& s, const int32_t* ids, int n, int E, int lane) {
  const int nwords = (E + 31) >> 5;
  for (int w = lane; w < nwords; w += 64) s.bits[w] = 0u;
  wave_lds_sync();
  for (int p = lane; p < n; p += 64) {
    const int e = ids[p];
    if (e >= 0 && e < E) atomicOr(&s.bits[e >> 5], 1u << (e & 31));
  }
  wave_lds_sync();
  int U = 0;
  for (int base = 0; base < E; base += 64) {
    const int e = base + lane;
    const bool in = e < E && ((s.bits[e >> 5] >> (e & 31)) & 1u);
    const uint64_t b = __ballot(in);
    if (in) s.keys[U + popc_below(b)] = e;
    U += __popcll(b);
  }
  wave_lds_sync();
  return U;
}

// ---------------------------------------------------------------------------
// observe_layer: obs[layer] = set-ordered unique experts of ids (one wave).
// ---------------------------------------------------------------------------
// ordered != 0: ids are stored as given (the caller's iteration order; ids
// outside [0, E) dropped, at most E kept).
__global__ __launch_bounds__(64) void observe_layer_kernel(wisp_cooccur t, int layer,
                                                           const int32_t* __restrict__ ids,
                                                           int n, int ordered) {
  __shared__ ObsSmem s;
  const int lane = threadIdx.x;
  const int E = t.experts;
  int U = 0;
  if (ordered) {
    for (int base = 0; base < n && U < E; base += 64) {
      const int p = base + lane;
      const int e = p < n ? ids[p] : -1;
      const bool ok = e >= 0 && e < E;
      const uint64_t b = __ballot(ok);
      const int at = U + popc_below(b);
      if (ok && at < E) s.order[at] = e;
      U = min(E, U + __popcll(b));
    }
    wave_lds_sync();
  } else {
    U = unique_sorted_wave(s, ids, n, E, lane);
    if (U > 0) set_order_wave(s.keys, U, s.order, s.table, lane);
  }
  if (U == 0) return;  // the forward records only a non-empty set
  for (int j = lane; j < U; j += 64) t.obs_keys[(size_t)layer * E + j] = s.order[j];
  if (lane == 0) {
    if (t.obs_n[layer] == 0) {  // a layer keeps its first position in the step
      t.obs_seq[layer] = t.meta[0];
      t.meta[0] = t.meta[0] + 1;
    }
    t.obs_n[layer] = U;
  }
}

// ---------------------------------------------------------------------------
// predict: top-k destinations at `target` from the step's observations.
// One block of 256 threads: thread per destination expert for the scores,
// then rank by counting.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void predict_kernel(wisp_cooccur t, int target, int k,
                                                      const double* __restrict__ weights,
                                                      int normalize, int only_prev,
                                                      int32_t* __restrict__ out_ids,
                                                      int32_t* __restrict__ out_n) {
  __shared__ double score[kMaxExperts];
  __shared__ int32_t present[kMaxExperts];
  __shared__ int32_t layers[kMaxLayers];
  __shared__ int32_t nlayers;
  __shared__ int32_t npresent;
  const int L = t.layers, E = t.experts;
  if (threadIdx.x == 0) {
    // source layers in the order the step saw them
    int n = 0;
    const int seen = t.meta[0];
    for (int q = 0; q < seen; ++q)
      for (int Ls = 0; Ls < L; ++Ls)
        if (t.obs_n[Ls] > 0 && t.obs_seq[Ls] == q) layers[n++] = Ls;
    nlayers = n;
    npresent = 0;
  }
  __syncthreads();
  for (int ed = threadIdx.x; ed < E; ed += 256) {
    double sc = 0.0;
    int pres = 0;
    for (int li = 0; li < nlayers; ++li) {
      const int Ls = layers[li];
      if (Ls >= target) continue;
      if (only_prev && Ls != target - 1) continue;
      const double w = weights[target - Ls - 1];
      const int ns = t.obs_n[Ls];
      for (int j = 0; j < ns; ++j) {
        const int es = t.obs_keys[(size_t)Ls * E + j];
        const int c = t.count[count_index(L, E, Ls, es, target, ed)];
        if (c <= 0) continue;
        const int tot = normalize ? t.total[(size_t)Ls * E + es] : 1;
        const double denom = (normalize && tot > 0) ? (double)tot : 1.0;
        sc += (w * (double)c) / denom;
        pres = 1;
      }
    }
    score[ed] = sc;
    present[ed] = pres;
    if (pres) atomicAdd(&npresent, 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) {
    if (!present[e]) continue;
    const double se = score[e];
    int r = 0;
    for (int q = 0; q < E; ++q)
      r += present[q] && (score[q] > se || (score[q] == se && q < e));
    if (r < k) out_ids[r] = e;
  }
  if (threadIdx.x == 0) *out_n = min(k, npresent);
}

// ---------------------------------------------------------------------------
// end of step: learn the step's pairs and marginals (grid L x L), then clear.
// A forward's observations are sets, but a caller's ordered lists may repeat
// an id (the reference then counts it twice), hence atomic increments.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void learn_kernel(wisp_cooccur t) {
  const int Ls = blockIdx.x, Ld = blockIdx.y;
  const int L = t.layers, E = t.experts;
  const int ns = t.obs_n[Ls], nd = t.obs_n[Ld];
  if (ns == 0) return;
  if (Ls == Ld) {
    for (int i = threadIdx.x; i < ns; i += 256)
      atomicAdd(&t.total[(size_t)Ls * E + t.obs_keys[(size_t)Ls * E + i]], 1);
    return;
  }
  if (Ls > Ld || nd == 0) return;
  for (int q = threadIdx.x; q < ns * nd; q += 256) {
    const int es = t.obs_keys[(size_t)Ls * E + q / nd];
    const int ed = t.obs_keys[(size_t)Ld * E + q % nd];
    atomicAdd(&t.count[count_index(L, E, Ls, es, Ld, ed)], 1);
  }
}

__global__ __launch_bounds__(256) void end_step_kernel(wisp_cooccur t, int learned) {
  for (int Ls = threadIdx.x; Ls < t.layers; Ls += 256) t.obs_n[Ls] = 0;
  if (threadIdx.x == 0) {
    t.meta[0] = 0;
    if (learned) t.meta[1] = t.meta[1] + 1;
  }
}

// ---------------------------------------------------------------------------
// prefetch_async decisions on one layer's state (one wave).
// rec: [0] evicted, [1] loaded, [2] clock advanced (0/1), [3] predictions
// taken, then max_pred evicted (expert, slot) pairs, then max_pred loaded
// pairs.  The loaded pairs and rec[1] feed the copy kernel.
// ---------------------------------------------------------------------------
struct PrefetchSmem {
  ObsSmem set;
  uint32_t last[kMaxExperts / 32];
  uint32_t pred[kMaxExperts / 32];
  int32_t s2e[kMaxExperts];
  int64_t tick[kMaxExperts];
  int32_t load[kMaxExperts];
  int32_t freel[kMaxExperts];
  int32_t cand[kMaxExperts];
  int32_t sorted[kMaxExperts];
};

__global__ __launch_bounds__(64) void prefetch_kernel(
    const int32_t* __restrict__ predicted, const int32_t* __restrict__ n_pred_ptr, int n_pred_arg,
    int ordered, int count_pred, const int32_t* __restrict__ last_ids, int n_last, int E, int cap,
    int max_pred, int32_t* __restrict__ map_g, int32_t* __restrict__ s2e_g,
    int64_t* __restrict__ tick_g, int64_t* __restrict__ ctr_g, int32_t* __restrict__ rec) {
  __shared__ PrefetchSmem sm;
  const int lane = threadIdx.x;
  const int nwords = (E + 31) >> 5;
  int n = n_pred_ptr ? *n_pred_ptr : n_pred_arg;
  n = max(0, min(n, max_pred));
  int32_t* rec_ev = rec + 4;
  int32_t* rec_ld = rec + 4 + 2 * max_pred;

  // Predictions in insertion order, first occurrence of each valid id kept.
  for (int w = lane; w < nwords; w += 64) {
    sm.pred[w] = 0u;
    sm.last[w] = 0u;
  }
  wave_lds_sync();
  int U = 0;
  for (int base = 0; base < n; base += 64) {
    const int p = base + lane;
    int e = p < n ? predicted[p] : -1;
    bool ok = e >= 0 && e < E;
    // drop a repeat of an id earlier in the list (within this chunk too);
    // every lane runs all 64 shuffles
    for (int q = 0; q < 64; ++q) {
      const int eq = __shfl(e, q);
      if (q < lane && eq == e) ok = false;
    }
    if (ok && ((sm.pred[e >> 5] >> (e & 31)) & 1u)) ok = false;
    const uint64_t b = __ballot(ok);
    if (ok) sm.set.keys[U + popc_below(b)] = e;
    U += __popcll(b);
    wave_lds_sync();
    if (ok) atomicOr(&sm.pred[e >> 5], 1u << (e & 31));
    wave_lds_sync();
  }
  if (lane == 0) {
    rec[0] = rec[1] = rec[2] = 0;
    rec[3] = U;
    if (count_pred && n > 0) ctr_g[kPredTotal] += n;
  }
  if (U == 0) return;
  const int32_t* order = sm.set.keys;
  if (!ordered) {
    set_order_wave(sm.set.keys, U, sm.set.order, sm.set.table, lane);
    order = sm.set.order;
  }
  for (int p = lane; p < n_last; p += 64) {
    const int e = last_ids[p];
    if (e >= 0 && e < E) atomicOr(&sm.last[e >> 5], 1u << (e & 31));
  }
  for (int s = lane; s < cap; s += 64) {
    sm.s2e[s] = s2e_g[s];
    sm.tick[s] = tick_g[s];
  }
  wave_lds_sync();

  // to_load: predictions not resident, in set order
  int nload = 0;
  for (int base = 0; base < U; base += 64) {
    const int j = base + lane;
    const int e = j < U ? order[j] : -1;
    const bool m = j < U && map_g[e] < 0;
    const uint64_t b = __ballot(m);
    if (m) sm.load[nload + popc_below(b)] = e;
    nload += __popcll(b);
  }
  if (nload == 0) return;
  // free slots and eviction candidates, ascending slot
  int nfree = 0, ncand = 0;
  for (int base = 0; base < cap; base += 64) {
    const int s = base + lane;
    bool f = false, c = false;
    if (s < cap) {
      const int cur = sm.s2e[s];
      f = cur < 0;
      c = cur >= 0 && !((sm.last[cur >> 5] >> (cur & 31)) & 1u) &&
          !((sm.pred[cur >> 5] >> (cur & 31)) & 1u);
    }
    const uint64_t fb = __ballot(f), cb = __ballot(c);
    if (f) sm.freel[nfree + popc_below(fb)] = s;
    if (c) sm.cand[ncand + popc_below(cb)] = s;
    nfree += __popcll(fb);
    ncand += __popcll(cb);
  }
  wave_lds_sync();
  int need = nload - nfree;
  int nev = 0;
  if (need > 0) {
    if (need > ncand) {  // speculative: keep only what fits, first in set order
      nload = ncand + nfree;
      need = nload - nfree;
    }
    for (int i = lane; i < ncand; i += 64) {  // stable sort of the candidates by tick
      const int64_t ti = sm.tick[sm.cand[i]];
      int r = 0;
      for (int j = 0; j < ncand; ++j) {
        const int64_t tj = sm.tick[sm.cand[j]];
        r += (tj < ti) || (tj == ti && j < i);
      }
      sm.sorted[r] = sm.cand[i];
    }
    wave_lds_sync();
    nev = need;
    for (int r = lane; r < nev; r += 64) {
      const int s = sm.sorted[r];
      const int victim = sm.s2e[s];
      map_g[victim] = -1;
      sm.s2e[s] = -1;
      sm.freel[nfree + r] = s;
      rec_ev[2 * r] = victim;
      rec_ev[2 * r + 1] = s;
    }
    nfree += nev;
    wave_lds_sync();
  }
  const int64_t clock = ctr_g[kClock] + 1;
  const int nput = min(nload, nfree);
  for (int j = lane; j < nput; j += 64) {
    const int s = sm.freel[nfree - 1 - j];
    const int e = sm.load[j];
    sm.s2e[s] = e;
    sm.tick[s] = clock;
    map_g[e] = s;
    rec_ld[2 * j] = e;
    rec_ld[2 * j + 1] = s;
  }
  wave_lds_sync();
  for (int s = lane; s < cap; s += 64) {
    s2e_g[s] = sm.s2e[s];
    tick_g[s] = sm.tick[s];
  }
  if (lane == 0) {
    ctr_g[kClock] = clock;
    ctr_g[kEvict] += nev;
    rec[0] = nev;
    rec[1] = nput;
    rec[2] = 1;
  }
}

}  // namespace

int prefetch_record_words(int max_pred) { return 4 + 4 * max_pred; }

int launch_prefetch(const int32_t* predicted, const int32_t* n_pred_ptr, int n_pred, int ordered,
                    int count_pred, const int32_t* last_ids, int n_last, int E, int cap,
                    int max_pred, int32_t* map, int32_t* s2e, int64_t* tick, int64_t* ctr,
                    int32_t* rec, hipStream_t st) {
  hipLaunchKernelGGL(prefetch_kernel, dim3(1), dim3(64), 0, st, predicted, n_pred_ptr, n_pred,
                     ordered, count_pred, last_ids, n_last, E, cap, max_pred, map, s2e, tick,
                     ctr, rec);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

}  // namespace wisp

using namespace wisp;

static int check_table(const wisp_cooccur* t) {
  if (!t || t->layers < 1 || t->layers > kMaxLayers || t->experts < 1 ||
      t->experts > kMaxExperts || !t->count || !t->total || !t->obs_keys || !t->obs_n ||
      !t->obs_seq || !t->meta)
    return WISP_ERR_INVALID;
  return WISP_OK;
}

extern "C" int wisp_cooccur_observe_layer(const wisp_cooccur* t, int layer, const int32_t* ids,
                                          int n, int ordered, wisp_stream_t stream) {
  if (check_table(t) != WISP_OK || layer < 0 || layer >= t->layers || n < 0 || (n > 0 && !ids))
    return WISP_ERR_INVALID;
  if (n == 0) return WISP_OK;
  hipLaunchKernelGGL(observe_layer_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, *t, layer,
                     ids, n, ordered);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

extern "C" int wisp_cooccur_predict(const wisp_cooccur* t, int target_layer, int k,
                                    const double* weights, int normalize, int only_prev_layer,
                                    int32_t* out_ids, int32_t* out_n, wisp_stream_t stream) {
  if (check_table(t) != WISP_OK || target_layer < 0 || target_layer >= t->layers || k < 0 ||
      !weights || !out_ids || !out_n)
    return WISP_ERR_INVALID;
  hipLaunchKernelGGL(predict_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, *t, target_layer,
                     k, weights, normalize, only_prev_layer, out_ids, out_n);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

extern "C" int wisp_cooccur_end_step(const wisp_cooccur* t, int learn, wisp_stream_t stream) {
  if (check_table(t) != WISP_OK) return WISP_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  if (learn)
    hipLaunchKernelGGL(learn_kernel, dim3(t->layers, t->layers), dim3(256), 0, st, *t);
  hipLaunchKernelGGL(end_step_kernel, dim3(1), dim3(256), 0, st, *t, learn ? 1 : 0);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

extern "C" int wisp_prefetch_record_words(int max_predicted) {
  return max_predicted < 0 ? -1 : wisp::prefetch_record_words(max_predicted);
}
