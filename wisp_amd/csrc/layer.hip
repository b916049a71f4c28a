// The paged MoE layer call: routing, the GPU pager, page-in on a side stream
// and the expert kernels, orchestrated on the host in C++.
//
// Replaces the reference's patched forward (src/wisp/integrations/vllm/
// fused_moe.py:930-987, 990-1237) and the copy half of ensure_resident
// (fused_moe.py:338-354).  Per paged call:
//   1. route (wisp_route_topk_softmax) and pager kernel on the caller's
//      stream; the pager writes its decision record to pinned host memory;
//   2. one event sync, then for each token group: the group's copies on the
//      layer's copy stream (after the previous group's expert kernels have
//      finished reading the scratch - write-after-read fence), an event, the
//      caller's stream waits on it (read-after-write fence), then the
//      group's expert kernels.
// Resident mode (cap == E, identity map) skips the pager and the sync and
// reads expert e from slot e.
#include <string.h>

#include <string>
#include <vector>

#include "common.h"
#include "pager_core.h"

static thread_local std::string g_last_error;

void wisp_set_last_error(const char* what, const char* where) {
  g_last_error = std::string(where) + ": " + what;
}

extern "C" const char* wisp_last_error(void) { return g_last_error.c_str(); }
extern "C" int wisp_abi_version(void) { return 1; }

namespace wisp {

int launch_pager(const int32_t* ids, int T, int K, int E, int cap, int single_group,
                 int32_t* map, int32_t* s2e, int64_t* tick, int64_t* ctr, int32_t* slots,
                 int32_t* rec, int rec_words, hipStream_t stream);
int experts_gemv(const void* x, int dtype, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, const void* w13, size_t w13_stride, const void* w2,
                 size_t w2_stride, void* act, void* out, hipStream_t st, const StageEvents* ev);
int experts_mfma(const void* x, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, const void* w13, size_t w13_stride, const void* w2,
                 size_t w2_stride, void* act, void* out, hipStream_t st, const StageEvents* ev);

namespace {

constexpr int kEventRing = 4;
constexpr int kProfRing = 256;

// Dispatch-timestamp timing of the two expert kernels of the first group of
// a call (see StageEvents).
struct ProfSlot {
  StageEvents se = {};
  bool pending = false;
};

size_t elem_size(int dtype) { return dtype == WISP_F32 ? 4 : 2; }

struct Layer {
  wisp_layer_desc d;
  hipStream_t copy_stream = nullptr;
  hipEvent_t ev_decided = nullptr;
  hipEvent_t ev_copy[kEventRing] = {};
  hipEvent_t ev_gemm[kEventRing] = {};
  hipEvent_t ev_pin_start = nullptr, ev_pin_end = nullptr;
  bool pin_pending = false;
  double pin_bytes_pending = 0;
  double pin_ms_total = 0, pin_bytes_total = 0;
  int64_t pin_calls = 0;
  bool fused_slab = false;
  size_t es = 2;
  bool profile = false;
  int prof_next = 0;
  ProfSlot prof[kProfRing];
  double prof_ms[2] = {0, 0};
  int64_t prof_n = 0;
};

void prof_harvest(Layer& L, ProfSlot& p) {
  if (!p.pending) return;
  float a = 0.f, b = 0.f;
  if (hipEventSynchronize(p.se.ev[3]) == hipSuccess &&
      hipEventElapsedTime(&a, p.se.ev[0], p.se.ev[1]) == hipSuccess &&
      hipEventElapsedTime(&b, p.se.ev[2], p.se.ev[3]) == hipSuccess) {
    L.prof_ms[0] += a;
    L.prof_ms[1] += b;
    L.prof_n += 1;
  }
  p.pending = false;
}

// Next free profiling slot (harvesting whatever it held), or null when off.
ProfSlot* prof_begin(Layer& L) {
  if (!L.profile) return nullptr;
  ProfSlot& p = L.prof[L.prof_next];
  L.prof_next = (L.prof_next + 1) % kProfRing;
  prof_harvest(L, p);
  if (!p.se.ev[0]) {
    for (int i = 0; i < 4; ++i)
      if (hipEventCreate(&p.se.ev[i]) != hipSuccess) return nullptr;
  }
  return &p;
}

__global__ void identity_kernel(int32_t* map, int32_t* s2e, int64_t* tick, int E) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < E) {
    map[e] = e;
    s2e[e] = e;
  }
}

// Copies of `n` loaded (expert, slot) pairs.
int issue_copies(Layer& L, const int32_t* pairs, int n, hipStream_t cs, double* bytes) {
  const size_t es = L.es;
  const size_t w13_bytes = L.d.w13_elems * es;
  const size_t w2_bytes = L.d.w2_elems * es;
  for (int j = 0; j < n; ++j) {
    const int e = pairs[2 * j], s = pairs[2 * j + 1];
    if (e < 0 || e >= L.d.num_experts || s < 0 || s >= L.d.cap) {
      wisp_set_last_error("decision record holds an out-of-range pair", "page-in");
      return WISP_ERR_INVALID;
    }
    char* d13 = (char*)L.d.scratch_w13 + (size_t)s * L.d.scratch_w13_stride * es;
    const char* m13 = (const char*)L.d.master_w13 + (size_t)e * L.d.master_w13_stride * es;
    if (L.fused_slab) {
      WISP_HIP_TRY(hipMemcpyAsync(d13, m13, w13_bytes + w2_bytes, hipMemcpyHostToDevice, cs));
    } else {
      char* d2 = (char*)L.d.scratch_w2 + (size_t)s * L.d.scratch_w2_stride * es;
      const char* m2 = (const char*)L.d.master_w2 + (size_t)e * L.d.master_w2_stride * es;
      WISP_HIP_TRY(hipMemcpyAsync(d13, m13, w13_bytes, hipMemcpyHostToDevice, cs));
      WISP_HIP_TRY(hipMemcpyAsync(d2, m2, w2_bytes, hipMemcpyHostToDevice, cs));
    }
    *bytes += (double)(w13_bytes + w2_bytes);
  }
  return WISP_OK;
}

void harvest_pagein_timing(Layer& L) {
  if (!L.pin_pending) return;
  float ms = 0.f;
  if (hipEventElapsedTime(&ms, L.ev_pin_start, L.ev_pin_end) == hipSuccess) {
    L.pin_ms_total += ms;
    L.pin_bytes_total += L.pin_bytes_pending;
    L.pin_calls += 1;
  }
  L.pin_pending = false;
  L.pin_bytes_pending = 0;
}

int experts(Layer& L, const void* x, int T, int K, const float* w, const int32_t* slots,
            void* act, void* out, int algo, hipStream_t st, bool timed) {
  const wisp_layer_desc& d = L.d;
  ProfSlot* p = timed && T > 0 ? prof_begin(L) : nullptr;
  const StageEvents* se = p ? &p->se : nullptr;
  int rc;
  if (algo == WISP_ALGO_MFMA)
    rc = experts_mfma(x, T, d.hidden, d.inter, K, w, slots, d.scratch_w13, d.scratch_w13_stride,
                      d.scratch_w2, d.scratch_w2_stride, act, out, st, se);
  else
    rc = experts_gemv(x, d.dtype, T, d.hidden, d.inter, K, w, slots, d.scratch_w13,
                      d.scratch_w13_stride, d.scratch_w2, d.scratch_w2_stride, act, out, st, se);
  if (rc != WISP_OK) return rc;
  if (p) p->pending = true;
  return WISP_OK;
}

// Kernel choice depends only on the whole call's T and the dtype, never on
// the grouping, so paged and resident runs of one batch use one kernel.
int choose_algo(int algo, int dtype, int T) {
  (void)dtype;
  (void)T;
  if (algo != WISP_ALGO_AUTO) return algo;
  return WISP_ALGO_GEMV;
}

// Copies and expert kernels for groups [0, ngroups) of a decision record.
int run_groups(Layer& L, const int32_t* rec, int T, int K, int ngroups, bool compute,
               const void* x, const float* topk_w, const int32_t* slots, void* act, void* out,
               int algo, hipStream_t st) {
  const RecordLayout RL(T, K);
  const size_t row = (size_t)L.d.hidden * L.es;
  int last_gemm = -1;
  bool timing_started = false;
  for (int g = 0; g < ngroups; ++g) {
    const int32_t* G = rec + RL.group_base(g);
    const int t0 = G[0], t1 = G[1], ld_off = G[6], n_ld = G[7];
    if (n_ld > 0) {
      if (last_gemm >= 0)
        WISP_HIP_TRY(hipStreamWaitEvent(L.copy_stream, L.ev_gemm[last_gemm % kEventRing], 0));
      if (!timing_started) {
        harvest_pagein_timing(L);
        WISP_HIP_TRY(hipEventRecord(L.ev_pin_start, L.copy_stream));
        timing_started = true;
      }
      int rc = issue_copies(L, rec + RL.loaded_base() + 2 * ld_off, n_ld, L.copy_stream,
                            &L.pin_bytes_pending);
      if (rc != WISP_OK) return rc;
      WISP_HIP_TRY(hipEventRecord(L.ev_copy[g % kEventRing], L.copy_stream));
      WISP_HIP_TRY(hipStreamWaitEvent(st, L.ev_copy[g % kEventRing], 0));
    }
    if (compute && t1 > t0) {
      int rc = experts(L, (const char*)x + (size_t)t0 * row, t1 - t0, K, topk_w + (size_t)t0 * K,
                       slots + (size_t)t0 * K, act, (char*)out + (size_t)t0 * row, algo, st,
                       g == 0);
      if (rc != WISP_OK) return rc;
      WISP_HIP_TRY(hipEventRecord(L.ev_gemm[g % kEventRing], st));
      last_gemm = g;
    }
  }
  if (timing_started) {
    WISP_HIP_TRY(hipEventRecord(L.ev_pin_end, L.copy_stream));
    L.pin_pending = true;
  }
  return WISP_OK;
}

// Device view of the (pinned host) decision record; device memory passes
// through unchanged.
int32_t* record_device_ptr(int32_t* rec) {
  void* dev = nullptr;
  if (hipHostGetDevicePointer(&dev, rec, 0) == hipSuccess && dev) return (int32_t*)dev;
  (void)hipGetLastError();
  return rec;
}

int check_ws(const wisp_workspace* ws, int T, int K) {
  if (!ws || (int64_t)T * K > ws->max_pairs || !ws->topk_w || !ws->topk_ids || !ws->slots ||
      !ws->act || !ws->record || ws->record_words < RecordLayout(T, K).words()) {
    wisp_set_last_error("workspace too small or missing", "wisp_layer_forward");
    return WISP_ERR_INVALID;
  }
  return WISP_OK;
}

}  // namespace
}  // namespace wisp

using wisp::Layer;

extern "C" int wisp_layer_create(const wisp_layer_desc* desc, void** handle) {
  using namespace wisp;
  if (!desc || !handle) return WISP_ERR_INVALID;
  const wisp_layer_desc& d = *desc;
  if (d.num_experts < 1 || d.num_experts > kMaxExperts || d.cap < 1 || d.cap > d.num_experts ||
      d.hidden < 0 || d.inter < 0 || d.w13_elems < 1 || d.w2_elems < 1 ||
      (d.hidden > 0 && (d.w13_elems != (size_t)2 * d.inter * d.hidden ||
                        d.w2_elems != (size_t)d.hidden * d.inter)) ||
      (d.dtype != WISP_F32 && d.dtype != WISP_BF16) ||
      (d.mode != WISP_MODE_PAGED && d.mode != WISP_MODE_RESIDENT) || !d.scratch_w13 ||
      !d.scratch_w2 || !d.master_w13 || !d.master_w2 || !d.expert_map || !d.slot_to_expert ||
      !d.lru_tick || !d.counters || d.scratch_w13_stride < d.w13_elems ||
      d.scratch_w2_stride < d.w2_elems || d.master_w13_stride < d.w13_elems ||
      d.master_w2_stride < d.w2_elems ||
      (d.mode == WISP_MODE_RESIDENT && d.cap != d.num_experts)) {
    wisp_set_last_error("invalid layer descriptor", "wisp_layer_create");
    return WISP_ERR_INVALID;
  }
  const size_t es = elem_size(d.dtype);
  Layer* L = new Layer();
  L->d = d;
  L->es = es;
  const size_t w13_elems = d.w13_elems;
  L->fused_slab = d.master_w13_stride == d.master_w2_stride &&
                  d.scratch_w13_stride == d.scratch_w2_stride &&
                  (const char*)d.master_w2 == (const char*)d.master_w13 + w13_elems * es &&
                  (const char*)d.scratch_w2 == (const char*)d.scratch_w13 + w13_elems * es;
  hipError_t e = hipStreamCreateWithFlags(&L->copy_stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&L->ev_decided, hipEventDisableTiming);
  for (int i = 0; i < kEventRing && e == hipSuccess; ++i) {
    e = hipEventCreateWithFlags(&L->ev_copy[i], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&L->ev_gemm[i], hipEventDisableTiming);
  }
  if (e == hipSuccess) e = hipEventCreate(&L->ev_pin_start);
  if (e == hipSuccess) e = hipEventCreate(&L->ev_pin_end);
  if (e != hipSuccess) {
    wisp_set_last_error(hipGetErrorString(e), "wisp_layer_create");
    wisp_layer_destroy(L);
    return WISP_ERR_HIP;
  }
  *handle = L;
  return WISP_OK;
}

extern "C" int wisp_layer_destroy(void* handle) {
  Layer* L = (Layer*)handle;
  if (!L) return WISP_OK;
  if (L->copy_stream) (void)hipStreamSynchronize(L->copy_stream);
  for (int i = 0; i < wisp::kEventRing; ++i) {
    if (L->ev_copy[i]) (void)hipEventDestroy(L->ev_copy[i]);
    if (L->ev_gemm[i]) (void)hipEventDestroy(L->ev_gemm[i]);
  }
  if (L->ev_decided) (void)hipEventDestroy(L->ev_decided);
  if (L->ev_pin_start) (void)hipEventDestroy(L->ev_pin_start);
  if (L->ev_pin_end) (void)hipEventDestroy(L->ev_pin_end);
  for (int i = 0; i < wisp::kProfRing; ++i)
    for (int j = 0; j < 4; ++j)
      if (L->prof[i].se.ev[j]) (void)hipEventDestroy(L->prof[i].se.ev[j]);
  if (L->copy_stream) (void)hipStreamDestroy(L->copy_stream);
  delete L;
  return WISP_OK;
}

extern "C" int wisp_layer_set_scratch(void* handle, void* scratch_w13, void* scratch_w2, int cap,
                                      int32_t* slot_to_expert, int64_t* lru_tick) {
  Layer* L = (Layer*)handle;
  if (!L || !scratch_w13 || !scratch_w2 || cap < 1 || cap > L->d.num_experts ||
      !slot_to_expert || !lru_tick)
    return WISP_ERR_INVALID;
  (void)hipStreamSynchronize(L->copy_stream);
  L->pin_pending = false;
  const size_t es = L->es, w13_elems = L->d.w13_elems;
  L->d.scratch_w13 = scratch_w13;
  L->d.scratch_w2 = scratch_w2;
  L->fused_slab = L->d.master_w13_stride == L->d.master_w2_stride &&
                  L->d.scratch_w13_stride == L->d.scratch_w2_stride &&
                  (const char*)L->d.master_w2 == (const char*)L->d.master_w13 + w13_elems * es &&
                  (const char*)scratch_w2 == (const char*)scratch_w13 + w13_elems * es;
  L->d.cap = cap;
  L->d.slot_to_expert = slot_to_expert;
  L->d.lru_tick = lru_tick;
  return WISP_OK;
}

extern "C" int wisp_layer_forward(void* handle, const void* x, const void* logits,
                                  int logits_dtype, int T, int K, int renormalize, void* out,
                                  const wisp_workspace* ws, int algo, wisp_stream_t stream) {
  using namespace wisp;
  Layer* L = (Layer*)handle;
  if (!L || T < 0 || (T > 0 && (!x || !logits || !out))) return WISP_ERR_INVALID;
  if (K < 1 || K > L->d.num_experts || K > kMaxTopK) {
    wisp_set_last_error("top_k outside [1, num_experts]", "wisp_layer_forward");
    return WISP_ERR_INVALID;
  }
  int rc = check_ws(ws, T, K);
  if (rc != WISP_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  const wisp_layer_desc& d = L->d;
  const size_t es = L->es;
  if (d.hidden < 1 || d.inter < 1 || (d.hidden * es) % 16 || (d.inter * es) % 16 ||
      (d.scratch_w13_stride * es) % 16 || (d.scratch_w2_stride * es) % 16 ||
      ((uintptr_t)d.scratch_w13) % 16 || ((uintptr_t)d.scratch_w2) % 16 ||
      (T > 0 && (((uintptr_t)x) % 16 || ((uintptr_t)out) % 16))) {
    wisp_set_last_error("expert shape/alignment outside the kernels' coverage (H and I must "
                        "be multiples of 16 bytes, buffers 16-byte aligned)",
                        "wisp_layer_forward");
    return WISP_ERR_UNSUPPORTED;
  }
  const int a = choose_algo(algo, d.dtype, T);
  if (a == WISP_ALGO_MFMA && d.dtype != WISP_BF16) return WISP_ERR_UNSUPPORTED;

  if (d.mode == WISP_MODE_RESIDENT) {
    rc = wisp_route_topk_softmax(logits, logits_dtype, T, d.num_experts, K, renormalize,
                                 ws->topk_w, ws->topk_ids, d.counters + kForward, stream);
    if (rc != WISP_OK) return rc;
    return experts(*L, x, T, K, ws->topk_w, ws->topk_ids, ws->act, out, a, st, true);
  }

  rc = wisp_route_topk_softmax(logits, logits_dtype, T, d.num_experts, K, renormalize,
                               ws->topk_w, ws->topk_ids, nullptr, stream);
  if (rc != WISP_OK) return rc;
  rc = launch_pager(ws->topk_ids, T, K, d.num_experts, d.cap, 0, d.expert_map,
                    d.slot_to_expert, d.lru_tick, d.counters, ws->slots,
                    record_device_ptr(ws->record), ws->record_words, st);
  if (rc != WISP_OK) return rc;
  WISP_HIP_TRY(hipEventRecord(L->ev_decided, st));
  WISP_HIP_TRY(hipEventSynchronize(L->ev_decided));
  const int32_t* rec = ws->record;
  const int status = rec[kRecStatus];
  if (status == WISP_ERR_INVALID) {
    wisp_set_last_error("routed expert id out of range", "wisp_layer_forward");
    return status;
  }
  rc = run_groups(*L, rec, T, K, rec[kRecGroupsDone], status == WISP_OK, x, ws->topk_w,
                  ws->slots, ws->act, out, a, st);
  if (rc != WISP_OK) return rc;
  if (status == WISP_ERR_SUBBATCH)
    wisp_set_last_error("one token routes to more experts than cap; sub-batching cannot help",
                        "wisp_layer_forward");
  return status;
}

extern "C" int wisp_layer_ensure_resident(void* handle, const int32_t* ids, int n,
                                          const wisp_workspace* ws, wisp_stream_t stream) {
  using namespace wisp;
  Layer* L = (Layer*)handle;
  if (!L || n < 0 || (n > 0 && !ids) || !ws || !ws->record ||
      ws->record_words < RecordLayout(n, 1).words())
    return WISP_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const wisp_layer_desc& d = L->d;
  int rc = launch_pager(ids, n, 1, d.num_experts, d.cap, 1, d.expert_map, d.slot_to_expert,
                        d.lru_tick, d.counters, nullptr, record_device_ptr(ws->record),
                        ws->record_words, st);
  if (rc != WISP_OK) return rc;
  WISP_HIP_TRY(hipEventRecord(L->ev_decided, st));
  WISP_HIP_TRY(hipEventSynchronize(L->ev_decided));
  const int32_t* rec = ws->record;
  const int status = rec[kRecStatus];
  if (status == WISP_ERR_INVALID) return status;
  // ensure_resident is a single call: one group, planned over n tokens x 1.
  const RecordLayout RL(n, 1);
  const int32_t* G = rec + RL.group_base(0);
  if (rec[kRecGroupsDone] > 0 && G[7] > 0) {
    harvest_pagein_timing(*L);
    WISP_HIP_TRY(hipEventRecord(L->ev_pin_start, L->copy_stream));
    rc = issue_copies(*L, rec + RL.loaded_base() + 2 * G[6], G[7], L->copy_stream,
                      &L->pin_bytes_pending);
    if (rc != WISP_OK) return rc;
    WISP_HIP_TRY(hipEventRecord(L->ev_pin_end, L->copy_stream));
    L->pin_pending = true;
    WISP_HIP_TRY(hipEventRecord(L->ev_copy[0], L->copy_stream));
    WISP_HIP_TRY(hipStreamWaitEvent(st, L->ev_copy[0], 0));
  }
  if (status == WISP_ERR_SUBBATCH)
    wisp_set_last_error("working set exceeds cap_experts; the caller must sub-batch",
                        "wisp_layer_ensure_resident");
  return status;
}

extern "C" int wisp_layer_prime_identity(void* handle, wisp_stream_t stream) {
  using namespace wisp;
  Layer* L = (Layer*)handle;
  if (!L) return WISP_ERR_INVALID;
  const wisp_layer_desc& d = L->d;
  if (d.cap != d.num_experts) {
    wisp_set_last_error("prime_identity requires cap == num_experts", "wisp_layer_prime_identity");
    return WISP_ERR_INVALID;
  }
  hipStream_t st = (hipStream_t)stream;
  std::vector<int32_t> pairs(2 * (size_t)d.num_experts);
  for (int e = 0; e < d.num_experts; ++e) {
    pairs[2 * e] = e;
    pairs[2 * e + 1] = e;
  }
  double bytes = 0;
  int rc = issue_copies(*L, pairs.data(), d.num_experts, L->copy_stream, &bytes);
  if (rc != WISP_OK) return rc;
  WISP_HIP_TRY(hipEventRecord(L->ev_copy[0], L->copy_stream));
  WISP_HIP_TRY(hipStreamWaitEvent(st, L->ev_copy[0], 0));
  hipLaunchKernelGGL(identity_kernel, dim3((d.num_experts + 255) / 256), dim3(256), 0, st,
                     d.expert_map, d.slot_to_expert, d.lru_tick, d.num_experts);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

extern "C" int wisp_layer_last_pagein(void* handle, float* ms, double* bytes) {
  Layer* L = (Layer*)handle;
  if (!L) return WISP_ERR_INVALID;
  wisp::harvest_pagein_timing(*L);
  if (ms) *ms = (float)L->pin_ms_total;
  if (bytes) *bytes = L->pin_bytes_total;
  L->pin_ms_total = 0;
  L->pin_bytes_total = 0;
  L->pin_calls = 0;
  return WISP_OK;
}

extern "C" int wisp_layer_profile(void* handle, int enable, double* w13_ms, double* w2_ms,
                                  int64_t* launches) {
  Layer* L = (Layer*)handle;
  if (!L) return WISP_ERR_INVALID;
  for (int i = 0; i < wisp::kProfRing; ++i) wisp::prof_harvest(*L, L->prof[i]);
  if (w13_ms) *w13_ms = L->prof_ms[0];
  if (w2_ms) *w2_ms = L->prof_ms[1];
  if (launches) *launches = L->prof_n;
  L->prof_ms[0] = L->prof_ms[1] = 0;
  L->prof_n = 0;
  L->profile = enable != 0;
  return WISP_OK;
}

extern "C" int wisp_pagein_issue(const int32_t* record, int record_words, int T, int K,
                                 int group, const void* master_w13, size_t master_w13_stride,
                                 const void* master_w2, size_t master_w2_stride,
                                 void* scratch_w13, size_t scratch_w13_stride, void* scratch_w2,
                                 size_t scratch_w2_stride, size_t w13_bytes, size_t w2_bytes,
                                 int fused_slab, wisp_stream_t copy_stream) {
  using namespace wisp;
  const RecordLayout RL(T, K);
  if (!record || record_words < RL.words() || group < 0 || group >= record[kRecGroupsDone] ||
      !master_w13 || !scratch_w13 || (!fused_slab && (!master_w2 || !scratch_w2)))
    return WISP_ERR_INVALID;
  const int32_t* G = record + RL.group_base(group);
  const int32_t* pairs = record + RL.loaded_base() + 2 * G[6];
  hipStream_t cs = (hipStream_t)copy_stream;
  for (int j = 0; j < G[7]; ++j) {
    const int e = pairs[2 * j], s = pairs[2 * j + 1];
    char* d13 = (char*)scratch_w13 + (size_t)s * scratch_w13_stride;
    const char* m13 = (const char*)master_w13 + (size_t)e * master_w13_stride;
    if (fused_slab) {
      WISP_HIP_TRY(hipMemcpyAsync(d13, m13, w13_bytes + w2_bytes, hipMemcpyHostToDevice, cs));
    } else {
      WISP_HIP_TRY(hipMemcpyAsync(d13, m13, w13_bytes, hipMemcpyHostToDevice, cs));
      WISP_HIP_TRY(hipMemcpyAsync((char*)scratch_w2 + (size_t)s * scratch_w2_stride,
                                  (const char*)master_w2 + (size_t)e * master_w2_stride,
                                  w2_bytes, hipMemcpyHostToDevice, cs));
    }
  }
  return WISP_OK;
}

extern "C" int wisp_moe_experts(const void* x, int dtype, int T, int H, int I, int K,
                                const float* topk_w, const int32_t* slots, const void* w13,
                                size_t w13_stride, const void* w2, size_t w2_stride, void* act,
                                void* out, int algo, wisp_stream_t stream) {
  using namespace wisp;
  if (T < 0 || H < 1 || I < 1 || K < 1 || (dtype != WISP_F32 && dtype != WISP_BF16) ||
      (T > 0 && (!x || !topk_w || !slots || !w13 || !w2 || !act || !out)))
    return WISP_ERR_INVALID;
  const size_t es = elem_size(dtype);
  if ((H * es) % 16 || (I * es) % 16 || (w13_stride * es) % 16 || (w2_stride * es) % 16 ||
      ((uintptr_t)w13) % 16 || ((uintptr_t)w2) % 16 ||
      (T > 0 && (((uintptr_t)x) % 16 || ((uintptr_t)act) % 16 || ((uintptr_t)out) % 16))) {
    wisp_set_last_error("H, I and buffers must be 16-byte aligned", "wisp_moe_experts");
    return WISP_ERR_UNSUPPORTED;
  }
  const int a = choose_algo(algo, dtype, T);
  if (a == WISP_ALGO_MFMA) {
    if (dtype != WISP_BF16) return WISP_ERR_UNSUPPORTED;
    return experts_mfma(x, T, H, I, K, topk_w, slots, w13, w13_stride, w2, w2_stride, act, out,
                        (hipStream_t)stream, nullptr);
  }
  return experts_gemv(x, dtype, T, H, I, K, topk_w, slots, w13, w13_stride, w2, w2_stride, act,
                      out, (hipStream_t)stream, nullptr);
}
