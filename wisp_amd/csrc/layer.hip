// The paged MoE layer call: routing, the GPU pager, page-in and the expert
// kernels, orchestrated on the host in C++.
//
// Replaces the reference's patched forward (src/wisp/integrations/vllm/
// fused_moe.py:930-987, 990-1237) and the copy half of ensure_resident
// (fused_moe.py:338-354).
//
// Paged call, one token group guaranteed (T*K <= cap, e.g. bs=1 decode),
// kernel page-in engine:
//   caller's stream: [route+pager] [page-in copy kernel] [w13] [w2]
// The pager leaves the (expert, slot) load list and its length in device
// memory and the copy kernel reads them there, so the host enqueues the four
// launches and returns: no host round trip, no copy-engine hand-off.  A call
// that loads nothing pays one near-empty launch.
//
// Same call, memcpy engine (hipMemcpyAsync):
//   caller's stream: [route+pager] [w13, pairs that hit] [w2 unless loads]
//   host:            wait for the decision record; if experts were loaded:
//                    the copies, then [w13, loaded pairs] [w2].
// The expert kernels of an all-hit call are already queued behind the pager,
// so the GPU never waits for the host; on a miss call the hit experts'
// gate/up GEMV runs while the host reads the record.  Nothing on the GPU
// waits on a flag: the guards are a per-pair filter and a skip word the
// pager kernel wrote.
//
// Paged call, several groups possible: route (fused into the pager for
// T <= 8), pager, one sync, then per group: copies (copy kernel or
// hipMemcpyAsync), the group's expert kernels.
//
// hipMemcpyAsync copies run by default on the caller's stream, where stream order
// is both fences (a copy follows the kernels that read the slot before it;
// the kernels that read the slot follow the copy).  With side streams
// (pagein_streams 1 or 2) each copy stream first waits on an event recorded
// after the last kernels that read the scratch (write-after-read) and the
// caller's stream waits on an event after the copies (read-after-write).
// Measured on MI355X, each cross-queue event hop adds ~20 us of latency, so
// side streams only pay off when there is independent work to overlap.
//
// Resident mode (cap == E, identity map) skips the pager and the sync and
// reads expert e from slot e.
#include <string.h>

#include <string>
#include <vector>

#include "common.h"
#include "pagein.h"
#include "pager_core.h"

static thread_local std::string g_last_error;

void wisp_set_last_error(const char* what, const char* where) {
  g_last_error = std::string(where) + ": " + what;
}

extern "C" const char* wisp_last_error(void) { return g_last_error.c_str(); }
extern "C" int wisp_abi_version(void) { return 4; }

namespace wisp {

int launch_pager(const int32_t* ids, const void* logits, int logits_dtype, int renorm,
                 float* topk_w, int32_t* topk_ids, int T, int K, int E, int cap,
                 int single_group, int32_t* map, int32_t* s2e, int64_t* tick, int64_t* ctr,
                 int32_t* slots, int32_t* flags, int32_t* loads, int32_t* rec, int rec_words,
                 hipStream_t stream, int32_t* rec_host);
int gemv_w13(const void* x, int dtype, int T, int H, int I, int K, const int32_t* slots,
             int nslots, const void* w13, size_t w13_stride, void* act, hipStream_t st,
             hipEvent_t ev_start, hipEvent_t ev_stop, const int32_t* pair_filter, int want);
int pagein_w13(const PageInArgs& a, const void* x, int dtype, int T, int H, int I, int K,
               const int32_t* flags, const void* w13, size_t w13_stride, void* act,
               hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop);
int gemv_w2(const void* act, int dtype, int T, int H, int I, int K, const float* topk_w,
            const int32_t* slots, int nslots, const void* w2, size_t w2_stride, void* out,
            hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop, const int32_t* skip_if,
            int cap, const void* act_spec);
bool decode_w13_supported(int dtype, int H, int E, int K, int cap);
int decode_w13(const PageInArgs& a, const void* x, int dtype, int logits_dtype, int H, int I,
               int K, int32_t* flags, const void* w13, size_t w13_stride, void* act,
               const DecodePagerArgs& pa, hipStream_t st, hipEvent_t ev_start,
               hipEvent_t ev_stop);
int experts_gemv(const void* x, int dtype, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                 const void* w2, size_t w2_stride, void* act, void* out, hipStream_t st,
                 const StageEvents* ev);
int experts_mfma(const void* x, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                 const void* w2, size_t w2_stride, void* act, void* out, void* work,
                 size_t work_bytes, hipStream_t st, const StageEvents* ev);
size_t mfma_work_bytes(int T, int K, int H, int nslots);
size_t fp8_work_bytes(int T, int K, int H, int I, int nslots);
int experts_fp8(const void* x, int T, int H, int I, int K, const float* topk_w,
                const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                const float* s13, size_t s13_stride, const void* w2, size_t w2_stride,
                const float* s2, size_t s2_stride, int block_n, void* act, void* out,
                hipStream_t st, const StageEvents* ev, bool pager_slots);
int experts_fp8_w2(const void* act, int T, int H, int I, int K, const float* topk_w,
                   const int32_t* slots, int nslots, const void* w2, size_t w2_stride,
                   const float* s2, size_t s2_stride, int block_n, void* out, hipStream_t st,
                   hipEvent_t e0, hipEvent_t e1, bool pager_slots);
int pagein_fp8_w13(const PageInArgs& a, const void* x, int H, int I, int K,
                   const int32_t* slots, const int32_t* flags, int nslots, const void* w13,
                   size_t w13_stride, const float* s13, size_t s13_stride, int block_n,
                   size_t s13_off, void* act, hipStream_t st, hipEvent_t e0, hipEvent_t e1,
                   bool pager_slots);
bool fp8_fused_supported(int H);
const char* fp8_unsupported(int H, int I, int K, int block_n, int block_k);
int experts_fp8_grouped(const void* x, int T, int H, int I, int K, const float* topk_w,
                        const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                        const float* s13, size_t s13_stride, const void* w2, size_t w2_stride,
                        const float* s2, size_t s2_stride, int block_n, void* act, void* out,
                        void* work, size_t work_bytes, hipStream_t st, const StageEvents* ev);
int launch_prefetch(const int32_t* predicted, const int32_t* n_pred_ptr, int n_pred, int ordered,
                    int count_pred, const int32_t* last_ids, int n_last, int E, int cap,
                    int max_pred, int32_t* map, int32_t* s2e, int64_t* tick, int64_t* ctr,
                    int32_t* rec, hipStream_t st);
int prefetch_record_words(int max_pred);
bool mfma_supported(int H, int I);
bool gemv_supported(int dtype, int H, int K);

// Calls of at least this many tokens run the bf16 experts on the MFMA grouped
// GEMM; fewer run the GEMV kernels, which stream each routed expert once per
// token and win while the tokens of a call share few experts.  Measured on
// MI355X at the Qwen3 shape with uniform routing (resident, us per call):
// GEMV 136 / 158 / 178 and MFMA 141 / 147 / 153 at 12 / 14 / 16 tokens.
constexpr int kMfmaMinTokens = 14;
// The block-FP8 grouped path takes over from its decode kernels from here.
constexpr int kFp8GroupedMinTokens = 16;

// The automatic expert-kernel choice, or -1 when no kernel family covers the
// call.  It depends only on the call's dtype, shape, token count and top-k,
// never on the grouping or the slots, so paged and resident runs of one batch
// use one kernel.  A bf16 call the GEMV pair does not cover (more routed
// experts per token than its w2 block holds, or rows longer than its w13
// registers) takes the MFMA path whenever that covers the shape.
int auto_algo(int dtype, int H, int I, int T, int K) {
  if (dtype == WISP_FP8_E4M3)
    return T >= kFp8GroupedMinTokens ? WISP_ALGO_MFMA : WISP_ALGO_GEMV;
  const bool gemv = gemv_supported(dtype, H, K);
  if (dtype == WISP_BF16 && mfma_supported(H, I) && (T >= kMfmaMinTokens || !gemv))
    return WISP_ALGO_MFMA;
  return gemv ? WISP_ALGO_GEMV : -1;
}

namespace {

constexpr int kEventRing = 4;
constexpr int kCopyStreams = 2;
constexpr int kProfRing = 512;
constexpr int kPinRing = 64;

// Bytes of one weight element, and of one activation element (x, act, out).
size_t elem_size(int dtype) { return dtype == WISP_F32 ? 4 : dtype == WISP_FP8_E4M3 ? 1 : 2; }
size_t act_size(int dtype) { return dtype == WISP_F32 ? 4 : 2; }

// One tensor of an expert as the page-in moves it (see PageInPlane): host
// master address (and its device mapping, for the copy kernel), scratch
// address, byte strides and bytes per expert.
struct Plane {
  const char* host = nullptr;
  const char* dev = nullptr;
  size_t m_stride = 0;
  char* d = nullptr;
  size_t d_stride = 0;
  size_t bytes = 0;
};

// One timed kernel launch (dispatch timestamps).
struct ProfLaunch {
  hipEvent_t start = nullptr, stop = nullptr;
  int kind = 0;          // 0: w13 kernel, 1: w2 kernel
  bool pending = false;
  bool counted = true;   // false for a speculative launch that found nothing to do
  uint64_t gen = 0;      // the layer's launch number that last took this slot
};

// One copy-kernel launch: dispatch timestamps and the pinned word its first
// block sets to the number of experts it copied.  A fused page-in + w13
// launch that copied nothing is pure w13 work and is timed as such.
struct PinLaunch {
  hipEvent_t start = nullptr, stop = nullptr;
  bool pending = false;
  bool fused = false;
  // the w2 launch of the same call (fused launches), so that a call that
  // copied nothing adds its w2 time to the no-load pair statistics
  ProfLaunch* w2 = nullptr;
  uint64_t w2_gen = 0;
};

struct Layer {
  wisp_layer_desc d;
  bool fp8 = false;
  // the tensors one page-in moves per expert, merged where they are adjacent
  int nplanes = 0;
  Plane planes[kMaxPlanes];
  size_t expert_bytes = 0;  // weight (and scale) bytes of one expert
  // kernel page-in (engine WISP_PAGEIN_KERNEL and eligible masters)
  bool kpin = false;
  // with kpin: the device address of the packed masters, or null
  const char* packed_dev = nullptr;
  // the fused page-in + w13 launch applies (plane 0 starts with the whole
  // w13 of an expert, in master and scratch alike; for block-FP8 experts
  // the plane is the whole [w13 | w2 | s13 | s2] slab, the w13 scales at
  // byte s13_off of it)
  bool fused_ok = false;
  size_t s13_off = 0;
  int32_t* hist = nullptr;        // pinned host [kPinRing]
  int32_t* hist_dev = nullptr;
  int pin_next = 0;
  PinLaunch pin[kPinRing];
  // where the last layer call's decision record went: the workspace's device
  // copy (one-group calls on the copy-kernel engine) or its pinned record
  bool rec_on_device = false;
  // cross-layer prefetch: copies on copy[0], fenced by events
  hipEvent_t ev_pf_decided = nullptr, ev_pf_done = nullptr;
  bool pf_pending = false;
  int nstreams = 0;  // side copy streams in use (0: the caller's stream)
  hipStream_t copy[kCopyStreams] = {};
  hipEvent_t ev_decided = nullptr;
  hipEvent_t ev_copy[kCopyStreams][kEventRing] = {};
  hipEvent_t ev_gemm[kEventRing] = {};
  hipEvent_t ev_pin_start = nullptr, ev_pin_end = nullptr;
  bool pin_pending = false;
  double pin_bytes_pending = 0;
  double pin_ms_total = 0, pin_bytes_total = 0;
  size_t es = 2;  // bytes of one weight element
  bool profile = false;
  int prof_next = 0;
  ProfLaunch prof[kProfRing];
  double prof_ms[2] = {0, 0};
  int64_t prof_calls = 0;
  int64_t prof_w13_calls = 0;  // calls whose w13 time is in prof_ms[0]
  uint64_t prof_gen = 0;
  // w2 time of the fused calls that copied nothing: the calls whose w13 time
  // a fused launch adds to prof_ms[0]
  double prof_w2_nl_ms = 0;
  int64_t prof_w2_nl_calls = 0;
  // The fused decode launch (pager, page-in and w13 in one grid, for
  // one-token calls with top-k == cap): w13 per slot [spec_cap][inter] in
  // the activation dtype, and the word its pager wave publishes the
  // launch's epoch in (device memory, allocated with the layer).
  void* act_spec = nullptr;
  int spec_cap = 0;
  uint32_t* decode_sync = nullptr;
  uint32_t decode_epoch = 0;
  bool decode_fused = false;  // wisp_layer_set_decode_fused
};

void prof_harvest(Layer& L, ProfLaunch& p) {
  if (!p.pending) return;
  float ms = 0.f;
  if (p.counted && hipEventSynchronize(p.stop) == hipSuccess &&
      hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess)
    L.prof_ms[p.kind] += ms;
  p.pending = false;
}

// An event that only timestamps a launch.  Without the system-scope fence
// that a default event performs when it is recorded (an L2 writeback and
// invalidation), the timed launch runs as it does untimed: with default
// events the page-in + w13 launch of a Qwen3 bs=1 call measured ~0.7 us
// longer than the same launch in a run without events.
hipError_t timing_event(hipEvent_t* e) {
  return hipEventCreateWithFlags(e, hipEventDisableSystemFence);
}

// Next timing slot for a launch of `kind` (harvesting what it held), or null
// when timing is off.
ProfLaunch* prof_begin(Layer& L, int kind) {
  if (!L.profile) return nullptr;
  ProfLaunch& p = L.prof[L.prof_next];
  L.prof_next = (L.prof_next + 1) % kProfRing;
  prof_harvest(L, p);
  if (!p.start && timing_event(&p.start) != hipSuccess) {
    p.start = nullptr;
    (void)hipGetLastError();
    return nullptr;
  }
  if (!p.stop && timing_event(&p.stop) != hipSuccess) {
    p.stop = nullptr;
    (void)hipGetLastError();
    return nullptr;  // the slot keeps its start event and retries the stop next time
  }
  p.kind = kind;
  p.counted = true;
  p.gen = ++L.prof_gen;
  return &p;
}

__global__ void identity_kernel(int32_t* map, int32_t* s2e, int E) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < E) {
    map[e] = e;
    s2e[e] = e;
  }
}

// Copies of `n` loaded (expert, slot) pairs on `st`, or alternating over the
// side streams so one engine's per-copy setup overlaps the other's transfer.
int issue_copies(Layer& L, const int32_t* pairs, int n, double* bytes, hipStream_t st) {
  for (int j = 0; j < n; ++j) {
    const int e = pairs[2 * j], s = pairs[2 * j + 1];
    if (e < 0 || e >= L.d.num_experts || s < 0 || s >= L.d.cap) {
      wisp_set_last_error("decision record holds an out-of-range pair", "page-in");
      return WISP_ERR_INVALID;
    }
    hipStream_t cs = L.nstreams ? L.copy[j % L.nstreams] : st;
    for (int q = 0; q < L.nplanes; ++q) {
      const Plane& p = L.planes[q];
      WISP_HIP_TRY(hipMemcpyAsync(p.d + (size_t)s * p.d_stride, p.host + (size_t)e * p.m_stride,
                                  p.bytes, hipMemcpyHostToDevice, cs));
    }
    *bytes += (double)L.expert_bytes;
  }
  return WISP_OK;
}

// The layer's tensors as page-in planes: w13, w2 and (block-FP8) the two
// scale tensors, merged when one starts where the previous ends in both the
// master and the scratch with equal strides, so a [w13 | w2 | s13 | s2] slab
// per expert moves as one copy.  A single merged plane is padded to 16 bytes
// when both strides leave room, so the copy kernel can move it.
void build_planes(Layer& L) {
  const wisp_layer_desc& d = L.d;
  const size_t wb = L.es;
  Plane raw[kMaxPlanes];
  int n = 0;
  raw[n++] = {(const char*)d.master_w13, nullptr, d.master_w13_stride * wb,
              (char*)d.scratch_w13, d.scratch_w13_stride * wb, d.w13_elems * wb};
  raw[n++] = {(const char*)d.master_w2, nullptr, d.master_w2_stride * wb, (char*)d.scratch_w2,
              d.scratch_w2_stride * wb, d.w2_elems * wb};
  if (L.fp8) {
    raw[n++] = {(const char*)d.master_s13, nullptr, d.master_s13_stride * 4,
                (char*)d.scratch_s13, d.scratch_s13_stride * 4, d.s13_elems * 4};
    raw[n++] = {(const char*)d.master_s2, nullptr, d.master_s2_stride * 4, (char*)d.scratch_s2,
                d.scratch_s2_stride * 4, d.s2_elems * 4};
  }
  L.expert_bytes = 0;
  for (int i = 0; i < n; ++i) L.expert_bytes += raw[i].bytes;
  L.nplanes = 0;
  for (int i = 0; i < n; ++i) {
    Plane* cur = L.nplanes ? &L.planes[L.nplanes - 1] : nullptr;
    if (cur && raw[i].host == cur->host + cur->bytes && raw[i].d == cur->d + cur->bytes &&
        raw[i].m_stride == cur->m_stride && raw[i].d_stride == cur->d_stride)
      cur->bytes += raw[i].bytes;
    else
      L.planes[L.nplanes++] = raw[i];
  }
  if (L.nplanes == 1) {
    Plane& p = L.planes[0];
    const size_t padded = (p.bytes + 15) & ~(size_t)15;
    if (padded <= p.m_stride && padded <= p.d_stride) p.bytes = padded;
  }
}

void harvest_pagein_timing(Layer& L) {
  if (!L.pin_pending) return;
  float ms = 0.f;
  if (hipEventSynchronize(L.ev_pin_end) == hipSuccess &&
      hipEventElapsedTime(&ms, L.ev_pin_start, L.ev_pin_end) == hipSuccess) {
    L.pin_ms_total += ms;
    L.pin_bytes_total += L.pin_bytes_pending;
  }
  L.pin_pending = false;
  L.pin_bytes_pending = 0;
}

void harvest_pin(Layer& L, int i) {
  PinLaunch& p = L.pin[i];
  if (!p.pending) return;
  float ms = 0.f;
  if (hipEventSynchronize(p.stop) == hipSuccess &&
      hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
    const int n = ((volatile int32_t*)L.hist)[i];
    if (n > 0) {
      L.pin_ms_total += ms;
      L.pin_bytes_total += (double)n * (double)L.expert_bytes;
    } else if (p.fused) {
      L.prof_ms[0] += ms;
      L.prof_w13_calls += 1;
      // the call's w2 launch, unless its timing slot was taken since
      float m2 = 0.f;
      if (p.w2 && p.w2->gen == p.w2_gen && p.w2->counted &&
          hipEventSynchronize(p.w2->stop) == hipSuccess &&
          hipEventElapsedTime(&m2, p.w2->start, p.w2->stop) == hipSuccess) {
        L.prof_w2_nl_ms += m2;
        L.prof_w2_nl_calls += 1;
      }
    }
  }
  p.pending = false;
  p.w2 = nullptr;
}

// Orders `st` after the layer's outstanding prefetch copies (before anything
// that reads or writes the scratch).
int wait_prefetch(Layer& L, hipStream_t st) {
  if (!L.pf_pending) return WISP_OK;
  WISP_HIP_TRY(hipStreamWaitEvent(st, L.ev_pf_done, 0));
  L.pf_pending = false;
  return WISP_OK;
}

// The w13 half of a fused page-in + w13 launch (one-token GEMV calls).
struct FusedW13 {
  const void* x;
  int T, K;
  const int32_t* flags;
  void* act;
  const int32_t* slots;
  // with dec: the pager runs in the same launch (Kernel A'')
  const DecodePagerArgs* dec = nullptr;
  int logits_dtype = WISP_F32;
};

// Copy-kernel page-in on `st` of the (expert, slot) pairs at `loads` (device
// memory); their number is *count (device) when count is non-null, else n.
// With `fw`, the same launch also runs the call's w13 stage (Kernel A').
int page_in_kernel(Layer& L, const int32_t* loads, const int32_t* count, int n, hipStream_t st,
                   const FusedW13* fw = nullptr) {
  const wisp_layer_desc& d = L.d;
  const int i = L.pin_next;
  L.pin_next = (L.pin_next + 1) % kPinRing;
  harvest_pin(L, i);
  PinLaunch& p = L.pin[i];
  p.fused = fw != nullptr;
  p.w2 = nullptr;
  PageInArgs a;
  a.loads = loads;
  a.count = count;
  a.n = n;
  a.num_experts = d.num_experts;
  a.cap = d.cap;
  a.nplanes = L.nplanes;
  for (int q = 0; q < L.nplanes; ++q) {
    const Plane& pl = L.planes[q];
    a.p[q] = {pl.dev, pl.m_stride, pl.d, pl.d_stride, pl.bytes};
  }
  a.pk = {L.packed_dev, d.packed_stride, d.hidden, d.inter, (char*)d.scratch_w13,
          d.scratch_w13_stride * L.es, (char*)d.scratch_w2, d.scratch_w2_stride * L.es};
  // The pinned word that tells the timing how many experts a launch copied
  // is written (with a system-scope fence, a host-link round trip inside the
  // kernel) only while timing is on, like the dispatch-timestamp events: each
  // timed launch costs the stream ~4.5 us (measured at the Qwen3 bs=1 decode
  // step).
  a.hist = L.profile ? L.hist_dev + i : nullptr;
  hipEvent_t e0 = L.profile ? p.start : nullptr, e1 = L.profile ? p.stop : nullptr;
  int rc;
  if (fw && fw->dec)
    rc = decode_w13(a, fw->x, d.dtype, fw->logits_dtype, d.hidden, d.inter, fw->K,
                    const_cast<int32_t*>(fw->flags), d.scratch_w13, d.scratch_w13_stride, fw->act,
                    *fw->dec, st, e0, e1);
  else if (fw && L.fp8)
    rc = pagein_fp8_w13(a, fw->x, d.hidden, d.inter, fw->K, fw->slots, fw->flags, d.cap,
                        d.scratch_w13, d.scratch_w13_stride, d.scratch_s13, d.scratch_s13_stride,
                        d.block_n, L.s13_off, fw->act, st, e0, e1, true);
  else if (fw)
    rc = pagein_w13(a, fw->x, d.dtype, fw->T, d.hidden, d.inter, fw->K, fw->flags, d.scratch_w13,
                    d.scratch_w13_stride, fw->act, st, e0, e1);
  else
    rc = launch_pagein(a, st, e0, e1);
  if (rc == WISP_OK && L.profile) p.pending = true;
  return rc;
}

// Whether the fused page-in + w13 launch can serve this layer: a bf16 or
// fp32 layer whose first page-in plane begins with the expert's w13 rows in
// both the master and the scratch; a block-FP8 layer whose one plane is the
// expert's whole slab, with its w13 scales at the same offset in master and
// scratch.
void set_fused_ok(Layer& L) {
  const wisp_layer_desc& d = L.d;
  const Plane& p0 = L.planes[0];
  const size_t w13_bytes = d.w13_elems * L.es;
  L.fused_ok = L.kpin && L.nplanes >= 1 && p0.host == (const char*)d.master_w13 &&
               p0.d == (char*)d.scratch_w13 && p0.bytes >= w13_bytes &&
               p0.m_stride == d.master_w13_stride * L.es &&
               p0.d_stride == d.scratch_w13_stride * L.es;
  L.s13_off = 0;
  if (L.fused_ok && L.fp8) {
    const ptrdiff_t om = (const char*)d.master_s13 - (const char*)d.master_w13;
    const ptrdiff_t od = (const char*)d.scratch_s13 - (const char*)d.scratch_w13;
    L.fused_ok = fp8_fused_supported(d.hidden) && L.nplanes == 1 && om == od &&
                 om >= (ptrdiff_t)w13_bytes && om % 4 == 0 &&
                 (size_t)om + d.s13_elems * 4 <= p0.bytes &&
                 d.master_s13_stride * 4 == p0.m_stride && d.scratch_s13_stride * 4 == p0.d_stride;
    if (L.fused_ok) L.s13_off = (size_t)om;
  }
}

// Enables the copy kernel when every master range is pinned, device-mapped
// host memory and every copy is a whole number of aligned 16-byte units.
void setup_kernel_pagein(Layer& L) {
  const wisp_layer_desc& d = L.d;
  if (d.pagein_engine != WISP_PAGEIN_KERNEL) return;
  const size_t last = (size_t)(d.num_experts - 1);
  const char* dev[kMaxPlanes] = {};
  for (int q = 0; q < L.nplanes; ++q) {
    const Plane& p = L.planes[q];
    if (p.bytes % 16 || p.m_stride % 16 || p.d_stride % 16 || (uintptr_t)p.host % 16 ||
        (uintptr_t)p.d % 16)
      return;
    dev[q] = mapped_host_range(p.host, last * p.m_stride + p.bytes);
    if (!dev[q]) return;
  }
  void* h = nullptr;
  if (hipHostMalloc(&h, kPinRing * sizeof(int32_t), hipHostMallocMapped) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  void* hd = nullptr;
  if (hipHostGetDevicePointer(&hd, h, 0) != hipSuccess || !hd) {
    (void)hipGetLastError();
    (void)hipHostFree(h);
    return;
  }
  for (int i = 0; i < kPinRing; ++i) {
    if (timing_event(&L.pin[i].start) != hipSuccess ||
        timing_event(&L.pin[i].stop) != hipSuccess) {
      (void)hipGetLastError();
      (void)hipHostFree(h);
      return;  // the events made so far are released by wisp_layer_destroy
    }
  }
  memset(h, 0, kPinRing * sizeof(int32_t));
  L.hist = (int32_t*)h;
  L.hist_dev = (int32_t*)hd;
  for (int q = 0; q < L.nplanes; ++q) L.planes[q].dev = dev[q];
  L.kpin = true;
  // a packed copy that is not pinned and mapped leaves the plain masters
  if (d.packed_master)
    L.packed_dev = mapped_host_range(d.packed_master, (size_t)d.num_experts * d.packed_stride);
  set_fused_ok(L);
}

// Page-in of `n` pairs.  On the caller's stream the copies simply follow
// the queued kernels.  On side streams every copy stream first waits on
// `after` (if any), copies run, and `st` waits for all of them; `slot` picks
// the event ring entry.  Copy time and bytes are accumulated only while
// timing is on.
int page_in(Layer& L, const int32_t* pairs, int n, hipEvent_t after, int slot, hipStream_t st) {
  harvest_pagein_timing(L);
  double untimed = 0;
  double* bytes = L.profile ? &L.pin_bytes_pending : &untimed;
  if (L.nstreams == 0) {
    if (L.profile) WISP_HIP_TRY(hipEventRecord(L.ev_pin_start, st));
    int rc = issue_copies(L, pairs, n, bytes, st);
    if (rc != WISP_OK) return rc;
    if (L.profile) {
      WISP_HIP_TRY(hipEventRecord(L.ev_pin_end, st));
      L.pin_pending = true;
    }
    return WISP_OK;
  }
  if (after)
    for (int c = 0; c < L.nstreams; ++c)
      WISP_HIP_TRY(hipStreamWaitEvent(L.copy[c], after, 0));
  WISP_HIP_TRY(hipEventRecord(L.ev_pin_start, L.copy[0]));
  for (int c = 1; c < L.nstreams; ++c)
    WISP_HIP_TRY(hipStreamWaitEvent(L.copy[c], L.ev_pin_start, 0));
  int rc = issue_copies(L, pairs, n, bytes, st);
  if (rc != WISP_OK) return rc;
  for (int c = 1; c < L.nstreams; ++c) {
    WISP_HIP_TRY(hipEventRecord(L.ev_copy[c][slot % kEventRing], L.copy[c]));
    WISP_HIP_TRY(hipStreamWaitEvent(L.copy[0], L.ev_copy[c][slot % kEventRing], 0));
  }
  WISP_HIP_TRY(hipEventRecord(L.ev_pin_end, L.copy[0]));
  L.pin_pending = L.profile;
  WISP_HIP_TRY(hipStreamWaitEvent(st, L.ev_pin_end, 0));
  return WISP_OK;
}

int w13(Layer& L, const void* x, int T, int K, const int32_t* slots, void* act, hipStream_t st,
        const int32_t* filter, int want) {
  const wisp_layer_desc& d = L.d;
  ProfLaunch* p = prof_begin(L, 0);
  // a call's w13 may take two launches (pairs that hit, then loaded pairs);
  // the first of them counts the call
  if (p && !(filter && want == 1)) L.prof_w13_calls += 1;
  int rc = gemv_w13(x, d.dtype, T, d.hidden, d.inter, K, slots, d.cap, d.scratch_w13,
                    d.scratch_w13_stride, act, st, p ? p->start : nullptr,
                    p ? p->stop : nullptr, filter, want);
  if (p && rc == WISP_OK) p->pending = true;
  return rc;
}

int w2(Layer& L, const void* act, int T, int K, const float* w, const int32_t* slots, void* out,
       hipStream_t st, const int32_t* skip_if, ProfLaunch** launched,
       const void* act_spec = nullptr) {
  const wisp_layer_desc& d = L.d;
  if (L.fp8 && skip_if) return WISP_ERR_INVALID;  // no speculative block-FP8 launches
  ProfLaunch* p = prof_begin(L, 1);
  // the slots come from the pager, so a one-token call with K == cap fills
  // every slot and the w2 kernel may run one wave per slot
  int rc = L.fp8 ? experts_fp8_w2(act, T, d.hidden, d.inter, K, w, slots, d.cap, d.scratch_w2,
                                  d.scratch_w2_stride, d.scratch_s2, d.scratch_s2_stride,
                                  d.block_n, out, st, p ? p->start : nullptr,
                                  p ? p->stop : nullptr, true)
                 : gemv_w2(act, d.dtype, T, d.hidden, d.inter, K, w, slots, d.cap, d.scratch_w2,
                           d.scratch_w2_stride, out, st, p ? p->start : nullptr,
                           p ? p->stop : nullptr, skip_if, d.cap, act_spec);
  if (p && rc == WISP_OK) p->pending = true;
  if (launched) *launched = p;
  return rc;
}

// Both expert stages for T tokens (any algorithm, no filters).
int experts(Layer& L, const void* x, int T, int K, const float* w, const int32_t* slots,
            void* act, void* out, int algo, const wisp_workspace* ws, hipStream_t st) {
  const wisp_layer_desc& d = L.d;
  if (L.fp8) {
    ProfLaunch* p13 = prof_begin(L, 0);
    ProfLaunch* p2 = prof_begin(L, 1);
    if (p13 && p2) L.prof_w13_calls += 1;
    StageEvents ev = {{p13 ? p13->start : nullptr, p13 ? p13->stop : nullptr,
                       p2 ? p2->start : nullptr, p2 ? p2->stop : nullptr}};
    const StageEvents* pe = (p13 && p2) ? &ev : nullptr;
    int rc = algo == WISP_ALGO_MFMA
                 ? experts_fp8_grouped(x, T, d.hidden, d.inter, K, w, slots, d.cap,
                                       d.scratch_w13, d.scratch_w13_stride, d.scratch_s13,
                                       d.scratch_s13_stride, d.scratch_w2, d.scratch_w2_stride,
                                       d.scratch_s2, d.scratch_s2_stride, d.block_n, act, out,
                                       ws->work, ws->work_bytes, st, pe)
                 : experts_fp8(x, T, d.hidden, d.inter, K, w, slots, d.cap, d.scratch_w13,
                               d.scratch_w13_stride, d.scratch_s13, d.scratch_s13_stride,
                               d.scratch_w2, d.scratch_w2_stride, d.scratch_s2,
                               d.scratch_s2_stride, d.block_n, act, out, st, pe, true);
    if (rc == WISP_OK && p13 && p2) p13->pending = p2->pending = true;
    return rc;
  }
  if (algo == WISP_ALGO_MFMA) {
    ProfLaunch* p13 = prof_begin(L, 0);
    ProfLaunch* p2 = prof_begin(L, 1);
    if (p13 && p2) L.prof_w13_calls += 1;
    StageEvents ev = {{p13 ? p13->start : nullptr, p13 ? p13->stop : nullptr,
                       p2 ? p2->start : nullptr, p2 ? p2->stop : nullptr}};
    int rc = experts_mfma(x, T, d.hidden, d.inter, K, w, slots, d.cap, d.scratch_w13,
                          d.scratch_w13_stride, d.scratch_w2, d.scratch_w2_stride, act, out,
                          ws->work, ws->work_bytes, st, (p13 && p2) ? &ev : nullptr);
    if (rc == WISP_OK && p13 && p2) p13->pending = p2->pending = true;
    return rc;
  }
  int rc = w13(L, x, T, K, slots, act, st, nullptr, 0);
  if (rc != WISP_OK) return rc;
  return w2(L, act, T, K, w, slots, out, st, nullptr, nullptr);
}

// The expert algorithm of a layer call (-1: the request does not cover it).
// Decided before the pager runs, so a call the kernels cannot compute fails
// without touching the pager state.
int choose_algo(const Layer& L, int algo, int T, int K) {
  const wisp_layer_desc& d = L.d;
  if (algo == WISP_ALGO_AUTO) return auto_algo(d.dtype, d.hidden, d.inter, T, K);
  if (algo == WISP_ALGO_MFMA && d.dtype == WISP_F32) return -1;
  if (algo == WISP_ALGO_MFMA && d.dtype == WISP_BF16 && !mfma_supported(d.hidden, d.inter))
    return -1;
  if (algo == WISP_ALGO_GEMV && d.dtype != WISP_FP8_E4M3 && !gemv_supported(d.dtype, d.hidden, K))
    return -1;
  if (algo != WISP_ALGO_GEMV && algo != WISP_ALGO_MFMA) return -1;
  return algo;
}

// Copies and expert kernels for groups [0, ngroups) of a decision record.
// Every group's copies are issued even after a failed expert launch, so the
// map the pager already wrote never points at a slot that was not filled.
int run_groups(Layer& L, const int32_t* rec, const int32_t* loads, int T, int K, int ngroups,
               bool compute, const void* x, const float* topk_w, const int32_t* slots, void* act,
               void* out, int algo, const wisp_workspace* ws, hipStream_t st) {
  const RecordLayout RL(T, K);
  const size_t row = (size_t)L.d.hidden * act_size(L.d.dtype);
  int last_gemm = -1;
  int failed = WISP_OK;
  for (int g = 0; g < ngroups; ++g) {
    const int32_t* G = rec + RL.group_base(g);
    const int t0 = G[0], t1 = G[1], ld_off = G[6], n_ld = G[7];
    if (n_ld > 0) {
      int rc = L.kpin ? page_in_kernel(L, loads + 2 * ld_off, nullptr, n_ld, st)
                      : page_in(L, rec + RL.loaded_base() + 2 * ld_off, n_ld,
                                last_gemm >= 0 ? L.ev_gemm[last_gemm % kEventRing] : nullptr, g,
                                st);
      if (rc != WISP_OK) return rc;
    }
    if (compute && failed == WISP_OK && t1 > t0) {
      failed = experts(L, (const char*)x + (size_t)t0 * row, t1 - t0, K,
                       topk_w + (size_t)t0 * K, slots + (size_t)t0 * K, act,
                       (char*)out + (size_t)t0 * row, algo, ws, st);
      if (failed != WISP_OK) continue;
      WISP_HIP_TRY(hipEventRecord(L.ev_gemm[g % kEventRing], st));
      last_gemm = g;
    }
  }
  return failed;
}

// Whether the workspace's work buffer holds what algorithm `a` needs for a
// call of T tokens (checked before the pager runs).
bool work_ok(const Layer& L, int a, int T, int K, const wisp_workspace* ws) {
  const wisp_layer_desc& d = L.d;
  size_t need = 0;
  if (a == WISP_ALGO_MFMA && d.dtype == WISP_BF16)
    need = mfma_work_bytes(T, K, d.hidden, d.cap);
  else if (a == WISP_ALGO_MFMA && d.dtype == WISP_FP8_E4M3)
    need = fp8_work_bytes(T, K, d.hidden, d.inter, d.cap);
  if (need == 0 || T == 0) return true;
  return ws->work && ws->work_bytes >= need && ((uintptr_t)ws->work) % 256 == 0;
}

// Device view of the (pinned host) decision record; device memory passes
// through unchanged.
int32_t* record_device_ptr(int32_t* rec) {
  void* dev = nullptr;
  if (hipHostGetDevicePointer(&dev, rec, 0) == hipSuccess && dev) return (int32_t*)dev;
  (void)hipGetLastError();
  return rec;
}

// A workspace laid out as this library's (its trailing struct_bytes).
bool ws_layout_ok(const wisp_workspace* ws, const char* where) {
  if (ws && ws->struct_bytes == sizeof(wisp_workspace)) return true;
  wisp_set_last_error("wisp_workspace.struct_bytes is not sizeof(wisp_workspace) of this "
                      "library's header", where);
  return false;
}

int check_ws(const wisp_workspace* ws, int T, int K) {
  if (!ws_layout_ok(ws, "wisp_layer_forward")) return WISP_ERR_INVALID;
  if (!ws || (int64_t)T * K > ws->max_pairs || !ws->topk_w || !ws->topk_ids || !ws->slots ||
      !ws->flags || !ws->loads || !ws->act || !ws->record ||
      ws->record_words < RecordLayout(T, K).words()) {
    wisp_set_last_error("workspace too small or missing", "wisp_layer_forward");
    return WISP_ERR_INVALID;
  }
  return WISP_OK;
}

}  // namespace
}  // namespace wisp

using wisp::Layer;

namespace wisp {
// The fused decode launch's buffers for a scratch of `cap` slots: act_spec
// [cap][inter] and the epoch word (zero, an epoch no launch uses).  Called at
// creation and on a resize to more slots, both points where no kernel of the
// layer is in flight.
static int alloc_decode(Layer& L, int cap) {
  const wisp_layer_desc& d = L.d;
  if (L.fp8 || d.hidden < 1 || d.mode != WISP_MODE_PAGED || cap <= L.spec_cap) return WISP_OK;
  if (L.act_spec) WISP_HIP_TRY(hipFree(L.act_spec));
  L.act_spec = nullptr;
  L.spec_cap = 0;
  WISP_HIP_TRY(hipMalloc(&L.act_spec, (size_t)cap * d.inter * act_size(d.dtype)));
  L.spec_cap = cap;
  if (!L.decode_sync) {
    WISP_HIP_TRY(hipMalloc((void**)&L.decode_sync, 256));
    WISP_HIP_TRY(hipMemset(L.decode_sync, 0, 256));
    L.decode_epoch = 0;
  }
  return WISP_OK;
}

// Block-FP8 fields of a descriptor: scale shapes consistent with the MLP
// shape and the block, scale buffers present.
static bool fp8_desc_ok(const wisp_layer_desc& d) {
  if (d.block_n < 1 || d.block_k < 1 || !d.scratch_s13 || !d.scratch_s2 || !d.master_s13 ||
      !d.master_s2 || d.s13_elems < 1 || d.s2_elems < 1 ||
      d.scratch_s13_stride < d.s13_elems || d.scratch_s2_stride < d.s2_elems ||
      d.master_s13_stride < d.s13_elems || d.master_s2_stride < d.s2_elems)
    return false;
  if (d.hidden == 0) return true;
  const size_t H = d.hidden, I = d.inter, bn = d.block_n, bk = d.block_k;
  return d.s13_elems == 2 * ((I + bn - 1) / bn) * ((H + bk - 1) / bk) &&
         d.s2_elems == ((H + bn - 1) / bn) * ((I + bk - 1) / bk);
}
}  // namespace wisp

extern "C" int wisp_layer_create(const wisp_layer_desc* desc, void** handle) {
  using namespace wisp;
  if (!desc || !handle) return WISP_ERR_INVALID;
  if (desc->struct_bytes != sizeof(wisp_layer_desc)) {
    wisp_set_last_error("wisp_layer_desc.struct_bytes is not sizeof(wisp_layer_desc) of this "
                        "library's header", "wisp_layer_create");
    return WISP_ERR_INVALID;
  }
  const wisp_layer_desc& d = *desc;
  if (d.num_experts < 1 || d.num_experts > kMaxExperts || d.cap < 1 || d.cap > kMaxExperts ||
      d.hidden < 0 || d.inter < 0 || d.w13_elems < 1 || d.w2_elems < 1 ||
      (d.hidden > 0 && (d.w13_elems != (size_t)2 * d.inter * d.hidden ||
                        d.w2_elems != (size_t)d.hidden * d.inter)) ||
      (d.dtype != WISP_F32 && d.dtype != WISP_BF16 && d.dtype != WISP_FP8_E4M3) ||
      (d.dtype == WISP_FP8_E4M3 && !fp8_desc_ok(d)) ||
      (d.mode != WISP_MODE_PAGED && d.mode != WISP_MODE_RESIDENT) || !d.scratch_w13 ||
      !d.scratch_w2 || !d.master_w13 || !d.master_w2 || !d.expert_map || !d.slot_to_expert ||
      !d.lru_tick || !d.counters || d.scratch_w13_stride < d.w13_elems ||
      d.scratch_w2_stride < d.w2_elems || d.master_w13_stride < d.w13_elems ||
      d.master_w2_stride < d.w2_elems ||
      (d.mode == WISP_MODE_RESIDENT && d.cap != d.num_experts) || d.pagein_streams < 0 ||
      d.pagein_streams > kCopyStreams ||
      (d.pagein_engine != WISP_PAGEIN_MEMCPY && d.pagein_engine != WISP_PAGEIN_KERNEL)) {
    wisp_set_last_error("invalid layer descriptor", "wisp_layer_create");
    return WISP_ERR_INVALID;
  }
  if (d.packed_master &&
      (d.dtype != WISP_BF16 || d.hidden < 64 || d.inter < 64 || d.hidden % 64 ||
       d.inter % 64 || d.packed_stride % 256 ||
       d.packed_stride < packed::Layout(d.hidden, d.inter).exc_off ||
       ((uintptr_t)d.packed_master) % 16)) {
    wisp_set_last_error("packed masters need a bf16 layer with hidden and inter multiples of 64 "
                        "and the stride wisp_pack_bf16_stride gives", "wisp_layer_create");
    return WISP_ERR_INVALID;
  }
  Layer* L = new Layer();
  L->d = d;
  L->fp8 = d.dtype == WISP_FP8_E4M3;
  L->es = elem_size(d.dtype);
  L->nstreams = d.pagein_streams;
  build_planes(*L);
  hipError_t e = hipEventCreateWithFlags(&L->ev_decided, hipEventDisableTiming);
  for (int c = 0; c < kCopyStreams && e == hipSuccess; ++c) {
    e = hipStreamCreateWithFlags(&L->copy[c], hipStreamNonBlocking);
    for (int i = 0; i < kEventRing && e == hipSuccess; ++i)
      e = hipEventCreateWithFlags(&L->ev_copy[c][i], hipEventDisableTiming);
  }
  for (int i = 0; i < kEventRing && e == hipSuccess; ++i)
    e = hipEventCreateWithFlags(&L->ev_gemm[i], hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&L->ev_pf_decided, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&L->ev_pf_done, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreate(&L->ev_pin_start);
  if (e == hipSuccess) e = hipEventCreate(&L->ev_pin_end);
  if (e != hipSuccess) {
    wisp_set_last_error(hipGetErrorString(e), "wisp_layer_create");
    wisp_layer_destroy(L);
    return WISP_ERR_HIP;
  }
  if (d.hidden > 0) setup_kernel_pagein(*L);
  if (alloc_decode(*L, d.cap) != WISP_OK) {
    wisp_layer_destroy(L);
    return WISP_ERR_HIP;
  }
  *handle = L;
  return WISP_OK;
}

extern "C" int wisp_layer_destroy(void* handle) {
  using namespace wisp;
  Layer* L = (Layer*)handle;
  if (!L) return WISP_OK;
  for (int c = 0; c < kCopyStreams; ++c)
    if (L->copy[c]) (void)hipStreamSynchronize(L->copy[c]);
  for (int i = 0; i < kEventRing; ++i) {
    for (int c = 0; c < kCopyStreams; ++c)
      if (L->ev_copy[c][i]) (void)hipEventDestroy(L->ev_copy[c][i]);
    if (L->ev_gemm[i]) (void)hipEventDestroy(L->ev_gemm[i]);
  }
  if (L->ev_decided) (void)hipEventDestroy(L->ev_decided);
  if (L->ev_pf_decided) (void)hipEventDestroy(L->ev_pf_decided);
  if (L->ev_pf_done) (void)hipEventDestroy(L->ev_pf_done);
  if (L->ev_pin_start) (void)hipEventDestroy(L->ev_pin_start);
  if (L->ev_pin_end) (void)hipEventDestroy(L->ev_pin_end);
  for (int i = 0; i < kProfRing; ++i) {
    if (L->prof[i].start) (void)hipEventDestroy(L->prof[i].start);
    if (L->prof[i].stop) (void)hipEventDestroy(L->prof[i].stop);
  }
  for (int i = 0; i < kPinRing; ++i) {
    if (L->pin[i].pending) (void)hipEventSynchronize(L->pin[i].stop);
    if (L->pin[i].start) (void)hipEventDestroy(L->pin[i].start);
    if (L->pin[i].stop) (void)hipEventDestroy(L->pin[i].stop);
  }
  if (L->hist) (void)hipHostFree(L->hist);
  if (L->act_spec) (void)hipFree(L->act_spec);
  if (L->decode_sync) (void)hipFree(L->decode_sync);
  for (int c = 0; c < kCopyStreams; ++c)
    if (L->copy[c]) (void)hipStreamDestroy(L->copy[c]);
  delete L;
  return WISP_OK;
}

extern "C" int wisp_layer_set_scratch(void* handle, void* scratch_w13, void* scratch_w2, int cap,
                                      int32_t* slot_to_expert, int64_t* lru_tick) {
  using namespace wisp;
  Layer* L = (Layer*)handle;
  if (!L || !scratch_w13 || !scratch_w2 || cap < 1 || cap > kMaxExperts ||
      !slot_to_expert || !lru_tick)
    return WISP_ERR_INVALID;
  if (L->fp8) {
    wisp_set_last_error("block-FP8 layers are not resized", "wisp_layer_set_scratch");
    return WISP_ERR_UNSUPPORTED;
  }
  for (int c = 0; c < kCopyStreams; ++c) (void)hipStreamSynchronize(L->copy[c]);
  harvest_pagein_timing(*L);
  for (int i = 0; i < kPinRing; ++i) harvest_pin(*L, i);
  L->d.scratch_w13 = scratch_w13;
  L->d.scratch_w2 = scratch_w2;
  // the masters (and their device mappings) are unchanged; only the scratch
  // side of each plane moves
  const char* dev[kMaxPlanes];
  for (int q = 0; q < L->nplanes; ++q) dev[q] = L->planes[q].dev;
  const int old_n = L->nplanes;
  build_planes(*L);
  if (L->nplanes != old_n) {
    L->kpin = false;
  } else {
    for (int q = 0; q < L->nplanes; ++q) {
      L->planes[q].dev = dev[q];
      if (((uintptr_t)L->planes[q].d) % 16 || L->planes[q].d_stride % 16) L->kpin = false;
    }
  }
  L->d.cap = cap;
  L->d.slot_to_expert = slot_to_expert;
  L->d.lru_tick = lru_tick;
  set_fused_ok(*L);
  if (alloc_decode(*L, cap) != WISP_OK) return WISP_ERR_HIP;
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
  const size_t es = L->es, as = act_size(d.dtype);
  if (d.hidden < 1 || d.inter < 1 || (d.hidden * es) % 16 || (d.inter * es) % 16 ||
      (d.hidden * as) % 16 || (d.inter * as) % 16 ||
      (d.scratch_w13_stride * es) % 16 || (d.scratch_w2_stride * es) % 16 ||
      ((uintptr_t)d.scratch_w13) % 16 || ((uintptr_t)d.scratch_w2) % 16 ||
      (T > 0 && (((uintptr_t)x) % 16 || ((uintptr_t)out) % 16))) {
    wisp_set_last_error("expert shape/alignment outside the kernels' coverage (H and I must "
                        "be multiples of 16 bytes, buffers 16-byte aligned)",
                        "wisp_layer_forward");
    return WISP_ERR_UNSUPPORTED;
  }
  if (L->fp8) {
    const char* why = fp8_unsupported(d.hidden, d.inter, K, d.block_n, d.block_k);
    if (!why && (((uintptr_t)d.scratch_s13) % 16 || ((uintptr_t)d.scratch_s2) % 16))
      why = "scale scratch must be 16-byte aligned";
    if (why) {
      wisp_set_last_error(why, "wisp_layer_forward");
      return WISP_ERR_UNSUPPORTED;
    }
  }
  const int a = choose_algo(*L, algo, T, K);
  if (a < 0) {
    wisp_set_last_error("no expert kernel covers this call (shape, top_k or requested "
                        "algorithm)", "wisp_layer_forward");
    return WISP_ERR_UNSUPPORTED;
  }
  if (!work_ok(*L, a, T, K, ws)) {
    wisp_set_last_error("work buffer missing, misaligned or too small for the grouped path",
                        "wisp_layer_forward");
    return WISP_ERR_INVALID;
  }
  if (L->profile) L->prof_calls += 1;

  L->rec_on_device = false;
  if (d.mode == WISP_MODE_RESIDENT) {
    rc = wisp_route_topk_softmax(logits, logits_dtype, T, d.num_experts, K, renormalize,
                                 ws->topk_w, ws->topk_ids, d.counters + kForward, stream);
    if (rc != WISP_OK) return rc;
    return experts(*L, x, T, K, ws->topk_w, ws->topk_ids, ws->act, out, a, ws, st);
  }

  const bool fuse_route = T <= kFusedRouteTokens;
  if (!fuse_route) {
    rc = wisp_route_topk_softmax(logits, logits_dtype, T, d.num_experts, K, renormalize,
                                 ws->topk_w, ws->topk_ids, nullptr, stream);
    if (rc != WISP_OK) return rc;
  }
  // One group is certain when every routed pair could be distinct and still
  // fit (the ids come from the router, so they are in range and the pager
  // cannot fail): then the rest of the call goes in right behind the pager.
  // On the copy-kernel engine such a call never reads its decision record on
  // the host, so the pager writes it to device memory (stores to pinned host
  // memory would hold the kernel's end for a host-link round trip);
  // wisp_layer_sync_record brings it to the pinned record on demand.
  // Every other call mirrors the record to the pinned one at the pager's end.
  const bool one_group = T > 0 && (int64_t)T * K <= d.cap;
  const bool rec_dev_only = one_group && L->kpin && ws->record_dev;
  int32_t* rec_dev = ws->record_dev ? ws->record_dev : record_device_ptr(ws->record);
  int32_t* rec_host = ws->record_dev && !rec_dev_only ? record_device_ptr(ws->record) : nullptr;
  L->rec_on_device = rec_dev_only;
  if (L->decode_fused && T == 1 && fuse_route && rec_dev_only && a == WISP_ALGO_GEMV &&
      L->fused_ok && !L->fp8 && L->act_spec && L->spec_cap >= d.cap &&
      (logits_dtype == WISP_F32 || logits_dtype == WISP_BF16) &&
      decode_w13_supported(d.dtype, d.hidden, d.num_experts, K, d.cap)) {
    // [route + pager + page-in + w13 per slot] [w2]: the launch's w13
    // blocks need nothing from the pager (the call fills every slot), so the
    // routing and the decisions run under their weight stream
    rc = wait_prefetch(*L, st);
    if (rc != WISP_OK) return rc;
    if (++L->decode_epoch == 0) L->decode_epoch = 1;  // 0 is the word's initial value
    const DecodePagerArgs pa{logits, renormalize, d.num_experts, ws->topk_w, ws->topk_ids,
                             d.expert_map, d.slot_to_expert, d.lru_tick, d.counters, ws->slots,
                             ws->loads, rec_dev, L->decode_sync, L->decode_epoch, L->act_spec};
    FusedW13 fw{x, T, K, ws->flags, ws->act, ws->slots};
    fw.dec = &pa;
    fw.logits_dtype = logits_dtype;
    const int pin_slot = L->pin_next;
    rc = page_in_kernel(*L, ws->loads, ws->flags, 0, st, &fw);
    if (rc != WISP_OK) return rc;
    ProfLaunch* p2 = nullptr;
    rc = w2(*L, ws->act, T, K, ws->topk_w, ws->flags + 1, out, st, nullptr, &p2, L->act_spec);
    if (rc == WISP_OK && p2) {
      L->pin[pin_slot].w2 = p2;
      L->pin[pin_slot].w2_gen = p2->gen;
    }
    return rc;
  }
  rc = launch_pager(ws->topk_ids, fuse_route ? logits : nullptr, logits_dtype, renormalize,
                    ws->topk_w, ws->topk_ids, T, K, d.num_experts, d.cap, 0, d.expert_map,
                    d.slot_to_expert, d.lru_tick, d.counters, ws->slots, ws->flags, ws->loads,
                    rec_dev, ws->record_words, st, rec_host);
  if (rc != WISP_OK) return rc;

  rc = wait_prefetch(*L, st);
  if (rc != WISP_OK) return rc;
  if (T == 1 && one_group && L->kpin && a == WISP_ALGO_GEMV && L->fused_ok) {
    // [route+pager] [page-in + w13] [w2]
    const FusedW13 fw{x, T, K, ws->flags, ws->act, ws->slots};
    const int pin_slot = L->pin_next;
    rc = page_in_kernel(*L, ws->loads, ws->flags, 0, st, &fw);
    if (rc != WISP_OK) return rc;
    ProfLaunch* p2 = nullptr;
    rc = w2(*L, ws->act, T, K, ws->topk_w, ws->slots, out, st, nullptr, &p2);
    if (rc == WISP_OK && p2) {
      L->pin[pin_slot].w2 = p2;
      L->pin[pin_slot].w2_gen = p2->gen;
    }
    return rc;
  }
  if (one_group && L->kpin) {
    rc = page_in_kernel(*L, ws->loads, ws->flags, 0, st);
    if (rc != WISP_OK) return rc;
    return experts(*L, x, T, K, ws->topk_w, ws->slots, ws->act, out, a, ws, st);
  }
  WISP_HIP_TRY(hipEventRecord(L->ev_decided, st));

  const bool speculate = a == WISP_ALGO_GEMV && one_group && !L->fp8;
  ProfLaunch* spec_w2 = nullptr;
  int spec_rc = WISP_OK;
  if (speculate) {
    // a failed launch here still lets the copies below run (the map already
    // names the slots they fill); its error is returned after them
    spec_rc = w13(*L, x, T, K, ws->slots, ws->act, st, ws->flags + 1, 0);
    if (spec_rc == WISP_OK)
      spec_rc = w2(*L, ws->act, T, K, ws->topk_w, ws->slots, out, st, ws->flags, &spec_w2);
  }

  WISP_HIP_TRY(hipEventSynchronize(L->ev_decided));
  const int32_t* rec = ws->record;
  const int status = rec[kRecStatus];
  if (status == WISP_ERR_INVALID) {
    wisp_set_last_error("routed expert id out of range", "wisp_layer_forward");
    return status;
  }
  if (speculate) {
    if (status != WISP_OK) return status;
    const RecordLayout RL(T, K);
    const int32_t* G = rec + RL.group_base(0);
    const int n_ld = rec[kRecGroupsDone] > 0 ? G[7] : 0;
    if (n_ld == 0) return spec_rc;  // the queued kernels computed everything
    if (spec_w2) spec_w2->counted = false;  // it found loads and exited
    rc = page_in(*L, rec + RL.loaded_base() + 2 * G[6], n_ld, nullptr, 0, st);
    if (rc != WISP_OK || spec_rc != WISP_OK) return rc != WISP_OK ? rc : spec_rc;
    rc = w13(*L, x, T, K, ws->slots, ws->act, st, ws->flags + 1, 1);
    if (rc == WISP_OK) rc = w2(*L, ws->act, T, K, ws->topk_w, ws->slots, out, st, nullptr, nullptr);
    return rc;
  }
  rc = run_groups(*L, rec, ws->loads, T, K, rec[kRecGroupsDone], status == WISP_OK, x,
                  ws->topk_w, ws->slots, ws->act, out, a, ws, st);
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
  if (!ws_layout_ok(ws, "wisp_layer_ensure_resident")) return WISP_ERR_INVALID;
  if (!L || n < 0 || (n > 0 && !ids) || !ws || !ws->record ||
      ws->record_words < RecordLayout(n, 1).words())
    return WISP_ERR_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const wisp_layer_desc& d = L->d;
  L->rec_on_device = false;
  int32_t* rec_dev = ws->record_dev ? ws->record_dev : record_device_ptr(ws->record);
  int32_t* rec_host = ws->record_dev ? record_device_ptr(ws->record) : nullptr;
  int rc = launch_pager(ids, nullptr, WISP_F32, 0, nullptr, nullptr, n, 1, d.num_experts, d.cap,
                        1, d.expert_map, d.slot_to_expert, d.lru_tick, d.counters, nullptr,
                        nullptr, nullptr, rec_dev, ws->record_words, st, rec_host);
  if (rc != WISP_OK) return rc;
  WISP_HIP_TRY(hipEventRecord(L->ev_decided, st));
  WISP_HIP_TRY(hipEventSynchronize(L->ev_decided));
  const int32_t* rec = ws->record;
  const int status = rec[kRecStatus];
  if (status == WISP_ERR_INVALID) return status;
  // ensure_resident is a single call: one group, planned over n tokens x 1.
  const RecordLayout RL(n, 1);
  const int32_t* G = rec + RL.group_base(0);
  rc = wait_prefetch(*L, st);
  if (rc != WISP_OK) return rc;
  if (rec[kRecGroupsDone] > 0 && G[7] > 0) {
    rc = page_in(*L, rec + RL.loaded_base() + 2 * G[6], G[7], nullptr, 0, st);
    if (rc != WISP_OK) return rc;
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
  int rc = wait_prefetch(*L, st);
  if (rc != WISP_OK) return rc;
  rc = page_in(*L, pairs.data(), d.num_experts, nullptr, 0, st);
  if (rc != WISP_OK) return rc;
  hipLaunchKernelGGL(identity_kernel, dim3((d.num_experts + 255) / 256), dim3(256), 0, st,
                     d.expert_map, d.slot_to_expert, d.num_experts);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

extern "C" int wisp_layer_last_pagein(void* handle, float* ms, double* bytes) {
  Layer* L = (Layer*)handle;
  if (!L) return WISP_ERR_INVALID;
  wisp::harvest_pagein_timing(*L);
  for (int i = 0; i < wisp::kPinRing; ++i) wisp::harvest_pin(*L, i);
  if (ms) *ms = (float)L->pin_ms_total;
  if (bytes) *bytes = L->pin_bytes_total;
  L->pin_ms_total = 0;
  L->pin_bytes_total = 0;
  return WISP_OK;
}

extern "C" int wisp_layer_prefetch(void* handle, const int32_t* predicted,
                                   const int32_t* n_predicted, int n, int ordered,
                                   int count_pred, const int32_t* last_ids, int n_last,
                                   int32_t* record, int record_words, wisp_stream_t stream) {
  using namespace wisp;
  Layer* L = (Layer*)handle;
  if (!L || n < 0 || n > kMaxExperts || (n > 0 && !predicted) || n_last < 0 ||
      (n_last > 0 && !last_ids) || !record || record_words < prefetch_record_words(n))
    return WISP_ERR_INVALID;
  const wisp_layer_desc& d = L->d;
  if (d.mode == WISP_MODE_RESIDENT || d.hidden < 1) return WISP_OK;  // nothing to page
  hipStream_t st = (hipStream_t)stream;
  // The previous prefetch's copies (side stream) still read their count and
  // load list from the caller's record, which this call's decisions rewrite:
  // order the decisions after those copies.
  int rc = wait_prefetch(*L, st);
  if (rc != WISP_OK) return rc;
  rc = launch_prefetch(predicted, n_predicted, n, ordered, count_pred, last_ids, n_last,
                           d.num_experts, d.cap, n, d.expert_map, d.slot_to_expert, d.lru_tick,
                           d.counters, record, st);
  if (rc != WISP_OK) return rc;
  int32_t* loads = record + 4 + 2 * n;
  WISP_HIP_TRY(hipEventRecord(L->ev_pf_decided, st));
  hipStream_t side = L->copy[0];
  WISP_HIP_TRY(hipStreamWaitEvent(side, L->ev_pf_decided, 0));
  if (L->kpin) {
    rc = page_in_kernel(*L, loads, record + 1, 0, side);
    if (rc != WISP_OK) return rc;
  } else {
    // hipMemcpyAsync needs the decisions on the host
    std::vector<int32_t> h(4 + 4 * (size_t)n);
    WISP_HIP_TRY(hipEventSynchronize(L->ev_pf_decided));
    WISP_HIP_TRY(hipMemcpy(h.data(), record, h.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
    double bytes = 0;
    rc = issue_copies(*L, h.data() + 4 + 2 * n, h[1], &bytes, side);
    if (rc != WISP_OK) return rc;
  }
  WISP_HIP_TRY(hipEventRecord(L->ev_pf_done, side));
  L->pf_pending = true;
  return WISP_OK;
}

extern "C" int wisp_layer_sync_record(void* handle, const wisp_workspace* ws) {
  using namespace wisp;
  Layer* L = (Layer*)handle;
  if (!ws_layout_ok(ws, "wisp_layer_sync_record")) return WISP_ERR_INVALID;
  if (!L || !ws || !ws->record || ws->record_words < 8) return WISP_ERR_INVALID;
  WISP_HIP_TRY(hipDeviceSynchronize());
  if (L->rec_on_device) {
    if (!ws->record_dev) return WISP_ERR_INVALID;
    WISP_HIP_TRY(hipMemcpy(ws->record, ws->record_dev, (size_t)ws->record_words * sizeof(int32_t),
                           hipMemcpyDeviceToHost));
  }
  return WISP_OK;
}

extern "C" int wisp_layer_set_decode_fused(void* handle, int enable) {
  Layer* L = (Layer*)handle;
  if (!L) return WISP_ERR_INVALID;
  L->decode_fused = enable != 0;
  return WISP_OK;
}

extern "C" int wisp_layer_pagein_engine(void* handle) {
  Layer* L = (Layer*)handle;
  if (!L) return -1;
  return L->kpin ? WISP_PAGEIN_KERNEL : WISP_PAGEIN_MEMCPY;
}

extern "C" int wisp_layer_profile(void* handle, int enable, double* w13_ms, double* w2_ms,
                                  int64_t* calls, int64_t* w13_calls) {
  Layer* L = (Layer*)handle;
  if (!L) return WISP_ERR_INVALID;
  for (int i = 0; i < wisp::kProfRing; ++i) wisp::prof_harvest(*L, L->prof[i]);
  for (int i = 0; i < wisp::kPinRing; ++i) wisp::harvest_pin(*L, i);
  if (w13_ms) *w13_ms = L->prof_ms[0];
  if (w2_ms) *w2_ms = L->prof_ms[1];
  if (calls) *calls = L->prof_calls;
  if (w13_calls) *w13_calls = L->prof_w13_calls;
  L->prof_ms[0] = L->prof_ms[1] = 0;
  L->prof_calls = 0;
  L->prof_w13_calls = 0;
  L->prof_w2_nl_ms = 0;
  L->prof_w2_nl_calls = 0;
  L->profile = enable != 0;
  return WISP_OK;
}

extern "C" int wisp_layer_profile_noload(void* handle, double* w2_ms, int64_t* calls) {
  Layer* L = (Layer*)handle;
  if (!L) return WISP_ERR_INVALID;
  for (int i = 0; i < wisp::kPinRing; ++i) wisp::harvest_pin(*L, i);
  if (w2_ms) *w2_ms = L->prof_w2_nl_ms;
  if (calls) *calls = L->prof_w2_nl_calls;
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
                                const float* topk_w, const int32_t* slots, int nslots,
                                const void* w13, size_t w13_stride, const void* w2,
                                size_t w2_stride, void* act, void* out, void* work,
                                size_t work_bytes, int algo, wisp_stream_t stream) {
  using namespace wisp;
  if (T < 0 || H < 1 || I < 1 || K < 1 || nslots < 1 ||
      (dtype != WISP_F32 && dtype != WISP_BF16) ||
      (T > 0 && (!x || !topk_w || !slots || !w13 || !w2 || !act || !out)))
    return WISP_ERR_INVALID;
  const size_t es = elem_size(dtype);
  if ((H * es) % 16 || (I * es) % 16 || (w13_stride * es) % 16 || (w2_stride * es) % 16 ||
      ((uintptr_t)w13) % 16 || ((uintptr_t)w2) % 16 ||
      (T > 0 && (((uintptr_t)x) % 16 || ((uintptr_t)act) % 16 || ((uintptr_t)out) % 16))) {
    wisp_set_last_error("H, I and buffers must be 16-byte aligned", "wisp_moe_experts");
    return WISP_ERR_UNSUPPORTED;
  }
  const int a = algo == WISP_ALGO_AUTO ? auto_algo(dtype, H, I, T, K) : algo;
  if (a < 0 || (a == WISP_ALGO_GEMV && !gemv_supported(dtype, H, K))) {
    wisp_set_last_error("no expert kernel covers this shape and top_k", "wisp_moe_experts");
    return WISP_ERR_UNSUPPORTED;
  }
  if (a == WISP_ALGO_MFMA) {
    if (dtype != WISP_BF16) {
      wisp_set_last_error("the MFMA path computes in bf16 only", "wisp_moe_experts");
      return WISP_ERR_UNSUPPORTED;
    }
    return experts_mfma(x, T, H, I, K, topk_w, slots, nslots, w13, w13_stride, w2, w2_stride,
                        act, out, work, work_bytes, (hipStream_t)stream, nullptr);
  }
  if (a != WISP_ALGO_GEMV) return WISP_ERR_INVALID;
  return experts_gemv(x, dtype, T, H, I, K, topk_w, slots, nslots, w13, w13_stride, w2,
                      w2_stride, act, out, (hipStream_t)stream, nullptr);
}

extern "C" size_t wisp_moe_work_bytes(int T, int K, int H, int nslots) {
  return wisp::mfma_work_bytes(T, K, H, nslots);
}
