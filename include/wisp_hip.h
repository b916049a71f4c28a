/*
 * wisp_hip — C ABI of the MI355X (gfx950) paged fused-MoE layer.
 *
 * Every entry point takes plain pointers, sizes and a hipStream_t, returns an
 * int status (WISP_OK = 0) and never allocates device memory: the caller
 * owns all buffers (wisp_moe_experts_noalloc instead works in a static device
 * array of the library).  On failure wisp_last_error() returns a message.
 *
 * Tensor pointers are device memory of the stream's device unless an entry
 * point says otherwise (expert masters live in host memory, pinned for the
 * copy-kernel engine; decision records may be pinned host memory).  The
 * kernels read what they are given as device addresses, so host memory passed
 * where device memory is expected is not detected here: the Python layer
 * checks devices before it calls in.
 *
 * Each function names the reference code it replaces; paths are relative to
 * the reference checkout (nokia-applied-research/WiSP).
 */
#ifndef WISP_HIP_H_
#define WISP_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* wisp_stream_t; /* == hipStream_t */

/* status codes */
#define WISP_OK 0
#define WISP_ERR_INVALID 1     /* bad argument (shape, id out of range, ...) */
#define WISP_ERR_SUBBATCH 2    /* a call's working set exceeds cap; the
                                  reference raises RuntimeError("... sub-batch")
                                  at fused_moe.py:315-327 */
#define WISP_ERR_HIP 3         /* HIP runtime error */
#define WISP_ERR_UNSUPPORTED 4 /* shape/dtype outside what the kernels cover */

/* element types */
#define WISP_F32 0
#define WISP_BF16 1
#define WISP_FP8_E4M3 2 /* layer dtype: expert weights float8_e4m3fn (OCP) with
                           float32 block scales; x, act and out bfloat16 */

/* layer modes (WISP_MODE, fused_moe.py:76-79) */
#define WISP_MODE_PAGED 0
#define WISP_MODE_RESIDENT 1

/* expert-stage algorithms */
#define WISP_ALGO_AUTO 0
#define WISP_ALGO_GEMV 1  /* wave-per-row GEMV, decode shapes */
#define WISP_ALGO_MFMA 2  /* bf16 MFMA grouped GEMM, batched/prefill shapes */

/* page-in engines */
#define WISP_PAGEIN_MEMCPY 0 /* hipMemcpyAsync per loaded expert, issued by the
                                host after it has read the decision record */
#define WISP_PAGEIN_KERNEL 1 /* a copy kernel reads the pinned masters through
                                their device mapping; the load list stays on
                                the GPU, so a call that is certain to be one
                                token group (T*top_k <= cap) never waits for
                                the host */

/* ---- library -------------------------------------------------------- */

/* Message of the last failing call on this thread ("" if none). */
const char* wisp_last_error(void);
/* ABI version of this library: 4 (wisp_layer_desc carries the block-FP8
 * fields and the packed masters; wisp_layer_desc and wisp_workspace end
 * with struct_bytes, which the caller sets to the struct's sizeof and the
 * library checks, so that a caller built against another layout is refused
 * instead of misread). */
int wisp_abi_version(void);
/* int32 words a decision record needs for a call of T tokens x K experts. */
int wisp_record_words(int T, int K);

/* ---- group 1: routing and the pager -------------------------------- */

/* Router softmax -> top-k -> optional renormalisation, one wave per token.
 * logits [T, E] (WISP_F32 or WISP_BF16) -> topk_w f32 [T, K], topk_ids i32
 * [T, K] in routing order (logit descending, ties to the lower id).
 * If forward_counter is non-null, it is incremented once (layer-call count).
 * Replaces: layer.select_experts(..., renormalize, scoring_func="softmax")
 *           at src/wisp/integrations/vllm/fused_moe.py:1054-1076. */
int wisp_route_topk_softmax(const void* logits, int logits_dtype, int T, int E, int K,
                            int renormalize, float* topk_w, int32_t* topk_ids,
                            int64_t* forward_counter, wisp_stream_t stream);

/* The expert pager on the GPU (one workgroup).  Plans the greedy token
 * groups (or one group if single_group), then for each group in order makes
 * the LRU hit / evict / load decisions, updates the device state
 * (expert_map [E], slot_to_expert [cap], lru_tick [cap], counters [8] =
 * {clock, forward, miss, evict, hits, ...}), writes the slot each
 * (token, k) reads into slots [T, K] (may be NULL), and writes the decision
 * record (layout: wisp_amd/csrc/pager_core.h) to `record`, which may be
 * pinned host memory.  Decisions are bit-exact with the reference.
 * Replaces: WispMoEState.ensure_resident (fused_moe.py:264-358), the greedy
 *           sub-batch planner (fused_moe.py:1119-1140) and the
 *           torch.unique(...).cpu() syncs at fused_moe.py:279,1102,1174. */
int wisp_pager_decide(const int32_t* topk_ids, int T, int K, int E, int cap,
                      int single_group, int32_t* expert_map, int32_t* slot_to_expert,
                      int64_t* lru_tick, int64_t* counters, int32_t* slots,
                      int32_t* record, int record_words, wisp_stream_t stream);

/* Same decisions computed sequentially on the host (host pointers).  The
 * specification the GPU pager is tested against. */
int wisp_pager_decide_host(const int32_t* topk_ids, int T, int K, int E, int cap,
                           int single_group, int32_t* expert_map, int32_t* slot_to_expert,
                           int64_t* lru_tick, int64_t* counters, int32_t* slots,
                           int32_t* record, int record_words);

/* Iteration order of CPython's set built from ascending keys (the order of
 * the reference's `missing` list, fused_moe.py:279-283).  Host only.
 * Returns n, or -1 if n is outside [0, 512]. */
int wisp_cpython_set_order(const int32_t* keys, int n, int32_t* order);

/* Greedy first-fit token grouping (host): group_end[g] = one past the last
 * token of group g.  Returns the number of groups.
 * Replaces: fused_moe.py:1119-1140. */
int wisp_subbatch_plan(const int32_t* topk_ids, int T, int K, int cap, int32_t* group_end);

/* Issue the page-in copies of one group of a decision record on copy_stream
 * (hipMemcpyAsync from pinned host masters into HBM scratch slots).  Strides
 * are in bytes.  When fused_slab != 0 the w2 bytes of an expert directly
 * follow its w13 bytes in both the master and the slot, and one copy of
 * w13_bytes + w2_bytes moves both.
 * Replaces: scratch_w13[slot].copy_(cpu_w13[e]); scratch_w2[slot].copy_(...)
 *           at fused_moe.py:351-352. */
int wisp_pagein_issue(const int32_t* record, int record_words, int T, int K, int group,
                      const void* master_w13, size_t master_w13_stride,
                      const void* master_w2, size_t master_w2_stride,
                      void* scratch_w13, size_t scratch_w13_stride,
                      void* scratch_w2, size_t scratch_w2_stride,
                      size_t w13_bytes, size_t w2_bytes, int fused_slab,
                      wisp_stream_t copy_stream);

/* ---- group 2: expert compute --------------------------------------- */

/* Slot-remapped SwiGLU experts with the routing-order combine:
 *   act[t,k] = silu(W13[s] x[t])[:I] * (W13[s] x[t])[I:],  s = slots[t,k]
 *   out[t]   = sum_{k=0..K-1} topk_w[t,k] * (W2[s] act[t,k])  (k ascending)
 * A slot of -1 contributes zero; slots are < nslots.  W13 of slot s is at
 * w13 + s*w13_stride ([2I, H] row-major), W2 at w2 + s*w2_stride ([H, I]
 * row-major); strides in elements.  act: workspace of T*K*I elements.  dtype
 * WISP_F32 or WISP_BF16 (x, weights, act and out share it).  work: device
 * buffer, 256-byte aligned, of wisp_moe_work_bytes(T, K, H, nslots) bytes
 * (used by WISP_ALGO_MFMA; may be NULL for the GEMV kernels).
 * Replaces: vLLM fused_experts(..., expert_map=...) at
 *           fused_moe.py:1106-1118 and 1155-1167. */
int wisp_moe_experts(const void* x, int dtype, int T, int H, int I, int K,
                     const float* topk_w, const int32_t* slots, int nslots,
                     const void* w13, size_t w13_stride, const void* w2, size_t w2_stride,
                     void* act, void* out, void* work, size_t work_bytes, int algo,
                     wisp_stream_t stream);

/* Block-FP8 (w8a8) SwiGLU experts with the routing-order combine, as vLLM's
 * fused_experts computes them with an fp8_w8a8 block quant config:
 *   activations quantised per token and group of 128 columns to e4m3fn
 *   (s = max(max|x|, 1e-10) / 448), then per k-block kb
 *   acc += (dot(q_x[kb], W[n, kb]) * s_x[kb]) * S[n / block_n][kb];
 *   h13 = bf16(acc); act = bf16(bf16(silu(gate)) * up); act quantised as x;
 *   y = bf16(W2-stage acc * topk_w); out[t] = moe_sum_k y[t,k] (bf16 adds
 *   for K in {2,3,4}, else one float32 sum rounded once), k ascending.
 * x, act, out: bfloat16.  W13 of slot s: w13 + s*w13_stride bytes
 * ([2I, H] e4m3fn), its scales s13 + s*s13_stride floats
 * ([2I/block_n, H/128]); W2 [H, I] and s2 [H/block_n, I/128] likewise.
 * Requires block_k == 128, block_n a multiple of 16 dividing I, H and I
 * multiples of 128.  A slot of -1 contributes zero.  algo: WISP_ALGO_GEMV
 * runs the decode kernels (MFMA tiles of one token column per pair, no work
 * buffer); WISP_ALGO_MFMA the grouped path (per-slot token lists, each
 * weight tile once per 64 tokens), which needs work: device, 256-byte
 * aligned, wisp_moe_fp8_work_bytes(T, K, H, I, nslots) bytes; AUTO picks
 * the grouped path from 16 tokens.
 * Replaces: vLLM fused_experts(..., quant_config=fp8_w8a8_moe_quant_config(
 *           w1_scale=scratch_s13, w2_scale=scratch_s2, block_shape=...))
 *           at src/wisp/integrations/vllm/fused_moe_fp8.py:245-249,316-326. */
int wisp_moe_experts_fp8(const void* x, int T, int H, int I, int K, const float* topk_w,
                         const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                         const float* s13, size_t s13_stride, const void* w2, size_t w2_stride,
                         const float* s2, size_t s2_stride, int block_n, int block_k, void* act,
                         void* out, void* work, size_t work_bytes, int algo,
                         wisp_stream_t stream);

/* Bytes of the work buffer the grouped block-FP8 path needs: per-slot pair
 * lists, bf16 per-pair outputs, and the quantised x and act with their
 * scales.  No reference counterpart (vLLM allocates its own). */
size_t wisp_moe_fp8_work_bytes(int T, int K, int H, int I, int nslots);

/* Dynamic per-row, per-group fp8 quantisation: x [rows, cols] (WISP_F32 or
 * WISP_BF16, row stride cols) -> q [rows, cols] e4m3fn codes and
 * scales [rows, cols / group] float32, s = max(max|x_g|, 1e-10) / 448,
 * q = e4m3fn(clamp(x / s, -448, 448)) rounded to nearest even.  group == 128
 * and cols a multiple of it.
 * Replaces: vLLM per_token_group_quant_fp8 (the activation quantisation of
 *           the fp8_w8a8 block path at fused_moe_fp8.py:316-326). */
int wisp_quant_fp8_groups(const void* x, int dtype, int rows, int cols, int group, uint8_t* q,
                          float* scales, wisp_stream_t stream);

/* Bytes of the device array wisp_moe_experts_noalloc works in, per GPU, in
 * a default build; building with WISP_NOALLOC_SCRATCH_MIB=n sets n MiB, and
 * wisp_noalloc_scratch_bytes() returns the size the library was built with.
 * Every process that loads the library holds this much HBM on each GPU it
 * runs on, from the code object's load there until the process ends,
 * whether or not it calls wisp_moe_experts_noalloc: count it in the HBM
 * budget beside the layers' scratch (cap slots each). */
#ifndef WISP_NOALLOC_SCRATCH_BYTES
#define WISP_NOALLOC_SCRATCH_BYTES (64u << 20)
#endif
/* The size of that array in this build, in bytes. */
size_t wisp_noalloc_scratch_bytes(void);

/* wisp_moe_experts without act and work arguments, allocating nothing.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (work captured into a HIP graph, serving loops or harnesses
 * that forbid hipMalloc).  The act intermediate and the MFMA work buffer live
 * in a static device array of the library, wisp_noalloc_scratch_bytes()
 * per GPU, held from the code object's load on that GPU until the process
 * ends.  A call needing more than that (T*K*I act elements, 256-byte
 * aligned, plus wisp_moe_work_bytes(T, K, H, nslots) on the MFMA path)
 * returns WISP_ERR_INVALID before any launch.  Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (on different streams
 * without ordering between them) race: order them on one stream or with
 * events.  Arguments, algorithms and results are those of wisp_moe_experts
 * (bit-identical outputs). */
int wisp_moe_experts_noalloc(const void* x, int dtype, int T, int H, int I, int K,
                             const float* topk_w, const int32_t* slots, int nslots,
                             const void* w13, size_t w13_stride, const void* w2,
                             size_t w2_stride, void* out, int algo, wisp_stream_t stream);

/* Bytes of the work buffer the MFMA expert path needs for T tokens x K over
 * nslots slots at hidden size H: per-slot pair lists and fp32 per-pair
 * outputs.  No reference counterpart (vLLM allocates its own). */
size_t wisp_moe_work_bytes(int T, int K, int H, int nslots);

/* ---- group 3: the layer call --------------------------------------- */

typedef struct wisp_layer_desc {
  int num_experts, cap;          /* cap in [1, 512]; it may exceed
                                    num_experts (the FP8 clamp
                                    max(8, min(cap, E)), fused_moe_fp8.py:58);
                                    resident mode needs cap == num_experts */
  int hidden, inter;             /* expert MLP shape; 0 for a pager-only
                                    state (the forward call then fails)  */
  int dtype, mode;
  int pagein_streams;            /* 0: page-in copies run on the caller's
                                    stream (stream order fences them);
                                    1 or 2: on that many side streams,
                                    fenced with events (memcpy engine)    */
  int pagein_engine;             /* WISP_PAGEIN_*; KERNEL falls back to
                                    MEMCPY when the masters are not pinned,
                                    device-mapped and 16-byte aligned     */
  size_t w13_elems, w2_elems;    /* elements of one expert's w13 / w2    */
  void* scratch_w13;             /* device, slot s at +s*stride [2I, H]  */
  size_t scratch_w13_stride;     /* elements                             */
  void* scratch_w2;              /* device, slot s at +s*stride [H, I]   */
  size_t scratch_w2_stride;      /* elements                             */
  const void* master_w13;        /* pinned host, expert e at +e*stride   */
  size_t master_w13_stride;      /* elements                             */
  const void* master_w2;
  size_t master_w2_stride;       /* elements                             */
  int32_t* expert_map;           /* device [num_experts]                 */
  int32_t* slot_to_expert;       /* device [cap]                         */
  int64_t* lru_tick;             /* device [cap]                         */
  int64_t* counters;             /* device [8]                           */
  /* block-FP8 experts (dtype WISP_FP8_E4M3; zero / NULL otherwise).  The
     weights above are then float8_e4m3fn (strides in bytes) and each expert
     carries float32 block scales: s13 [2*ceil(I/bn), ceil(H/bk)],
     s2 [ceil(H/bn), ceil(I/bk)] (fused_moe_fp8.py:188-202). */
  int block_n, block_k;          /* weight block [rows, cols]            */
  size_t s13_elems, s2_elems;    /* scale elements of one expert         */
  float* scratch_s13;            /* device, slot s at +s*stride          */
  size_t scratch_s13_stride;     /* elements                             */
  float* scratch_s2;
  size_t scratch_s2_stride;      /* elements                             */
  const float* master_s13;       /* host, expert e at +e*stride          */
  size_t master_s13_stride;      /* elements                             */
  const float* master_s2;
  size_t master_s2_stride;       /* elements                             */
  /* bf16 layers: the masters' packed copy (wisp_pack_bf16), pinned host,
     expert e at +e*packed_stride bytes, or NULL.  The copy-kernel engine
     then pages in from it; the memcpy engine ignores it.  It must hold
     exactly master_w13 / master_w2 as packed. */
  const void* packed_master;
  size_t packed_stride;          /* bytes                                */
  size_t struct_bytes;           /* sizeof(wisp_layer_desc); another value
                                    is refused (WISP_ERR_INVALID)         */
} wisp_layer_desc;

typedef struct wisp_workspace {
  int max_pairs;                 /* T*K the buffers below are sized for  */
  float* topk_w;                 /* device [max_pairs]                   */
  int32_t* topk_ids;             /* device [max_pairs]                   */
  int32_t* slots;                /* device [max_pairs]                   */
  int32_t* flags;                /* device [1 + max_pairs]: experts loaded
                                    by the call, then per pair a word: its
                                    slot in bits 0-15 (0xFFFF: none) and,
                                    if this call loaded its expert, that
                                    expert id + 1 in bits 16-30            */
  int32_t* loads;                /* device [2*max_pairs]: (expert, slot)
                                    pairs loaded by the call              */
  void* act;                     /* device [max_pairs*inter]             */
  int32_t* record;               /* pinned host [record_words]           */
  int record_words;
  int32_t* record_dev;           /* device [record_words] or NULL: where
                                    one-group calls on the copy-kernel
                                    engine write their record instead
                                    (read it back with
                                    wisp_layer_sync_record)               */
  void* work;                    /* device, 256-byte aligned: MFMA path
                                    work buffer (wisp_moe_work_bytes with
                                    nslots = cap)                         */
  size_t work_bytes;
  size_t struct_bytes;           /* sizeof(wisp_workspace); another value
                                    is refused (WISP_ERR_INVALID)         */
} wisp_workspace;

/* Packed bf16 masters.  No reference counterpart: the reference pages the
 * bf16 masters as they are (fused_moe.py:338-354).  The packed copy holds
 * the same values in ~0.77x the bytes (typical weights), so the copy-kernel
 * engine's page-in moves fewer bytes over the host link and unpacks them
 * into the slot; the slot's bytes are the master's exactly.  Per row of L
 * values and block of 64 values: the sign and mantissa bytes, a 4-bit
 * exponent code above the block's smallest nonzero exponent (code 15:
 * exponent 0), the block's base exponent; a block whose exponents span more
 * than 15 values keeps its 64 exponent bytes in the expert's exception
 * area.  Experts are [E, 2I, H] (w13) and [E, H, I] (w2) bf16 at the given
 * element strides; H and I must be multiples of 64.  Host-only calls (no
 * device work), threaded over experts.
 * wisp_pack_bf16_stride: bytes per packed expert (a multiple of 256) for
 * these masters, 0 when the shape does not pack. */
size_t wisp_pack_bf16_stride(int E, int H, int I, const void* master_w13,
                             size_t master_w13_stride, const void* master_w2,
                             size_t master_w2_stride);
/* Packs the masters into out (E * stride bytes, host memory); stride at
 * least wisp_pack_bf16_stride of the same masters. */
int wisp_pack_bf16(int E, int H, int I, const void* master_w13, size_t master_w13_stride,
                   const void* master_w2, size_t master_w2_stride, void* out, size_t stride);

/* Create / destroy the per-layer context (copy stream, events). */
int wisp_layer_create(const wisp_layer_desc* desc, void** handle);
int wisp_layer_destroy(void* handle);
/* Re-point the context at a new scratch / cap (after a resize).  Layers of
 * dtype WISP_FP8_E4M3 have no resize (the reference's FP8 state has none):
 * WISP_ERR_UNSUPPORTED. */
int wisp_layer_set_scratch(void* handle, void* scratch_w13, void* scratch_w2, int cap,
                           int32_t* slot_to_expert, int64_t* lru_tick);

/* One MoE layer call on `stream` for T tokens routed to top_k experts each:
 * route, page (paged mode) and compute.  Returns WISP_ERR_SUBBATCH when one
 * token alone needs more than cap experts.
 * Replaces: _patched_forward_cuda / _wisp_forward_cuda_paged
 *           (fused_moe.py:930-987, 990-1237). */
int wisp_layer_forward(void* handle, const void* x, const void* logits, int logits_dtype,
                       int T, int top_k, int renormalize, void* out, const wisp_workspace* ws,
                       int algo, wisp_stream_t stream);

/* Wait for the device, then make the decision record of the layer's last
 * call readable at ws->record (pinned host), copying it from ws->record_dev
 * when the call wrote it there.  No reference counterpart (the reference
 * pager runs on the host). */
int wisp_layer_sync_record(void* handle, const wisp_workspace* ws);

/* Make the experts in ids[n] resident as one call (no sub-batching).
 * Replaces: WispMoEState.ensure_resident (fused_moe.py:264-358). */
int wisp_layer_ensure_resident(void* handle, const int32_t* ids, int n,
                               const wisp_workspace* ws, wisp_stream_t stream);

/* Copy every expert into slot e and set the identity map (cap == E).
 * Replaces: WispMoEState.prime_identity (fused_moe.py:242-258). */
int wisp_layer_prime_identity(void* handle, wisp_stream_t stream);

/* Milliseconds the page-in copies of the layer calls since the last query
 * took (memcpy engine: from the first copy to the last; kernel engine: the
 * copy kernels' execution) and the bytes they moved; then reset both.  Only
 * calls made while timing is on (wisp_layer_profile) are counted. */
int wisp_layer_last_pagein(void* handle, float* ms, double* bytes);

/* The page-in engine the layer uses (WISP_PAGEIN_*), or -1 for a bad handle. */
int wisp_layer_pagein_engine(void* handle);

/* Run the first half of a one-token paged call whose top-k equals cap
 * (routing fused, copy-kernel engine, at most 128 experts, bf16 or fp32
 * rows of 2 or 4 16-byte chunks per lane) as one launch: the pager in one
 * wave, the page-in copies once it has decided, and w13 per slot from the
 * slots' contents, which need no decision (enable != 0); or as the pager
 * launch then the page-in + w13 launch (0, the default).  The outputs and
 * decisions are the same; the fused launch shortens a call that loads
 * nothing by ~2 us, but its pager runs behind the w13 stream's loads.
 * No counterpart in the reference (the reference's forward is one vLLM
 * call): a launch-structure choice of this implementation. */
int wisp_layer_set_decode_fused(void* handle, int enable);

/* Read and reset the accumulated execution time (dispatch timestamps) of the
 * w13+SiLU kernels and of the w2+combine kernels of all layer calls since the
 * last read, the number of layer calls, and the number of calls whose w13
 * time is in w13_ms; then switch timing on (enable != 0) or off.  A
 * speculative w2 launch that found experts to load and exited is not counted.
 * One-group GEMV calls on the copy-kernel engine run page-in and w13 as one
 * launch: it counts as w13 time when it copied nothing, else as page-in time
 * (wisp_layer_last_pagein).  The switch also covers the page-in timing.
 * Timing is off by default: every timed launch carries dispatch-timestamp
 * events, which lengthen the stream. */
int wisp_layer_profile(void* handle, int enable, double* w13_ms, double* w2_ms,
                       int64_t* calls, int64_t* w13_calls);

/* The w2 time (ms, dispatch timestamps) of the calls whose fused page-in +
 * w13 launch copied nothing, and their number, since the last
 * wisp_layer_profile: the same calls whose w13 time wisp_layer_profile
 * reports in w13_ms on that path, so the two stages are averaged over one
 * set of calls.  Read it before wisp_layer_profile, which resets it.
 * No counterpart in the reference: measurement only. */
int wisp_layer_profile_noload(void* handle, double* w2_ms, int64_t* calls);

/* ---- group 4: cross-layer speculative prefetch ------------------------ */

/* Dense expert co-activation table and the current step's observations, all
 * in device memory (owned by the caller). */
typedef struct wisp_cooccur {
  int layers, experts;
  int32_t* count;     /* [layers][experts][layers][experts]: steps in which
                         expert e_src fired at L_src and e_dst at L_dst, for
                         L_dst > L_src                                        */
  int32_t* total;     /* [layers][experts]: steps in which (L, e) fired        */
  int32_t* obs_keys;  /* [layers][experts]: the current step's experts of each
                         layer, in the iteration order of the set the forward
                         built (ascending insertion)                           */
  int32_t* obs_n;     /* [layers]: their number, 0 when not seen this step     */
  int32_t* obs_seq;   /* [layers]: the order in which the step saw the layers  */
  int32_t* meta;      /* [4]: [0] layers seen this step, [1] steps learned     */
} wisp_cooccur;

/* Record layer `layer`'s experts for the current step (nothing for n == 0):
 * ordered == 0: the set built from the ascending unique of ids[n] (what the
 * forward does); ordered != 0: ids[n] as given, in that iteration order.
 * Replaces: _CURRENT_STEP_OBS[layer_idx] = last_set (fused_moe.py:1174-1199). */
int wisp_cooccur_observe_layer(const wisp_cooccur* table, int layer, const int32_t* ids, int n,
                               int ordered, wisp_stream_t stream);

/* Top-k experts predicted at target_layer from the step's observations:
 * out_ids[0..*out_n) in rank order.  weights[d] (device, double) weighs
 * sources d+1 layers below the target (decay ** d).
 * Replaces: predict_layer (src/wisp/oracle/cooccur.py:233-287). */
int wisp_cooccur_predict(const wisp_cooccur* table, int target_layer, int k,
                         const double* weights, int normalize, int only_prev_layer,
                         int32_t* out_ids, int32_t* out_n, wisp_stream_t stream);

/* End of a step: add its pairs and marginals to the table when `learn`, then
 * clear the observations.  Replaces: table.observe_step(_CURRENT_STEP_OBS);
 * _CURRENT_STEP_OBS.clear() (fused_moe.py:1224-1233, cooccur.py:79-104). */
int wisp_cooccur_end_step(const wisp_cooccur* table, int learn, wisp_stream_t stream);

/* Words of a prefetch record for up to max_predicted predictions:
 * [0] evicted, [1] loaded, [2] clock advanced, [3] predictions taken, then
 * max_predicted evicted (expert, slot) pairs, then max_predicted loaded. */
int wisp_prefetch_record_words(int max_predicted);

/* Speculatively page predicted[0..n) (device; length *n_predicted when that
 * device pointer is non-NULL, else n) into the layer: the decisions run on
 * `stream`, the copies on the layer's side stream; the layer's next call
 * waits for them before it touches its scratch.  ordered != 0: the list is
 * already a set's iteration order; else it is the insertion order of
 * set(predicted).  last_ids[n_last] (device): the layer's last routed
 * experts (never evicted here).  count_pred != 0 adds the prediction count
 * to the layer's counters.  record: device [wisp_prefetch_record_words(n)].
 * Replaces: WispMoEState.prefetch_async (fused_moe.py:360-433). */
int wisp_layer_prefetch(void* handle, const int32_t* predicted, const int32_t* n_predicted,
                        int n, int ordered, int count_pred, const int32_t* last_ids,
                        int n_last, int32_t* record, int record_words, wisp_stream_t stream);

/* ---- group 5: probes ----------------------------------------------- */

/* Pinned host -> device hipMemcpyAsync bandwidth: `iters` copies of `bytes`
 * on `streams` streams; writes the per-iteration milliseconds.
 * Replaces: scripts/m3_11_anvil_bandwidth_probe.py:42-82. */
int wisp_probe_h2d(void* dst, const void* src_host, size_t bytes, int iters, int streams,
                   float* ms_per_iter);

/* Streaming device copy kernel (dst <- src, bytes multiple of 16), for the
 * HBM read+write calibration of the byte counters. */
int wisp_probe_hbm_copy(void* dst, const void* src, size_t bytes, wisp_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* WISP_HIP_H_ */
