// Shared definitions for the wisp_hip library (gfx950 only).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <atomic>

#include "../../include/wisp_hip.h"

#define WISP_HD __host__ __device__

namespace wisp {

// Upper bounds baked into the single-workgroup pager kernel's LDS layout.
constexpr int kMaxExperts = 512;
constexpr int kMaxTopK = 64;
// A CPython set of n <= kMaxExperts small ints never needs a table larger
// than the smallest power of two above 4n, which is <= 8n.
constexpr int kMaxSetTable = 8 * kMaxExperts;
// Calls of at most this many tokens are routed inside the pager kernel.
constexpr int kFusedRouteTokens = 8;
// Routed experts per token the decode GEMV pair handles (its w2 kernel runs
// one wave per expert in one block and keeps their partial sums in LDS).
constexpr int kGemvMaxTopK = 16;

// Per-layer counters kept on the device, in this order.
enum Counter : int {
  kClock = 0,     // LRU clock (one tick per ensure_resident call)
  kForward = 1,   // layer calls
  kMiss = 2,
  kEvict = 3,
  kHits = 4,
  kPredTotal = 5,  // experts predicted for this layer by cross-layer prefetch
  kNumCounters = 8,
};

// Orders this wavefront's LDS accesses across lanes without waiting for its
// outstanding global or host-memory stores (a block barrier would: on CDNA
// the barrier's wait counts stores too).  Only valid where every LDS
// producer and consumer is in the same wavefront.
__device__ inline void wave_lds_sync() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt/expcnt left at max
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// A wave-uniform word through the scalar data cache, for memory that no
// kernel writes while this one runs.  Where the compiler cannot prove that
// (a kernel that also stores through other pointers) it reads such a word
// with a vector load and a readfirstlane, a vector memory round trip that a
// weight stream then queues behind.
__device__ inline int32_t scalar_word(const int32_t* p) {
  int32_t v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}

// v of the lane that DPP control kCtrl names (all rows and banks enabled).
template <int kCtrl>
__device__ inline float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, false));
}

// v of lane `lane` (wave-uniform), through a scalar register.
__device__ inline float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Max over each 16-lane row of the wave, in every lane of the row: xor 1,
// xor 2, half-row mirror, row mirror.  Register-only (DPP), where a lane
// shuffle goes through the LDS crossbar; max is exact and commutative, so
// the order of the steps does not change the result.
__device__ inline float row16_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  return v;
}

// Block barrier for LDS data only: this wave's LDS accesses complete, then
// every wave meets.  __syncthreads() also waits for the wave's outstanding
// global loads (on CDNA its fence waits for the whole vector memory
// counter), so a block that has weight loads in flight while it stages data
// in LDS would wait for the weights at the barrier.
__device__ inline void block_lds_sync() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt/expcnt left at max
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Sum over each 16-lane row, the same bits in every lane of the row (after
// each step both partners hold the same bits, since IEEE add is
// commutative).  Register-only (DPP).
__device__ inline float row16_sum_f32(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  return v;
}

// Sum over the 64 lanes, the same bits in every lane: the four row sums
// combined in a fixed order through scalar registers.
__device__ inline float wave_sum_f32(float v) {
  v = row16_sum_f32(v);
  return ((readlane_f32(v, 0) + readlane_f32(v, 16)) + readlane_f32(v, 32)) +
         readlane_f32(v, 48);
}

// Sum over each 32-lane half of the wave, the same bits in every lane of
// the half.
__device__ inline float half_sum_f32(float v) {
  v = row16_sum_f32(v);
  const float lo = readlane_f32(v, 0) + readlane_f32(v, 16);
  const float hi = readlane_f32(v, 32) + readlane_f32(v, 48);
  return (__lane_id() < 32) ? lo : hi;
}

// float -> bfloat16 bits, round to nearest even (a NaN stays a quiet NaN).
// Branch-free: both results are formed and one is selected.
__device__ inline uint16_t bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
  return (uint16_t)(nan ? ((u >> 16) | 0x40u) : r);
}

// bfloat16 bits -> float.
__device__ inline float bf16f(uint32_t b) { return __uint_as_float(b << 16); }

// SiLU in float32 as vLLM's silu_and_mul computes it: g / (1 + exp(-g)).
__device__ inline float silu(float g) { return g / (1.0f + expf(-g)); }

// Optional kernel timing: {w13 start, w13 stop, w2 start, w2 stop}, recorded
// by the dispatch itself (hipExtLaunchKernelGGL), so the elapsed time is the
// kernel's own execution time.
struct StageEvents {
  hipEvent_t ev[4];
};

// Per slot s < nslots, the ascending list of the pairs p < P with
// slots[p] == s (lists[s * P + j]) and its length (counts[s]); one wave per
// slot, ballot compaction (deterministic).  Defined with the bf16 grouped
// GEMM; the block-FP8 grouped path shares it.
void launch_gather(const int32_t* slots, int P, int nslots, int32_t* lists, int32_t* counts,
                   hipStream_t st);

// Raises `kernel`'s dynamic-LDS limit to `max_lds` when a launch needs more
// than the default 64 KiB, once per device (bit d of *done marks device d;
// safe when several host threads launch at once).
template <typename Kern>
inline hipError_t allow_lds(Kern kernel, size_t lds, size_t max_lds,
                            std::atomic<uint64_t>* done) {
  if (lds <= 64 * 1024) return hipSuccess;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (done->load(std::memory_order_acquire) & bit) return hipSuccess;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds);
  if (e == hipSuccess) done->fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

// Launch with or without dispatch timestamps.
template <typename Kern, typename... Args>
inline void launch_timed(Kern kernel, dim3 grid, dim3 block, hipStream_t st, hipEvent_t start,
                         hipEvent_t stop, Args... args) {
  if (start)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, st, start, stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, st, args...);
}

// launch_timed with lds bytes of dynamic LDS per block.
template <typename Kern, typename... Args>
inline void launch_timed_lds(Kern kernel, dim3 grid, dim3 block, unsigned lds, hipStream_t st,
                             hipEvent_t start, hipEvent_t stop, Args... args) {
  if (start)
    hipExtLaunchKernelGGL(kernel, grid, block, lds, st, start, stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

}  // namespace wisp

#define WISP_HIP_TRY(expr)                               \
  do {                                                   \
    hipError_t _e = (expr);                              \
    if (_e != hipSuccess) {                              \
      wisp_set_last_error(hipGetErrorString(_e), #expr); \
      return WISP_ERR_HIP;                               \
    }                                                    \
  } while (0)

// Records a message retrievable through wisp_last_error().
void wisp_set_last_error(const char* what, const char* where);
