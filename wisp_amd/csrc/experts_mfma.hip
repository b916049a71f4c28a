// Batched/prefill expert kernels on the bf16 MFMA units: a grouped GEMM over
// the slots present in the call.
//
// Replaces vLLM fused_experts for multi-token calls
// (src/wisp/integrations/vllm/fused_moe.py:1106-1118, 1155-1167); same
// arithmetic as the decode GEMV kernels:
//   act[p]  = bf16(silu(W13[s][:I] x[t]) * (W13[s][I:] x[t]))   p = (t, k)
//   y[p]    = W2[s] act[p]                                        (fp32)
//   out[t]  = bf16(sum_{k ascending} w[t,k] * y[(t, k)])
//
// Four launches:
//   1. gather: per slot s, the ascending list of pairs routed to s and its
//      length (one wave per slot, ballot compaction - stable, deterministic);
//   2. w13: block (i-panel of 64, slot s) streams the 64 gate rows and 64 up
//      rows of the panel once per 64 tokens of s and multiplies them against
//      those tokens, 16 per MFMA tile (v_mfma_f32_16x16x32_bf16), with the
//      token fragments read from the L2-resident x rows; epilogue silu(g) * u;
//   3. w2: block (h-panel of 64, slot s) likewise over act, writing fp32 y;
//   4. combine: out[t] from y in routing order.
// Each output element is one MFMA dot product chain over K in a fixed order,
// independent of which other tokens share its tile, so a token's bytes do not
// depend on the grouping or the slot numbers: paged calls (split into token
// groups) give the same bytes as resident calls.
//
// At the Qwen3-30B-A3B shapes the expert weights are 9 MiB and a prefill
// chunk routes ~32 tokens to each expert, about 32 FLOP per weight byte: far
// below the bf16 ridge (~315 FLOP/B), so these kernels are HBM-bound and are
// built to stream each weight byte once per call.
#include "common.h"

namespace wisp {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kKAlign = 256;         // H and I must be multiples (up to 8 k-steps per iteration)
constexpr int kPanel = 64;           // output columns per block: 4 waves x 16
constexpr int kMaxMT = 4;            // 16-token tiles per pass (64 tokens); more tokens
                                     // on a slot take further passes over its weights

// Weight and token fragments alike use plain loads: here the nontemporal
// hint made every variant slower (measured on MI355X at the Qwen3 shape: -8 %
// at 16 and 32 tokens, -4 % at 512), unlike the decode GEMV.
__device__ inline u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ inline bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ inline uint16_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ inline float silu(float g) { return g / (1.0f + expf(-g)); }

// Work buffer carve-up (bytes, each piece 256-byte aligned).
struct WorkLayout {
  size_t lists, counts, y, total;
  WorkLayout(int P, int H, int nslots) {
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    lists = 0;
    counts = up((size_t)nslots * P * 4);
    y = counts + up((size_t)nslots * 4);
    total = y + up((size_t)P * H * 4);
  }
};

// ---------------------------------------------------------------------------
// 1. gather: lists[s * P + j] = j-th pair (ascending) with slots[p] == s.
// grid = nslots, block = one wave.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void gather_kernel(const int32_t* __restrict__ slots, int P,
                                                    int32_t* __restrict__ lists,
                                                    int32_t* __restrict__ counts) {
  const int s = blockIdx.x, lane = threadIdx.x;
  int32_t* L = lists + (size_t)s * P;
  int n = 0;
  for (int base = 0; base < P; base += 64) {
    const int p = base + lane;
    const bool m = p < P && slots[p] == s;
    const uint64_t b = __ballot(m);
    if (m) L[n + __popcll(b & ((1ull << lane) - 1ull))] = p;
    n += __popcll(b);
  }
  if (lane == 0) counts[s] = n;
}

// Row pointers of this lane's A rows (row lane%16 of each 16-token tile of
// the pass starting at m0), offset to the lane's 8 columns of a k-step; null
// for rows past the slot's last token (they read as zero).
template <int MT, bool kTokenRows>
__device__ inline void a_rows(const uint16_t* (&ap)[MT], const uint16_t* __restrict__ A, int ld,
                              int K, const int32_t* __restrict__ list, int m0, int mrows,
                              int lane) {
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int r = t * 16 + (lane & 15);
    ap[t] = nullptr;
    if (r < mrows) {
      const int p = list[m0 + r];
      ap[t] = A + (size_t)(kTokenRows ? p / K : p) * ld + (lane >> 4) * 8;
    }
  }
}

__device__ inline u32x4 ld16_or_zero(const uint16_t* p, int off) {
  if (!p) return u32x4{0u, 0u, 0u, 0u};
  return ld16(p + off);
}

// ---------------------------------------------------------------------------
// 2. w13 + SiLU*mul.  grid = (I / 64, nslots); wave w owns i in
// [blockIdx.x*64 + 16w, +16): gate rows i and up rows I + i.  Each wave
// streams its 32 weight rows once per pass of up to MT*16 tokens, U k-steps
// of 32 columns per iteration (16-byte loads per lane), and fetches the token
// fragments of the same k-steps from x (small and shared: L2-resident).
// No LDS, no barriers: waves are independent streams.
// ---------------------------------------------------------------------------
template <int MT, int U>
__global__ __launch_bounds__(256) void mfma_w13_kernel(
    const uint16_t* __restrict__ x, int H, int I, int K, int P, const int32_t* __restrict__ lists,
    const int32_t* __restrict__ counts, const uint16_t* __restrict__ w13, size_t w13_stride,
    uint16_t* __restrict__ act) {
  const int s = blockIdx.y;
  const int M = counts[s];
  if (M == 0) return;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i0 = blockIdx.x * kPanel + wave * 16;
  const uint16_t* Wg = w13 + (size_t)s * w13_stride + (size_t)(i0 + (lane & 15)) * H +
                       (lane >> 4) * 8;
  const uint16_t* Wu = Wg + (size_t)I * H;

  for (int m0 = 0; m0 < M; m0 += MT * 16) {
    const int mrows = min(M - m0, MT * 16);
    const uint16_t* ap[MT];
    a_rows<MT, true>(ap, x, H, K, list, m0, mrows, lane);
    f32x4 ag[MT], au[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      ag[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      au[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int k0 = 0; k0 < H; k0 += 32 * U) {
      u32x4 bg[U], bu[U], a[U][MT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        bg[u] = ld16(Wg + k0 + u * 32);
        bu[u] = ld16(Wu + k0 + u * 32);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) a[u][t] = ld16_or_zero(ap[t], k0 + u * 32);
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t * 16 < mrows) {
            ag[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[u][t]), as_bf16x8(bg[u]),
                                                            ag[t], 0, 0, 0);
            au[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[u][t]), as_bf16x8(bu[u]),
                                                            au[t], 0, 0, 0);
          }
        }
      }
    }
    // C[row][col]: row = 16t + 4*(lane/16) + q, col = lane % 16
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = t * 16 + (lane >> 4) * 4 + q;
        if (r < mrows) {
          const int p = list[m0 + r];
          act[(size_t)p * I + i0 + (lane & 15)] = bf16_rne(silu(ag[t][q]) * au[t][q]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 3. w2: y[p, h] = W2[s][h, :] . act[p, :].  grid = (H / 64, nslots); wave w
// owns h in [blockIdx.x*64 + 16w, +16); same streaming scheme over act.
// ---------------------------------------------------------------------------
template <int MT, int U>
__global__ __launch_bounds__(256) void mfma_w2_kernel(
    const uint16_t* __restrict__ act, int H, int I, int P, const int32_t* __restrict__ lists,
    const int32_t* __restrict__ counts, const uint16_t* __restrict__ w2, size_t w2_stride,
    float* __restrict__ y) {
  const int s = blockIdx.y;
  const int M = counts[s];
  if (M == 0) return;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h0 = blockIdx.x * kPanel + wave * 16;
  const uint16_t* Wr = w2 + (size_t)s * w2_stride + (size_t)(h0 + (lane & 15)) * I +
                       (lane >> 4) * 8;

  for (int m0 = 0; m0 < M; m0 += MT * 16) {
    const int mrows = min(M - m0, MT * 16);
    const uint16_t* ap[MT];
    a_rows<MT, false>(ap, act, I, 1, list, m0, mrows, lane);
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < I; k0 += 32 * U) {
      u32x4 b[U], a[U][MT];
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = ld16(Wr + k0 + u * 32);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) a[u][t] = ld16_or_zero(ap[t], k0 + u * 32);
#pragma unroll
      for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t * 16 < mrows)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[u][t]), as_bf16x8(b[u]),
                                                             acc[t], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = t * 16 + (lane >> 4) * 4 + q;
        if (r < mrows) y[(size_t)list[m0 + r] * H + h0 + (lane & 15)] = acc[t][q];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Software-pipelined variants for slots with many tokens (prefill).  The
// token tile of the pass (MT*16 rows) is staged through double-buffered LDS,
// 32*U columns at a time and shared by the four waves; each wave keeps the
// next chunk's weight fragments in flight in registers while it runs the
// MFMAs of the current chunk.  One barrier per chunk, and it waits only for
// LDS operations, so the weight loads stay in flight across it; the token
// loads of a chunk are issued before its weight loads, so storing them to
// LDS does not wait for the weights either.  Each thread's token rows are
// resolved once per pass.  Measured on MI355X at the Qwen3 shape, resident
// 512-token chunk: w13 231 -> 178 us and w2 136 -> 99 us against a block
// barrier, weight-then-token issue order, per-chunk row lookups and
// nontemporal weight loads.
// ---------------------------------------------------------------------------

// Block barrier that waits only for this wave's LDS operations.
__device__ inline void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt/expcnt left at max
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
template <int MT, int U>
struct PipeA {
  static constexpr int kCols = 32 * U;
  static constexpr int kLd = kCols + 8;                  // padded row (bf16)
  static constexpr int kVecs = MT * 16 * kCols / 8;      // 16-byte vectors per chunk
  static constexpr int kPer = (kVecs + 255) / 256;       // per thread
};

// Row pointers of this thread's share of the A tile: vector q of the thread
// is row idx / kRowVecs, 8 columns at (idx % kRowVecs) * 8 of each chunk
// (null past the pass's last row: loads as zero).
template <int MT, int U, bool kTokenRows, int NPER>
__device__ inline void pipe_rows(const uint16_t* (&rp)[NPER], const uint16_t* __restrict__ A,
                                 int ld, int K, const int32_t* __restrict__ list, int m0,
                                 int mrows) {
  constexpr int kRowVecs = PipeA<MT, U>::kCols / 8;
#pragma unroll
  for (int q = 0; q < PipeA<MT, U>::kPer; ++q) {
    const int idx = threadIdx.x + q * 256;
    const int row = idx / kRowVecs, c = idx % kRowVecs;
    rp[q] = nullptr;
    if (idx < PipeA<MT, U>::kVecs && row < mrows) {
      const int p = list[m0 + row];
      rp[q] = A + (size_t)(kTokenRows ? p / K : p) * ld + c * 8;
    }
  }
}

// Loads this thread's share of the A chunk at column k0 into registers.
template <int MT, int U, int NPER>
__device__ inline void pipe_load_a(u32x4 (&r)[NPER], const uint16_t* const (&rp)[NPER], int k0) {
#pragma unroll
  for (int q = 0; q < PipeA<MT, U>::kPer; ++q)
    r[q] = rp[q] ? ld16(rp[q] + k0) : u32x4{0u, 0u, 0u, 0u};
}

template <int MT, int U, int NPER, int LD>
__device__ inline void pipe_store_a(uint16_t (*As)[LD], const u32x4 (&r)[NPER]) {
  constexpr int kRowVecs = PipeA<MT, U>::kCols / 8;
#pragma unroll
  for (int q = 0; q < PipeA<MT, U>::kPer; ++q) {
    const int idx = threadIdx.x + q * 256;
    if (idx < PipeA<MT, U>::kVecs)
      *reinterpret_cast<u32x4*>(&As[idx / kRowVecs][(idx % kRowVecs) * 8]) = r[q];
  }
}

// NB: the weight operand rows of one wave are W[row0 + lane%16]; NW such row
// groups (NW = 2 for gate/up, 1 for w2) share the A tile.
template <int MT, int U, int NW, bool kTokenRows, int LD>
__device__ inline void pipe_gemm(const uint16_t* __restrict__ A, int ld_a, int K, int Kdim,
                                 const int32_t* __restrict__ list, int m0, int mrows,
                                 const uint16_t* const (&Wr)[NW], f32x4 (&acc)[NW][MT],
                                 uint16_t (*As)[MT * 16][LD]) {
  using PA = PipeA<MT, U>;
  const int lane = threadIdx.x & 63;
  const int kq = (lane >> 4) * 8;
  const uint16_t* rp[PA::kPer];
  pipe_rows<MT, U, kTokenRows>(rp, A, ld_a, K, list, m0, mrows);
  u32x4 b[NW][U], bn[NW][U], ar[PA::kPer];
  pipe_load_a<MT, U>(ar, rp, 0);
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int u = 0; u < U; ++u) b[w][u] = ld16(Wr[w] + u * 32);
  lds_barrier();  // the previous pass's readers of buffer 0 are done
  pipe_store_a<MT, U>(As[0], ar);
  lds_barrier();
  int buf = 0;
  for (int k0 = 0; k0 < Kdim; k0 += PA::kCols) {
    const bool more = k0 + PA::kCols < Kdim;
    if (more) {
      pipe_load_a<MT, U>(ar, rp, k0 + PA::kCols);
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int u = 0; u < U; ++u) bn[w][u] = ld16(Wr[w] + k0 + PA::kCols + u * 32);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        if (t * 16 < mrows) {
          const bf16x8 a =
              *reinterpret_cast<const bf16x8*>(&As[buf][t * 16 + (lane & 15)][u * 32 + kq]);
#pragma unroll
          for (int w = 0; w < NW; ++w)
            acc[w][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(b[w][u]), acc[w][t],
                                                                0, 0, 0);
        }
      }
    }
    if (more) {
      pipe_store_a<MT, U>(As[buf ^ 1], ar);
      lds_barrier();
      buf ^= 1;
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int u = 0; u < U; ++u) b[w][u] = bn[w][u];
    }
  }
}

template <int MT, int U>
__global__ __launch_bounds__(256) void mfma_w13_pipe_kernel(
    const uint16_t* __restrict__ x, int H, int I, int K, int P, const int32_t* __restrict__ lists,
    const int32_t* __restrict__ counts, const uint16_t* __restrict__ w13, size_t w13_stride,
    uint16_t* __restrict__ act) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][MT * 16][PipeA<MT, U>::kLd];
  const int s = blockIdx.y;
  const int M = counts[s];
  if (M == 0) return;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i0 = blockIdx.x * kPanel + wave * 16;
  const uint16_t* Wg = w13 + (size_t)s * w13_stride + (size_t)(i0 + (lane & 15)) * H +
                       (lane >> 4) * 8;
  const uint16_t* const Wr[2] = {Wg, Wg + (size_t)I * H};
  for (int m0 = 0; m0 < M; m0 += MT * 16) {
    const int mrows = min(M - m0, MT * 16);
    f32x4 acc[2][MT];
#pragma unroll
    for (int w = 0; w < 2; ++w)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[w][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    pipe_gemm<MT, U, 2, true>(x, H, K, H, list, m0, mrows, Wr, acc, As);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = t * 16 + (lane >> 4) * 4 + q;
        if (r < mrows) {
          const int p = list[m0 + r];
          act[(size_t)p * I + i0 + (lane & 15)] = bf16_rne(silu(acc[0][t][q]) * acc[1][t][q]);
        }
      }
    }
  }
}

template <int MT, int U>
__global__ __launch_bounds__(256) void mfma_w2_pipe_kernel(
    const uint16_t* __restrict__ act, int H, int I, int P, const int32_t* __restrict__ lists,
    const int32_t* __restrict__ counts, const uint16_t* __restrict__ w2, size_t w2_stride,
    float* __restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][MT * 16][PipeA<MT, U>::kLd];
  const int s = blockIdx.y;
  const int M = counts[s];
  if (M == 0) return;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h0 = blockIdx.x * kPanel + wave * 16;
  const uint16_t* const Wr[1] = {w2 + (size_t)s * w2_stride + (size_t)(h0 + (lane & 15)) * I +
                                 (lane >> 4) * 8};
  for (int m0 = 0; m0 < M; m0 += MT * 16) {
    const int mrows = min(M - m0, MT * 16);
    f32x4 acc[1][MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[0][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    pipe_gemm<MT, U, 1, false>(act, I, 1, I, list, m0, mrows, Wr, acc, As);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = t * 16 + (lane >> 4) * 4 + q;
        if (r < mrows) y[(size_t)list[m0 + r] * H + h0 + (lane & 15)] = acc[0][t][q];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 4. combine: out[t, h] = bf16(sum_k w[t,k] * y[(t,k), h]), k ascending,
// skipping pairs without a slot.  grid = (ceil(H / 256), T).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, int H, int K,
                                                     int nslots, const float* __restrict__ topk_w,
                                                     const int32_t* __restrict__ slots,
                                                     uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const int p = t * K + k;
    const int s = slots[p];
    if (s < 0 || s >= nslots) continue;
    acc = fmaf(topk_w[p], y[(size_t)p * H + h], acc);
  }
  out[(size_t)t * H + h] = bf16_rne(acc);
}

template <int MT, int U, bool kPipe>
void launch_gemms(const uint16_t* x, int H, int I, int K, int P, int nslots, const int32_t* lists,
                  const int32_t* counts, const uint16_t* w13, size_t w13_stride,
                  const uint16_t* w2, size_t w2_stride, uint16_t* act, float* y, hipStream_t st,
                  const StageEvents* ev) {
  hipEvent_t e0 = ev ? ev->ev[0] : nullptr, e1 = ev ? ev->ev[1] : nullptr;
  hipEvent_t e2 = ev ? ev->ev[2] : nullptr, e3 = ev ? ev->ev[3] : nullptr;
  if (kPipe) {
    launch_timed(mfma_w13_pipe_kernel<MT, U>, dim3(I / kPanel, nslots), dim3(256), st, e0, e1, x,
                 H, I, K, P, lists, counts, w13, w13_stride, act);
    launch_timed(mfma_w2_pipe_kernel<MT, U>, dim3(H / kPanel, nslots), dim3(256), st, e2, e3, act,
                 H, I, P, lists, counts, w2, w2_stride, y);
  } else {
    launch_timed(mfma_w13_kernel<MT, U>, dim3(I / kPanel, nslots), dim3(256), st, e0, e1, x, H, I,
                 K, P, lists, counts, w13, w13_stride, act);
    launch_timed(mfma_w2_kernel<MT, U>, dim3(H / kPanel, nslots), dim3(256), st, e2, e3, act, H,
                 I, P, lists, counts, w2, w2_stride, y);
  }
}

}  // namespace

void launch_gather(const int32_t* slots, int P, int nslots, int32_t* lists, int32_t* counts,
                   hipStream_t st) {
  hipLaunchKernelGGL(gather_kernel, dim3(nslots), dim3(64), 0, st, slots, P, lists, counts);
}

size_t mfma_work_bytes(int T, int K, int H, int nslots) {
  if (T < 1 || K < 1 || H < 1 || nslots < 1) return 0;
  return WorkLayout(T * K, H, nslots).total;
}

// Shapes the MFMA path covers (else the caller uses the GEMV kernels).
bool mfma_supported(int H, int I) {
  return H >= kKAlign && I >= kKAlign && H % kKAlign == 0 && I % kKAlign == 0;
}

int experts_mfma(const void* x, int T, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                 const void* w2, size_t w2_stride, void* act, void* out, void* work,
                 size_t work_bytes, hipStream_t st, const StageEvents* ev) {
  if (T == 0) return WISP_OK;
  if (!mfma_supported(H, I)) {
    wisp_set_last_error("MFMA path needs hidden and intermediate sizes that are multiples of 256",
                        "MFMA experts");
    return WISP_ERR_UNSUPPORTED;
  }
  const int P = T * K;
  const WorkLayout W(P, H, nslots);
  if (nslots < 1 || nslots > 65535 || !work || work_bytes < W.total ||
      ((uintptr_t)work) % 256) {
    wisp_set_last_error("MFMA work buffer missing, misaligned or too small", "MFMA experts");
    return WISP_ERR_INVALID;
  }
  int32_t* lists = (int32_t*)((char*)work + W.lists);
  int32_t* counts = (int32_t*)((char*)work + W.counts);
  float* y = (float*)((char*)work + W.y);
  hipLaunchKernelGGL(gather_kernel, dim3(nslots), dim3(64), 0, st, slots, P, lists, counts);
  // A slot holds a token at most once (a token's top-k experts are
  // distinct), so T bounds the rows of any slot.
  const uint16_t* xb = (const uint16_t*)x;
  const uint16_t* a13 = (const uint16_t*)w13;
  const uint16_t* a2 = (const uint16_t*)w2;
  uint16_t* ab = (uint16_t*)act;
  // (tiles per pass, k-steps per iteration, pipelined), measured at the Qwen3
  // shapes on MI355X: more tiles per pass cost registers (fewer waves in
  // flight) but save passes over the weights once slots hold more than 32
  // tokens, where staging the token tile in LDS also pays.
  if (T <= 16)
    launch_gemms<1, 8, false>(xb, H, I, K, P, nslots, lists, counts, a13, w13_stride, a2,
                              w2_stride, ab, y, st, ev);
  else if (T <= 128)
    launch_gemms<2, 4, false>(xb, H, I, K, P, nslots, lists, counts, a13, w13_stride, a2,
                              w2_stride, ab, y, st, ev);
  else
    launch_gemms<kMaxMT, 2, true>(xb, H, I, K, P, nslots, lists, counts, a13, w13_stride, a2,
                                  w2_stride, ab, y, st, ev);
  hipLaunchKernelGGL(combine_kernel, dim3((H + 255) / 256, T), dim3(256), 0, st, y, H, K, nslots,
                     topk_w, slots, (uint16_t*)out);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

}  // namespace wisp
