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
//      length (block-wide ballot compaction - stable, deterministic);
//   2. w13: block (i-panel of 64, slot s) streams the 64 gate rows and 64 up
//      rows of the panel once per 64 tokens of s and multiplies them against
//      those tokens, 16 per MFMA tile (v_mfma_f32_16x16x32_bf16); epilogue
//      silu(g) * u.  Both operands are staged through LDS by asynchronous
//      global->LDS copies (dma_pipeline.h);
//   3. w2: block (h-panel of 128, slot s) likewise over act, writing fp32 y;
//   4. combine: out[t] from y in routing order.
// Each output element is one MFMA dot product chain over K in a fixed order
// (ascending 32-column k-steps from a start column set by the output panel,
// wrapping around), independent of which other tokens share its tile, so a
// token's bytes do not depend on the grouping or the slot numbers: paged
// calls (split into token groups) give the same bytes as resident calls.
//
// At the Qwen3-30B-A3B shapes the expert weights are 9 MiB and a prefill
// chunk routes ~32 tokens to each expert, about 32 FLOP per weight byte: far
// below the bf16 ridge (~315 FLOP/B), so these kernels are HBM-bound and are
// built to stream each weight byte once per call.
#include <type_traits>

#include <algorithm>

#include "common.h"
#include "dma_pipeline.h"

namespace wisp {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kKAlign = 256;         // H and I must be multiples
constexpr int kPanel = 64;           // output columns per block: 4 waves x 16
// The LDS-staged w2 kernel's blocks own 128 output rows (4 waves x 32): a
// w2 row is only 12 chunks long at the Qwen3 shape, so per-block setup and
// the token tile weigh more than in w13, and 32 rows per wave halve both.
// Calls with enough (slot, panel) work for two rounds of blocks use 256 rows
// per block (two copy stages, two blocks per CU).
constexpr int kW2PanelsPer = 2;      // 64-row panels per LDS-staged w2 block
constexpr int kW2PanelsBig = 4;

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
// grid = nslots, block = 512 threads; each iteration covers 4096 pairs, 8
// consecutive ones per thread, and places the matches by a block-wide
// exclusive prefix of the per-thread counts (counts <= 8: four ballots per
// wave for the bits, one LDS exchange across the eight waves).
// ---------------------------------------------------------------------------
constexpr int kGatherPer = 8;
constexpr int kGatherWaves = 8;

__global__ __launch_bounds__(64 * kGatherWaves) void gather_kernel(
    const int32_t* __restrict__ slots, int P, int32_t* __restrict__ lists,
    int32_t* __restrict__ counts) {
  __shared__ int wave_total[kGatherWaves];
  const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int32_t* L = lists + (size_t)s * P;
  const uint64_t below = (1ull << lane) - 1ull;
  int n = 0;  // matches before this iteration (block-uniform)
  for (int base = 0; base < P; base += 64 * kGatherWaves * kGatherPer) {
    const int p0 = base + tid * kGatherPer;
    int v[kGatherPer];
#pragma unroll
    for (int q = 0; q < kGatherPer; ++q) v[q] = p0 + q < P ? slots[p0 + q] : -1;
    unsigned hit = 0;
#pragma unroll
    for (int q = 0; q < kGatherPer; ++q) hit |= (unsigned)(v[q] == s) << q;
    const int c = __popc(hit);
    int pre = 0, tot = 0;
#pragma unroll
    for (int bit = 0; bit < 4; ++bit) {
      const uint64_t m = __ballot((c >> bit) & 1);
      pre += __popcll(m & below) << bit;
      tot += __popcll(m) << bit;
    }
    if (lane == 0) wave_total[wave] = tot;
    __syncthreads();
    int off = n, all = 0;
#pragma unroll
    for (int w = 0; w < kGatherWaves; ++w) {
      off += w < wave ? wave_total[w] : 0;
      all += wave_total[w];
    }
    __syncthreads();  // wave_total is rewritten by the next iteration
    int o = off + pre;
#pragma unroll
    for (int q = 0; q < kGatherPer; ++q)
      if (hit >> q & 1u) L[o++] = p0 + q;
    n += all;
  }
  if (tid == 0) counts[s] = n;
}

// Where the k loop of an output panel starts.  Every block streams its rows
// chunk by chunk; when all blocks start at column 0, the reads in flight share
// their low address bits and crowd a few memory channels (a pure read of the
// Qwen3 w13 tensor in this order, non-temporal loads: 6.27 TB/s on MI355X).
// Starting each panel at its own multiple of 64 columns, evenly spread over
// the row, and wrapping around gives 6.99 TB/s.  The start depends only on the panel (blockIdx.x),
// never on the slot, so an output's dot-product order is the same for any
// slot placement or token grouping.
__device__ inline int k_rotation(int Kdim) {
  return (int)(blockIdx.x * (unsigned)(Kdim / 64) / gridDim.x) * 64;
}

// The w2 kernel's rotation: by the block's 256-row group of H (NG 64-row
// panels per block, NG = 2 or 4), so that blocks of 128 and of 256 rows give
// every output row the same k order and the same bytes.
template <int NG>
__device__ inline int k_rotation_w2(int Kdim) {
  static_assert(NG == 2 || NG == 4, "64-row panels per w2 block");
  const unsigned group = blockIdx.x * NG / 4, groups = gridDim.x * NG / 4;
  return (int)(group * (unsigned)(Kdim / 64) / groups) * 64;
}

// Column of k-step offset k (0 <= k < Kdim) in a loop rotated by rot columns.
__device__ inline int k_col(int k, int rot, int Kdim) {
  const int c = k + rot;
  return c >= Kdim ? c - Kdim : c;
}

// ---------------------------------------------------------------------------
// w13 and w2 kernels: the chunk pipeline of dma_pipeline.h over 64-column
// (128-byte) chunks, two 32-column k-steps of MFMA per chunk, the k rotation
// of the output panel.  w13 blocks own a 64-row panel (each wave 16 gate and
// 16 up rows); w2 blocks own 128 rows (32 per wave).
// What bounds them: a pure read of the Qwen3 w13 tensor with these copies
// (non-temporal), chunk order, rotation and occupancy runs at 6.95 TB/s on
// MI355X and w13 here at 6.18 TB/s of weights; the w2 tensor reads at
// 6.45 TB/s and w2 here at 4.90 TB/s.
// ---------------------------------------------------------------------------

// The pass's GEMM over Kdim columns for mrows tokens (the pass's pair list
// held one entry per lane in `held`, dma::list_entries): acc[g][t] +=
// W(row group g) . A(token tile t)^T for the NT = ceil(mrows / 16) tiles the
// pass fills, NG row groups of 16 per wave, the k loop starting rot columns
// in.  A is the token matrix (leading dimension ld); with kTokenRows, pair p
// reads row p / K.  With the weights as the MFMA's first
// operand, lane l holds rows 4 (l / 16) + q, q < 4, of its group for token
// column l % 16: four consecutive outputs of one token, stored at once.
template <int NG, int S, bool kTokenRows>
__device__ inline void dma_gemm(unsigned char* smem,
                                const unsigned char* const (&wrow)[16 * NG / dma::kRowsPerCopy],
                                const uint16_t* __restrict__ A, int ld, int K, int held,
                                int mrows, int Kdim, int rot, bool first,
                                f32x4 (&acc)[NG][4]) {
  const int lane = threadIdx.x & 63;
  auto row_of = [&](int r) {
    const int p = dma::list_entry(held, r);
    return reinterpret_cast<const unsigned char*>(A + (size_t)(kTokenRows ? p / K : p) * ld);
  };
  auto off = [&](int c) { return (size_t)k_col(c * 64, rot, Kdim) * sizeof(uint16_t); };
  auto run = [&](auto nt) {
    constexpr int NT = decltype(nt)::value;
    dma::pass<16 * NG, S, NT>(
        smem, wrow, mrows, row_of, Kdim / 64, off,
        [&](const unsigned char* ws, const unsigned char* as, int) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int cb = u * 4 + (lane >> 4);
            bf16x8 b[NG], a[NT];
#pragma unroll
            for (int g = 0; g < NG; ++g)
              b[g] = *reinterpret_cast<const bf16x8*>(ws + dma::swz(g * 16 + (lane & 15), cb));
#pragma unroll
            for (int t = 0; t < NT; ++t)
              a[t] = *reinterpret_cast<const bf16x8*>(as + dma::swz(t * 16 + (lane & 15), cb));
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
              for (int g = 0; g < NG; ++g)
                acc[g][t] =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[g], a[t], acc[g][t], 0, 0, 0);
          }
        },
        dma::NoSetup{}, first);
  };
  const int nt = (mrows + 15) >> 4;
  if (nt == 1)
    run(std::integral_constant<int, 1>{});
  else if (nt == 2)
    run(std::integral_constant<int, 2>{});
  else if (nt == 3)
    run(std::integral_constant<int, 3>{});
  else
    run(std::integral_constant<int, 4>{});
}

// The pairs of the token columns this lane stores after the pass (tile t,
// column lane % 16; columns past mrows repeat the last), from the pass's
// lane-held pair list.
__device__ inline void epilogue_pairs(int held, int mrows, int (&pr)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int t = 0; t < 4; ++t) pr[t] = dma::list_entry(held, min(t * 16 + (lane & 15), mrows - 1));
}

// bf16(silu(g) * u) of four consecutive columns, one 8-byte store at p.
__device__ inline void store_act4(uint16_t* p, const f32x4& g, const f32x4& u) {
  uint32_t h[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) h[q] = bf16_rne(silu(g[q]) * u[q]);
  *reinterpret_cast<uint2*>(p) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
}

template <int S>
__global__ __launch_bounds__(256) void mfma_w13_dma_kernel(
    const uint16_t* __restrict__ x, int H, int I, int K, int P, const int32_t* __restrict__ lists,
    const int32_t* __restrict__ counts, const uint16_t* __restrict__ w13, size_t w13_stride,
    uint16_t* __restrict__ act) {
  extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
  const int s = blockIdx.y;
  const int32_t* list = lists + (size_t)s * P;
  // the slot's count and the first pass's pair list, loaded together
  const int M = counts[s];
  int held = dma::list_entries(list, 0, P);
  if (M == 0) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i0 = blockIdx.x * kPanel + wave * 16;
  const uint16_t* W = w13 + (size_t)s * w13_stride;
  // this lane's weight copy rows: slice rows 0-15 gate, 16-31 up
  const unsigned char* wrow[32 / dma::kRowsPerCopy];
#pragma unroll
  for (int i = 0; i < 32 / dma::kRowsPerCopy; ++i) {
    const int r = i * dma::kRowsPerCopy + lane / dma::kLanesPerRow;
    wrow[i] = reinterpret_cast<const unsigned char*>(
        W + (size_t)(r < 16 ? i0 + r : I + i0 + r - 16) * H);
  }
  const int rot = k_rotation(H);
  for (int m0 = 0; m0 < M; m0 += dma::kTokRows) {
    const int mrows = min(M - m0, dma::kTokRows);
    if (m0 > 0) held = dma::list_entries(list, m0, P);
    f32x4 acc[2][4];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    int pr[4];
    epilogue_pairs(held, mrows, pr);
    dma_gemm<2, S, true>(dsm, wrow, x, H, K, held, mrows, H, rot, m0 == 0, acc);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (t * 16 + (lane & 15) < mrows)
        store_act4(act + (size_t)pr[t] * I + i0 + (lane >> 4) * 4, acc[0][t], acc[1][t]);
  }
}

template <int S, int NG>
__global__ __launch_bounds__(256) void mfma_w2_dma_kernel(
    const uint16_t* __restrict__ act, int H, int I, int P, const int32_t* __restrict__ lists,
    const int32_t* __restrict__ counts, const uint16_t* __restrict__ w2, size_t w2_stride,
    float* __restrict__ y) {
  extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
  const int s = blockIdx.y;
  const int32_t* list = lists + (size_t)s * P;
  // the slot's count and the first pass's pair list, loaded together
  const int M = counts[s];
  int held = dma::list_entries(list, 0, P);
  if (M == 0) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // NG row groups of 16 per wave
  const int h0 = blockIdx.x * kPanel * NG + wave * 16 * NG;
  const uint16_t* W = w2 + (size_t)s * w2_stride;
  const unsigned char* wrow[16 * NG / dma::kRowsPerCopy];
#pragma unroll
  for (int i = 0; i < 16 * NG / dma::kRowsPerCopy; ++i)
    wrow[i] = reinterpret_cast<const unsigned char*>(
        W + (size_t)(h0 + i * dma::kRowsPerCopy + lane / dma::kLanesPerRow) * I);
  const int rot = k_rotation_w2<NG>(I);
  for (int m0 = 0; m0 < M; m0 += dma::kTokRows) {
    const int mrows = min(M - m0, dma::kTokRows);
    if (m0 > 0) held = dma::list_entries(list, m0, P);
    f32x4 acc[NG][4];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    int pr[4];
    epilogue_pairs(held, mrows, pr);
    dma_gemm<NG, S, false>(dsm, wrow, act, I, 1, held, mrows, I, rot, m0 == 0, acc);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (t * 16 + (lane & 15) < mrows) {
        float* yr = y + (size_t)pr[t] * H + h0 + (lane >> 4) * 4;
#pragma unroll
        for (int g = 0; g < NG; ++g) *reinterpret_cast<f32x4*>(yr + g * 16) = acc[g][t];
      }
  }
}

// ---------------------------------------------------------------------------
// 4. combine: out[t, h] = bf16(sum_k w[t,k] * y[(t,k), h]), k ascending,
// skipping pairs without a slot (their y rows are never written: selected
// out, not multiplied by zero).  8 columns per thread, every k's slot,
// weight and y loads issued before the sums.  grid = (ceil(H / 2048), T).
// ---------------------------------------------------------------------------
constexpr int kCombineK = 16;  // top-k handled with all loads up front; more loop

template <bool kVecStore>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ y, int H, int K,
                                                     int nslots, const float* __restrict__ topk_w,
                                                     const int32_t* __restrict__ slots,
                                                     uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (h >= H) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += kCombineK) {
    const int kn = min(K - k0, kCombineK);
    f32x4 lo[kCombineK], hi[kCombineK];
    float w[kCombineK];
    bool ok[kCombineK];
#pragma unroll
    for (int k = 0; k < kCombineK; ++k) {
      if (k < kn) {
        const int p = t * K + k0 + k;
        const int sl = slots[p];
        ok[k] = sl >= 0 && sl < nslots;
        w[k] = topk_w[p];
        const f32x4* yr = reinterpret_cast<const f32x4*>(y + (size_t)p * H + h);
        lo[k] = yr[0];
        hi[k] = yr[1];
      }
    }
#pragma unroll
    for (int k = 0; k < kCombineK; ++k) {
      if (k < kn && ok[k]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[j] = fmaf(w[k], lo[k][j], acc[j]);
          acc[4 + j] = fmaf(w[k], hi[k][j], acc[4 + j]);
        }
      }
    }
  }
  uint16_t* o = out + (size_t)t * H + h;
  if constexpr (kVecStore) {
    u32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = (uint32_t)bf16_rne(acc[2 * j]) | ((uint32_t)bf16_rne(acc[2 * j + 1]) << 16);
    *reinterpret_cast<u32x4*>(o) = v;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = bf16_rne(acc[j]);
  }
}

void launch_combine(const float* y, int T, int H, int K, int nslots, const float* topk_w,
                    const int32_t* slots, uint16_t* out, hipStream_t st) {
  const dim3 grid((H + 2047) / 2048, T);
  if (((uintptr_t)out | ((size_t)H * 2)) % 16 == 0)
    hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, st, y, H, K, nslots, topk_w,
                       slots, out);
  else
    hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, st, y, H, K, nslots, topk_w,
                       slots, out);
}

template <int S2, int NG>
hipError_t launch_w2_dma(const uint16_t* act, int H, int I, int P, int nslots,
                         const int32_t* lists, const int32_t* counts, const uint16_t* w2,
                         size_t w2_stride, float* y, hipStream_t st, hipEvent_t e2,
                         hipEvent_t e3) {
  constexpr unsigned b2 = dma::Smem<16 * NG, S2>::kBytes;
  static_assert(b2 <= 160 * 1024, "LDS per block");
  static std::atomic<uint64_t> big2{0};
  hipError_t e = allow_lds(&mfma_w2_dma_kernel<S2, NG>, b2, b2, &big2);
  if (e != hipSuccess) return e;
  launch_timed_lds(mfma_w2_dma_kernel<S2, NG>, dim3(H / (kPanel * NG), nslots), dim3(256), b2,
                   st, e2, e3, act, H, I, P, lists, counts, w2, w2_stride, y);
  return hipSuccess;
}

template <int S13>
hipError_t launch_dma(const uint16_t* x, int H, int I, int K, int P, int nslots,
                      const int32_t* lists, const int32_t* counts, const uint16_t* w13,
                      size_t w13_stride, const uint16_t* w2, size_t w2_stride, uint16_t* act,
                      float* y, hipStream_t st, const StageEvents* ev) {
  constexpr unsigned b13 = dma::Smem<32, S13>::kBytes;
  static_assert(b13 <= 160 * 1024, "LDS per block");
  static std::atomic<uint64_t> big13{0};
  hipError_t e = allow_lds(&mfma_w13_dma_kernel<S13>, b13, b13, &big13);
  if (e != hipSuccess) return e;
  hipEvent_t e0 = ev ? ev->ev[0] : nullptr, e1 = ev ? ev->ev[1] : nullptr;
  hipEvent_t e2 = ev ? ev->ev[2] : nullptr, e3 = ev ? ev->ev[3] : nullptr;
  launch_timed_lds(mfma_w13_dma_kernel<S13>, dim3(I / kPanel, nslots), dim3(256), b13, st, e0,
                   e1, x, H, I, K, P, lists, counts, w13, w13_stride, act);
  // 256-row w2 blocks (two stages) when the call's slots could give two
  // blocks per CU of them; else 128-row blocks (three stages).  Measured at
  // the Qwen3 512-token chunk: 83 against 89 us; the smaller blocks keep
  // calls with few slots (Mixtral, paged token groups) spread over the GPU.
  const int64_t busy = (int64_t)std::min(P, nslots) * (H / (kPanel * kW2PanelsBig));
  return busy >= 512 ? launch_w2_dma<2, kW2PanelsBig>(act, H, I, P, nslots, lists, counts, w2,
                                                      w2_stride, y, st, e2, e3)
                     : launch_w2_dma<3, kW2PanelsPer>(act, H, I, P, nslots, lists, counts, w2,
                                                      w2_stride, y, st, e2, e3);
}

}  // namespace

void launch_gather(const int32_t* slots, int P, int nslots, int32_t* lists, int32_t* counts,
                   hipStream_t st) {
  hipLaunchKernelGGL(gather_kernel, dim3(nslots), dim3(64 * kGatherWaves), 0, st, slots, P, lists,
                     counts);
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
  hipLaunchKernelGGL(gather_kernel, dim3(nslots), dim3(64 * kGatherWaves), 0, st, slots, P, lists,
                     counts);
  // A slot holds a token at most once (a token's top-k experts are
  // distinct), so T bounds the rows of any slot.
  const uint16_t* xb = (const uint16_t*)x;
  const uint16_t* a13 = (const uint16_t*)w13;
  const uint16_t* a2 = (const uint16_t*)w2;
  uint16_t* ab = (uint16_t*)act;
  // w13 with two copy stages (three blocks per CU: 241 against 244 us at the
  // Qwen3 512-token chunk), w2 with three (its shorter rows gain nothing from
  // a third block per CU).  Measured on MI355X, these kernels also beat
  // register-streaming ones at every call size, down to 4 tokens (71 against
  // 109 us at the Qwen3 shape).
  WISP_HIP_TRY((launch_dma<2>(xb, H, I, K, P, nslots, lists, counts, a13, w13_stride, a2,
                              w2_stride, ab, y, st, ev)));
  launch_combine(y, T, H, K, nslots, topk_w, slots, (uint16_t*)out, st);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

}  // namespace wisp
