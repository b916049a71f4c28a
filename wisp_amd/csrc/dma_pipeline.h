// Global->LDS chunk pipeline shared by the LDS-staged grouped GEMMs (bf16
// and block-FP8).
//
// A block of four waves streams, chunk by chunk, 128 bytes of each of its
// weight rows (NWR rows per wave, one slice per wave and stage, read only by
// that wave) and 128 bytes of each row of the pass's token tile (up to 64
// rows, shared by the waves, copy j issued by wave j % 4) straight into LDS
// with the asynchronous global->LDS loads (global_load_lds_dwordx4), S - 1
// chunks ahead of their use.  Neither operand passes through registers.
// One copy instruction moves 1 KiB: 8 rows of 128 bytes.  Each LDS row holds
// its 16-byte column blocks XOR-swizzled by the row (block cb at position
// cb ^ (row & 7)), so MFMA operand reads of 16 rows at one column block
// spread over the banks.  Token rows past the pass's last token copy a valid
// row; their results are never stored.  Each wave waits for its own copies
// by vmcnt (a constant per chunk), then one barrier per chunk: after it,
// every wave's copies of the chunk have landed and every wave is done with
// the stage the next copy overwrites.  The weight copies are non-temporal
// (each weight byte is read once per launch); the token copies are not.
// Each loop step names its copy stage and its compute stage as distinct
// (restrict), so the compiler does not hold a chunk's LDS reads behind the
// copies just issued for a later one.
#pragma once

#include "common.h"

namespace wisp {
namespace dma {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kRowBytes = 128;     // bytes of one row in one chunk
constexpr int kRowsPerCopy = 8;    // one 1 KiB copy: 8 rows x 128 bytes
constexpr int kLanesPerRow = 8;    // 16 bytes per lane
constexpr int kTokRows = 64;       // token tile: four MFMA tiles of 16
constexpr int kMaxTokCopies = 2;   // 64 rows / 8 per copy / 4 waves

// Block barrier that waits only for this wave's LDS operations (its
// global->LDS copies are waited for by vmcnt, explicitly, beforehand).
__device__ inline void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt/expcnt left at max
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Cache policy of a copy: the weights stream through once (non-temporal);
// the token rows, which every panel of a slot reads, stay cached.
constexpr int kPolicyDefault = 0;
constexpr int kPolicyNontemporal = 2;  // the instruction's nt bit

// 16 bytes per lane from g into LDS at dst + 16 * lane.  Measured on MI355X
// with a pure read of the Qwen3 w13 tensor in these kernels' chunk order at
// 3 blocks per CU: 6.10 TB/s with the default policy, 6.87 TB/s non-temporal
// (register loads: 6.16 and 7.11 TB/s).
template <int POLICY = kPolicyDefault>
__device__ inline void dma16(const void* g, void* dst) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)dst, 16, 0, POLICY);
}

// Waits until at most N of this wave's vector memory operations are
// outstanding.
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Waits for the copies of the chunk that has `ahead` later chunks issued
// behind it (each chunk is PER copy instructions per wave).
template <int PER, int A>
__device__ inline void wait_chunk(int ahead) {
  if constexpr (A > 0) {
    if (ahead >= A) {
      wait_vm<A * PER>();
      return;
    }
    wait_chunk<PER, A - 1>(ahead);
  } else {
    wait_vm<0>();
  }
}

// Byte offset of 16-byte column block cb of row r in a swizzled slice.
__device__ inline int swz(int r, int cb) { return r * kRowBytes + ((cb ^ (r & 7)) << 4); }

// 16 bytes of row r, column block cb, of a swizzled slice.
__device__ inline uint4 ld_swz(const unsigned char* slice, int r, int cb) {
  return *reinterpret_cast<const uint4*>(slice + swz(r, cb));
}

// LDS of one stage: the four waves' weight slices, then the token tile.
template <int NWR, int S>
struct Smem {
  static constexpr int kW = 4 * NWR * kRowBytes;
  static constexpr int kA = kTokRows * kRowBytes;
  static constexpr int kStage = kW + kA;
  static constexpr int kBytes = S * kStage;
};

// A chunk's byte offsets into the weight rows (w) and the token rows (t).
// A chunk offset given as one number applies to both.
struct Offs {
  size_t w, t;
};
__device__ inline Offs offs_of(size_t o) { return Offs{o, o}; }
__device__ inline Offs offs_of(Offs o) { return o; }

// One stage's copies of the chunk at offsets o: this wave's NWR weight rows
// and its TCW token copies.  wrow[i] / arow[i] are the lane's source rows
// (copy i covers rows [8i, 8i + 8) of the wave's weights; token copy
// wave + 4i covers tile rows [8 (wave + 4i), +8)).
template <int NWR, int TCW>
__device__ inline void chunk_copies(unsigned char* stage,
                                    const unsigned char* const (&wrow)[NWR / kRowsPerCopy],
                                    const unsigned char* const (&arow)[kMaxTokCopies], int wave,
                                    int lane, Offs o) {
  const int pos = lane % kLanesPerRow, sub = lane / kLanesPerRow;
#pragma unroll
  for (int i = 0; i < NWR / kRowsPerCopy; ++i) {
    const int r = i * kRowsPerCopy + sub;
    dma16<kPolicyNontemporal>(wrow[i] + o.w + ((pos ^ (r & 7)) << 4),
                              stage + (wave * NWR + i * kRowsPerCopy) * kRowBytes);
  }
  unsigned char* at = stage + 4 * NWR * kRowBytes;
#pragma unroll
  for (int i = 0; i < TCW; ++i) {
    const int r0 = (wave + 4 * i) * kRowsPerCopy;
    dma16(arow[i] + o.t + ((pos ^ ((r0 + sub) & 7)) << 4), at + r0 * kRowBytes);
  }
}

struct NoSetup {
  __device__ void operator()() const {}
};

// One step of the pipeline: the copies of a later chunk into stage `wr`
// (when `issue`), then the compute of chunk c from stage `rd`.  The two
// stages never overlap, and the restrict parameters say so: the compiler's
// memory-counter pass then sees that the compute's LDS reads do not depend
// on the copies just issued.  Without that it waits for every copy in
// flight before the first LDS read, so a block held one chunk in flight
// whatever the stage count.
template <int NWR, int TCW, typename F>
__device__ __attribute__((always_inline)) inline void step(
    unsigned char* __restrict__ wr, const unsigned char* __restrict__ rd, bool issue,
    const unsigned char* const (&wrow)[NWR / kRowsPerCopy],
    const unsigned char* const (&arow)[kMaxTokCopies], int wave, int lane, Offs o, F& compute,
    int c) {
  if (issue) chunk_copies<NWR, TCW>(wr, wrow, arow, wave, lane, o);
  compute(rd + wave * NWR * kRowBytes, rd + 4 * NWR * kRowBytes, c);
}

// The S-stage pipeline over n chunks; chunk c starts off(c) bytes into every
// row (or off(c).w into the weight rows and off(c).t into the token rows).
// after_prologue() runs once the first S - 1 chunks' copies are issued
// (setup whose loads should travel with them: what it writes to LDS is seen
// by every wave from chunk 0's compute on, after the loop's barrier);
// compute(ws, as, c) runs once chunk c has landed, with ws this wave's weight
// slice and as the token tile of its stage.
template <int NWR, int S, int TCW, typename Off, typename F, typename G = NoSetup>
__device__ inline void pipeline(unsigned char* smem,
                                const unsigned char* const (&wrow)[NWR / kRowsPerCopy],
                                const unsigned char* const (&arow)[kMaxTokCopies], int n, Off off,
                                F&& compute, G&& after_prologue = G{}) {
  using Sm = Smem<NWR, S>;
  constexpr int PER = NWR / kRowsPerCopy + TCW;  // copies per wave and chunk
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int c = 0; c < S - 1; ++c)
    if (c < n)
      chunk_copies<NWR, TCW>(smem + c * Sm::kStage, wrow, arow, wave, lane, offs_of(off(c)));
  after_prologue();
  for (int c = 0; c < n; ++c) {
    wait_chunk<PER, S - 2>(min(S - 2, n - 1 - c));
    lds_barrier();
    const bool issue = c + S - 1 < n;
    step<NWR, TCW>(smem + ((c + S - 1) % S) * Sm::kStage, smem + (c % S) * Sm::kStage, issue,
                   wrow, arow, wave, lane, offs_of(off(issue ? c + S - 1 : c)), compute, c);
  }
}

// One pass for mrows tokens (NT = ceil(mrows / 16) tiles): the lane's token
// source rows (row_of(r) for tile row r, called by every lane; rows past
// mrows repeat the last), a drain of the previous pass (its copies and its
// readers of every stage and of anything after_prologue writes), then the
// pipeline with this wave's share of the tile's copies.
// A block's first pass (`first`) has no earlier pass to drain.  (Issuing
// its chunk 0 weight copies before the token rows are resolved measured
// slower: the compiler's wait for the pair list, which row_of permutes, also
// waits for those copies.)
template <int NWR, int S, int NT, typename RowOf, typename Off, typename F,
          typename G = NoSetup>
__device__ inline void pass(unsigned char* smem,
                            const unsigned char* const (&wrow)[NWR / kRowsPerCopy], int mrows,
                            RowOf row_of, int n, Off off, F&& compute,
                            G&& after_prologue = G{}, bool first = false) {
  constexpr int copies = 16 * NT / kRowsPerCopy;  // token copies of the tile, all waves
  static_assert(copies <= 4 * kMaxTokCopies, "token copies per wave");
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const unsigned char* arow[kMaxTokCopies];
#pragma unroll
  for (int i = 0; i < kMaxTokCopies; ++i)
    arow[i] = row_of(min((wave + 4 * i) * kRowsPerCopy + lane / kLanesPerRow, mrows - 1));
  if (!first) {
    wait_vm<0>();   // nothing but this pass's copies is outstanding below
    lds_barrier();  // the previous pass's readers of every stage are done
  }
  const int tcw = (copies - wave + 3) / 4;  // copies j = wave + 4i < copies: 0, 1 or 2
  if (tcw <= 0)
    pipeline<NWR, S, 0>(smem, wrow, arow, n, off, compute, after_prologue);
  else if (tcw == 1)
    pipeline<NWR, S, 1>(smem, wrow, arow, n, off, compute, after_prologue);
  else
    pipeline<NWR, S, 2>(smem, wrow, arow, n, off, compute, after_prologue);
}

// A load issued where it is written: the compiler neither sinks a relaxed
// atomic load below later control flow (a kernel's early exit on an empty
// slot) nor moves it after later loads, where plain loads of restrict data
// may go.
__device__ inline int32_t load_early(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ inline float load_early(const float* p) {
  return __int_as_float(load_early(reinterpret_cast<const int32_t*>(p)));
}

// A pass's pair list held one entry per lane: lane r holds list[m0 + r]
// (entries at or past the slot's count, read clamped to the list's length,
// are never used), so a tile row's entry is a lane permute rather than a
// dependent global load.  A kernel loads the first pass's entries together
// with the slot's count.
__device__ inline int list_entries(const int32_t* __restrict__ list, int m0, int len) {
  return load_early(list + min(m0 + (int)(threadIdx.x & 63), len - 1));
}
__device__ inline int list_entry(int held, int r) { return __shfl(held, r); }

}  // namespace dma
}  // namespace wisp
