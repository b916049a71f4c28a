// Decode-shape expert kernels (GEMV): w13 with fused SiLU*mul, then w2 with
// the routing-order combine.
//
// Replaces vLLM fused_experts as called by the reference with the slot
// remap (src/wisp/integrations/vllm/fused_moe.py:1106-1118, 1155-1167):
//   act[t,k] = silu(W13[s][:I] x[t]) * (W13[s][I:] x[t]),   s = slots[t,k]
//   out[t]   = sum_{k=0..K-1} w[t,k] * (W2[s] act[t,k])     (k ascending)
//
// Both kernels stream weight rows with 16-byte loads, one wavefront (or half
// of one) per row, and reduce in a fixed order, so the bytes of
// out[t] depend only on x[t], the routing of token t and the weights read -
// never on the slot numbers, on cap or on the other tokens of the launch.
// That is what makes paged output byte-identical to resident output.
#include "common.h"
#include "pagein.h"
#include "pager_core.h"
#include "pager_wave.h"

namespace wisp {
namespace {

template <typename T>
struct Vec;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <>
struct Vec<float> {
  static constexpr int N = 4;
  __device__ static inline void unpack(const uint4& u, float* f) {
    f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
  }
  __device__ static inline void unpack(const u32x4& u, float* f) {
    f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
  }
};
template <>
struct Vec<uint16_t> {  // bf16 bits
  static constexpr int N = 8;
  __device__ static inline void unpack(const uint4& u, float* f) {
    f[0] = __uint_as_float(u.x << 16); f[1] = __uint_as_float(u.x & 0xffff0000u);
    f[2] = __uint_as_float(u.y << 16); f[3] = __uint_as_float(u.y & 0xffff0000u);
    f[4] = __uint_as_float(u.z << 16); f[5] = __uint_as_float(u.z & 0xffff0000u);
    f[6] = __uint_as_float(u.w << 16); f[7] = __uint_as_float(u.w & 0xffff0000u);
  }
  __device__ static inline void unpack(const u32x4& u, float* f) {
    f[0] = __uint_as_float(u.x << 16); f[1] = __uint_as_float(u.x & 0xffff0000u);
    f[2] = __uint_as_float(u.y << 16); f[3] = __uint_as_float(u.y & 0xffff0000u);
    f[4] = __uint_as_float(u.z << 16); f[5] = __uint_as_float(u.z & 0xffff0000u);
    f[6] = __uint_as_float(u.w << 16); f[7] = __uint_as_float(u.w & 0xffff0000u);
  }
};

template <typename T>
__device__ inline void store_elem(T* p, float v);
template <>
__device__ inline void store_elem<float>(float* p, float v) { *p = v; }
template <>
__device__ inline void store_elem<uint16_t>(uint16_t* p, float v) { *p = bf16_rne(v); }

__device__ inline uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// A word loaded before the loads that follow it in the source: the compiler
// neither sinks nor reorders a relaxed atomic load (plain loads of
// restrict-qualified data it may move below later loads).
__device__ inline int32_t load_first(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Streaming load for weight rows: each byte is read once per launch, so the
// nontemporal hint keeps the rows from displacing cached data (measured on
// MI355X: w13 at the Qwen3 decode shape 9.2 us instead of 10.2 us).
__device__ inline uint4 ld16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------------------
// Kernel A: act = silu(gate) * up.  Block = 4 waves, each wave owns one i
// (gate row i and up row I + i) of one (token, k) pair; each lane covers CH
// chunks of 16 bytes of a row (chunk c*64 + lane).  grid = (ceil(I / 4),
// T * K).  One row pair per wave gives the most waves in flight, which is
// what a pure weight stream needs.  FULL: a row is exactly CH chunks per lane,
// so the loads carry no bounds guard (a guarded load sits in its own
// exec-masked block, which costs ~0.7 us per launch at the Qwen3 shape by
// keeping the loads from issuing back to back).
//
// The row loads and the dot products are shared with the fused page-in
// kernel below, which computes the same act values from rows it copies.
// ---------------------------------------------------------------------------
template <typename T, int CH, bool FULL, bool STREAM>
__device__ inline void load_row(const T* __restrict__ row, int nch, int lane, uint4 (&v)[CH]) {
  constexpr int V = Vec<T>::N;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = c * 64 + lane;
    v[c] = (FULL || ch < nch) ? (STREAM ? ld16_stream(row + (size_t)ch * V)
                                        : ld16(row + (size_t)ch * V))
                              : make_uint4(0, 0, 0, 0);
  }
}

// silu(gate . x) * (up . x) for the rows and x chunks a wave holds: fp32 FMA
// over each lane's chunks in order, then wave_sum_f32 over the 64 lanes (DPP
// row sums, then the four rows in order); every lane returns the result.
template <typename T, int CH, typename VW>
__device__ inline float swiglu_rows(const VW (&wg)[CH], const VW (&wu)[CH],
                                    const uint4 (&xv)[CH]) {
  constexpr int V = Vec<T>::N;
  float ag = 0.f, au = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float xf[V], gf[V], uf[V];
    Vec<T>::unpack(xv[c], xf);
    Vec<T>::unpack(wg[c], gf);
    Vec<T>::unpack(wu[c], uf);
#pragma unroll
    for (int q = 0; q < V; ++q) {
      ag = fmaf(gf[q], xf[q], ag);
      au = fmaf(uf[q], xf[q], au);
    }
  }
  return silu(wave_sum_f32(ag)) * wave_sum_f32(au);
}

// The same dot product one row at a time: this lane's FMA chain over its
// chunks, then wave_sum_f32.  Each of swiglu_rows' two accumulators follows
// exactly this sequence, so silu(row_dot(gate)) * row_dot(up) equals
// swiglu_rows bit for bit.
template <typename T, int CH>
__device__ inline float row_dot(const u32x4 (&w)[CH], const uint4 (&xv)[CH]) {
  constexpr int V = Vec<T>::N;
  float a = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float xf[V], wf[V];
    Vec<T>::unpack(xv[c], xf);
    Vec<T>::unpack(w[c], wf);
#pragma unroll
    for (int q = 0; q < V; ++q) a = fmaf(wf[q], xf[q], a);
  }
  return wave_sum_f32(a);
}

// One wave: act[pair][i] of a pair whose expert sits in slot s, stored only
// when `keep` (the loads and the arithmetic happen either way, so a caller
// can load `keep` together with s instead of before it).
template <typename T, int CH, bool FULL>
__device__ inline void w13_wave(const T* __restrict__ x, int H, int I, int K, int pair, int i,
                                int s, const T* __restrict__ w13, size_t w13_stride,
                                T* __restrict__ act, int lane, bool keep = true) {
  constexpr int V = Vec<T>::N;
  T* arow = act + (size_t)pair * I;
  if (s < 0) {
    if (lane == 0 && keep) store_elem(arow + i, 0.f);
    return;
  }
  const int nch = H / V;
  const T* W = w13 + (size_t)s * w13_stride;
  uint4 xv[CH], wg[CH], wu[CH];
  load_row<T, CH, FULL, false>(x + (size_t)(pair / K) * H, nch, lane, xv);
  load_row<T, CH, FULL, true>(W + (size_t)i * H, nch, lane, wg);
  load_row<T, CH, FULL, true>(W + (size_t)(I + i) * H, nch, lane, wu);
  const float v = swiglu_rows<T, CH, uint4>(wg, wu, xv);
  if (lane == 0 && keep) store_elem(arow + i, v);
}

template <typename T, int CH, bool FULL>
__global__ __launch_bounds__(256) void w13_silu_kernel(const T* __restrict__ x, int H, int I,
                                                        int K, const int32_t* __restrict__ slots,
                                                        const T* __restrict__ w13,
                                                        size_t w13_stride, T* __restrict__ act,
                                                        const int32_t* __restrict__ pair_filter,
                                                        int want, int nslots) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pair = blockIdx.y;
  // the pager's per-pair words: run only the pairs whose expert this call
  // loaded (want != 0) or only the others (want == 0)
  if (pair_filter && (pair_word_loaded(pair_filter[pair]) >= 0) != (want != 0)) return;
  const int i = blockIdx.x * 4 + wave;
  if (i >= I) return;
  // a slot outside [0, nslots) reads no expert, as a slot of -1
  const int s = slots[pair];
  w13_wave<T, CH, FULL>(x, H, I, K, pair, i, (unsigned)s < (unsigned)nslots ? s : -1, w13,
                        w13_stride, act, lane);
}

// ---------------------------------------------------------------------------
// Kernel A': page-in and w13 in one launch, for one-token calls on the
// copy-kernel engine (a token's routed experts are distinct, so each expert
// serves exactly one pair).
//   * Blocks [0, kPageInBlocks) copy each expert the pager loaded from its
//     pinned master into its slot, in load order: first its w13 rows, one
//     row pair (gate i, up I + i) per wave and iteration, computing act[p][i]
//     of the expert's pair p from the rows the wave holds (Kernel A's
//     arithmetic on the same bytes, so the output equals a resident call's);
//     then the rest of its bytes as a plain copy.  Streaming the experts in
//     order keeps ~2 MiB of host reads in flight, which holds the host link
//     at its copy rate (reading every loaded expert at once from all the
//     w13 waves cost ~4 % of it).
//   * Blocks from kPageInBlocks on are Kernel A's blocks in (i-block, pair)
//     order, for the pairs whose expert was already resident.  A wave reads
//     its pair's slot and loaded flag from one word the pager wrote
//     (pair_word), so its row loads wait for a single load, as in Kernel A.
// A call that loads nothing costs the w13 work plus 64 blocks that exit
// after one load; one that loads experts runs the resident pairs' w13 under
// the copies.
// ---------------------------------------------------------------------------
// The w13 blocks' arguments come first in the kernel's argument segment (and
// the page-in blocks' 200-byte PageInArgs after them), so the blocks that
// stream weights find theirs at the front.
struct FusedW13Args {
  const void* x;
  const int32_t* words;  // the pager's flags + 1: pair_word(slot, loaded expert)
  const void* w13;       // scratch base, slot s at + s * w13_stride elements
  size_t w13_stride;
  void* act;
  int H, I, K, cap;
};

// The copy blocks' work when the masters are packed (packed.h): each loaded
// expert's w13 rows unpacked into its slot, one row pair per wave and
// iteration; the expert's pair then reads the two rows back from the slot
// with the resident blocks' own w13_wave, so its act bytes are theirs.
// (Computing act from the unpacked registers instead held more registers
// than the w13 blocks' budget, and all blocks of the launch get the most
// any path needs.)  Then each loaded expert's w2 rows.
template <int CH, bool FULL, int NCB>
__device__ inline void pagein_w13_packed(const FusedW13Args& f, const PageInArgs& a, int cb,
                                         int mine) {
  // wave-uniform (readfirstlane), so that the row bases sit in scalar
  // registers
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int H = f.H, I = f.I, nch = H / 8;
  const PackedSrc& pk = a.pk;
  const packed::Layout Lp(H, I);
  const int n = *a.count;
  int jcur = -1, e = -1, s = -1, pair = -1;
  for (int q = cb * 4 + wave; q < n * I; q += NCB * 4) {
    const int j = q / I, i = q - j * I;
    if (j != jcur) {
      jcur = j;
      e = __builtin_amdgcn_readfirstlane(a.loads[2 * j]);
      s = __builtin_amdgcn_readfirstlane(a.loads[2 * j + 1]);
      const uint64_t m = __ballot(mine == e);
      pair = m ? __builtin_ctzll(m) : -1;
    }
    if (e < 0 || e >= a.num_experts || s < 0 || s >= a.cap) continue;
    const char* ex = pk.m + (size_t)e * pk.m_stride;
    char* slot = pk.d13 + (size_t)s * pk.d13_stride;
#pragma unroll 1
    for (int r = 0; r < 2; ++r) {
      const int row = r ? I + i : i;
      const char* src = ex + (size_t)row * Lp.rs13;
      u32x4* dst = reinterpret_cast<u32x4*>(slot + (size_t)row * H * sizeof(uint16_t));
      const __amdgpu_buffer_rsrc_t rs = packed::row_rsrc(src, H);
      packed::Chunk c[CH];
      packed::for_each_chunk<CH>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        c[k] = packed::load_lane_chunk<k>(rs, H, lane);
      });
      // exception blocks are rare: a row without any takes the plain unpack
      bool exc = false;
#pragma unroll
      for (int k = 0; k < CH; ++k)
        exc |= (FULL || k * 64 + lane < nch) && packed::is_exception(c[k], k * 64 + lane);
      const bool slow = __ballot(exc) != 0;
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int ch = k * 64 + lane;
        if (FULL || ch < nch) {
          const uint4 v = packed::unpack_plain(c[k]);
          __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, dst + ch);
        }
      }
      // a row with exception blocks rewrites their chunks afterwards (a
      // separate pass: inline in the one above, it spilled registers of the
      // w13 blocks that share this launch)
      if (slow) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const int ch = k * 64 + lane;
          if ((FULL || ch < nch) && packed::is_exception(c[k], ch)) {
            const uint4 v = packed::unpack_chunk(c[k], src, H, ch, ex + Lp.exc_off);
            __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, dst + ch);
          }
        }
      }
    }
    if (pair >= 0) {
      // each lane reads back the chunks it stored: its own stores, in order
      __threadfence_block();
      w13_wave<uint16_t, CH, FULL>((const uint16_t*)f.x, H, I, f.K, pair, i, 0,
                                   reinterpret_cast<const uint16_t*>(slot), 0,
                                   (uint16_t*)f.act, lane);
    }
  }
  for (int j = 0; j < n; ++j) {
    const int ej = a.loads[2 * j], sj = a.loads[2 * j + 1];
    if (ej < 0 || ej >= a.num_experts || sj < 0 || sj >= a.cap) continue;
    const char* ex = pk.m + (size_t)ej * pk.m_stride;
    unpack_rows_wide<256, 1>(ex + Lp.w2_off, H, I, ex + Lp.exc_off,
                             pk.d2 + (size_t)sj * pk.d2_stride, cb, NCB);
  }
}

// Copy block `cb` (of kPageInBlocks, or NCB with PACKED) of a fused
// page-in + w13 launch (PACKED: from the packed masters).
template <typename T, int CH, bool FULL, bool PACKED = false, int NCB = kPageInBlocks>
__device__ inline void pagein_w13_copy_block(const FusedW13Args& f, const PageInArgs& a, int cb) {
  constexpr int V = Vec<T>::N;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int H = f.H, I = f.I, nch = H / V;
  const int n = *a.count;
  if (a.hist && cb == 0 && threadIdx.x == 0) {
    *a.hist = n;
    __threadfence_system();
  }
  if (n <= 0) return;
  // lane p < K holds the expert pair p's word says was loaded (or -1)
  const int mine = lane < f.K ? pair_word_loaded(f.words[lane]) : -1;
  const PageInPlane& p0 = a.p[0];  // starts with the expert's w13 rows
  const size_t row_bytes = (size_t)H * sizeof(T);
  uint4 xv[CH];
  load_row<T, CH, FULL, false>((const T*)f.x, nch, lane, xv);  // the call's one token
  if constexpr (PACKED && sizeof(T) == 2) {
    pagein_w13_packed<CH, FULL, NCB>(f, a, cb, mine);
    return;
  }
  int jcur = -1, e = -1, s = -1, pair = -1;
  for (int q = cb * 4 + wave; q < n * I; q += kPageInBlocks * 4) {
    const int j = q / I, i = q - j * I;
    if (j != jcur) {
      jcur = j;
      e = a.loads[2 * j];
      s = a.loads[2 * j + 1];
      const uint64_t m = __ballot(mine == e);
      pair = m ? __builtin_ctzll(m) : -1;
    }
    if (e < 0 || e >= a.num_experts || s < 0 || s >= a.cap) continue;
    const u32x4* src_g = reinterpret_cast<const u32x4*>(p0.m + (size_t)e * p0.m_stride +
                                                        (size_t)i * row_bytes);
    const u32x4* src_u = reinterpret_cast<const u32x4*>(p0.m + (size_t)e * p0.m_stride +
                                                        (size_t)(I + i) * row_bytes);
    u32x4* dst_g = reinterpret_cast<u32x4*>(p0.d + (size_t)s * p0.d_stride + (size_t)i * row_bytes);
    u32x4* dst_u = reinterpret_cast<u32x4*>(p0.d + (size_t)s * p0.d_stride +
                                            (size_t)(I + i) * row_bytes);
    // One row at a time, straight from the load registers to the slot and
    // the dot product: 256 copy waves with 4 KiB each in flight keep the
    // host link busy, and the registers stay within the w13 blocks' budget.
    float dot[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const u32x4* src = r ? src_u : src_g;
      u32x4* dst = r ? dst_u : dst_g;
      u32x4 w[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int ch = c * 64 + lane;
        w[c] = (FULL || ch < nch) ? src[ch] : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int ch = c * 64 + lane;
        if (FULL || ch < nch) __builtin_nontemporal_store(w[c], dst + ch);
      }
      dot[r] = pair >= 0 ? row_dot<T, CH>(w, xv) : 0.f;
    }
    if (pair >= 0 && lane == 0) store_elem((T*)f.act + (size_t)pair * I + i, silu(dot[0]) * dot[1]);
  }
  // the rest of each loaded expert: plane 0 past its w13 rows, other planes
  const size_t w13_bytes = 2 * (size_t)I * row_bytes;
  for (int j = 0; j < n; ++j) {
    const int ej = a.loads[2 * j], sj = a.loads[2 * j + 1];
    if (ej < 0 || ej >= a.num_experts || sj < 0 || sj >= a.cap) continue;
    copy_range(p0.m + (size_t)ej * p0.m_stride + w13_bytes,
               p0.d + (size_t)sj * p0.d_stride + w13_bytes, p0.bytes - w13_bytes, cb,
               kPageInBlocks);
    for (int q = 1; q < a.nplanes; ++q) {
      const PageInPlane& pl = a.p[q];
      copy_range(pl.m + (size_t)ej * pl.m_stride, pl.d + (size_t)sj * pl.d_stride, pl.bytes,
                 cb, kPageInBlocks);
    }
  }
}

template <typename T, int CH, bool FULL, bool PACKED, int NCB>
__device__ inline void pagein_w13_body(const FusedW13Args& f, const PageInArgs& a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (blockIdx.x >= NCB) {
    const int I = f.I, nbx = (I + 3) / 4;
    const int local = blockIdx.x - NCB;
    const int pair = local / nbx;
    const int i = (local - pair * nbx) * 4 + wave;
    if (i >= I) return;
    const int32_t word = scalar_word(f.words + pair);
    if (pair_word_loaded(word) >= 0) return;  // the copy blocks compute it
    const int s = pair_word_slot(word);
    w13_wave<T, CH, FULL>((const T*)f.x, f.H, I, f.K, pair, i, s < f.cap ? s : -1,
                          (const T*)f.w13, f.w13_stride, (T*)f.act, lane);
    return;
  }
  pagein_w13_copy_block<T, CH, FULL, PACKED, NCB>(f, a, blockIdx.x);
}

template <typename T, int CH, bool FULL>
__global__ __launch_bounds__(256) void pagein_w13_kernel(FusedW13Args f, PageInArgs a) {
  pagein_w13_body<T, CH, FULL, false, kPageInBlocks>(f, a);
}

// The same launch paging in from packed masters.  The unpack would take
// more registers than the w13 blocks (which then hold fewer waves per SIMD
// than they need to stream their weights in one round), so the launch is
// held at the waves per SIMD the plain launch gets for the same row length.
// Copy blocks of the packed launch: twice the plain launch's, since each
// wave has less of the host link in flight (a packed row is ~3 KiB, and
// the unpack and the read-back of the rows sit between its loads).
// Measured at the Qwen3 decode shape: 51.8 GB/s of link with 64 blocks,
// 54.0 with 128, the same with 192.
constexpr int kPackedPageInBlocks = 128;

constexpr int packed_waves_per_eu(int ch) { return ch <= 3 ? 7 : ch == 4 ? 6 : ch <= 6 ? 4 : 3; }

template <int CH, bool FULL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(packed_waves_per_eu(CH))))
void pagein_w13_packed_kernel(FusedW13Args f, PageInArgs a) {
  pagein_w13_body<uint16_t, CH, FULL, true, kPackedPageInBlocks>(f, a);
}

// ---------------------------------------------------------------------------
// Kernel A'': the whole first half of a one-token call in one launch, for a
// call that fills every slot (top-k == cap, one token: after the pager, the
// slots hold exactly the token's experts) with routing fused:
//   * block 0: the pager (pager_wave, wave 0): routing, the LRU decisions,
//     the pair words and the load list; then it publishes the launch's
//     epoch in `sync` (release at agent scope);
//   * blocks 1 .. kPageInBlocks: Kernel A''s copy blocks, started when they
//     see the epoch (acquire at agent scope): each loaded expert's act rows,
//     per pair, from the bytes they copy;
//   * the other blocks: Kernel A's blocks per (i-block, slot), writing
//     act_spec[s][i] from whatever slot s holds at launch.  They need
//     nothing from the pager, so the routing and the decisions run under
//     their weight stream.  For a slot that this call loads, the value is
//     computed from the old expert (or the bytes being copied) and is never
//     read: the w2 kernel takes the copy blocks' act of that pair instead.
// A call that loads nothing therefore costs the longer of the pager and the
// w13 stream in one launch, where it cost a pager launch and then the w13
// launch.
// ---------------------------------------------------------------------------
// Polls of the epoch word before a copy block gives up (about a second):
// the pager wave never waits on anything, so the word arrives within
// microseconds; the bound only keeps a broken launch from hanging the GPU.
constexpr int kDecodeSpinLimit = 1 << 20;

template <typename T, typename TL, int CH, bool PACKED = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6))) void decode_w13_kernel(FusedW13Args f, PageInArgs a,
                                                         DecodePagerArgs pa) {
  // the pager wave's LDS for at most 128 experts and one token's pairs
  __shared__ PagerSmemT<128> sm;
  __shared__ FusedRouteSmemT<kMaxTopK> fr;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (blockIdx.x == 0) {
    if (wave != 0) return;
    pager_wave<TL, 2, true, 128, kMaxTopK, true>(
        nullptr, (const TL*)pa.logits, pa.renorm, pa.topk_w, pa.topk_ids, 1, f.K, pa.E, f.cap, 0,
        pa.map, pa.s2e, pa.tick, pa.ctr, pa.slots, const_cast<int32_t*>(f.words) - 1, pa.loads,
        pa.rec, nullptr, sm, fr);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    if (lane == 0) __hip_atomic_store(pa.sync, pa.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (blockIdx.x <= kPageInBlocks) {
    __shared__ int seen;
    if (threadIdx.x == 0) {
      int it = 0;
      while (__hip_atomic_load(pa.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != pa.epoch &&
             ++it < kDecodeSpinLimit)
        __builtin_amdgcn_s_sleep(2);
      seen = it < kDecodeSpinLimit;
    }
    __syncthreads();
    if (!seen) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    pagein_w13_copy_block<T, CH, true, PACKED, kPageInBlocks>(f, a, blockIdx.x - 1);
    return;
  }
  const int I = f.I, nbx = (I + 3) / 4;
  const int local = blockIdx.x - 1 - kPageInBlocks;
  const int s = local / nbx;
  const int i = (local - s * nbx) * 4 + wave;
  if (i >= I) return;
  // one token, K == cap: act_spec row s is "pair" s of a call of K pairs
  w13_wave<T, CH, true>((const T*)f.x, f.H, I, f.K, s, i, s, (const T*)f.w13, f.w13_stride,
                        (T*)pa.act_spec, lane);
}

// ---------------------------------------------------------------------------
// Kernel B: out[t, h] = sum_k w[t,k] * dot(W2[s_k][h, :], act[t,k,:]).
// Block = K waves, wave k computes the dot products of expert k for the
// (64/LPR)*RPH rows of this block: LPR lanes per row group, each group RPH
// consecutive rows, CH chunks per lane (or a runtime chunk loop when
// CH == 0).  A group loads its act chunks once for its RPH rows.  The
// partials meet in LDS and one lane per row sums them in routing order, with
// the routing weights staged in LDS by the waves at the start (0 for an
// absent slot).  grid = (ceil(H / ((64 / LPR) * RPH)), T).
//
// Each row's arithmetic (chunk order, then the sum over the LPR lanes,
// then the k-ordered sum) does not depend on RPH, so the row grouping is a
// launch-shape choice only.  Measured on MI355X inside the Qwen3 bs=1 decode
// step (dispatch events, the kernel following the w13 kernel): one row per
// half-wave 5.89 us, two rows 5.78 us; non-temporal weight loads made both
// slower (6.36 and 6.33 us), unlike in the w13 kernel, whose waves read whole
// rows.  A pure read of the same 25 MB in this launch shape takes 5.1-5.3 us.
// ---------------------------------------------------------------------------
constexpr int kMaxKw2 = kGemvMaxTopK;

// The RPH weight rows from h0 of one expert (rows past H read row H - 1 and
// are dropped), CH chunks per lane of an LPR-lane row group.
template <typename T, int LPR, int CH, int RPH, bool FULL>
__device__ inline void w2_load_rows(const T* __restrict__ wbase, int h0, int H, int I, int l,
                                    uint4 (&wv)[RPH][CH]) {
  constexpr int V = Vec<T>::N;
  const int nch = I / V;
#pragma unroll
  for (int r = 0; r < RPH; ++r) {
    const T* wrow = wbase + (size_t)min(h0 + r, H - 1) * I;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int ch = c * LPR + l;
      wv[r][c] = (FULL || ch < nch) ? ld16(wrow + (size_t)ch * V) : make_uint4(0, 0, 0, 0);
    }
  }
}

// This lane's CH act chunks of one act row (chunks past the row read 0).
template <typename T, int LPR, int CH, bool FULL>
__device__ inline void w2_load_act(const T* __restrict__ arow, int I, int l, uint4 (&av)[CH]) {
  constexpr int V = Vec<T>::N;
  const int nch = I / V;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = c * LPR + l;
    av[c] = (FULL || ch < nch) ? ld16(arow + (size_t)ch * V) : make_uint4(0, 0, 0, 0);
  }
}

// This lane's part of the RPH dot products of the rows in wv with the act
// chunks in av: the FMA chain over its chunks in order.
template <typename T, int CH, int RPH>
__device__ inline void w2_dots_av(const uint4 (&wv)[RPH][CH], const uint4 (&av)[CH],
                                  float (&d)[RPH]) {
  constexpr int V = Vec<T>::N;
#pragma unroll
  for (int r = 0; r < RPH; ++r) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      float wf[V], af[V];
      Vec<T>::unpack(wv[r][c], wf);
      Vec<T>::unpack(av[c], af);
#pragma unroll
      for (int q = 0; q < V; ++q) d[r] = fmaf(wf[q], af[q], d[r]);
    }
  }
}

// This lane's part of the RPH dot products of the rows in wv with one act
// row: the FMA chain over its chunks in order.
template <typename T, int LPR, int CH, int RPH, bool FULL>
__device__ inline void w2_dots(const uint4 (&wv)[RPH][CH], const T* __restrict__ arow, int I,
                               int l, float (&d)[RPH]) {
  uint4 av[CH];
  w2_load_act<T, LPR, CH, FULL>(arow, I, l, av);
  w2_dots_av<T, CH, RPH>(wv, av, d);
}

// SLOTS (one token whose top-k equals cap, CH > 0): wave k streams slot k
// instead of pair k's slot.  It issues its row loads right after the pairs'
// slots and weights, without waiting for them, then finds the pair the slot
// serves and dots its rows with that pair's act row.  Each row's arithmetic
// is the same as with one wave per pair, so the output bytes are too.
// Without SPEC the K act rows are staged in LDS first: wave k loads act row
// k before anything else, so the act row a wave dots with comes from LDS
// once the slot table names it, instead of a global load issued only then.
// SPEC (with SLOTS, after Kernel A''): `slots` holds the pager's pair words;
// the act row of slot k is act_spec row k, or the pair's own act row when the
// call loaded that pair's expert (the copy blocks computed it).
template <typename T, int LPR, int CH, int RPH, bool FULL, bool SLOTS, bool SPEC = false>
__global__ __launch_bounds__(1024) void w2_combine_kernel(const T* __restrict__ act, int H, int I,
                                                           int K, const float* __restrict__ topk_w,
                                                           const int32_t* __restrict__ slots,
                                                           const T* __restrict__ w2,
                                                           size_t w2_stride,
                                                           T* __restrict__ out,
                                                           const int32_t* __restrict__ skip_if,
                                                           const T* __restrict__ act_spec,
                                                           int nslots) {
  static_assert(LPR == 32 || LPR == 64, "a row spans half a wave or a whole wave");
  constexpr int V = Vec<T>::N;
  constexpr int RPB = 64 / LPR * RPH;  // rows per block
  constexpr int CHA = CH > 0 ? CH : 1;
  __shared__ float part[kMaxKw2][RPB];
  __shared__ float wk[kMaxKw2];
  // the staged act rows: [k][chunk][lane of a row group]
  constexpr bool kStageAct = SLOTS && !SPEC && CH > 0 && kMaxKw2 * CHA * LPR * 16 <= 32768;
  __shared__ uint4 act_s[kStageAct ? kMaxKw2 * CHA * LPR : 1];
  // every pointer with the first kernel arguments (an empty asm statement
  // that takes them): the skip test below otherwise made the rest a second
  // round trip
  asm volatile("" ::"s"(act), "s"(topk_w), "s"(slots), "s"(w2), "s"(out), "s"(skip_if), "s"(H),
               "s"(I), "s"(K), "s"(w2_stride), "s"(act_spec));
  if (skip_if && *skip_if != 0) return;
  const int k = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane / LPR, l = lane % LPR;
  const int t = blockIdx.y;
  const int h0 = blockIdx.x * RPB + sub * RPH;
  float d[RPH];
#pragma unroll
  for (int r = 0; r < RPH; ++r) d[r] = 0.f;
  int p = k;  // the pair whose dot products this wave computes (-1: none)
  if (SLOTS) {
    // lane j < K: pair j's slot and routing weight
    // (both loaded ahead of the rows, so that waiting for them does not wait
    // for the rows: loads complete in order)
    const int jl = min(lane, K - 1);
    uint4 av_k[CHA];  // act row k (staged)
    if constexpr (kStageAct) {
      w2_load_act<T, LPR, CHA, FULL>(act + ((size_t)t * K + k) * I, I, l, av_k);
      // the act loads stay first: waiting for them waits for nothing after
      __builtin_amdgcn_sched_barrier(0);
    }
    const int32_t wd = load_first(slots + t * K + jl);
    const int sj = SPEC ? pair_word_slot(wd) : wd;
    const float wj = __int_as_float(load_first((const int32_t*)topk_w + t * K + jl));
    uint4 wv[RPH][CHA];
    w2_load_rows<T, LPR, CHA, RPH, FULL>(w2 + (size_t)k * w2_stride, h0, H, I, l, wv);
    // nothing that waits for sj or wj may be scheduled above the row loads
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kStageAct) {
      if (sub == 0) {
#pragma unroll
        for (int c = 0; c < CHA; ++c) act_s[(k * CHA + c) * LPR + l] = av_k[c];
      }
      block_lds_sync();  // every wave's row; the weight rows stay in flight
    }
    const uint64_t mine = __ballot(lane < K && sj == k);
    p = mine ? __builtin_ctzll(mine) : -1;
    const int sk = __shfl(sj, k);
    const float wsk = __shfl(wj, k);
    // unconditional (a wave whose slot serves no pair dots with pair 0's act
    // and drops the result): rows used under a branch would be loaded there
    if constexpr (kStageAct) {
      const int pp = p < 0 ? 0 : p;
      uint4 av[CHA];
#pragma unroll
      for (int c = 0; c < CHA; ++c) av[c] = act_s[(pp * CHA + c) * LPR + l];
      w2_dots_av<T, CHA, RPH>(wv, av, d);
    } else {
      const T* arow = act + ((size_t)t * K + (p < 0 ? 0 : p)) * I;
      if (SPEC) {
        const uint64_t loaded = __ballot(lane < K && pair_word_loaded(wd) >= 0);
        if (!(p >= 0 && ((loaded >> p) & 1ull))) arow = act_spec + (size_t)k * I;
      }
      w2_dots<T, LPR, CHA, RPH, FULL>(wv, arow, I, l, d);
    }
    if (lane == 0) wk[k] = sk >= 0 ? wsk : 0.f;
    if (sk < 0 && l == 0) {  // pair k reads no expert: its partials are 0
#pragma unroll
      for (int r = 0; r < RPH; ++r) part[k][sub * RPH + r] = 0.f;
    }
  } else {
    // a slot outside [0, nslots) reads no expert, as a slot of -1
    const int raw = slots[t * K + k];
    const int s = (unsigned)raw < (unsigned)nslots ? raw : -1;
    if (lane == 0) wk[k] = s >= 0 ? topk_w[t * K + k] : 0.f;
    if (s >= 0 && h0 < H) {
      const T* wbase = w2 + (size_t)s * w2_stride;
      const T* arow = act + ((size_t)t * K + k) * I;
      if (CH > 0) {
        uint4 wv[RPH][CHA];
        w2_load_rows<T, LPR, CHA, RPH, FULL>(wbase, h0, H, I, l, wv);
        w2_dots<T, LPR, CHA, RPH, FULL>(wv, arow, I, l, d);
      } else {
        // long rows (Mixtral's 14336): the lane's chunks in order, each act
        // chunk loaded once for the RPH rows (each row's FMA chain is the
        // same as alone).  Measured at the Mixtral shape: 40.1-40.4 us
        // against 40.7 us for a row at a time with 4 chunks unrolled; two,
        // four or eight rows per wave, or each row split over four waves
        // (all its loads in flight, partial sums in order), were no faster.
        const int nch = I / V;
        const T* wrow[RPH];
#pragma unroll
        for (int r = 0; r < RPH; ++r) wrow[r] = wbase + (size_t)min(h0 + r, H - 1) * I;
#pragma unroll 2
        for (int ch = l; ch < nch; ch += LPR) {
          float af[V];
          Vec<T>::unpack(ld16(arow + (size_t)ch * V), af);
#pragma unroll
          for (int r = 0; r < RPH; ++r) {
            float wf[V];
            Vec<T>::unpack(ld16(wrow[r] + (size_t)ch * V), wf);
#pragma unroll
            for (int q = 0; q < V; ++q) d[r] = fmaf(wf[q], af[q], d[r]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPH; ++r) d[r] = LPR == 64 ? wave_sum_f32(d[r]) : half_sum_f32(d[r]);
  if (l == 0 && p >= 0) {
#pragma unroll
    for (int r = 0; r < RPH; ++r) part[p][sub * RPH + r] = d[r];
  }
  __syncthreads();
  if (threadIdx.x < RPB) {
    const int r = threadIdx.x;
    const int hh = blockIdx.x * RPB + r;
    if (hh < H) {
      float acc = 0.f;
      for (int kk = 0; kk < K; ++kk) acc = fmaf(wk[kk], part[kk][r], acc);
      store_elem(out + (size_t)t * H + hh, acc);
    }
  }
}

// Optional controls of a launch: kernel timing events, the pair filter of
// the w13 kernel (run only pairs with pair_filter[p] == want) and the skip
// word of the w2 kernel (exit when *skip_if != 0), and the w2 kernel's
// one-wave-per-slot layout (a one-token call whose top-k equals cap).
struct LaunchCtl {
  hipEvent_t start = nullptr, stop = nullptr;
  const int32_t* pair_filter = nullptr;
  int want = 0;
  const int32_t* skip_if = nullptr;
  bool slots = false;
  const void* act_spec = nullptr;  // with slots: the w2 kernel's SPEC mode
  int nslots = 0;                  // slot ids at or above it read no expert
};

template <typename T, int CH>
void launch_w13(const T* x, int T_, int H, int I, int K, const int32_t* slots, const T* w13,
                size_t w13_stride, T* act, hipStream_t st, const LaunchCtl& c) {
  dim3 grid((I + 3) / 4, T_ * K);
  if (H == CH * 64 * Vec<T>::N)
    launch_timed(w13_silu_kernel<T, CH, true>, grid, dim3(256), st, c.start, c.stop, x, H, I, K,
                 slots, w13, w13_stride, act, c.pair_filter, c.want, c.nslots);
  else
    launch_timed(w13_silu_kernel<T, CH, false>, grid, dim3(256), st, c.start, c.stop, x, H, I, K,
                 slots, w13, w13_stride, act, c.pair_filter, c.want, c.nslots);
}

template <typename T, int CH>
void launch_pagein_w13(const PageInArgs& a, const FusedW13Args& f, hipStream_t st,
                       hipEvent_t ev_start, hipEvent_t ev_stop) {
  const dim3 grid(kPageInBlocks + (f.I + 3) / 4 * f.K);
  const bool full = f.H == CH * 64 * Vec<T>::N;
  if constexpr (sizeof(T) == 2) {
    if (a.pk.m) {
      const dim3 grid(kPackedPageInBlocks + (f.I + 3) / 4 * f.K);
      if (full)
        launch_timed(pagein_w13_packed_kernel<CH, true>, grid, dim3(256), st, ev_start, ev_stop,
                     f, a);
      else
        launch_timed(pagein_w13_packed_kernel<CH, false>, grid, dim3(256), st, ev_start,
                     ev_stop, f, a);
      return;
    }
  }
  if (full)
    launch_timed(pagein_w13_kernel<T, CH, true>, grid, dim3(256), st, ev_start, ev_stop, f, a);
  else
    launch_timed(pagein_w13_kernel<T, CH, false>, grid, dim3(256), st, ev_start, ev_stop, f, a);
}

template <typename T, typename TL, int CH>
void launch_decode_w13(const PageInArgs& a, const FusedW13Args& f, const DecodePagerArgs& pa,
                       hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
  const dim3 grid(1 + kPageInBlocks + (f.I + 3) / 4 * f.cap);
  if (sizeof(T) == 2 && a.pk.m)
    launch_timed(decode_w13_kernel<T, TL, CH, true>, grid, dim3(256), st, ev_start, ev_stop, f, a,
                 pa);
  else
    launch_timed(decode_w13_kernel<T, TL, CH>, grid, dim3(256), st, ev_start, ev_stop, f, a, pa);
}

// The per-lane chunk count of the w13 kernels for a row of H elements (0 when
// a row is longer than 8 chunks per lane).
template <typename T>
int w13_chunks(int H) {
  const int ch = (H / Vec<T>::N + 63) / 64;
  return ch <= 4 ? ch : ch <= 6 ? 6 : ch <= 8 ? 8 : 0;
}

template <typename T>
int dispatch_w13(const T* x, int T_, int H, int I, int K, const int32_t* slots, const T* w13,
                 size_t w13_stride, T* act, hipStream_t st, const LaunchCtl& c) {
  switch (w13_chunks<T>(H)) {
    case 1: launch_w13<T, 1>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 2: launch_w13<T, 2>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 3: launch_w13<T, 3>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 4: launch_w13<T, 4>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 6: launch_w13<T, 6>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 8: launch_w13<T, 8>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    default: return WISP_ERR_UNSUPPORTED;
  }
  return WISP_OK;
}

template <typename T>
int dispatch_pagein_w13(const PageInArgs& a, const FusedW13Args& f, hipStream_t st,
                        hipEvent_t ev_start, hipEvent_t ev_stop) {
  switch (w13_chunks<T>(f.H)) {
    case 1: launch_pagein_w13<T, 1>(a, f, st, ev_start, ev_stop); break;
    case 2: launch_pagein_w13<T, 2>(a, f, st, ev_start, ev_stop); break;
    case 3: launch_pagein_w13<T, 3>(a, f, st, ev_start, ev_stop); break;
    case 4: launch_pagein_w13<T, 4>(a, f, st, ev_start, ev_stop); break;
    case 6: launch_pagein_w13<T, 6>(a, f, st, ev_start, ev_stop); break;
    case 8: launch_pagein_w13<T, 8>(a, f, st, ev_start, ev_stop); break;
    default: return WISP_ERR_UNSUPPORTED;
  }
  return WISP_OK;
}

// Kernel A'' for whole rows of 2 or 4 chunks per lane (the other shapes keep
// the separate pager launch: at 8 chunks the launch's 80 VGPRs spill).
template <typename T, typename TL>
int dispatch_decode_w13(const PageInArgs& a, const FusedW13Args& f, const DecodePagerArgs& pa,
                        hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
  const int ch = w13_chunks<T>(f.H);
  if (f.H != ch * 64 * Vec<T>::N) return WISP_ERR_UNSUPPORTED;
  switch (ch) {
    case 2: launch_decode_w13<T, TL, 2>(a, f, pa, st, ev_start, ev_stop); break;
    case 4: launch_decode_w13<T, TL, 4>(a, f, pa, st, ev_start, ev_stop); break;
    default: return WISP_ERR_UNSUPPORTED;
  }
  return WISP_OK;
}

template <typename T, int LPR, int CH, int RPH = 1>
void launch_w2(const T* act, int T_, int H, int I, int K, const float* w, const int32_t* slots,
               const T* w2, size_t w2_stride, T* out, hipStream_t st, const LaunchCtl& c) {
  constexpr int RPB = 64 / LPR * RPH;
  dim3 grid((H + RPB - 1) / RPB, T_);
  const bool full = CH > 0 && I == CH * LPR * Vec<T>::N;
  const T* spec = (const T*)c.act_spec;
  if (CH > 0 && c.slots && spec) {
    if (full)
      launch_timed(w2_combine_kernel<T, LPR, CH, RPH, true, true, true>, grid, dim3(64 * K), st,
                   c.start, c.stop, act, H, I, K, w, slots, w2, w2_stride, out, c.skip_if, spec, c.nslots);
    else
      launch_timed(w2_combine_kernel<T, LPR, CH, RPH, false, true, true>, grid, dim3(64 * K),
                   st, c.start, c.stop, act, H, I, K, w, slots, w2, w2_stride, out, c.skip_if,
                   spec, c.nslots);
  } else if (CH > 0 && c.slots) {
    if (full)
      launch_timed(w2_combine_kernel<T, LPR, CH, RPH, true, true>, grid, dim3(64 * K), st,
                   c.start, c.stop, act, H, I, K, w, slots, w2, w2_stride, out, c.skip_if, spec, c.nslots);
    else
      launch_timed(w2_combine_kernel<T, LPR, CH, RPH, false, true>, grid, dim3(64 * K), st,
                   c.start, c.stop, act, H, I, K, w, slots, w2, w2_stride, out, c.skip_if, spec, c.nslots);
  } else if (full) {
    launch_timed(w2_combine_kernel<T, LPR, CH, RPH, true, false>, grid, dim3(64 * K), st,
                 c.start, c.stop, act, H, I, K, w, slots, w2, w2_stride, out, c.skip_if, spec, c.nslots);
  } else {
    launch_timed(w2_combine_kernel<T, LPR, CH, RPH, false, false>, grid, dim3(64 * K), st,
                 c.start, c.stop, act, H, I, K, w, slots, w2, w2_stride, out, c.skip_if, spec, c.nslots);
  }
}

template <typename T>
int dispatch_w2(const T* act, int T_, int H, int I, int K, const float* w, const int32_t* slots,
                const T* w2, size_t w2_stride, T* out, hipStream_t st, const LaunchCtl& c) {
  if (K > kMaxKw2) return WISP_ERR_UNSUPPORTED;
  const int nch = I / Vec<T>::N;
  if (nch <= 32 * 4) {  // half a wave per row group of two rows, up to 4 chunks per lane
    switch ((nch + 31) / 32) {
      case 1: launch_w2<T, 32, 1, 2>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
      case 2: launch_w2<T, 32, 2, 2>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
      case 3: launch_w2<T, 32, 3, 2>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
      default: launch_w2<T, 32, 4, 2>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
    }
  } else {
    launch_w2<T, 64, 0>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c);
  }
  return WISP_OK;
}

}  // namespace

// Shapes the GEMV pair covers: the w13 kernel holds up to 8 chunks of 16
// bytes of a row per lane (H up to 4096 bf16 / 2048 fp32 elements), and the
// w2 kernel runs one wave per routed expert in a block of at most 16 waves.
bool gemv_supported(int dtype, int H, int K) {
  const int V = dtype == WISP_F32 ? 4 : 8;
  const int ch = (H / V + 63) / 64;
  return K >= 1 && K <= kMaxKw2 && ch >= 1 && ch <= 8;
}

// The fused page-in + w13 launch (Kernel A'): `a` as for the copy kernel,
// with a.count the pager's flags word; plane 0 of `a` must start with the
// expert's w13 rows.
int pagein_w13(const PageInArgs& a, const void* x, int dtype, int T_, int H, int I, int K,
               const int32_t* flags, const void* w13, size_t w13_stride, void* act,
               hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop) {
  if (T_ != 1) {
    wisp_set_last_error("the fused page-in + w13 launch serves one-token calls",
                        "page-in + w13 kernel");
    return WISP_ERR_INVALID;
  }
  FusedW13Args f{x, flags + 1, w13, w13_stride, act, H, I, K, a.cap};
  const int rc = dtype == WISP_F32 ? dispatch_pagein_w13<float>(a, f, st, ev_start, ev_stop)
                                   : dispatch_pagein_w13<uint16_t>(a, f, st, ev_start, ev_stop);
  if (rc != WISP_OK) {
    wisp_set_last_error("hidden size outside the GEMV kernels' coverage", "page-in + w13 kernel");
    return rc;
  }
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

// Whether Kernel A'' serves a layer: a one-token call with top-k == cap <=
// 64, at most 128 experts, rows of 2 or 4 chunks per lane.
bool decode_w13_supported(int dtype, int H, int E, int K, int cap) {
  const int V = dtype == WISP_F32 ? 4 : 8;
  const int ch = H / V / 64;
  return K == cap && cap <= 64 && E <= 128 && H % (64 * V) == 0 && (ch == 2 || ch == 4);
}

// Kernel A'': `a` as for pagein_w13 (a.count = flags), pager arguments in pa.
int decode_w13(const PageInArgs& a, const void* x, int dtype, int logits_dtype, int H, int I,
               int K, int32_t* flags, const void* w13, size_t w13_stride, void* act,
               const DecodePagerArgs& pa, hipStream_t st, hipEvent_t ev_start,
               hipEvent_t ev_stop) {
  FusedW13Args f{x, flags + 1, w13, w13_stride, act, H, I, K, a.cap};
  int rc;
  if (dtype == WISP_F32)
    rc = logits_dtype == WISP_BF16
             ? dispatch_decode_w13<float, uint16_t>(a, f, pa, st, ev_start, ev_stop)
             : dispatch_decode_w13<float, float>(a, f, pa, st, ev_start, ev_stop);
  else
    rc = logits_dtype == WISP_BF16
             ? dispatch_decode_w13<uint16_t, uint16_t>(a, f, pa, st, ev_start, ev_stop)
             : dispatch_decode_w13<uint16_t, float>(a, f, pa, st, ev_start, ev_stop);
  if (rc != WISP_OK) {
    wisp_set_last_error("hidden size outside the fused decode launch's coverage",
                        "decode w13 kernel");
    return rc;
  }
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

int gemv_w13(const void* x, int dtype, int T_, int H, int I, int K, const int32_t* slots,
             int nslots, const void* w13, size_t w13_stride, void* act, hipStream_t st,
             hipEvent_t ev_start, hipEvent_t ev_stop, const int32_t* pair_filter, int want) {
  if (T_ == 0) return WISP_OK;
  LaunchCtl c;
  c.nslots = nslots;
  c.start = ev_start;
  c.stop = ev_stop;
  c.pair_filter = pair_filter;
  c.want = want;
  const int rc = dtype == WISP_F32
      ? dispatch_w13<float>((const float*)x, T_, H, I, K, slots, (const float*)w13, w13_stride,
                            (float*)act, st, c)
      : dispatch_w13<uint16_t>((const uint16_t*)x, T_, H, I, K, slots, (const uint16_t*)w13,
                               w13_stride, (uint16_t*)act, st, c);
  if (rc != WISP_OK) {
    wisp_set_last_error("hidden size outside the GEMV kernels' coverage", "w13 kernel");
    return rc;
  }
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

// With `cap` > 0, a one-token call whose top-k equals cap uses every slot
// and runs the w2 kernel one wave per slot (cap 0: one wave per pair).
int gemv_w2(const void* act, int dtype, int T_, int H, int I, int K, const float* topk_w,
            const int32_t* slots, int nslots, const void* w2, size_t w2_stride, void* out,
            hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop, const int32_t* skip_if,
            int cap, const void* act_spec) {
  if (T_ == 0) return WISP_OK;
  LaunchCtl c;
  c.nslots = nslots;
  c.start = ev_start;
  c.stop = ev_stop;
  c.skip_if = skip_if;
  c.slots = T_ == 1 && K == cap;
  c.act_spec = c.slots ? act_spec : nullptr;
  const int rc = dtype == WISP_F32
      ? dispatch_w2<float>((const float*)act, T_, H, I, K, topk_w, slots, (const float*)w2,
                           w2_stride, (float*)out, st, c)
      : dispatch_w2<uint16_t>((const uint16_t*)act, T_, H, I, K, topk_w, slots,
                              (const uint16_t*)w2, w2_stride, (uint16_t*)out, st, c);
  if (rc != WISP_OK) {
    wisp_set_last_error("top_k above 16 is outside the GEMV kernels' coverage", "w2 kernel");
    return rc;
  }
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

int experts_gemv(const void* x, int dtype, int T_, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                 const void* w2, size_t w2_stride, void* act, void* out, hipStream_t st,
                 const StageEvents* ev) {
  int rc = gemv_w13(x, dtype, T_, H, I, K, slots, nslots, w13, w13_stride, act, st,
                    ev ? ev->ev[0] : nullptr, ev ? ev->ev[1] : nullptr, nullptr, 0);
  if (rc != WISP_OK) return rc;
  return gemv_w2(act, dtype, T_, H, I, K, topk_w, slots, nslots, w2, w2_stride, out, st,
                 ev ? ev->ev[2] : nullptr, ev ? ev->ev[3] : nullptr, nullptr, 0, nullptr);
}

}  // namespace wisp
