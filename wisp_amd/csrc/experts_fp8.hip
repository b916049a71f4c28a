// Block-FP8 (w8a8) expert kernels for decode and small batches on gfx950.
//
// Replaces vLLM's fused_experts with an fp8_w8a8 block quant config, as the
// reference's FP8 path calls it on the Triton backend
// (src/wisp/integrations/vllm/fused_moe_fp8.py:245-249, 316-326):
//   x quantised per token and 128-column group (per_token_group_quant_fp8):
//     s = max(max|x_g|, 1e-10) / 448,  q = e4m3fn(clamp(x / s, -448, 448))
//   h = bf16(sum_kb (dot(q_x[kb], W13[n, kb]) * s_x[kb]) * S13[n / bn][kb])
//   act = bf16(bf16(silu(gate)) * up)                         (silu_and_mul)
//   y_k = bf16((W2-stage sum on the quantised act) * topk_w[t, k])
//   out[t] = moe_sum_k y_k: bf16 adds for K in {2, 3, 4}, otherwise one
//            float32 sum rounded once; k ascending.
//
// Both GEMMs run on v_mfma_f32_16x16x128_f8f6f4.  One instruction multiplies
// a 16-row weight tile by up to 16 activation columns over one 128-wide
// k-block, which is exactly one block of the weight scales, so the scaling
// happens once per instruction result, in the order vLLM's kernel uses:
//   acc += (D * s_act[column]) * s_w[tile's row block][kb]
// Operand layout (checked on MI355X): lane l feeds row (A) / column (B)
// l % 16 with the 32 consecutive k at 32 * (l / 16); the result lane l holds
// rows 4 * (l / 16) + j, j < 4, of column l % 16.  The instruction does not
// round like an exact float32 sum (measured: up to ~1e-4 of the largest
// result on full-range codes), but it is deterministic and its result for
// one output does not depend on the other columns, so outputs depend only on
// the pair's token and the weights read: paged and resident runs agree byte
// for byte.
//
// w13 kernel: grid (I / 16 row tiles, T*K pairs).  The block of the lowest
// pair routed to a slot computes every pair of that slot, up to NCOL per
// MFMA column set, and the other pairs' blocks exit, so each weight tile is
// read once per launch.  NW waves split the k-blocks of H; each wave
// quantises the activation groups it consumes into its own LDS slice, so no
// separate quantisation launch precedes the GEMM.  Partial sums meet in LDS
// in wave order; the epilogue rounds gate and up to bf16 and applies
// silu_and_mul with vLLM's roundings.
//
// w2 kernel: grid (H / 16 row tiles, T tokens).  The block quantises the
// token's K act rows into LDS, waves take (pair, k-range) jobs over I, and
// the block scales each pair by its routing weight, rounds to bf16 and sums
// the K results in routing order.
#include <type_traits>

#include "common.h"
#include "dma_pipeline.h"
#include "pagein.h"
#include "pager_core.h"

#pragma clang fp contract(off)  // keep vLLM's separate multiply and add roundings

namespace wisp {

int experts_fp8(const void* x, int T, int H, int I, int K, const float* topk_w,
                const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                const float* s13, size_t s13_stride, const void* w2, size_t w2_stride,
                const float* s2, size_t s2_stride, int block_n, void* act, void* out,
                hipStream_t st, const StageEvents* ev, bool pager_slots);
const char* fp8_unsupported(int H, int I, int K, int block_n, int block_k);
int experts_fp8_grouped(const void* x, int T, int H, int I, int K, const float* topk_w,
                        const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                        const float* s13, size_t s13_stride, const void* w2, size_t w2_stride,
                        const float* s2, size_t s2_stride, int block_n, void* act, void* out,
                        void* work, size_t work_bytes, hipStream_t st, const StageEvents* ev);
size_t fp8_work_bytes(int T, int K, int H, int I, int nslots);
int auto_algo(int dtype, int H, int I, int T, int K);
int experts_fp8_w2(const void* act, int T, int H, int I, int K, const float* topk_w,
                   const int32_t* slots, int nslots, const void* w2, size_t w2_stride,
                   const float* s2, size_t s2_stride, int block_n, void* out, hipStream_t st,
                   hipEvent_t e0, hipEvent_t e1, bool pager_slots);
int pagein_fp8_w13(const PageInArgs& a, const void* x, int H, int I, int K,
                   const int32_t* slots, const int32_t* flags, int nslots, const void* w13,
                   size_t w13_stride, const float* s13, size_t s13_stride, int block_n,
                   size_t s13_off, void* act, hipStream_t st, hipEvent_t e0, hipEvent_t e1,
                   bool pager_slots);

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr float kE4m3Max = 448.f;
constexpr float kQuantEps = 1e-10f;
constexpr int kKB = 128;         // k-block: the MFMA's K and the scale block's width
constexpr int kKC = 4;           // k-blocks a w13 wave loads before it computes
constexpr int kW2Waves = 8;
constexpr size_t kMaxLds = 160 * 1024;

__device__ inline float round_bf16(float f) { return bf16f(bf16_rne(f)); }

// Four values as bf16 to the 8 consecutive, 8-byte aligned bytes at p, in
// one store (an MFMA lane holds four consecutive output columns).
__device__ inline void store_bf16x4(uint16_t* p, float a, float b, float c, float d) {
  *reinterpret_cast<uint2*>(p) =
      make_uint2((uint32_t)bf16_rne(a) | ((uint32_t)bf16_rne(b) << 16),
                 (uint32_t)bf16_rne(c) | ((uint32_t)bf16_rne(d) << 16));
}

// act = bf16(bf16(silu(bf16(g))) * bf16(u)) for four consecutive columns.
__device__ inline void store_act4(uint16_t* p, const f32x4& g, const f32x4& u) {
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float hg = round_bf16(g[j]), hu = round_bf16(u[j]);
    v[j] = round_bf16(silu(hg)) * hu;
  }
  store_bf16x4(p, v[0], v[1], v[2], v[3]);
}

__device__ inline f32x4 mfma_fp8(const i32x8& a, const i32x8& b) {
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  // formats 0/0: both operands e4m3; zero scale operands select the
  // unscaled instruction
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

__device__ inline i32x8 join(const u32x4& a, const u32x4& b) {
  i32x8 r;
  r[0] = (int)a.x; r[1] = (int)a.y; r[2] = (int)a.z; r[3] = (int)a.w;
  r[4] = (int)b.x; r[5] = (int)b.y; r[6] = (int)b.z; r[7] = (int)b.w;
  return r;
}

// 32 bytes of a weight row.  Plain loads: with the nontemporal hint the
// decode kernels ran ~1.4 us slower each (measured on MI355X at the Qwen3
// shape), and the register-streaming grouped kernels 24.4 -> 28.3 us (w13)
// and 11.7 -> 13.4 us (w2) per ~4-token group of 32 slots; unlike the bf16
// GEMV, whose rows are read whole by one wave, and the global->LDS copies.
__device__ inline i32x8 ld32(const uint8_t* p) {
  const u32x4 a = *reinterpret_cast<const u32x4*>(p);
  const u32x4 b = *reinterpret_cast<const u32x4*>(p + 16);
  return join(a, b);
}

__device__ inline i32x8 lds32(const uint8_t* p) {
  return join(*reinterpret_cast<const u32x4*>(p), *reinterpret_cast<const u32x4*>(p + 16));
}

// 32 bytes to p (16-byte aligned) by two non-temporal 16-byte stores.
__device__ inline void st32_nt(uint8_t* p, const i32x8& v) {
  const u32x4 lo = {(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
  const u32x4 hi = {(uint32_t)v[4], (uint32_t)v[5], (uint32_t)v[6], (uint32_t)v[7]};
  __builtin_nontemporal_store(lo, reinterpret_cast<u32x4*>(p));
  __builtin_nontemporal_store(hi, reinterpret_cast<u32x4*>(p + 16));
}

__device__ inline i32x8 zero8() {
  i32x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = 0;
  return r;
}

// Max over the 16 lanes of this lane's quarter-wave (one DPP row).
__device__ inline float quarter_max(float v) { return row16_max_f32(v); }

// Quantises one 128-value group held 8 values per lane by the 16 lanes of a
// quarter-wave (per_token_group_quant_fp8): returns the scale and the 8 codes
// of this lane as two words (code of value i in byte i).
__device__ inline float quant8(const float* v, uint32_t* q) {
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
  m = quarter_max(m);
  const float s = fmaxf(m, kQuantEps) / kE4m3Max;
  float c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = fminf(fmaxf(v[i] / s, -kE4m3Max), kE4m3Max);
  int w0 = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
  w0 = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], w0, true);
  int w1 = __builtin_amdgcn_cvt_pk_fp8_f32(c[4], c[5], 0, false);
  w1 = __builtin_amdgcn_cvt_pk_fp8_f32(c[6], c[7], w1, true);
  q[0] = (uint32_t)w0;
  q[1] = (uint32_t)w1;
  return s;
}

__device__ inline void unpack_bf16x8(const u32x4& u, float* f) {
  f[0] = bf16f(u.x & 0xffffu); f[1] = bf16f(u.x >> 16);
  f[2] = bf16f(u.y & 0xffffu); f[3] = bf16f(u.y >> 16);
  f[4] = bf16f(u.z & 0xffffu); f[5] = bf16f(u.z >> 16);
  f[6] = bf16f(u.w & 0xffffu); f[7] = bf16f(u.w >> 16);
}

// ---------------------------------------------------------------------------
// Standalone group quantiser: one quarter-wave per 128-value group.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void quant_groups_kernel(const T* __restrict__ x, int rows,
                                                           int cols, uint8_t* __restrict__ q,
                                                           float* __restrict__ scales) {
  const int ng = cols / kKB;
  const long job = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  if (job >= (long)rows * ng) return;
  const int r = (int)(job / ng), g = (int)(job % ng), sub = threadIdx.x & 15;
  const size_t off = (size_t)r * cols + (size_t)g * kKB + sub * 8;
  float v[8];
  if constexpr (sizeof(T) == 2) {
    unpack_bf16x8(*reinterpret_cast<const u32x4*>(x + off), v);
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4*>(x + off);
    const u32x4 b = *reinterpret_cast<const u32x4*>(x + off + 4);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
    v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
    v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  }
  uint32_t c[2];
  const float s = quant8(v, c);
  *reinterpret_cast<uint2*>(q + off) = make_uint2(c[0], c[1]);
  if (sub == 0) scales[(size_t)r * ng + g] = s;
}

// ---------------------------------------------------------------------------
// The launch's slot table.  Up to kPairRegs * 64 pairs it is read once into
// registers (lane l holds pairs l, 64 + l, ...), so a block knows its slot,
// whether it leads and its column set after one memory round trip; larger
// launches (BIG) scan it in memory.
// ---------------------------------------------------------------------------
constexpr int kPairRegs = 4;

template <bool BIG>
__device__ inline void load_pairs(const int32_t* __restrict__ slots, int P, int lane,
                                  int (&v)[kPairRegs]) {
  // unguarded loads at clamped indices (no exec-masked branches), masked after
  int raw[kPairRegs];
#pragma unroll
  for (int c = 0; c < kPairRegs; ++c) raw[c] = BIG ? -1 : slots[min(c * 64 + lane, P - 1)];
#pragma unroll
  for (int c = 0; c < kPairRegs; ++c) v[c] = (!BIG && c * 64 + lane < P) ? raw[c] : -1;
}

// Slot of pair p (wave-uniform).
template <bool BIG>
__device__ inline int slot_of(const int32_t* __restrict__ slots, const int (&v)[kPairRegs],
                              int p) {
  if constexpr (BIG) {
    return slots[p];
  } else {
    int r = -1;
#pragma unroll
    for (int c = 0; c < kPairRegs; ++c)
      if (p / 64 == c) r = __builtin_amdgcn_readlane(v[c], p % 64);
    return r;
  }
}

// Pair index of rank `rank` (per lane) among the pairs routed to slot s >= 0
// (-1 if none), and their number.
template <bool BIG>
__device__ inline int pair_of_rank(const int32_t* __restrict__ slots, const int (&v)[kPairRegs],
                                   int P, int s, int rank, int lane, int* total) {
  int found = -1, seen = 0;
  auto step = [&](int b, bool m) {
    unsigned long long bal = __ballot(m);
    const int c = __popcll(bal);
    const int want = rank - seen;
    if (found < 0 && want >= 0 && want < c) {
      for (int i = 0; i < want; ++i) bal &= bal - 1;
      found = b + __ffsll((long long)bal) - 1;
    }
    seen += c;
  };
  if constexpr (BIG) {
    for (int b = 0; b < P; b += 64) {
      const int q = b + lane;
      step(b, q < P && slots[q] == s);
    }
  } else {
#pragma unroll
    for (int c = 0; c < kPairRegs; ++c) step(c * 64, v[c] == s);  // -1 past P never matches
  }
  *total = seen;
  return found;
}

// ---------------------------------------------------------------------------
// w13 + silu_and_mul.
// NCOL: MFMA columns per pass over the weights (1 for a one-token launch, 4,
// or 16), a compile-time width so that every load is unguarded: a column or
// k-block past the live ones loads a clamped copy that is never stored.
// Dynamic LDS: red [NW][2][64][4] f32, then per wave xs [kKC][NCOL] f32 and
// xq [kKC][NCOL][kKB] codes.
// ---------------------------------------------------------------------------
template <int NW, int NCOL, bool BIG>
__global__ __launch_bounds__(NW * 64) void fp8_w13_kernel(
    const uint16_t* __restrict__ x, int H, int I, int K, int P, const int32_t* __restrict__ slots,
    int nslots, const uint8_t* __restrict__ w13, size_t w13_stride, const float* __restrict__ s13,
    size_t s13_stride, int block_n, uint16_t* __restrict__ act) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* red = reinterpret_cast<float*>(smem);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int p = blockIdx.y, i0 = blockIdx.x * 16;
  int sv[kPairRegs];
  load_pairs<BIG>(slots, P, lane, sv);
  const int s = slot_of<BIG>(slots, sv, p);
  if (s < 0 || s >= nslots) {  // this pair reads no expert
    if (threadIdx.x < 16) act[(size_t)p * I + i0 + threadIdx.x] = 0;
    return;
  }
  int total = 0;
  if (pair_of_rank<BIG>(slots, sv, P, s, 0, lane, &total) != p) return;  // not the leader

  float* xs = reinterpret_cast<float*>(smem + NW * 2 * 64 * 4 * sizeof(float) +
                                       (size_t)wave * kKC * NCOL * (4 + kKB));
  uint8_t* xq = reinterpret_cast<uint8_t*>(xs + kKC * NCOL);
  const int nkb = H / kKB;
  const int per = (nkb + NW - 1) / NW;
  const int kb0 = min(nkb, wave * per), kb1 = min(nkb, kb0 + per);
  const uint8_t* W = w13 + (size_t)s * w13_stride;
  const float* Sg = s13 + (size_t)s * s13_stride + (size_t)(i0 / block_n) * nkb;
  const float* Su = s13 + (size_t)s * s13_stride + (size_t)((I + i0) / block_n) * nkb;
  const uint8_t* rowg = W + (size_t)(i0 + col) * H + grp * 32;
  const uint8_t* rowu = W + (size_t)(I + i0 + col) * H + grp * 32;

  for (int rank0 = 0; rank0 < total; rank0 += NCOL) {
    const int npc = min(NCOL, total - rank0);
    // column `col` of this set computes the pair of rank rank0 + col (every
    // lane runs the ballots; lanes past the set's width get -1)
    const int r = pair_of_rank<BIG>(slots, sv, P, s, rank0 + col, lane, &total);
    const int mypair = col < npc ? r : -1;
    const int mytok = mypair >= 0 ? mypair / K : 0;
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    for (int kc = kb0; kc < kb1; kc += kKC) {
      const int nk = min(kKC, kb1 - kc);
      // activations: pass c quantises column c, quarter-wave g its k-block g
      // (lane & 15 is then the lane's eighth of the 128-value group); the
      // activation loads go first, then the weights and scales, so the
      // quantisation waits only for the activations
      u32x4 xv[NCOL];
#pragma unroll
      for (int c = 0; c < NCOL; ++c) {
        const int tok = __builtin_amdgcn_readlane(mytok, min(c, npc - 1));
        xv[c] = *reinterpret_cast<const u32x4*>(x + (size_t)tok * H +
                                                (size_t)(kc + min(grp, nk - 1)) * kKB + col * 8);
      }
      i32x8 wg[kKC], wu[kKC];
      float sg[kKC], su[kKC];
#pragma unroll
      for (int kbi = 0; kbi < kKC; ++kbi) {
        const int kb = kc + min(kbi, nk - 1);
        wg[kbi] = ld32(rowg + (size_t)kb * kKB);
        wu[kbi] = ld32(rowu + (size_t)kb * kKB);
        sg[kbi] = Sg[kb];
        su[kbi] = Su[kb];
      }
#pragma unroll
      for (int c = 0; c < NCOL; ++c) {
        float v[8];
        unpack_bf16x8(xv[c], v);
        uint32_t q[2];
        const float sc = quant8(v, q);
        if (c < npc && grp < nk) {
          *reinterpret_cast<uint2*>(xq + ((size_t)grp * NCOL + c) * kKB + col * 8) =
              make_uint2(q[0], q[1]);
          if (col == 0) xs[grp * NCOL + c] = sc;
        }
      }
      wave_lds_sync();
#pragma unroll
      for (int kbi = 0; kbi < kKC; ++kbi) {
        if (kbi < nk) {
          const i32x8 b = col < npc ? lds32(xq + ((size_t)kbi * NCOL + col) * kKB + grp * 32)
                                    : zero8();
          const float sa = col < npc ? xs[kbi * NCOL + col] : 0.f;
          const f32x4 dg = mfma_fp8(wg[kbi], b);
          const f32x4 du = mfma_fp8(wu[kbi], b);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            ag[j] = ag[j] + (dg[j] * sa) * sg[kbi];
            au[j] = au[j] + (du[j] * sa) * su[kbi];
          }
        }
      }
      wave_lds_sync();  // the slice is rewritten by the next chunk
    }
    float* rw = red + ((size_t)wave * 2 * 64 + lane) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      rw[j] = ag[j];
      rw[64 * 4 + j] = au[j];
    }
    __syncthreads();
    if (wave == 0 && col < npc) {
      float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
      for (int w = 0; w < NW; ++w) {
        const float* rr = red + ((size_t)w * 2 * 64 + lane) * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          g[j] = g[j] + rr[j];
          u[j] = u[j] + rr[64 * 4 + j];
        }
      }
      store_act4(act + (size_t)mypair * I + i0 + grp * 4, f32x4{g[0], g[1], g[2], g[3]},
                 f32x4{u[0], u[1], u[2], u[3]});
    }
    __syncthreads();  // red is rewritten by the next column set
  }
}

// The NW waves' partial sums of this lane's four gate and four up outputs
// (red [NW][2][64][4] f32), added in wave order to zero, read four waves at
// a time: all eight at once would hold 64 registers (one 512-thread block per
// CU), one at a time would make eight LDS round trips.
template <int NW>
__device__ inline void sum_partials(const float* red, int lane, f32x4& g, f32x4& u) {
  g = f32x4{0.f, 0.f, 0.f, 0.f};
  u = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int w0 = 0; w0 < NW; w0 += 4) {
    f32x4 pg[4], pu[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = min(w0 + i, NW - 1);
      pg[i] = *reinterpret_cast<const f32x4*>(red + ((size_t)w * 2 * 64 + lane) * 4);
      pu[i] = *reinterpret_cast<const f32x4*>(red + ((size_t)w * 2 * 64 + 64 + lane) * 4);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (w0 + i < NW) {
        g = g + pg[i];
        u = u + pu[i];
      }
    }
  }
}

// A word loaded before the loads that follow it in the source: the compiler
// neither sinks nor reorders a relaxed atomic load (plain loads of
// restrict-qualified data it may move below later loads).
__device__ inline int32_t load_first(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ---------------------------------------------------------------------------
// w13 + silu_and_mul for a one-token call.  A token's routed experts are
// distinct, so every block computes its own pair (no search for other pairs
// of its slot), and the token's activation loads go out first, with no wait
// before them.  A block owns 8 outputs i0 .. i0 + 7 (blockIdx.x = i0 / 8) and
// puts their gate and up rows into one MFMA operand: operand rows 0-7 are
// gate rows i0 .. i0 + 7, rows 8-15 the up rows I + i0 .. I + i0 + 7.  Each
// output's steps are fp8_w13_kernel's (one MFMA column, the same k-block
// ranges per wave, the waves' partial sums in wave order), with half the
// weight registers of a 16-output block that holds gate and up in two
// operands; so a Qwen3-shaped call (I 768, top-8) runs 768 blocks, three per
// CU, where 16-output blocks ran 384, two or one per CU.  SLOTS (the call
// fills every slot: top-k == cap and the slots come from the pager):
// blockIdx.y is a slot, whose weight and scale loads go out before the slot
// table is read; the table then names the pair to store (slot 0's blocks
// store zeros for pairs that name no slot of the scratch).  Each of the NW
// waves takes KC k-blocks of H per chunk.  Dynamic LDS: red [NW][2][64][4]
// f32 (this block uses its first half), then per wave xs [KC] f32 and xq
// [KC][kKB] codes.
// ---------------------------------------------------------------------------
// The block of 8-output tile `tile` and pair (or, with SLOTS, slot) `by`.
// With `words` (the pager's per-pair words; a fused page-in launch), a pair
// whose expert this call loaded is left to the copy blocks, which compute it
// from the bytes they copy.
template <int NW, int KC, bool SLOTS>
__device__ inline void w13_one_block(const uint16_t* __restrict__ x, int H, int I, int K,
                                     const int32_t* __restrict__ slots, int nslots,
                                     const uint8_t* __restrict__ w13, size_t w13_stride,
                                     const float* __restrict__ s13, size_t s13_stride,
                                     int block_n, uint16_t* __restrict__ act,
                                     unsigned char* smem, int tile, int by,
                                     const int32_t* __restrict__ words) {
  float* red = reinterpret_cast<float*>(smem);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int i0 = tile * 8;
  const int nkb = H / kKB;
  const int per = (nkb + NW - 1) / NW;
  const int kb0 = min(nkb, wave * per), kb1 = min(nkb, kb0 + per);
  float* xs = reinterpret_cast<float*>(smem + NW * 2 * 64 * 4 * sizeof(float) +
                                       (size_t)wave * KC * (4 + kKB));
  uint8_t* xq = reinterpret_cast<uint8_t*>(xs + KC);

  // The first chunk's activation loads go out first, then its weight and
  // scale loads, then (SLOTS) the slot table, with nothing that waits in
  // between: loads complete in order, so the quantisation waits for x only,
  // and the weights stream while it runs.  (Left to itself the compiler
  // waited for x and the table before issuing any weight load, which held
  // every block's weights back by that round trip.)  A wave without k-blocks
  // loads the last one and drops it.
  const int kbx = min(kb0 + min(grp, max(min(KC, kb1 - kb0), 1) - 1), nkb - 1);
  u32x4 xv = *reinterpret_cast<const u32x4*>(x + (size_t)kbx * kKB + col * 8);
  int s, sl = -1, wd = -1;
  bool absent = false;  // this block's pair reads no expert: it stores zeros
  if (SLOTS) {
    s = by;
  } else {
    if (words && pair_word_loaded(scalar_word(words + by)) >= 0) return;
    s = scalar_word(slots + by);
    absent = s < 0 || s >= nslots;
    if (absent) s = 0;  // loads from slot 0, dropped (no branch around them)
  }
  const uint8_t* W = w13 + (size_t)s * w13_stride;
  // operand row `col`: gate row i0 + col, or up row I + i0 + col - 8; result
  // rows 4 * grp .. 4 * grp + 3 are gate rows for grp < 2, up rows above
  const uint8_t* row = W + (size_t)(col < 8 ? i0 + col : I + i0 + col - 8) * H + grp * 32;
  const float* Sw = s13 + (size_t)s * s13_stride +
                    (size_t)((grp < 2 ? i0 : I + i0) / block_n) * nkb;
  i32x8 w[KC];
  float sw[KC];
  auto load_chunk = [&](int kc) {
    const int nk = min(KC, kb1 - kc);
#pragma unroll
    for (int kbi = 0; kbi < KC; ++kbi) {
      const int kb = min(kc + min(kbi, nk - 1), nkb - 1);
      w[kbi] = ld32(row + (size_t)kb * kKB);
      sw[kbi] = Sw[kb];
    }
  };
  load_chunk(kb0);
  if (SLOTS) {
    sl = load_first(slots + min(lane, K - 1));  // lane j < K: pair j's slot
    // unconditional (read from the slots when there are no words): a load
    // under a branch made the compiler wait for every load before it
    wd = load_first((words ? words : slots) + min(lane, K - 1));
  }
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int kc = kb0; kc < kb1; kc += KC) {
    const int nk = min(KC, kb1 - kc);
    if (kc != kb0) {
      xv = *reinterpret_cast<const u32x4*>(x + (size_t)(kc + min(grp, nk - 1)) * kKB + col * 8);
      load_chunk(kc);
    }
    {
      float v[8];
      unpack_bf16x8(xv, v);
      uint32_t q[2];
      const float sc = quant8(v, q);
      if (grp < nk) {
        *reinterpret_cast<uint2*>(xq + (size_t)grp * kKB + col * 8) = make_uint2(q[0], q[1]);
        if (col == 0) xs[grp] = sc;
      }
    }
    wave_lds_sync();
    // every lane reads its group's column-0 operand (the other columns'
    // results are never used, and one column's result does not depend on
    // the others), so the reads and MFMAs of the chunk are independent;
    // only the scaled sums run in k-block order
    i32x8 b[KC];
    float sa[KC];
#pragma unroll
    for (int kbi = 0; kbi < KC; ++kbi) {
      b[kbi] = lds32(xq + (size_t)min(kbi, nk - 1) * kKB + grp * 32);
      sa[kbi] = xs[min(kbi, nk - 1)];
    }
    f32x4 d[KC];
#pragma unroll
    for (int kbi = 0; kbi < KC; ++kbi) d[kbi] = mfma_fp8(w[kbi], b[kbi]);
#pragma unroll
    for (int kbi = 0; kbi < KC; ++kbi) {
      if (kbi < nk) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = acc[j] + (d[kbi][j] * sa[kbi]) * sw[kbi];
      }
    }
    wave_lds_sync();  // the slice is rewritten by the next chunk
  }
  *reinterpret_cast<f32x4*>(red + ((size_t)wave * 64 + lane) * 4) = acc;
  int p = by;
  uint64_t none = 0;  // SLOTS: pairs whose slot lies outside the scratch
  if (SLOTS) {
    const uint64_t mine = __ballot(lane < K && sl == s);
    p = mine ? __builtin_ctzll(mine) : -1;
    none = s == 0 ? __ballot(lane < K && (sl < 0 || sl >= nslots)) : 0;
    if (words && __ballot(lane < K && sl == s && pair_word_loaded(wd) >= 0)) p = -1;
  }
  const int zp = absent ? p : -1;  // stored as zeros below
  if (absent) p = -1;
  block_lds_sync();
  if (wave == 0 && col == 0 && grp < 2 && p >= 0) {
    // this lane's four gate outputs and, 32 lanes on, their up outputs,
    // each summed over the waves in wave order from zero
    f32x4 g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int w0 = 0; w0 < NW; w0 += 4) {
      f32x4 pg[4], pu[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int w = min(w0 + i, NW - 1);
        pg[i] = *reinterpret_cast<const f32x4*>(red + ((size_t)w * 64 + lane) * 4);
        pu[i] = *reinterpret_cast<const f32x4*>(red + ((size_t)w * 64 + lane + 32) * 4);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (w0 + i < NW) {
          g = g + pg[i];
          u = u + pu[i];
        }
      }
    }
    store_act4(act + (size_t)p * I + i0 + grp * 4, g, u);
  }
  for (; none; none &= none - 1)
    if (threadIdx.x < 8) act[(size_t)__builtin_ctzll(none) * I + i0 + threadIdx.x] = 0;
  if (zp >= 0 && threadIdx.x < 8) act[(size_t)zp * I + i0 + threadIdx.x] = 0;
}

template <int NW, int KC, bool SLOTS>
__global__ __launch_bounds__(NW * 64) void fp8_w13_one_kernel(
    const uint16_t* __restrict__ x, int H, int I, int K, const int32_t* __restrict__ slots,
    int nslots, const uint8_t* __restrict__ w13, size_t w13_stride, const float* __restrict__ s13,
    size_t s13_stride, int block_n, uint16_t* __restrict__ act) {
  extern __shared__ __align__(16) unsigned char smem[];
  w13_one_block<NW, KC, SLOTS>(x, H, I, K, slots, nslots, w13, w13_stride, s13, s13_stride,
                               block_n, act, smem, blockIdx.x, blockIdx.y, nullptr);
}

// ---------------------------------------------------------------------------
// Page-in and w13 in one launch for one-token calls on the copy-kernel
// engine, the block-FP8 twin of the bf16 page-in + w13 launch (one slab per
// expert, [w13 | w2 | s13 | s2], in master and scratch alike).
//   * Blocks [0, kFp8CopyBlocks) copy each expert the pager loaded: its w13
//     rows in 16-row tiles (gate rows i0 .. i0 + 15 and the matching up
//     rows), each tile from the pinned master into the slot, computing the
//     tile's act of the expert's pair from the codes the block holds with
//     w13_one_block's steps (the same k-block ranges per wave, k-blocks in
//     ascending order within a wave, the waves' partial sums in wave order),
//     so the output equals a resident call's; then the rest of the slab as
//     a plain copy.  The token is quantised once per block, into LDS.
//   * Blocks from kFp8CopyBlocks on are w13_one_block's for the pairs whose
//     expert was already resident (grid order: tile fastest, then pair or
//     slot).
// Dynamic LDS: the larger of w13_one_block's and the copy blocks' (red
// [NW][2][64][4] f32, then xq [nkb][kKB] codes and xs [nkb] f32).
// ---------------------------------------------------------------------------
// Copy blocks of the fused launch (512 threads each; 4 MiB of host reads in
// flight).  32 blocks measured 1 % slower page-in.
constexpr int kFp8CopyBlocks = 64;

struct Fp8FusedArgs {
  const uint16_t* x;
  const int32_t* slots;  // the call's per-pair slots
  const int32_t* words;  // the pager's per-pair words: pair_word(slot, loaded expert)
  const uint8_t* w13;    // scratch, slot s at + s * w13_stride bytes
  size_t w13_stride;
  const float* s13;
  size_t s13_stride;     // floats
  uint16_t* act;
  size_t s13_off;        // byte offset of the w13 scales in an expert's slab
  int H, I, K, nslots, block_n;
};

// Byte offset of the copy blocks' per-wave staging in the fused launch's
// LDS: after red [NW][2][64][4] f32 and the token's codes and scales.
constexpr size_t fp8_copy_stage_off(int nw, int nkb) {
  return ((size_t)nw * 2 * 64 * 4 * sizeof(float) + (size_t)nkb * (4 + kKB) + 15) / 16 * 16;
}

// Copy blocks of the fused launch, for NW * PER == H / kKB (every wave PER
// k-blocks).  A tile's 32 rows (16 gate, 16 up) are read over the host link
// as whole PER * 128-byte row segments, 16 bytes a lane (requests of 1 KiB
// per instruction, where the MFMA layout, 16 rows x 32 bytes per
// instruction, would cut them into 64-byte pieces and cost ~15 % of the
// link); each wave stores its segments to the slot and, gate rows then up
// rows, puts the PER k-blocks of 16 rows in its own PER * 2 KiB of LDS,
// whence it reads its MFMA operands.  Staging a half's k-blocks at once lets
// its load registers go before the MFMAs: one k-block at a time kept all
// of them live through the tile (98 VGPRs, two blocks per CU for the whole
// launch; 60 now, with the w13 blocks' 8-output tiles).
template <int NW, int PER>
__device__ inline void fp8_copy_w13_blocks(const Fp8FusedArgs& f, const PageInArgs& a,
                                           unsigned char* smem, int cb) {
  constexpr int SEG = PER * kKB;     // bytes of a row a wave holds
  constexpr int LPR = SEG / 16;      // lanes per row segment
  constexpr int RPI = 64 / LPR;      // rows per load instruction
  constexpr int NI = 32 / RPI;       // load instructions per tile
  const int n = *a.count;
  if (a.hist && cb == 0 && threadIdx.x == 0) {
    *a.hist = n;
    __threadfence_system();
  }
  if (n <= 0) return;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int H = f.H, I = f.I, nkb = H / kKB, ntile = I / 16;
  float* red = reinterpret_cast<float*>(smem);
  uint8_t* xq = reinterpret_cast<uint8_t*>(red + NW * 2 * 64 * 4);
  float* xs = reinterpret_cast<float*>(xq + (size_t)nkb * kKB);
  // this wave's staging: PER k-blocks of 16 rows x kKB
  uint8_t* ws = smem + fp8_copy_stage_off(NW, nkb) + (size_t)wave * PER * 16 * kKB;
  // lane p < K holds the expert pair p's word says was loaded (or -1)
  const int mine = lane < f.K ? pair_word_loaded(f.words[lane]) : -1;
  // the token's k-blocks, one per 16-lane row
  for (int base = wave * 4; base < nkb; base += NW * 4) {
    const int kb = base + grp;
    float v[8];
    unpack_bf16x8(*reinterpret_cast<const u32x4*>(f.x + (size_t)min(kb, nkb - 1) * kKB + col * 8),
                  v);
    uint32_t q[2];
    const float sc = quant8(v, q);
    if (kb < nkb) {
      *reinterpret_cast<uint2*>(xq + (size_t)kb * kKB + col * 8) = make_uint2(q[0], q[1]);
      if (col == 0) xs[kb] = sc;
    }
  }
  block_lds_sync();
  const int kb0 = wave * PER;  // this wave's k-blocks: kb0 .. kb0 + PER - 1
  const int seg_row = lane / LPR, seg_cb = lane % LPR;  // a load's row and 16-byte block
  const PageInPlane& p0 = a.p[0];
  for (int q = cb; q < n * ntile; q += kFp8CopyBlocks) {
    const int j = q / ntile, tile = q - j * ntile;
    const int e = a.loads[2 * j], s = a.loads[2 * j + 1];
    if (e < 0 || e >= a.num_experts || s < 0 || s >= a.cap) continue;
    const uint64_t m = __ballot(mine == e);
    const int pair = m ? __builtin_ctzll(m) : -1;
    const int i0 = tile * 16;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(p0.m) + (size_t)e * p0.m_stride;
    uint8_t* dst = reinterpret_cast<uint8_t*>(p0.d) + (size_t)s * p0.d_stride;
    const float* S = reinterpret_cast<const float*>(src + f.s13_off);
    float sg[PER], su[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      sg[k] = S[(size_t)(i0 / f.block_n) * nkb + kb0 + k];
      su[k] = S[(size_t)((I + i0) / f.block_n) * nkb + kb0 + k];
    }
    // byte offset of load ii's 16 bytes in the slab (recomputed for the
    // store rather than held: the registers bound the launch's occupancy)
    auto off = [&](int ii) {
      const int rr = ii * RPI + seg_row;  // tile row: 0-15 gate, 16-31 up
      return (uint32_t)((rr < 16 ? i0 + rr : I + i0 + rr - 16) * H + kb0 * kKB + seg_cb * 16);
    };
    u32x4 v[NI];
#pragma unroll
    for (int ii = 0; ii < NI; ++ii) v[ii] = *reinterpret_cast<const u32x4*>(src + off(ii));
#pragma unroll
    for (int ii = 0; ii < NI; ++ii)
      __builtin_nontemporal_store(v[ii], reinterpret_cast<u32x4*>(dst + off(ii)));
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
    // LDS row r (0-15) of staged k-block k: its 8 16-byte blocks at
    // (block ^ (r & 7))
    auto at = [&](int k, int r, int cb) {
      return ws + (k * 16 + r) * kKB + ((cb ^ (r & 7)) << 4);
    };
    const int cb = grp * 2;  // the lane's 32 bytes of a k-block
    // rows [16 h, 16 h + 16) of the tile (h 0: gate, 1: up), every k-block
    // of their segments at once, then that half's MFMAs in k-block order;
    // the wave's own LDS, so its reads of the gate half come first in order
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int ii = 0; ii < NI; ++ii) {
        const int rr = ii * RPI + seg_row;
        if ((rr >> 4) == h)
          *reinterpret_cast<u32x4*>(at(seg_cb >> 3, rr & 15, seg_cb & 7)) = v[ii];
      }
      wave_lds_sync();
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const i32x8 w = join(*reinterpret_cast<const u32x4*>(at(k, col, cb)),
                             *reinterpret_cast<const u32x4*>(at(k, col, cb + 1)));
        const int kb = kb0 + k;
        const i32x8 b = lds32(xq + (size_t)kb * kKB + grp * 32);
        const float sa = xs[kb];
        const f32x4 d = mfma_fp8(w, b);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          if (h == 0)
            ag[jj] = ag[jj] + (d[jj] * sa) * sg[k];
          else
            au[jj] = au[jj] + (d[jj] * sa) * su[k];
        }
      }
      wave_lds_sync();  // the up half overwrites the staging
    }
    float* rw = red + ((size_t)wave * 2 * 64 + lane) * 4;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      rw[jj] = ag[jj];
      rw[64 * 4 + jj] = au[jj];
    }
    block_lds_sync();
    if (wave == 0 && col == 0 && pair >= 0) {
      f32x4 g, u;
      sum_partials<NW>(red, lane, g, u);
      store_act4(f.act + (size_t)pair * I + i0 + grp * 4, g, u);
    }
    block_lds_sync();  // red and the segments are rewritten by the next tile
  }
  // the rest of each loaded expert's slab (w2 and the scales), other planes
  const size_t w13_bytes = (size_t)2 * I * H;
  for (int j = 0; j < n; ++j) {
    const int ej = a.loads[2 * j], sj = a.loads[2 * j + 1];
    if (ej < 0 || ej >= a.num_experts || sj < 0 || sj >= a.cap) continue;
    copy_range<NW * 64>(p0.m + (size_t)ej * p0.m_stride + w13_bytes,
                        p0.d + (size_t)sj * p0.d_stride + w13_bytes, p0.bytes - w13_bytes,
                        cb, kFp8CopyBlocks);
    for (int qq = 1; qq < a.nplanes; ++qq) {
      const PageInPlane& pl = a.p[qq];
      copy_range<NW * 64>(pl.m + (size_t)ej * pl.m_stride, pl.d + (size_t)sj * pl.d_stride,
                          pl.bytes, cb, kFp8CopyBlocks);
    }
  }
}

// w13 blocks of KC k-blocks per wave chunk; copy blocks of PER k-blocks per
// wave (NW * PER == H / kKB).  Six waves per SIMD (at most 80 VGPRs, which
// the copy blocks reach without spilling): three 8-wave blocks per CU, so
// the Qwen3-shaped launch's 768 w13 blocks run in one round.
template <int NW, int KC, int PER, bool SLOTS>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(6)))
void pagein_fp8_w13_kernel(Fp8FusedArgs f, PageInArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  if (blockIdx.x >= kFp8CopyBlocks) {
    const int ntile = f.I / 8;  // 8-output tiles
    const int local = blockIdx.x - kFp8CopyBlocks;
    const int by = local / ntile;
    w13_one_block<NW, KC, SLOTS>(f.x, f.H, f.I, f.K, f.slots, f.nslots, f.w13, f.w13_stride,
                                 f.s13, f.s13_stride, f.block_n, f.act, smem,
                                 local - by * ntile, by, f.words);
    return;
  }
  fp8_copy_w13_blocks<NW, PER>(f, a, smem, blockIdx.x);
}

// ---------------------------------------------------------------------------
// w2 + routing weight + moe_sum.
// KC2: k-blocks a wave loads before it computes (the job's k-range is a
// whole number of chunks, or the last chunk loads clamped copies that are
// never used).  QP: quantisation passes per round (4 act groups per pass),
// sized so that a wave quantises few clamped copies.
// Dynamic LDS: aq [K][I] codes, as [K][nkb] f32, part [K][WP][16] f32.
// ---------------------------------------------------------------------------
template <int NW, int KC2, int QP>
__global__ __launch_bounds__(NW * 64) void fp8_w2_kernel(
    const uint16_t* __restrict__ act, int H, int I, int K, const float* __restrict__ topk_w,
    const int32_t* __restrict__ slots, int nslots, const uint8_t* __restrict__ w2,
    size_t w2_stride, const float* __restrict__ s2, size_t s2_stride, int block_n, int WP,
    uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int t = blockIdx.y, h0 = blockIdx.x * 16;
  const int nkb = I / kKB;
  uint8_t* aq = smem;
  float* as = reinterpret_cast<float*>(smem + (size_t)K * I);
  float* part = as + (size_t)K * nkb;

  // the token's slots and routing weights, lane k holding pair k (K <= 64;
  // lanes past K hold copies and are never read), loaded without branches; a
  // slot outside the scratch contributes zero
  const int kl = min(lane, K - 1);
  int sk = slots[(size_t)t * K + kl];
  const float wk = topk_w[(size_t)t * K + kl];
  if (sk >= nslots) sk = -1;

  // act groups to quantise: one quarter-wave per 128-value group, four per
  // pass, QP passes per round; clamped copies past the last group are
  // quantised and dropped
  const int ngroups = K * nkb;
  u32x4 av[QP];
  auto load_round = [&](int g0) {
#pragma unroll
    for (int it = 0; it < QP; ++it) {
      const int g = min(g0 + it * NW * 4 + grp, ngroups - 1);
      const int k = g / nkb, kb = g % nkb;
      av[it] = *reinterpret_cast<const u32x4*>(act + ((size_t)t * K + k) * I +
                                               (size_t)kb * kKB + col * 8);
    }
  };
  auto quant_round = [&](int g0) {
#pragma unroll
    for (int it = 0; it < QP; ++it) {
      const int g = g0 + it * NW * 4 + grp;
      float v[8];
      unpack_bf16x8(av[it], v);
      uint32_t q[2];
      const float sc = quant8(v, q);
      if (g < ngroups) {
        const int k = g / nkb, kb = g % nkb;
        *reinterpret_cast<uint2*>(aq + (size_t)k * I + (size_t)kb * kKB + col * 8) =
            make_uint2(q[0], q[1]);
        if (col == 0) as[k * nkb + kb] = sc;
      }
    }
  };
  load_round(wave * 4);

  // this wave's jobs: (pair k, k-block part q), q < WP; the first job's first
  // chunk of weights and scales is in flight while the act is quantised
  const int njob = K * WP;
  const int per = (nkb + WP - 1) / WP;
  i32x8 a[KC2];
  float sw[KC2];
  // The loads are unconditional (a wave without a first job, an absent slot
  // or an empty k-range reads slot 0's first block and drops it): loads
  // under a branch would make the wait before the quantisation below count
  // them too.
  const int j0 = wave;
  const int s0 = j0 < njob ? __builtin_amdgcn_readlane(sk, min(j0, njob - 1) / WP) : -1;
  const int kbs0 = min(nkb, (j0 % WP) * per);
  const int kbe0 = min(nkb, kbs0 + per);
  {
    const bool live = s0 >= 0 && kbe0 > kbs0;
    const int sl = live ? s0 : 0;
    const uint8_t* row = w2 + (size_t)sl * w2_stride + (size_t)(h0 + col) * I + grp * 32;
    const float* S = s2 + (size_t)sl * s2_stride + (size_t)(h0 / block_n) * nkb;
    const int last = live ? min(KC2, kbe0 - kbs0) - 1 : 0;
    const int base = live ? kbs0 : 0;
#pragma unroll
    for (int kbi = 0; kbi < KC2; ++kbi) {
      const int kb = base + min(kbi, last);
      a[kbi] = ld32(row + (size_t)kb * kKB);
      sw[kbi] = S[kb];
    }
  }
  quant_round(wave * 4);
  for (int g0 = wave * 4 + QP * NW * 4; g0 < ngroups; g0 += QP * NW * 4) {
    load_round(g0);
    quant_round(g0);
  }
  block_lds_sync();  // the first job's weights stay in flight

  for (int j = wave; j < njob; j += NW) {
    const int k = j / WP;
    const int s = j == j0 ? s0 : __builtin_amdgcn_readlane(sk, k);
    const int kbs = j == j0 ? kbs0 : min(nkb, (j % WP) * per);
    const int kbe = j == j0 ? kbe0 : min(nkb, kbs + per);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (s >= 0) {
      const uint8_t* row = w2 + (size_t)s * w2_stride + (size_t)(h0 + col) * I + grp * 32;
      const float* S = s2 + (size_t)s * s2_stride + (size_t)(h0 / block_n) * nkb;
      const float* sa = as + (size_t)k * nkb;
      const uint8_t* aqk = aq + (size_t)k * I + grp * 32;
      for (int kc = kbs; kc < kbe; kc += KC2) {
        const int nk = min(KC2, kbe - kc);
        if (!(j == j0 && kc == kbs)) {
#pragma unroll
          for (int kbi = 0; kbi < KC2; ++kbi) {
            const int kb = kc + min(kbi, nk - 1);
            a[kbi] = ld32(row + (size_t)kb * kKB);
            sw[kbi] = S[kb];
          }
        }
#pragma unroll
        for (int kbi = 0; kbi < KC2; ++kbi) {
          if (kbi < nk) {
            const i32x8 b = col == 0 ? lds32(aqk + (size_t)(kc + kbi) * kKB) : zero8();
            const f32x4 d = mfma_fp8(a[kbi], b);
            const float sc = sa[kc + kbi];
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = acc[q] + (d[q] * sc) * sw[kbi];
          }
        }
      }
    }
    if (col == 0) {
      float* pr = part + ((size_t)k * WP + (j % WP)) * 16 + grp * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) pr[q] = acc[q];
    }
  }
  __syncthreads();
  if (wave == 0) {  // lanes < 16 store
    // pair k's slot and weight come through scalar registers and every
    // job wrote its partials, so the k steps' LDS reads do not wait on each
    // other; only the sum runs in routing order
    const int r = lane & 15;
    const bool bf16_adds = K >= 2 && K <= 4;
    float sum = 0.f;
    for (int k0 = 0; k0 < K; k0 += 8) {
      float v[8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int k = min(k0 + kk, K - 1);
        v[kk] = 0.f;
        for (int q = 0; q < WP; ++q) v[kk] = v[kk] + part[((size_t)k * WP + q) * 16 + r];
      }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int k = k0 + kk;
        if (k < K) {
          const int s = __builtin_amdgcn_readlane(sk, k);
          const float y = s >= 0 ? round_bf16(v[kk] * readlane_f32(wk, k)) : 0.f;
          sum = bf16_adds ? round_bf16(sum + y) : sum + y;
        }
      }
    }
    if (lane < 16) out[(size_t)t * H + h0 + r] = bf16_rne(sum);
  }
}

// ---------------------------------------------------------------------------
// w2 + routing weight + moe_sum for a one-token call with K <= 16 and
// KB = I / 128 <= 8 k-blocks.  Block = K waves over one 16-row tile of H;
// wave w quantises pair w's act into LDS and streams one expert's tile: pair
// w's slot, or slot w with SLOTS (the call fills every slot: top-k == cap,
// slots from the pager), whose loads then go out before the slot table
// arrives.  (At the Qwen3 shape that is 128 blocks, half the CUs: 8-row
// blocks, 256 of them, measured no faster, 6.0 against 5.6-6.0 us; the
// kernel is bound by its chain of dependent steps, not by the CUs that
// stream.)  Everything a wave needs after the LDS barrier is read at once
// and its KB MFMAs are independent; only the scaled sums run in k-block
// order.  Per output the steps are fp8_w2_kernel's with one job per pair, so
// the bytes are the same.  Dynamic LDS: aq [K][I] codes, as [K][KB] f32,
// part [K][16] f32.
// ---------------------------------------------------------------------------
template <int KB, bool SLOTS>
__global__ __launch_bounds__(1024) void fp8_w2_one_kernel(
    const uint16_t* __restrict__ act, int H, int I, int K, const float* __restrict__ topk_w,
    const int32_t* __restrict__ slots, int nslots, const uint8_t* __restrict__ w2,
    size_t w2_stride, const float* __restrict__ s2, size_t s2_stride, int block_n,
    uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int h0 = blockIdx.x * 16;
  uint8_t* aq = smem;
  float* as = reinterpret_cast<float*>(smem + (size_t)K * I);
  float* part = as + (size_t)K * KB;

  // Load order: pair `wave`'s act (quarter-wave g quantises k-blocks g and
  // g + 4), then the tile's weights and scales, then (SLOTS) the slot table
  // and routing weights, with nothing that waits in between: loads complete
  // in order, so the quantisation waits for act only while the weights
  // stream.  (Left to itself the compiler put the quantisation, and its wait
  // for act, between the weight loads.)  Without SLOTS the tile's slot comes
  // from the table, which is then loaded first.
  // lane j < K: pair j's slot and routing weight (a slot outside the
  // scratch contributes zero)
  const int jl = min(lane, K - 1);
  int sj = SLOTS ? -1 : load_first(slots + jl);
  u32x4 av[2];
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int kb = min(grp + 4 * it, KB - 1);
    av[it] = *reinterpret_cast<const u32x4*>(act + (size_t)wave * I + (size_t)kb * kKB + col * 8);
  }
  // the tile this wave streams: slot `wave`, or pair `wave`'s slot
  if (!SLOTS && sj >= nslots) sj = -1;
  const int s = SLOTS ? wave : __builtin_amdgcn_readlane(sj, wave);
  const int sl = s >= 0 ? s : 0;  // an absent pair reads slot 0 and drops it
  const uint8_t* row = w2 + (size_t)sl * w2_stride + (size_t)(h0 + col) * I + grp * 32;
  const float* S = s2 + (size_t)sl * s2_stride + (size_t)(h0 / block_n) * KB;
  i32x8 a[KB];
  float sw[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    a[kb] = ld32(row + (size_t)kb * kKB);
    sw[kb] = S[kb];
  }
  if (SLOTS) sj = load_first(slots + jl);
  const float wj = __int_as_float(load_first((const int32_t*)topk_w + jl));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    float v[8];
    unpack_bf16x8(av[it], v);
    uint32_t q[2];
    const float sc = quant8(v, q);
    const int kb = grp + 4 * it;
    if (kb < KB) {
      *reinterpret_cast<uint2*>(aq + (size_t)wave * I + (size_t)kb * kKB + col * 8) =
          make_uint2(q[0], q[1]);
      if (col == 0) as[wave * KB + kb] = sc;
    }
  }
  block_lds_sync();  // the tile's loads stay in flight
  __builtin_amdgcn_sched_barrier(0);  // nothing that reads sj above the barrier
  if (SLOTS && sj >= nslots) sj = -1;
  // the pair this wave's tile serves (-1: none)
  int p = wave;
  if (SLOTS) {
    const uint64_t m = __ballot(lane < K && sj == s);
    p = m ? __builtin_ctzll(m) : -1;
  } else if (s < 0) {
    p = -1;
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (p >= 0) {
    // every lane reads its group's column-0 operand (the other columns'
    // results are never used, and one column's result does not depend on
    // the others)
    i32x8 b[KB];
    float sa[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      b[kb] = lds32(aq + (size_t)p * I + (size_t)kb * kKB + grp * 32);
      sa[kb] = as[p * KB + kb];
    }
    f32x4 d[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) d[kb] = mfma_fp8(a[kb], b[kb]);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = acc[q] + (d[kb][q] * sa[kb]) * sw[kb];
  }
  if (col == 0 && p >= 0) {  // an absent pair's partials are never read
    float* pr = part + (size_t)p * 16 + grp * 4;
#pragma unroll
    for (int q = 0; q < 4; ++q) pr[q] = acc[q];
  }
  block_lds_sync();
  if (wave == 0) {  // lanes < 16 store
    const int r = lane & 15;
    const bool bf16_adds = K >= 2 && K <= 4;
    float sum = 0.f;
    for (int k0 = 0; k0 < K; k0 += 8) {
      float v[8];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) v[kk] = 0.f + part[(size_t)min(k0 + kk, K - 1) * 16 + r];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int k = k0 + kk;
        if (k < K) {
          const float y = __builtin_amdgcn_readlane(sj, k) >= 0
                              ? round_bf16(v[kk] * readlane_f32(wj, k)) : 0.f;
          sum = bf16_adds ? round_bf16(sum + y) : sum + y;
        }
      }
    }
    if (lane < 16) out[(size_t)h0 + r] = bf16_rne(sum);
  }
}

// ---------------------------------------------------------------------------
// Grouped path for batches and prefill chunks: per slot, the pairs routed to
// it (gather), x and act quantised once by the group quantiser, and each
// weight tile streamed once per pass of up to MT * 16 token columns.
//   fp8_grouped_w13: grid (I / 64, nslots), wave w owns gate rows
//     [64 * bx + 16w, +16) and the matching up rows; act written as bf16;
//   fp8_grouped_w2: grid (H / 64, nslots), y[p] = bf16(acc * topk_w[p]);
//   fp8_combine: out[t] = moe_sum over k of y[(t, k)].
// An output element is one chain over the k-blocks in ascending order, the
// same for every MT, U and grouping, so bytes do not depend on which tokens
// share a launch.  U k-blocks are loaded per iteration (nkb % U == 0).
// ---------------------------------------------------------------------------
template <int MT, int U>
__global__ __launch_bounds__(256) void fp8_grouped_w13_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, int H, int I, int K, int P,
    const int32_t* __restrict__ lists, const int32_t* __restrict__ counts,
    const uint8_t* __restrict__ w13, size_t w13_stride, const float* __restrict__ s13,
    size_t s13_stride, int block_n, uint16_t* __restrict__ act) {
  const int s = blockIdx.y;
  const int M = counts[s];
  if (M == 0) return;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int i0 = blockIdx.x * 64 + wave * 16;
  const int nkb = H / kKB;
  const uint8_t* Wg = w13 + (size_t)s * w13_stride + (size_t)(i0 + col) * H + grp * 32;
  const uint8_t* Wu = Wg + (size_t)I * H;
  const float* Sg = s13 + (size_t)s * s13_stride + (size_t)(i0 / block_n) * nkb;
  const float* Su = s13 + (size_t)s * s13_stride + (size_t)((I + i0) / block_n) * nkb;
  for (int m0 = 0; m0 < M; m0 += MT * 16) {
    const int mrows = min(M - m0, MT * 16);
    // the pair and token of this lane's column in each tile (past the last
    // row: a clamped copy, computed and not stored)
    int pr[MT], tok[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      pr[t] = list[m0 + min(t * 16 + col, mrows - 1)];
      tok[t] = pr[t] / K;
    }
    f32x4 ag[MT], au[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      ag[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      au[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int kb0 = 0; kb0 < nkb; kb0 += U) {
      i32x8 wgr[U], wur[U], b[U][MT];
      float sg[U], su[U], sx[U][MT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        wgr[u] = ld32(Wg + (size_t)(kb0 + u) * kKB);
        wur[u] = ld32(Wu + (size_t)(kb0 + u) * kKB);
        sg[u] = Sg[kb0 + u];
        su[u] = Su[kb0 + u];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          b[u][t] = ld32(xq + (size_t)tok[t] * H + (size_t)(kb0 + u) * kKB + grp * 32);
          sx[u][t] = xs[(size_t)tok[t] * nkb + kb0 + u];
        }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t * 16 < mrows) {
            const f32x4 dg = mfma_fp8(wgr[u], b[u][t]);
            const f32x4 du = mfma_fp8(wur[u], b[u][t]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              ag[t][j] = ag[t][j] + (dg[j] * sx[u][t]) * sg[u];
              au[t][j] = au[t][j] + (du[j] * sx[u][t]) * su[u];
            }
          }
        }
    }
    // D[row][col]: weight row i0 + 4 * grp + j, token column col
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int r = t * 16 + col;
      if (r < mrows) {
        store_act4(act + (size_t)pr[t] * I + i0 + grp * 4, ag[t], au[t]);
      }
    }
  }
}

template <int MT, int U>
__global__ __launch_bounds__(256) void fp8_grouped_w2_kernel(
    const uint8_t* __restrict__ aq, const float* __restrict__ as, int H, int I, int P,
    const int32_t* __restrict__ lists, const int32_t* __restrict__ counts,
    const float* __restrict__ topk_w, const uint8_t* __restrict__ w2, size_t w2_stride,
    const float* __restrict__ s2, size_t s2_stride, int block_n, uint16_t* __restrict__ y) {
  const int s = blockIdx.y;
  const int M = counts[s];
  if (M == 0) return;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int h0 = blockIdx.x * 64 + wave * 16;
  const int nkb = I / kKB;
  const uint8_t* Wr = w2 + (size_t)s * w2_stride + (size_t)(h0 + col) * I + grp * 32;
  const float* S = s2 + (size_t)s * s2_stride + (size_t)(h0 / block_n) * nkb;
  for (int m0 = 0; m0 < M; m0 += MT * 16) {
    const int mrows = min(M - m0, MT * 16);
    int pr[MT];
    float pw[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      pr[t] = list[m0 + min(t * 16 + col, mrows - 1)];
      pw[t] = topk_w[pr[t]];
    }
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kb0 = 0; kb0 < nkb; kb0 += U) {
      i32x8 a[U], b[U][MT];
      float sw[U], sa[U][MT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        a[u] = ld32(Wr + (size_t)(kb0 + u) * kKB);
        sw[u] = S[kb0 + u];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          b[u][t] = ld32(aq + (size_t)pr[t] * I + (size_t)(kb0 + u) * kKB + grp * 32);
          sa[u][t] = as[(size_t)pr[t] * nkb + kb0 + u];
        }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          if (t * 16 < mrows) {
            const f32x4 d = mfma_fp8(a[u], b[u][t]);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[t][j] = acc[t][j] + (d[j] * sa[u][t]) * sw[u];
          }
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int r = t * 16 + col;
      if (r < mrows) {
        store_bf16x4(y + (size_t)pr[t] * H + h0 + grp * 4, acc[t][0] * pw[t],
                     acc[t][1] * pw[t], acc[t][2] * pw[t], acc[t][3] * pw[t]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-staged grouped path for calls of more than 16 tokens: the chunk
// pipeline of dma_pipeline.h, one chunk per 128-column k-block (128 bytes of
// e4m3fn per row), the weight rows and the token tile of each k-block copied
// straight into LDS two k-blocks ahead.  The k-blocks run in ascending order
// and every output takes exactly the grouped kernels' steps (same MFMA
// operands and orientation, acc + (D * s_act) * s_w per k-block), so its
// bytes equal theirs: paged calls, whose token groups may use either, match
// resident calls.  Per pass the token scales of the tile's 64 rows are
// staged in LDS beside the stages; the weight scales of a wave's row tiles
// are staged once per block.
//   fp8_w13_dma: grid (I / 64, nslots), wave w owns gate rows
//     [64 bx + 16w, +16) and the matching up rows;
//   fp8_w2_dma<S, NP>: grid (H / (128 NP), nslots); the block streams NP
//     consecutive 128-row panels of its slot as one chunk sequence (the
//     token tile is the same for all of them), wave w owning rows
//     [128 (NP bx + p) + 32w, +32) of panel p, stored at the panel's last
//     k-block.  A block's setup (count, pair list, scales) and its first
//     chunk's latency are paid once per NP panels.
// ---------------------------------------------------------------------------

// A lane's fp8 MFMA operand from a swizzled LDS slice: row r, the 32 bytes
// at 32 * grp of the k-block (column blocks 2 grp and 2 grp + 1).
__device__ inline i32x8 lds_operand(const unsigned char* slice, int r, int grp) {
  return join(*reinterpret_cast<const u32x4*>(slice + dma::swz(r, 2 * grp)),
              *reinterpret_cast<const u32x4*>(slice + dma::swz(r, 2 * grp + 1)));
}

// Dynamic LDS of the LDS-staged kernels: the stages, the pass's token scales
// [64][nkb], the four waves' weight scales [4][NP][2][nkb].
template <int S, int NP = 1>
inline size_t fp8_dma_lds(int nkb) {
  return dma::Smem<32, S>::kBytes + (size_t)dma::kTokRows * nkb * sizeof(float) +
         (size_t)4 * NP * 2 * nkb * sizeof(float);
}

// Stages the pass's token scales: row r < 64 of the tile reads the scales of
// tile row min(r, mrows - 1).  Runs inside the pass, after its first copies
// are issued (the pass's drain has seen the previous pass's readers out);
// row_of is called by every lane.
template <typename RowOf>
__device__ inline void stage_token_scales(float* xsl, const float* __restrict__ scales, int nkb,
                                          int mrows, RowOf row_of) {
  for (int q = threadIdx.x; q < dma::kTokRows * nkb; q += 256) {
    const int r = q / nkb, kb = q - r * nkb;
    xsl[q] = scales[(size_t)row_of(min(r, mrows - 1)) * nkb + kb];
  }
}

template <int S>
__global__ __launch_bounds__(256) void fp8_w13_dma_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, int H, int I, int K, int P,
    const int32_t* __restrict__ lists, const int32_t* __restrict__ counts,
    const uint8_t* __restrict__ w13, size_t w13_stride, const float* __restrict__ s13,
    size_t s13_stride, int block_n, uint16_t* __restrict__ act) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int s = blockIdx.y;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int i0 = blockIdx.x * 64 + wave * 16;
  const int nkb = H / kKB;
  const float* Sg = s13 + (size_t)s * s13_stride + (size_t)(i0 / block_n) * nkb;
  const float* Su = s13 + (size_t)s * s13_stride + (size_t)((I + i0) / block_n) * nkb;
  // loaded together: the slot's count, the first pass's pair list and the
  // first 64 of this wave's gate and up scales (staged into LDS after the
  // first copies are issued)
  const int M = counts[s];
  int held = dma::list_entries(list, 0, P);
  const float sg0 = dma::load_early(Sg + min(lane, nkb - 1));
  const float su0 = dma::load_early(Su + min(lane, nkb - 1));
  if (M == 0) return;
  float* xsl = reinterpret_cast<float*>(smem + dma::Smem<32, S>::kBytes);
  float* wsl = xsl + dma::kTokRows * nkb + wave * 2 * nkb;  // this wave's gate, up scales
  const uint8_t* W = w13 + (size_t)s * w13_stride;
  // this lane's weight copy rows: slice rows 0-15 gate, 16-31 up
  const unsigned char* wrow[32 / dma::kRowsPerCopy];
#pragma unroll
  for (int i = 0; i < 32 / dma::kRowsPerCopy; ++i) {
    const int r = i * dma::kRowsPerCopy + lane / dma::kLanesPerRow;
    wrow[i] = W + (size_t)(r < 16 ? i0 + r : I + i0 + r - 16) * H;
  }
  auto off = [](int c) { return (size_t)c * kKB; };
  for (int m0 = 0; m0 < M; m0 += dma::kTokRows) {
    const int mrows = min(M - m0, dma::kTokRows);
    if (m0 > 0) held = dma::list_entries(list, m0, P);
    // the pairs of this lane's output rows (tile t, row col)
    int pr[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) pr[t] = dma::list_entry(held, min(t * 16 + col, mrows - 1));
    auto tok_of = [&](int r) { return dma::list_entry(held, r) / K; };
    auto row_of = [&](int r) { return xq + (size_t)tok_of(r) * H; };
    // once the pass's first copies are issued: the token scales and, in the
    // first pass, this wave's weight scales
    auto stage = [&]() {
      stage_token_scales(xsl, xs, nkb, mrows, tok_of);
      if (m0 == 0) {
        for (int q = lane; q < nkb; q += 64) {
          wsl[q] = q < 64 ? sg0 : Sg[q];
          wsl[nkb + q] = q < 64 ? su0 : Su[q];
        }
      }
    };
    f32x4 ag[4], au[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      ag[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      au[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    auto run = [&](auto nt) {
      constexpr int NT = decltype(nt)::value;
      dma::pass<32, S, NT>(smem, wrow, mrows, row_of, nkb, off,
                           [&](const unsigned char* ws, const unsigned char* as, int c) {
                             const i32x8 wg = lds_operand(ws, col, grp);
                             const i32x8 wu = lds_operand(ws, 16 + col, grp);
                             const float sg = wsl[c], su = wsl[nkb + c];
#pragma unroll
                             for (int t = 0; t < NT; ++t) {
                               const i32x8 b = lds_operand(as, t * 16 + col, grp);
                               const float sx = xsl[(t * 16 + col) * nkb + c];
                               const f32x4 dg = mfma_fp8(wg, b);
                               const f32x4 du = mfma_fp8(wu, b);
#pragma unroll
                               for (int j = 0; j < 4; ++j) {
                                 ag[t][j] = ag[t][j] + (dg[j] * sx) * sg;
                                 au[t][j] = au[t][j] + (du[j] * sx) * su;
                               }
                             }
                           }, stage, m0 == 0);
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
    // D[row][col]: weight row i0 + 4 * grp + j, token column col
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int r = t * 16 + col;
      if (r < mrows) {
        store_act4(act + (size_t)pr[t] * I + i0 + grp * 4, ag[t], au[t]);
      }
    }
  }
}

// A wave's w2 outputs of one 32-row panel: D[row][col] is weight row
// h0 + 16 g + 4 grp + j, token column col of tile t.
__device__ inline void store_w2_tile(uint16_t* __restrict__ y, int H, int h0, const int (&pr)[4],
                                     const float (&pw)[4], int mrows, int col, int grp,
                                     const f32x4 (&acc)[2][4]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int r = t * 16 + col;
    if (r < mrows) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        store_bf16x4(y + (size_t)pr[t] * H + h0 + 16 * g + grp * 4, acc[g][t][0] * pw[t],
                     acc[g][t][1] * pw[t], acc[g][t][2] * pw[t], acc[g][t][3] * pw[t]);
      }
    }
  }
}

template <int S, int NP>
__global__ __launch_bounds__(256) void fp8_w2_dma_kernel(
    const uint8_t* __restrict__ aq, const float* __restrict__ as_, int H, int I, int P,
    const int32_t* __restrict__ lists, const int32_t* __restrict__ counts,
    const float* __restrict__ topk_w, const uint8_t* __restrict__ w2, size_t w2_stride,
    const float* __restrict__ s2, size_t s2_stride, int block_n, uint16_t* __restrict__ y) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int s = blockIdx.y;
  const int32_t* list = lists + (size_t)s * P;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int hb = blockIdx.x * NP * 128 + wave * 32;  // this wave's rows in panel 0
  const int nkb = I / kKB;
  // this wave's weight scale q < 2 NP nkb: panel q / (2 nkb), row group
  // (q / nkb) % 2, k-block q % nkb
  auto wscale_at = [&](int q) {
    const int pg = q / nkb, kb = q - pg * nkb;
    const int h = hb + (pg >> 1) * 128 + 16 * (pg & 1);
    return s2 + (size_t)s * s2_stride + (size_t)(h / block_n) * nkb + kb;
  };
  // loaded together: the slot's count, the first pass's pair list and the
  // first 64 of this wave's weight scales (staged into LDS after the first
  // copies are issued)
  const int M = counts[s];
  int held = dma::list_entries(list, 0, P);
  const float ws0 = dma::load_early(wscale_at(min(lane, 2 * NP * nkb - 1)));
  if (M == 0) return;
  float* asl = reinterpret_cast<float*>(smem + dma::Smem<32, S>::kBytes);
  float* wsl = asl + dma::kTokRows * nkb + wave * 2 * NP * nkb;  // [panel][row group][k-block]
  const uint8_t* W = w2 + (size_t)s * w2_stride;
  const unsigned char* wrow[32 / dma::kRowsPerCopy];
#pragma unroll
  for (int i = 0; i < 32 / dma::kRowsPerCopy; ++i)
    wrow[i] = W + (size_t)(hb + i * dma::kRowsPerCopy + lane / dma::kLanesPerRow) * I;
  // chunk q: panel q / nkb (128 rows further down per panel), k-block q % nkb
  auto off = [&](int q) {
    const int pn = q / nkb;
    const size_t kb = (size_t)(q - pn * nkb) * kKB;
    return dma::Offs{(size_t)pn * 128 * I + kb, kb};
  };
  for (int m0 = 0; m0 < M; m0 += dma::kTokRows) {
    const int mrows = min(M - m0, dma::kTokRows);
    if (m0 > 0) held = dma::list_entries(list, m0, P);
    // the pairs and routing weights of this lane's output rows (tile t, row
    // col); the weights load with the pass's first copies, not after the k
    // loop
    int pr[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) pr[t] = dma::list_entry(held, min(t * 16 + col, mrows - 1));
    auto pair_of = [&](int r) { return dma::list_entry(held, r); };
    auto row_of = [&](int r) { return aq + (size_t)pair_of(r) * I; };
    float pw[4];
    // once the pass's first copies are issued: the token scales, the routing
    // weights and, in the first pass, this wave's weight scales
    auto stage = [&]() {
      stage_token_scales(asl, as_, nkb, mrows, pair_of);
#pragma unroll
      for (int t = 0; t < 4; ++t) pw[t] = topk_w[pr[t]];
      if (m0 == 0)
        for (int q = lane; q < 2 * NP * nkb; q += 64) wsl[q] = q < 64 ? ws0 : *wscale_at(q);
    };
    f32x4 acc[2][4];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto run = [&](auto nt) {
      constexpr int NT = decltype(nt)::value;
      dma::pass<32, S, NT>(smem, wrow, mrows, row_of, NP * nkb, off,
                           [&](const unsigned char* ws, const unsigned char* ts, int q) {
                             const int pn = NP > 1 ? q / nkb : 0;
                             const int c = q - pn * nkb;
                             i32x8 a[2];
                             float sw[2];
#pragma unroll
                             for (int g = 0; g < 2; ++g) {
                               a[g] = lds_operand(ws, g * 16 + col, grp);
                               sw[g] = wsl[(2 * pn + g) * nkb + c];
                             }
#pragma unroll
                             for (int t = 0; t < NT; ++t) {
                               const i32x8 b = lds_operand(ts, t * 16 + col, grp);
                               const float sa = asl[(t * 16 + col) * nkb + c];
#pragma unroll
                               for (int g = 0; g < 2; ++g) {
                                 const f32x4 d = mfma_fp8(a[g], b);
#pragma unroll
                                 for (int j = 0; j < 4; ++j)
                                   acc[g][t][j] = acc[g][t][j] + (d[j] * sa) * sw[g];
                               }
                             }
                             if (NP > 1 && c == nkb - 1) {
                               // the panel's last k-block: its outputs, then
                               // fresh sums for the next panel
                               store_w2_tile(y, H, hb + pn * 128, pr, pw, mrows, col, grp, acc);
#pragma unroll
                               for (int g = 0; g < 2; ++g)
#pragma unroll
                                 for (int t = 0; t < 4; ++t) acc[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
                             }
                           }, stage, m0 == 0);
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
    if (NP == 1) store_w2_tile(y, H, hb, pr, pw, mrows, col, grp, acc);
  }
}

// out[t, h] = moe_sum over k ascending of y[(t, k), h]: bf16 adds for K in
// {2, 3, 4}, else one float32 sum rounded once.  grid = (ceil(H / 256), T).
__global__ __launch_bounds__(256) void fp8_combine_kernel(const uint16_t* __restrict__ y, int H,
                                                          int K, int nslots,
                                                          const int32_t* __restrict__ slots,
                                                          uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  const bool bf16_adds = K >= 2 && K <= 4;
  float sum = 0.f;
  for (int k = 0; k < K; ++k) {
    const int p = t * K + k;
    const int s = slots[p];
    const float v = (s < 0 || s >= nslots) ? 0.f : bf16f(y[(size_t)p * H + h]);
    sum = bf16_adds ? round_bf16(sum + v) : sum + v;
  }
  out[(size_t)t * H + h] = bf16_rne(sum);
}

// Work buffer of the grouped path (bytes, each piece 256-byte aligned).
struct Fp8Work {
  size_t lists, counts, y, xq, xs, aq, as, total;
  Fp8Work(int T, int K, int H, int I, int nslots) {
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t P = (size_t)T * K;
    lists = 0;
    counts = up((size_t)nslots * P * 4);
    y = counts + up((size_t)nslots * 4);
    xq = y + up(P * H * 2);
    xs = xq + up((size_t)T * H);
    aq = xs + up((size_t)T * (H / kKB) * 4);
    as = aq + up(P * I);
    total = as + up(P * (I / kKB) * 4);
  }
};

size_t w13_lds(int NW, int ncol) {
  return (size_t)NW * 2 * 64 * 4 * sizeof(float) + (size_t)NW * kKC * ncol * (4 + kKB);
}

size_t w2_lds(int K, int I, int WP) {
  return (size_t)K * I + (size_t)K * (I / kKB) * sizeof(float) +
         (size_t)K * WP * 16 * sizeof(float);
}

// Waves per w13 block: four up to H = 2048, eight above (a wave then loops
// over chunks of kKC k-blocks).
int w13_waves(int H) { return H / kKB <= 4 * kKC ? 4 : 8; }

struct W13Args {
  const uint16_t* x;
  int H, I, K, P;
  const int32_t* slots;
  int nslots;
  const uint8_t* w13;
  size_t w13_stride;
  const float* s13;
  size_t s13_stride;
  int block_n;
  uint16_t* act;
};

template <int NW, int NCOL, bool BIG>
hipError_t launch_w13(const W13Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  static std::atomic<uint64_t> big_lds{0};
  const auto kern = &fp8_w13_kernel<NW, NCOL, BIG>;
  const size_t lds = w13_lds(NW, NCOL);
  hipError_t e = allow_lds(kern, lds, kMaxLds, &big_lds);
  if (e != hipSuccess) return e;
  const dim3 grid(a.I / 16, a.P), block(NW * 64);
  if (e0)
    hipExtLaunchKernelGGL(kern, grid, block, lds, st, e0, e1, 0, a.x, a.H, a.I, a.K, a.P, a.slots,
                          a.nslots, a.w13, a.w13_stride, a.s13, a.s13_stride, a.block_n, a.act);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, st, a.x, a.H, a.I, a.K, a.P, a.slots, a.nslots,
                       a.w13, a.w13_stride, a.s13, a.s13_stride, a.block_n, a.act);
  return hipGetLastError();
}

// The one-token w13 kernel: one block per (8-output tile, pair), or per
// (tile, slot) with SLOTS.
template <int NW, int KC, bool SLOTS>
hipError_t launch_w13_one(const W13Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  static std::atomic<uint64_t> big_lds{0};
  const auto kern = &fp8_w13_one_kernel<NW, KC, SLOTS>;
  const size_t lds = (size_t)NW * 2 * 64 * 4 * sizeof(float) + (size_t)NW * KC * (4 + kKB);
  hipError_t e = allow_lds(kern, lds, kMaxLds, &big_lds);
  if (e != hipSuccess) return e;
  const dim3 grid(a.I / 8, SLOTS ? a.nslots : a.P), block(NW * 64);
  if (e0)
    hipExtLaunchKernelGGL(kern, grid, block, lds, st, e0, e1, 0, a.x, a.H, a.I, a.K, a.slots,
                          a.nslots, a.w13, a.w13_stride, a.s13, a.s13_stride, a.block_n, a.act);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, st, a.x, a.H, a.I, a.K, a.slots, a.nslots, a.w13,
                       a.w13_stride, a.s13, a.s13_stride, a.block_n, a.act);
  return hipGetLastError();
}

struct W2Args {
  const uint16_t* act;
  int H, I, K, T;
  const float* topk_w;
  const int32_t* slots;
  int nslots;
  const uint8_t* w2;
  size_t w2_stride;
  const float* s2;
  size_t s2_stride;
  int block_n, WP;
  uint16_t* out;
};

template <int KC2, int QP>
hipError_t launch_w2(const W2Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  static std::atomic<uint64_t> big_lds{0};
  const auto kern = &fp8_w2_kernel<kW2Waves, KC2, QP>;
  const size_t lds = w2_lds(a.K, a.I, a.WP);
  hipError_t e = allow_lds(kern, lds, kMaxLds, &big_lds);
  if (e != hipSuccess) return e;
  const dim3 grid(a.H / 16, a.T), block(kW2Waves * 64);
  if (e0)
    hipExtLaunchKernelGGL(kern, grid, block, lds, st, e0, e1, 0, a.act, a.H, a.I, a.K, a.topk_w,
                          a.slots, a.nslots, a.w2, a.w2_stride, a.s2, a.s2_stride, a.block_n,
                          a.WP, a.out);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, st, a.act, a.H, a.I, a.K, a.topk_w, a.slots,
                       a.nslots, a.w2, a.w2_stride, a.s2, a.s2_stride, a.block_n, a.WP, a.out);
  return hipGetLastError();
}

// The one-token w2 kernel for I = KB * 128.
template <int KB, bool SLOTS>
hipError_t launch_w2_one(const W2Args& a, hipStream_t st, hipEvent_t e0, hipEvent_t e1) {
  static std::atomic<uint64_t> big_lds{0};
  const auto kern = &fp8_w2_one_kernel<KB, SLOTS>;
  const size_t lds = (size_t)a.K * a.I + (size_t)a.K * KB * 4 + (size_t)a.K * 16 * 4;
  hipError_t e = allow_lds(kern, lds, kMaxLds, &big_lds);
  if (e != hipSuccess) return e;
  const dim3 grid(a.H / 16), block(a.K * 64);
  if (e0)
    hipExtLaunchKernelGGL(kern, grid, block, lds, st, e0, e1, 0, a.act, a.H, a.I, a.K, a.topk_w,
                          a.slots, a.nslots, a.w2, a.w2_stride, a.s2, a.s2_stride, a.block_n,
                          a.out);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, st, a.act, a.H, a.I, a.K, a.topk_w, a.slots,
                       a.nslots, a.w2, a.w2_stride, a.s2, a.s2_stride, a.block_n, a.out);
  return hipGetLastError();
}

using L2 = hipError_t (*)(const W2Args&, hipStream_t, hipEvent_t, hipEvent_t);

template <bool SLOTS>
L2 pick_w2_one(int kb) {
  switch (kb) {
    case 1: return &launch_w2_one<1, SLOTS>;
    case 2: return &launch_w2_one<2, SLOTS>;
    case 3: return &launch_w2_one<3, SLOTS>;
    case 4: return &launch_w2_one<4, SLOTS>;
    case 5: return &launch_w2_one<5, SLOTS>;
    case 6: return &launch_w2_one<6, SLOTS>;
    case 7: return &launch_w2_one<7, SLOTS>;
    case 8: return &launch_w2_one<8, SLOTS>;
    default: return nullptr;
  }
}

}  // namespace

const char* fp8_unsupported(int H, int I, int K, int block_n, int block_k) {
  if (block_k != kKB) return "block-FP8 kernels need block_k == 128";
  if (block_n < 16 || block_n % 16) return "block-FP8 kernels need block_n a multiple of 16";
  if (H < kKB || I < kKB || H % kKB || I % kKB)
    return "block-FP8 kernels need H and I multiples of 128";
  if (I % block_n)
    return "block-FP8 experts need I a multiple of block_n (the w13 scale rows of gate and up)";
  if (K < 1 || w2_lds(K, I, 1) > kMaxLds) return "top_k * I exceeds the w2 kernel's LDS";
  return nullptr;
}

// The LDS-staged kernels with the activation quantisation between them.
template <int S13, int S2, int NP2>
bool launch_grouped_dma(const uint8_t* xq, const float* xs, uint8_t* aq, float* as, int T, int H,
                        int I, int K, int nslots, const int32_t* lists, const int32_t* counts,
                        const float* topk_w, const uint8_t* w13, size_t w13_stride,
                        const float* s13, size_t s13_stride, const uint8_t* w2, size_t w2_stride,
                        const float* s2, size_t s2_stride, int block_n, uint16_t* act,
                        uint16_t* y, hipStream_t st, const StageEvents* ev) {
  const size_t l13 = fp8_dma_lds<S13>(H / kKB), l2 = fp8_dma_lds<S2, NP2>(I / kKB);
  if (l13 > kMaxLds || l2 > kMaxLds || H % (128 * NP2)) return false;
  static std::atomic<uint64_t> big13{0}, big2{0};
  if (allow_lds(&fp8_w13_dma_kernel<S13>, l13, kMaxLds, &big13) != hipSuccess ||
      allow_lds(&fp8_w2_dma_kernel<S2, NP2>, l2, kMaxLds, &big2) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const int P = T * K;
  hipEvent_t e0 = ev ? ev->ev[0] : nullptr, e1 = ev ? ev->ev[1] : nullptr;
  hipEvent_t e2 = ev ? ev->ev[2] : nullptr, e3 = ev ? ev->ev[3] : nullptr;
  launch_timed_lds(fp8_w13_dma_kernel<S13>, dim3(I / 64, nslots), dim3(256), (unsigned)l13, st,
                   e0, e1, xq, xs, H, I, K, P, lists, counts, w13, w13_stride, s13, s13_stride,
                   block_n, act);
  const long jobs = (long)P * (I / kKB);
  hipLaunchKernelGGL(quant_groups_kernel<uint16_t>, dim3((unsigned)((jobs + 15) / 16)),
                     dim3(256), 0, st, (const uint16_t*)act, P, I, aq, as);
  launch_timed_lds(fp8_w2_dma_kernel<S2, NP2>, dim3(H / (128 * NP2), nslots), dim3(256),
                   (unsigned)l2, st, e2,
                   e3, aq, as, H, I, P, lists, counts, topk_w, w2, w2_stride, s2, s2_stride,
                   block_n, y);
  return true;
}

template <int MT, int U>
void launch_grouped(const uint8_t* xq, const float* xs, uint8_t* aq, float* as, int T, int H,
                    int I, int K, int nslots, const int32_t* lists, const int32_t* counts,
                    const float* topk_w, const uint8_t* w13, size_t w13_stride, const float* s13,
                    size_t s13_stride, const uint8_t* w2, size_t w2_stride, const float* s2,
                    size_t s2_stride, int block_n, uint16_t* act, uint16_t* y, hipStream_t st,
                    const StageEvents* ev) {
  const int P = T * K;
  hipEvent_t e0 = ev ? ev->ev[0] : nullptr, e1 = ev ? ev->ev[1] : nullptr;
  hipEvent_t e2 = ev ? ev->ev[2] : nullptr, e3 = ev ? ev->ev[3] : nullptr;
  launch_timed(fp8_grouped_w13_kernel<MT, U>, dim3(I / 64, nslots), dim3(256), st, e0, e1, xq, xs,
               H, I, K, P, lists, counts, w13, w13_stride, s13, s13_stride, block_n, act);
  const long jobs = (long)P * (I / kKB);
  hipLaunchKernelGGL(quant_groups_kernel<uint16_t>, dim3((unsigned)((jobs + 15) / 16)),
                     dim3(256), 0, st, (const uint16_t*)act, P, I, aq, as);
  launch_timed(fp8_grouped_w2_kernel<MT, U>, dim3(H / 64, nslots), dim3(256), st, e2, e3, aq, as,
               H, I, P, lists, counts, topk_w, w2, w2_stride, s2, s2_stride, block_n, y);
}

size_t fp8_work_bytes(int T, int K, int H, int I, int nslots) {
  if (T < 1 || K < 1 || H < kKB || I < kKB || nslots < 1) return 0;
  return Fp8Work(T, K, H, I, nslots).total;
}

int experts_fp8_grouped(const void* x, int T, int H, int I, int K, const float* topk_w,
                        const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                        const float* s13, size_t s13_stride, const void* w2, size_t w2_stride,
                        const float* s2, size_t s2_stride, int block_n, void* act, void* out,
                        void* work, size_t work_bytes, hipStream_t st, const StageEvents* ev) {
  if (T == 0) return WISP_OK;
  const Fp8Work W(T, K, H, I, nslots);
  if (nslots > 65535 || !work || work_bytes < W.total || ((uintptr_t)work) % 256) {
    wisp_set_last_error("block-FP8 grouped path: work buffer missing, misaligned or too small",
                        "FP8 experts");
    return WISP_ERR_INVALID;
  }
  char* wb = (char*)work;
  int32_t* lists = (int32_t*)(wb + W.lists);
  int32_t* counts = (int32_t*)(wb + W.counts);
  uint16_t* y = (uint16_t*)(wb + W.y);
  uint8_t* xq = (uint8_t*)(wb + W.xq);
  float* xs = (float*)(wb + W.xs);
  uint8_t* aq = (uint8_t*)(wb + W.aq);
  float* as = (float*)(wb + W.as);
  const int P = T * K;
  launch_gather(slots, P, nslots, lists, counts, st);
  const long jobs = (long)T * (H / kKB);
  hipLaunchKernelGGL(quant_groups_kernel<uint16_t>, dim3((unsigned)((jobs + 15) / 16)),
                     dim3(256), 0, st, (const uint16_t*)x, T, H, xq, xs);
  const uint8_t* a13 = (const uint8_t*)w13;
  const uint8_t* a2 = (const uint8_t*)w2;
  uint16_t* ab = (uint16_t*)act;
  // above 16 tokens the LDS-staged kernels (at 16 the register-streaming
  // ones are faster here: 97 against 102 us at the Qwen3-FP8 shape, resident);
  // they return false where their LDS would not fit
  // w13 with two stages: an fp8 row is half a bf16 row's bytes, so its k
  // loop is short (16 chunks at the Qwen3 shape), and with 48 KiB of stages
  // three blocks fit per CU and overlap each other's setup (157 against
  // 172 us for the Qwen3-FP8 512-token chunk with three stages, measured on
  // MI355X).  w2 (6 chunks per 128-row panel) with four panels per block and
  // three stages: two blocks per CU, each with two chunks in flight.
  // Measured at the Qwen3-FP8 shape, two runs each: bs=32 step 30.4 / 30.4
  // against 33.7 / 33.7 us with one panel per block and 31.7 / 31.6 us with
  // four panels and two stages; 512-token chunk 47.9 / 48.0 against
  // 50.0 / 50.5 and 48.8 / 48.9 us.  Two panels per block with two stages
  // leave a tail (1,024 blocks over 768 block slots).
  constexpr int kNP = 4;
  const int np2 = H % (128 * kNP) == 0 ? kNP : H % 256 == 0 ? 2 : 1;
  auto dma = np2 == kNP ? &launch_grouped_dma<2, 3, kNP>
             : np2 == 2 ? &launch_grouped_dma<2, 3, 2>
                        : &launch_grouped_dma<2, 3, 1>;
  if (T > 16 && dma(xq, xs, aq, as, T, H, I, K, nslots, lists, counts, topk_w,
                    (const uint8_t*)w13, w13_stride, s13, s13_stride, (const uint8_t*)w2,
                    w2_stride, s2, s2_stride, block_n, (uint16_t*)act, y, st, ev)) {
    hipLaunchKernelGGL(fp8_combine_kernel, dim3((H + 255) / 256, T), dim3(256), 0, st, y, H, K,
                       nslots, slots, (uint16_t*)out);
    WISP_HIP_TRY(hipGetLastError());
    return WISP_OK;
  }
  // two k-blocks per iteration when both k extents allow it; 16-token tiles
  // per pass: a slot holds at most T tokens
  const bool u2 = (H / kKB) % 2 == 0 && (I / kKB) % 2 == 0;
  const int mt = T <= 16 ? 1 : T <= 128 ? 2 : 4;
#define WISP_GROUPED(MT_, U_)                                                                 \
  launch_grouped<MT_, U_>(xq, xs, aq, as, T, H, I, K, nslots, lists, counts, topk_w, a13,    \
                          w13_stride, s13, s13_stride, a2, w2_stride, s2, s2_stride, block_n, \
                          ab, y, st, ev)
  if (u2) {
    if (mt == 1) WISP_GROUPED(1, 2);
    else if (mt == 2) WISP_GROUPED(2, 2);
    else WISP_GROUPED(4, 2);
  } else {
    if (mt == 1) WISP_GROUPED(1, 1);
    else if (mt == 2) WISP_GROUPED(2, 1);
    else WISP_GROUPED(4, 1);
  }
#undef WISP_GROUPED
  hipLaunchKernelGGL(fp8_combine_kernel, dim3((H + 255) / 256, T), dim3(256), 0, st, y, H, K,
                     nslots, slots, (uint16_t*)out);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

// pager_slots: the slots come from the pager, so a token's pairs name
// distinct slots of the scratch, and a one-token call with K == nslots
// fills every slot (the one-token kernels then lay their work out by slot).
int experts_fp8(const void* x, int T, int H, int I, int K, const float* topk_w,
                const int32_t* slots, int nslots, const void* w13, size_t w13_stride,
                const float* s13, size_t s13_stride, const void* w2, size_t w2_stride,
                const float* s2, size_t s2_stride, int block_n, void* act, void* out,
                hipStream_t st, const StageEvents* ev, bool pager_slots) {
  if (T == 0) return WISP_OK;
  const int P = T * K;
  const W13Args a13 = {(const uint16_t*)x, H, I, K, P, slots, nslots, (const uint8_t*)w13,
                       w13_stride, s13, s13_stride, block_n, (uint16_t*)act};
  hipEvent_t e0 = ev ? ev->ev[0] : nullptr, e1 = ev ? ev->ev[1] : nullptr;
  const bool by_slot = T == 1 && pager_slots && K == nslots;
  // MFMA columns per pass: a decode token needs one; pairs sharing a slot
  // are at most T (a token's experts are distinct)
  const int ncol = T == 1 ? 1 : T <= 4 ? 4 : 16;
  const bool big = P > kPairRegs * 64;
  using L13 = hipError_t (*)(const W13Args&, hipStream_t, hipEvent_t, hipEvent_t);
  L13 l13;
  // one-token kernel: eight waves of two k-blocks each up to H = 2048
  // (measured at the Qwen3-FP8 decode shape: 7.48 us, against 7.61 us for
  // four waves of four and 7.77 us for sixteen waves of one), of four above
  if (ncol == 1)
    l13 = H / kKB <= 16 ? (by_slot ? &launch_w13_one<8, 2, true>
                                   : &launch_w13_one<8, 2, false>)
                        : (by_slot ? &launch_w13_one<8, kKC, true>
                                   : &launch_w13_one<8, kKC, false>);
  else if (w13_waves(H) == 4)
    l13 = ncol == 4 ? &launch_w13<4, 4, false>
        : big ? &launch_w13<4, 16, true> : &launch_w13<4, 16, false>;
  else
    l13 = ncol == 4 ? &launch_w13<8, 4, false>
        : big ? &launch_w13<8, 16, true> : &launch_w13<8, 16, false>;
  WISP_HIP_TRY(l13(a13, st, e0, e1));
  return experts_fp8_w2(act, T, H, I, K, topk_w, slots, nslots, w2, w2_stride, s2, s2_stride,
                        block_n, out, st, ev ? ev->ev[2] : nullptr, ev ? ev->ev[3] : nullptr,
                        pager_slots);
}

// The w2 stage of experts_fp8 (routing weights and moe_sum fused).
int experts_fp8_w2(const void* act, int T, int H, int I, int K, const float* topk_w,
                   const int32_t* slots, int nslots, const void* w2, size_t w2_stride,
                   const float* s2, size_t s2_stride, int block_n, void* out, hipStream_t st,
                   hipEvent_t e0, hipEvent_t e1, bool pager_slots) {
  if (T == 0) return WISP_OK;
  const bool by_slot = T == 1 && pager_slots && K == nslots;
  // waves per pair: split I's k-blocks when there are fewer pairs than waves
  int WP = K >= kW2Waves ? 1 : kW2Waves / K;
  while (WP > 1 && w2_lds(K, I, WP) > kMaxLds) WP >>= 1;
  const int per = (I / kKB + WP - 1) / WP;
  const int kc2 = per <= 4 ? 4 : per <= 6 ? 6 : per <= 8 || per % 8 == 0 ? 8 : per % 6 == 0 ? 6 : 8;
  const W2Args a2 = {(const uint16_t*)act, H, I, K, T, topk_w, slots, nslots, (const uint8_t*)w2,
                     w2_stride, s2, s2_stride, block_n, WP, (uint16_t*)out};
  // quantisation passes a wave needs (4 groups each), capped at 4 per round
  const int passes = (K * (I / kKB) + kW2Waves * 4 - 1) / (kW2Waves * 4);
  L2 l2 = nullptr;
  if (T == 1 && K <= 16)  // one wave per pair or slot
    l2 = by_slot ? pick_w2_one<true>(I / kKB) : pick_w2_one<false>(I / kKB);
  if (!l2) {
    if (passes <= 1)
      l2 = kc2 == 4 ? &launch_w2<4, 1> : kc2 == 6 ? &launch_w2<6, 1> : &launch_w2<8, 1>;
    else if (passes <= 2)
      l2 = kc2 == 4 ? &launch_w2<4, 2> : kc2 == 6 ? &launch_w2<6, 2> : &launch_w2<8, 2>;
    else
      l2 = kc2 == 4 ? &launch_w2<4, 4> : kc2 == 6 ? &launch_w2<6, 4> : &launch_w2<8, 4>;
  }
  WISP_HIP_TRY(l2(a2, st, e0, e1));
  return WISP_OK;
}

namespace {

template <int NW, int KC, int PER, bool SLOTS>
hipError_t launch_pagein_fp8_w13(const Fp8FusedArgs& f, const PageInArgs& a, hipStream_t st,
                                 hipEvent_t e0, hipEvent_t e1) {
  static std::atomic<uint64_t> big_lds{0};
  const auto kern = &pagein_fp8_w13_kernel<NW, KC, PER, SLOTS>;
  const int nkb = f.H / kKB;
  const size_t red = (size_t)NW * 2 * 64 * 4 * sizeof(float);
  const size_t lds = std::max(red + (size_t)NW * KC * (4 + kKB),
                              fp8_copy_stage_off(NW, nkb) + (size_t)NW * PER * 16 * kKB);
  hipError_t e = allow_lds(kern, lds, kMaxLds, &big_lds);
  if (e != hipSuccess) return e;
  const dim3 grid(kFp8CopyBlocks + f.I / 8 * (SLOTS ? f.nslots : f.K)), block(NW * 64);
  if (e0)
    hipExtLaunchKernelGGL(kern, grid, block, lds, st, e0, e1, 0, f, a);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, st, f, a);
  return hipGetLastError();
}

}  // namespace

// Whether pagein_fp8_w13 serves a layer of hidden size H (its copy blocks
// give every wave H / kKB / 8 whole k-blocks).
bool fp8_fused_supported(int H) { return H == 16 * kKB || H == 8 * kKB; }

// Page-in of the experts the pager loaded (a.count = flags) and the w13
// stage of a one-token call in one launch; the layer's masters and scratch
// hold one [w13 | w2 | s13 | s2] slab per expert (plane 0), the w13 scales
// at byte s13_off of it.
int pagein_fp8_w13(const PageInArgs& a, const void* x, int H, int I, int K,
                   const int32_t* slots, const int32_t* flags, int nslots, const void* w13,
                   size_t w13_stride, const float* s13, size_t s13_stride, int block_n,
                   size_t s13_off, void* act, hipStream_t st, hipEvent_t e0, hipEvent_t e1,
                   bool pager_slots) {
  const Fp8FusedArgs f = {(const uint16_t*)x, slots, flags + 1, (const uint8_t*)w13, w13_stride,
                          s13, s13_stride, (uint16_t*)act, s13_off, H, I, K, nslots, block_n};
  const bool by_slot = pager_slots && K == nslots;
  hipError_t e;
  if (H == 16 * kKB)
    e = by_slot ? launch_pagein_fp8_w13<8, 2, 2, true>(f, a, st, e0, e1)
                : launch_pagein_fp8_w13<8, 2, 2, false>(f, a, st, e0, e1);
  else if (H == 8 * kKB)
    e = by_slot ? launch_pagein_fp8_w13<8, 2, 1, true>(f, a, st, e0, e1)
                : launch_pagein_fp8_w13<8, 2, 1, false>(f, a, st, e0, e1);
  else
    return WISP_ERR_UNSUPPORTED;
  WISP_HIP_TRY(e);
  return WISP_OK;
}

}  // namespace wisp

extern "C" int wisp_quant_fp8_groups(const void* x, int dtype, int rows, int cols, int group,
                                     uint8_t* q, float* scales, wisp_stream_t stream) {
  using namespace wisp;
  if (rows < 0 || cols < 0 || (rows > 0 && cols > 0 && (!x || !q || !scales)) ||
      (dtype != WISP_F32 && dtype != WISP_BF16))
    return WISP_ERR_INVALID;
  if (group != kKB || cols % kKB || ((uintptr_t)x) % 16 || ((uintptr_t)q) % 8) {
    wisp_set_last_error("group must be 128, cols a multiple of it, x 16-byte and q 8-byte "
                        "aligned", "wisp_quant_fp8_groups");
    return WISP_ERR_UNSUPPORTED;
  }
  const long jobs = (long)rows * (cols / kKB);
  if (jobs == 0) return WISP_OK;
  const dim3 grid((unsigned)((jobs + 15) / 16));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == WISP_BF16)
    hipLaunchKernelGGL(quant_groups_kernel<uint16_t>, grid, dim3(256), 0, st,
                       (const uint16_t*)x, rows, cols, q, scales);
  else
    hipLaunchKernelGGL(quant_groups_kernel<float>, grid, dim3(256), 0, st, (const float*)x, rows,
                       cols, q, scales);
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

extern "C" int wisp_moe_experts_fp8(const void* x, int T, int H, int I, int K,
                                    const float* topk_w, const int32_t* slots, int nslots,
                                    const void* w13, size_t w13_stride, const float* s13,
                                    size_t s13_stride, const void* w2, size_t w2_stride,
                                    const float* s2, size_t s2_stride, int block_n, int block_k,
                                    void* act, void* out, void* work, size_t work_bytes,
                                    int algo, wisp_stream_t stream) {
  using namespace wisp;
  if (T < 0 || K < 1 || K > kMaxTopK || nslots < 1 ||
      (T > 0 && (!x || !topk_w || !slots || !w13 || !w2 || !s13 || !s2 || !act || !out)))
    return WISP_ERR_INVALID;
  if (algo != WISP_ALGO_AUTO && algo != WISP_ALGO_GEMV && algo != WISP_ALGO_MFMA)
    return WISP_ERR_INVALID;
  const char* why = fp8_unsupported(H, I, K, block_n, block_k);
  if (!why && (w13_stride % 16 || w2_stride % 16 || ((uintptr_t)w13) % 16 ||
               ((uintptr_t)w2) % 16 || ((uintptr_t)s13) % 4 || ((uintptr_t)s2) % 4 ||
               (T > 0 && (((uintptr_t)x) % 16 || ((uintptr_t)act) % 16 ||
                          ((uintptr_t)out) % 16))))
    why = "weights, strides and buffers must be 16-byte aligned";
  if (why) {
    wisp_set_last_error(why, "wisp_moe_experts_fp8");
    return WISP_ERR_UNSUPPORTED;
  }
  const int a = algo == WISP_ALGO_AUTO ? auto_algo(WISP_FP8_E4M3, H, I, T, K) : algo;
  if (a == WISP_ALGO_MFMA)
    return experts_fp8_grouped(x, T, H, I, K, topk_w, slots, nslots, w13, w13_stride, s13,
                               s13_stride, w2, w2_stride, s2, s2_stride, block_n, act, out, work,
                               work_bytes, (hipStream_t)stream, nullptr);
  return experts_fp8(x, T, H, I, K, topk_w, slots, nslots, w13, w13_stride, s13, s13_stride, w2,
                     w2_stride, s2, s2_stride, block_n, act, out, (hipStream_t)stream, nullptr,
                     false);
}

extern "C" size_t wisp_moe_fp8_work_bytes(int T, int K, int H, int I, int nslots) {
  return wisp::fp8_work_bytes(T, K, H, I, nslots);
}
