// Device-driven page-in (kernel copies from pinned host masters).
#pragma once

#include "common.h"
#include "packed.h"

namespace wisp {

constexpr int kPageInBlocks = 64;

// One tensor of an expert that moves as a unit: expert e's bytes
// [m + e*m_stride, +bytes) of the pinned master (device address of its
// mapping) go to slot s at [d + s*d_stride, +bytes) of the HBM scratch.
// Strides and sizes are in bytes, all multiples of 16.
struct PageInPlane {
  const char* m;
  size_t m_stride;
  char* d;
  size_t d_stride;
  size_t bytes;
};

// At most four tensors per expert: w13, w2 and, for block-FP8 experts,
// their two scale tensors.  A layer whose tensors sit back to back in one
// slab per expert (in master and scratch alike) copies them as one plane.
constexpr int kMaxPlanes = 4;

// A bf16 layer's packed masters (packed.h): expert e at m + e * m_stride
// (the device address of their pinned, mapped host copy); its w13 rows
// unpack to slot s at d13 + s * d13_stride, its w2 rows at d2 + s *
// d2_stride (bytes).  m null: the planes are copied as they are.
struct PackedSrc {
  const char* m;
  size_t m_stride;
  int H, I;
  char* d13;
  size_t d13_stride;
  char* d2;
  size_t d2_stride;
};

// One page-in launch.  The load list holds (expert, slot) pairs; its length
// is *count when count is non-null (written by the pager kernel), else n.
struct PageInArgs {
  const int32_t* loads;
  const int32_t* count;
  int n;
  int num_experts, cap;
  int nplanes;
  PageInPlane p[kMaxPlanes];
  int32_t* hist;  // device address of a pinned host word that receives n, or null
  PackedSrc pk;
};

int launch_pagein(const PageInArgs& a, hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop);

// The pager wave's arguments in a fused one-token decode launch (page-in,
// w13 and the pager in one grid; the layer's call with top-k == cap).
struct DecodePagerArgs {
  const void* logits;  // [E] of the call's one token
  int renorm, E;
  float* topk_w;
  int32_t* topk_ids;
  int32_t* map;
  int32_t* s2e;
  int64_t* tick;
  int64_t* ctr;
  int32_t* slots;
  int32_t* loads;
  int32_t* rec;       // the device decision record
  uint32_t* sync;     // the launch's epoch, published by the pager wave
  uint32_t epoch;
  void* act_spec;     // [cap][I]: w13 per slot
};

constexpr int kPageInUnroll = 4;

// Copies `bytes` (a multiple of 16) from src to dst, spread over `nblocks`
// blocks of NT threads; `blk` is this block's index among them.  Each
// thread keeps kPageInUnroll 16-byte loads in flight (64 blocks of 256
// threads: 1 MiB).
template <int NT = 256>
__device__ inline void copy_range(const char* __restrict__ src, char* __restrict__ dst,
                                  size_t bytes, int blk, int nblocks) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4* s = reinterpret_cast<const u32x4*>(src);
  u32x4* d = reinterpret_cast<u32x4*>(dst);
  const size_t n = bytes >> 4;
  const size_t step = (size_t)nblocks * NT * kPageInUnroll;
  for (size_t base = (size_t)blk * NT * kPageInUnroll + threadIdx.x; base < n; base += step) {
    u32x4 v[kPageInUnroll];
#pragma unroll
    for (int u = 0; u < kPageInUnroll; ++u) {
      const size_t i = base + (size_t)u * NT;
      if (i < n) v[u] = s[i];
    }
#pragma unroll
    for (int u = 0; u < kPageInUnroll; ++u) {
      const size_t i = base + (size_t)u * NT;
      if (i < n) __builtin_nontemporal_store(v[u], d + i);
    }
  }
}

// Unpacks `rows` packed rows of L values from src (row r at src + r *
// row_bytes(L)) into bf16 rows at dst (row r at dst + r * 2L bytes), spread
// over `nblocks` blocks of NT threads (`blk`: this block's index), 32
// consecutive values (four chunks, half a block) a thread and UNR such
// groups in flight: two 16-byte sign/mantissa loads and one 16-byte code
// load per group.  exc is the expert's exception area.  Index math is 32-bit
// (an expert's rows hold fewer than 2^32 values).
template <int NT = 256, int UNR = 2>
__device__ inline void unpack_rows_wide(const char* __restrict__ src, int rows, int L,
                                        const char* __restrict__ exc, char* __restrict__ dst,
                                        int blk, int nblocks) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const unsigned ng = (unsigned)L / 32u, rb = (unsigned)packed::row_bytes(L);
  const unsigned n = (unsigned)rows * ng, step = (unsigned)nblocks * NT * UNR;
  const unsigned hdr = (unsigned)(L + L / 2), mo = hdr + (unsigned)packed::align_up(L / 64, 4);
  for (unsigned base = (unsigned)blk * NT * UNR + threadIdx.x; base < n; base += step) {
    u32x4 l0[UNR], l1[UNR], cd[UNR];
    uint32_t bs[UNR], mk[UNR];
    unsigned off[UNR], g[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const unsigned i = base + (unsigned)u * NT;
      const unsigned r = i < n ? i / ng : 0u;
      g[u] = i < n ? i - r * ng : 0u;
      off[u] = r * rb;
      if (i < n) {
        const char* row = src + off[u];
        l0[u] = *reinterpret_cast<const u32x4*>(row + 32u * g[u]);
        l1[u] = *reinterpret_cast<const u32x4*>(row + 32u * g[u] + 16u);
        cd[u] = *reinterpret_cast<const u32x4*>(row + (unsigned)L + 16u * g[u]);
        bs[u] = *reinterpret_cast<const uint8_t*>(row + hdr + (g[u] >> 1));
        mk[u] = *reinterpret_cast<const uint32_t*>(row + mo + 4u * (g[u] >> 6));
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const unsigned i = base + (unsigned)u * NT;
      if (i >= n) continue;
      u32x4* d = reinterpret_cast<u32x4*>(dst) + 4u * i;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const u32x4& l = t < 2 ? l0[u] : l1[u];
        packed::Chunk c;
        c.lo = (uint64_t)l[2 * (t & 1)] | ((uint64_t)l[2 * (t & 1) + 1] << 32);
        c.cd = cd[u][t];
        c.base = bs[u];
        c.mask = mk[u];
        const int q = (int)(4u * g[u]) + t;
        const uint4 v = packed::is_exception(c, q)
                            ? packed::unpack_chunk(c, src + off[u], L, q, exc)
                            : packed::unpack_plain(c);
        __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, d + t);
      }
    }
  }
}

// One loaded expert's whole packed slab into its slot, over `nblocks`
// blocks.
template <int NT = 256>
__device__ inline void unpack_expert(const PackedSrc& pk, int e, int s, int blk, int nblocks) {
  const packed::Layout Lp(pk.H, pk.I);
  const char* ex = pk.m + (size_t)e * pk.m_stride;
  unpack_rows_wide<NT>(ex, 2 * pk.I, pk.H, ex + Lp.exc_off, pk.d13 + (size_t)s * pk.d13_stride,
                       blk, nblocks);
  unpack_rows_wide<NT>(ex + Lp.w2_off, pk.H, pk.I, ex + Lp.exc_off,
                       pk.d2 + (size_t)s * pk.d2_stride, blk, nblocks);
}

// Device address of host memory [base, base + bytes) when that range lies
// inside one pinned, device-mapped host allocation; null otherwise.
const char* mapped_host_range(const void* base, size_t bytes);

}  // namespace wisp
