// Wavefront helpers for CPython set iteration order (shared by the pager and
// the cross-layer prefetch kernels).
#pragma once

#include "common.h"
#include "pager_core.h"

namespace wisp {

__device__ inline int popc_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ inline uint64_t ballot(bool p) { return __ballot(p); }

// Insert `key` into a CPython set table of mask+1 <= 128 slots whose
// occupancy is the bitmask (lo, hi); returns the slot (same probe sequence as
// set_insert_clean).  All operands are wave-uniform.
__device__ inline int probe_insert(uint64_t& lo, uint64_t& hi, uint32_t mask, int key) {
  uint32_t perturb = (uint32_t)key;
  uint32_t i = (uint32_t)key & mask;
  for (;;) {
    if (i + 9 <= mask) {
      // the 10 linear probes at once: occupancy bits i .. i+9
      const uint64_t w = i >= 64 ? hi >> (i - 64) : i == 0 ? lo : (lo >> i) | (hi << (64 - i));
      const uint32_t free = ~(uint32_t)w & 0x3FFu;
      if (free) {
        const uint32_t s = i + (uint32_t)__builtin_ctz(free);
        if (s < 64) lo |= 1ull << s; else hi |= 1ull << (s - 64);
        return (int)s;
      }
    } else {
      uint64_t& w = i < 64 ? lo : hi;
      const uint64_t bit = 1ull << (i & 63);
      if (!(w & bit)) {
        w |= bit;
        return (int)i;
      }
    }
    perturb >>= 5;
    i = (i * 5 + 1 + perturb) & mask;
  }
}

// CPython set iteration position of each of U <= 64 ascending keys, key j
// held by lane j.  Tables stay <= 128 slots for U <= 64 (growth happens at 5
// and 19 keys), so the occupancy fits two 64-bit masks in scalar registers;
// a resize re-inserts the keys in old slot order.  Returns the position of
// this lane's key (lanes >= U return -1).
__device__ int set_positions_wave(int key, int U, int lane) {
  uint64_t lo = 0, hi = 0;
  uint32_t mask = 7;
  int myslot = -1;
  for (int j = 0; j < U; ++j) {
    const int kj = __builtin_amdgcn_readlane(key, j);
    const int s = probe_insert(lo, hi, mask, kj);
    if (lane == j) myslot = s;
    const int fill = j + 1;
    if ((uint32_t)fill * 5 >= mask * 3) {
      uint32_t newsize = 8;
      while (newsize <= (uint32_t)fill * 4) newsize <<= 1;
      uint64_t nlo = 0, nhi = 0;
      int newslot = -1;
      for (int half = 0; half < 2; ++half) {
        uint64_t bits = half ? hi : lo;
        while (bits) {
          const int sl = half * 64 + __builtin_ctzll(bits);
          bits &= bits - 1;
          const uint64_t who = __ballot(myslot == sl);
          const int l = __builtin_ctzll(who);
          const int kl = __builtin_amdgcn_readlane(key, l);
          const int ns = probe_insert(nlo, nhi, newsize - 1, kl);
          if (lane == l) newslot = ns;
        }
      }
      lo = nlo;
      hi = nhi;
      mask = newsize - 1;
      if (lane <= j) myslot = newslot;
    }
  }
  if (lane >= U) return -1;
  const uint64_t below_lo = myslot >= 64 ? lo : (lo & ((1ull << myslot) - 1));
  const uint64_t below_hi = myslot >= 64 ? (hi & ((1ull << (myslot - 64)) - 1)) : 0ull;
  return __popcll(below_lo) + __popcll(below_hi);
}

// Writes to order[0..n) the CPython iteration order of a set built by
// inserting keys[0..n) (distinct) in array order.  keys, order and table
// (kMaxSetTable words) live in LDS; all lanes of the wave call it.
__device__ inline void set_order_wave(const int32_t* keys, int n, int32_t* order, int32_t* table,
                                      int lane) {
  if (n <= 64) {
    const int key = lane < n ? keys[lane] : -1;
    const int pos = set_positions_wave(key, n, lane);
    if (lane < n) order[pos] = key;
  } else if (lane == 0) {
    cpython_set_order(keys, n, order, table, kMaxSetTable);
  }
  wave_lds_sync();
}

}  // namespace wisp
