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

// Inclusive prefix OR across the 64 lanes: OR of v over lanes 0..lane.
// Four DPP row shifts inside each 16-lane row, then the row totals by
// readlane.
__device__ inline uint32_t wave_prefix_or(uint32_t v, int lane) {
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 47);
  const int row = lane >> 4;
  return v | (row >= 1 ? r0 : 0u) | (row >= 2 ? r1 : 0u) | (row >= 3 ? r2 : 0u);
}

// OR of v over the 64 lanes (wave-uniform): the row prefix ORs of
// wave_prefix_or, then the four row totals by readlane.
__device__ inline uint32_t wave_or(uint32_t v) {
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);  // row_shr:8
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 15) |
         (uint32_t)__builtin_amdgcn_readlane((int)v, 31) |
         (uint32_t)__builtin_amdgcn_readlane((int)v, 47) |
         (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

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

// Slot of `key` inserted into a CPython set table of mask+1 <= 32 slots with
// occupancy `occ` (scalar); marks it occupied.  Same probe sequence as
// set_insert_clean: slot i, then i+1 .. i+9 when i + 9 <= mask, then the
// perturbed step.
__device__ inline int probe_insert32(uint32_t& occ, uint32_t mask, int key) {
  uint32_t perturb = (uint32_t)key;
  uint32_t i = (uint32_t)key & mask;
  for (;;) {
    const uint32_t win = i + 9 <= mask ? 0x3FFu : 1u;
    const uint32_t free = ~(occ >> i) & win;
    if (free) {
      const uint32_t s = i + (uint32_t)__builtin_ctz(free);
      occ |= 1u << s;
      return (int)s;
    }
    perturb >>= 5;
    i = (i * 5 + 1 + perturb) & mask;
  }
}

// set_positions_wave for U <= 18 keys, whose table is 8 slots up to 4 keys
// and 32 slots from the resize at the fifth.  Key j is held by lane j and
// inserted j-th.
//   * When no two keys share a home slot (key & mask of the final table),
//     no insertion probes, whatever the order: every key sits at its home
//     slot, and the order is the home slots ascending.
//   * Otherwise the insertions run in scalar registers (occupancy words, the
//     8-slot table's key per slot in a packed word, so the resize re-inserts
//     its keys by walking the occupied slots), the lanes touched only to hand
//     each key its slot.
__device__ inline int set_positions_small(int key, int U, int lane) {
  const bool mine = lane < U;
  const uint32_t home_mask = U < 5 ? 7u : 31u;
  const uint32_t home = mine ? 1u << ((uint32_t)key & home_mask) : 0u;
  const uint32_t homes = wave_or(home);
  if (__popc(homes) == U) return mine ? __popc(homes & (home - 1u)) : -1;
  uint32_t occ = 0, mask = 7;
  uint32_t key_at = 0;  // 8-slot table: index of the key in slot s, 4 bits per slot
  int myslot = -1;
  const int n8 = U < 5 ? U : 5;
  for (int j = 0; j < n8; ++j) {
    const int s = probe_insert32(occ, mask, __builtin_amdgcn_readlane(key, j));
    key_at |= (uint32_t)j << (4 * s);
    if (lane == j) myslot = s;
  }
  if (U >= 5) {
    // resize to 32 slots: the five keys again, in 8-slot table order
    uint32_t left = occ;
    occ = 0;
    mask = 31;
    while (left) {
      const int sl = __builtin_ctz(left);
      left &= left - 1u;
      const int j = (int)((key_at >> (4 * sl)) & 15u);
      const int s = probe_insert32(occ, mask, __builtin_amdgcn_readlane(key, j));
      if (lane == j) myslot = s;
    }
    for (int j = 5; j < U; ++j) {
      const int s = probe_insert32(occ, mask, __builtin_amdgcn_readlane(key, j));
      if (lane == j) myslot = s;
    }
  }
  if (!mine) return -1;
  return __popc(occ & ((1u << myslot) - 1u));
}

// Writes to order[0..n) the CPython iteration order of a set built by
// inserting keys[0..n) (distinct) in array order.  keys, order and table
// (kMaxSetTable words) live in LDS; all lanes of the wave call it.
__device__ inline void set_order_wave(const int32_t* keys, int n, int32_t* order, int32_t* table,
                                      int lane) {
  if (n <= 64) {
    const int key = lane < n ? keys[lane] : -1;
    const int pos = n <= 18 ? set_positions_small(key, n, lane) : set_positions_wave(key, n, lane);
    if (lane < n) order[pos] = key;
  } else if (lane == 0) {
    cpython_set_order(keys, n, order, table, kMaxSetTable);
  }
  wave_lds_sync();
}

}  // namespace wisp
