// Expert-pager semantics shared by the host and device implementations.
//
// The reference pager is WispMoEState.ensure_resident
// (src/wisp/integrations/vllm/fused_moe.py:264-358) driven by the greedy
// token sub-batching of _wisp_forward_cuda_paged (fused_moe.py:1102-1168).
// This header holds
//   * cpython_set_order: the iteration order of a CPython 3.10 set of small
//     non-negative ints inserted in ascending order (the order in which the
//     reference forms its `missing` list, fused_moe.py:279-283), computed
//     from CPython's published open-addressing scheme: table of 8 slots,
//     `i = hash & mask`, up to 9 linear probes when `i + 9 <= mask`, else
//     `perturb >>= 5; i = (5 i + 1 + perturb) & mask`; grow when
//     5 * fill >= 3 * mask to the smallest power of two above 4 * used,
//     re-inserting the old table in slot order;
//   * the decision-record layout the pager writes for the host;
//   * pager_decide_host: a sequential implementation of the whole layer call
//     used by CPU tests and as the specification the GPU kernel is checked
//     against.
#pragma once

#include <stdint.h>
#include <stddef.h>
#include <string.h>

#ifndef WISP_HD
#define WISP_HD __host__ __device__
#endif

namespace wisp {

// ---------------------------------------------------------------------------
// CPython set iteration order
// ---------------------------------------------------------------------------

WISP_HD inline void set_insert_clean(int32_t* table, uint32_t mask, int32_t key) {
  size_t perturb = (size_t)key;            // hash(i) == i for small ints
  size_t i = (size_t)key & mask;
  for (;;) {
    if (table[i] < 0) { table[i] = key; return; }
    if (i + 9 <= mask) {
      for (int j = 1; j <= 9; ++j) {
        if (table[i + j] < 0) { table[i + j] = key; return; }
      }
    }
    perturb >>= 5;
    i = (i * 5 + 1 + perturb) & mask;
  }
}

// keys: n distinct non-negative ints, ascending.  order: n outputs (must not
// alias keys).  table: scratch of table_cap ints.  Returns n, or -1 if the
// table would exceed table_cap.
WISP_HD inline int cpython_set_order(const int32_t* keys, int n, int32_t* order,
                                     int32_t* table, int table_cap) {
  if (table_cap < 8) return -1;
  uint32_t mask = 7;
  for (int s = 0; s < 8; ++s) table[s] = -1;
  int fill = 0;
  for (int j = 0; j < n; ++j) {
    set_insert_clean(table, mask, keys[j]);
    ++fill;
    if ((size_t)fill * 5 >= (size_t)mask * 3) {
      size_t minused = fill > 50000 ? (size_t)fill * 2 : (size_t)fill * 4;
      size_t newsize = 8;
      while (newsize <= minused) newsize <<= 1;
      if (newsize > (size_t)table_cap) return -1;
      int m = 0;
      for (uint32_t s = 0; s <= mask; ++s)
        if (table[s] >= 0) order[m++] = table[s];
      mask = (uint32_t)newsize - 1;
      for (uint32_t s = 0; s <= mask; ++s) table[s] = -1;
      for (int q = 0; q < m; ++q) set_insert_clean(table, mask, order[q]);
    }
  }
  int m = 0;
  for (uint32_t s = 0; s <= mask; ++s)
    if (table[s] >= 0) order[m++] = table[s];
  return m;
}

// ---------------------------------------------------------------------------
// Decision record (int32 words, written by the pager, read by the host)
// ---------------------------------------------------------------------------
//   header, 8 words:
//     [0] status (WISP_OK, WISP_ERR_SUBBATCH, WISP_ERR_INVALID)
//     [1] groups completed        [2] groups planned
//     [3] failing group or -1     [4] its unique-expert count
//     [5] evicted pairs in total  [6] loaded pairs in total
//     [7] reserved
//   groups, 8 words each, max_groups entries, starting at word 8:
//     t0, t1, n_needed, hits, evicted offset, n_evicted, loaded offset, n_loaded
//   evicted (expert, slot) pairs, max_pairs entries, in eviction order
//   loaded  (expert, slot) pairs, max_pairs entries, in load order
struct RecordLayout {
  int max_groups, max_pairs;
  WISP_HD RecordLayout(int T, int K)
      : max_groups(T > 0 ? T : 1), max_pairs(T * K > 0 ? T * K : 1) {}
  WISP_HD int group_base(int g) const { return 8 + 8 * g; }
  WISP_HD int evicted_base() const { return 8 + 8 * max_groups; }
  WISP_HD int loaded_base() const { return evicted_base() + 2 * max_pairs; }
  WISP_HD int words() const { return loaded_base() + 2 * max_pairs; }
};

enum RecordHeader : int {
  kRecStatus = 0,
  kRecGroupsDone = 1,
  kRecGroupsPlanned = 2,
  kRecFailGroup = 3,
  kRecFailUnique = 4,
  kRecEvicted = 5,
  kRecLoaded = 6,
};

// Per-pair word of the pager's flags array (flags[1 + p]): the pair's slot in
// the low 16 bits (0xFFFF: none) and, when the call loaded the pair's expert,
// that expert id + 1 in bits 16-30 (0 otherwise).  One load gives an expert
// kernel the slot, whether it was just loaded, and from which master.
WISP_HD inline int32_t pair_word(int slot, int loaded_expert) {
  return (int32_t)(((uint32_t)slot & 0xFFFFu) |
                   (loaded_expert >= 0 ? (uint32_t)(loaded_expert + 1) << 16 : 0u));
}
WISP_HD inline int pair_word_slot(int32_t w) {
  const int s = (int)((uint32_t)w & 0xFFFFu);
  return s == 0xFFFF ? -1 : s;
}
// The expert the call loaded for this pair, or -1.
WISP_HD inline int pair_word_loaded(int32_t w) { return (int)((uint32_t)w >> 16) - 1; }

// Device- or host-resident pager state for one layer.
struct PagerView {
  int E, cap;
  int32_t* map;    // [E]   expert -> slot, -1 if absent
  int32_t* s2e;    // [cap] slot -> expert, -1 if free
  int64_t* tick;   // [cap] LRU tick of the last touch
  int64_t* ctr;    // [kNumCounters]
};

}  // namespace wisp
