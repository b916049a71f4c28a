// Device-driven page-in (kernel copies from pinned host masters).
#pragma once

#include "common.h"

namespace wisp {

constexpr int kPageInBlocks = 64;

// One page-in launch.  The load list holds (expert, slot) pairs; its length
// is *count when count is non-null (written by the pager kernel), else n.
// m13/m2 are device addresses of the pinned masters (m2 null: each expert's
// w13 and w2 are one contiguous range of b13 bytes in both master and
// scratch).  Strides and sizes are in bytes, all multiples of 16.
struct PageInArgs {
  const int32_t* loads;
  const int32_t* count;
  int n;
  int num_experts, cap;
  const char* m13;
  size_t m13_stride;
  const char* m2;
  size_t m2_stride;
  char* s13;
  size_t s13_stride;
  char* s2;
  size_t s2_stride;
  size_t b13, b2;
  int32_t* hist;  // device address of a pinned host word that receives n, or null
};

int launch_pagein(const PageInArgs& a, hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop);

// Device address of host memory [base, base + bytes) when that range lies
// inside one pinned, device-mapped host allocation; null otherwise.
const char* mapped_host_range(const void* base, size_t bytes);

}  // namespace wisp
