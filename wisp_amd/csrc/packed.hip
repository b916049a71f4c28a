// Host side of the packed bf16 masters (the format is in packed.h): the
// per-expert stride and the packing itself, both threaded over experts.
// No reference counterpart: the reference pages the bf16 masters as they
// are (src/wisp/integrations/vllm/fused_moe.py:338-354); a packed copy
// moves the same values in fewer bytes over the host link.
#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "common.h"
#include "packed.h"

namespace wisp {
namespace {

inline int expo(uint16_t u) { return (u >> 7) & 0xFF; }

// Block of 64 values: lo bytes always; codes and base when the nonzero
// exponents span at most 15 values (returns true), else the 64 exponent
// bytes into ex (returns false).
bool pack_block(const uint16_t* v, uint8_t* lo, uint8_t* codes, uint8_t* base, uint8_t* ex) {
  int emin = 256, emax = -1;
  for (int j = 0; j < 64; ++j) {
    lo[j] = (uint8_t)(((v[j] >> 8) & 0x80) | (v[j] & 0x7F));
    const int e = expo(v[j]);
    if (e) {
      emin = std::min(emin, e);
      emax = std::max(emax, e);
    }
  }
  if (emax < 0 || emax - emin <= 14) {
    *base = (uint8_t)(emax < 0 ? 0 : emin);
    for (int j = 0; j < 32; ++j) {
      const int e0 = expo(v[2 * j]), e1 = expo(v[2 * j + 1]);
      const int c0 = e0 ? e0 - emin : 15, c1 = e1 ? e1 - emin : 15;
      codes[j] = (uint8_t)(c0 | (c1 << 4));
    }
    return true;
  }
  *base = 0;
  memset(codes, 0, 32);
  if (ex)
    for (int j = 0; j < 64; ++j) ex[j] = (uint8_t)expo(v[j]);
  return false;
}

// Exception blocks of one row (count only when out is null), written at
// out (the packed row) and exc (the next free exception slot of the expert).
int pack_row(const uint16_t* v, int L, uint8_t* out, uint8_t* exc, uint32_t exc_base) {
  const int nb = L / 64;
  uint8_t lo[64], codes[32], base;
  int nexc = 0;
  uint8_t* hdr = out ? out + L + L / 2 : nullptr;
  uint32_t* mask = out ? reinterpret_cast<uint32_t*>(hdr + packed::align_up(nb, 4)) : nullptr;
  if (out) memset(hdr, 0, packed::header_bytes(L));
  for (int b = 0; b < nb; ++b) {
    const bool fits = pack_block(v + 64 * b, lo, codes, &base, exc ? exc + 64 * nexc : nullptr);
    if (out) {
      memcpy(out + 64 * b, lo, 64);
      memcpy(out + L + 32 * b, codes, 32);
      hdr[b] = base;
      if (!fits) mask[b >> 5] |= 1u << (b & 31);
    }
    if (!fits) ++nexc;
  }
  if (out) mask[(nb + 31) / 32] = exc_base;
  return nexc;
}

struct Masters {
  int E, H, I;
  const uint16_t* w13;
  size_t s13;  // elements
  const uint16_t* w2;
  size_t s2;
};

// Exception blocks of expert e.
size_t count_expert(const Masters& m, int e) {
  size_t n = 0;
  for (int r = 0; r < 2 * m.I; ++r)
    n += pack_row(m.w13 + (size_t)e * m.s13 + (size_t)r * m.H, m.H, nullptr, nullptr, 0);
  for (int r = 0; r < m.H; ++r)
    n += pack_row(m.w2 + (size_t)e * m.s2 + (size_t)r * m.I, m.I, nullptr, nullptr, 0);
  return n;
}

void pack_expert(const Masters& m, int e, uint8_t* out) {
  const packed::Layout Lp(m.H, m.I);
  uint8_t* exc = out + Lp.exc_off;
  uint32_t nexc = 0;
  for (int r = 0; r < 2 * m.I; ++r)
    nexc += pack_row(m.w13 + (size_t)e * m.s13 + (size_t)r * m.H, m.H, out + r * Lp.rs13,
                     exc + 64 * (size_t)nexc, nexc);
  for (int r = 0; r < m.H; ++r)
    nexc += pack_row(m.w2 + (size_t)e * m.s2 + (size_t)r * m.I, m.I,
                     out + Lp.w2_off + r * Lp.rs2, exc + 64 * (size_t)nexc, nexc);
}

// Runs f(e) for every expert on up to 16 threads (on the calling thread
// alone when no thread can be started).
template <typename F>
void over_experts(int E, F f) {
  const int nt = std::max(1, std::min({E, 16, (int)std::thread::hardware_concurrency()}));
  std::vector<std::thread> th;
  int started = 0;
  try {
    for (; started < nt; ++started)
      th.emplace_back([&, started] {
        for (int e = started; e < E; e += nt) f(e);
      });
  } catch (...) {
  }
  for (auto& x : th) x.join();
  // experts of the threads that did not start
  for (int t = started; t < nt; ++t)
    for (int e = t; e < E; e += nt) f(e);
}

bool valid(int E, int H, int I, const void* w13, size_t s13, const void* w2, size_t s2) {
  return E >= 1 && H >= 64 && I >= 64 && H % 64 == 0 && I % 64 == 0 && w13 && w2 &&
         s13 >= 2 * (size_t)I * H && s2 >= (size_t)H * I;
}

}  // namespace
}  // namespace wisp

extern "C" size_t wisp_pack_bf16_stride(int E, int H, int I, const void* master_w13,
                                        size_t master_w13_stride, const void* master_w2,
                                        size_t master_w2_stride) {
  using namespace wisp;
  if (!valid(E, H, I, master_w13, master_w13_stride, master_w2, master_w2_stride)) return 0;
  const Masters m{E, H, I, (const uint16_t*)master_w13, master_w13_stride,
                  (const uint16_t*)master_w2, master_w2_stride};
  std::vector<size_t> n(E);
  over_experts(E, [&](int e) { n[e] = count_expert(m, e); });
  const size_t most = *std::max_element(n.begin(), n.end());
  return (packed::Layout(H, I).exc_off + 64 * most + 255) / 256 * 256;
}

extern "C" int wisp_pack_bf16(int E, int H, int I, const void* master_w13,
                              size_t master_w13_stride, const void* master_w2,
                              size_t master_w2_stride, void* out, size_t stride) {
  using namespace wisp;
  if (!valid(E, H, I, master_w13, master_w13_stride, master_w2, master_w2_stride) || !out ||
      stride % 256 || stride < packed::Layout(H, I).exc_off)
    return WISP_ERR_INVALID;
  const Masters m{E, H, I, (const uint16_t*)master_w13, master_w13_stride,
                  (const uint16_t*)master_w2, master_w2_stride};
  std::vector<size_t> n(E);
  over_experts(E, [&](int e) { n[e] = count_expert(m, e); });
  if (packed::Layout(H, I).exc_off + 64 * *std::max_element(n.begin(), n.end()) > stride) {
    wisp_set_last_error("stride below wisp_pack_bf16_stride for these masters", "wisp_pack_bf16");
    return WISP_ERR_INVALID;
  }
  over_experts(E, [&](int e) {
    uint8_t* o = (uint8_t*)out + (size_t)e * stride;
    pack_expert(m, e, o);
    const size_t used = packed::Layout(H, I).exc_off + 64 * n[e];
    memset(o + used, 0, stride - used);
  });
  return WISP_OK;
}
