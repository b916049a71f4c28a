// Packed bf16 masters: a lossless copy of an expert's weights that moves
// ~0.77x the bytes over the host link (page-in is the bound of paged decode).
//
// A bf16 value is sign (1) | exponent (8) | mantissa (7).  Weights spread
// over a few binades, so within a block of 64 consecutive values of a row
// the exponents fit 15 codes above the block's smallest nonzero exponent.
// Per row of L values (L a multiple of 64, nb = L / 64 blocks, nw =
// ceil(nb / 32) mask words):
//   lo     L bytes       value j: sign << 7 | mantissa
//   codes  L / 2 bytes   value j: nibble j % 2 (low first) of byte j / 2;
//                        exponent = base + code, code 15 = exponent 0
//                        (zeros and subnormals)
//   header base[nb] bytes, padded to 4; then nw u32 words whose bit b
//                        marks block b as an exception; then one u32: the
//                        row's first exception's index in the expert's
//                        exception area; padded to 16 bytes
// A block whose nonzero exponents span more than 15 values is an exception:
// its lo bytes stay in place and its 64 exponent bytes go to the expert's
// exception area (64 bytes per exception block, in row and block order).
// An expert is its 2I w13 rows (L = H), then its H w2 rows (L = I), then the
// exception area; experts sit at a fixed stride (the largest expert rounded
// up to 256 bytes).  Every row starts 16-byte aligned.
#pragma once

#include <type_traits>

#include "common.h"

namespace wisp {
namespace packed {

__host__ __device__ constexpr int align_up(int v, int a) { return (v + a - 1) / a * a; }

// Bytes of the header of a row of L values.
__host__ __device__ constexpr int header_bytes(int L) {
  return align_up(align_up(L / 64, 4) + 4 * ((L / 64 + 31) / 32) + 4, 16);
}
// Bytes of a packed row of L values.
__host__ __device__ constexpr int row_bytes(int L) { return L + L / 2 + header_bytes(L); }

// Where an expert's parts start (bytes from the expert's start).
struct Layout {
  int H, I;
  size_t rs13, rs2;  // packed row bytes of w13 (L = H) and w2 (L = I) rows
  size_t w2_off, exc_off;
  __host__ __device__ Layout(int H_, int I_) : H(H_), I(I_) {
    rs13 = (size_t)row_bytes(H);
    rs2 = (size_t)row_bytes(I);
    w2_off = 2 * (size_t)I * rs13;
    exc_off = w2_off + (size_t)H * rs2;
  }
};

// The loads of one chunk (8 values: q in [0, L / 8)) of a packed row.
struct Chunk {
  uint64_t lo;
  uint32_t cd, base, mask;
};

// Chunk k of a lane that owns chunks k * 64 + lane (the GEMV kernels' lane
// layout) of a row of L values, as buffer loads from the row's resource:
// the lane's offsets are one register per stream, the chunk's part an
// immediate, and loads past the row return 0.  A block's mask word is the
// same for all lanes of a chunk (blocks 8k .. 8k + 7 share word k / 4).
__device__ inline __amdgpu_buffer_rsrc_t row_rsrc(const char* row, int L) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(row), (short)0, row_bytes(L),
                                           0x00020000);
}
// f(std::integral_constant<int, k>) for k = 0 .. N - 1.
template <int N, int K = 0, typename F>
__device__ inline void for_each_chunk(F&& f) {
  if constexpr (K < N) {
    f(std::integral_constant<int, K>{});
    for_each_chunk<N, K + 1>(f);
  }
}

template <int K>
__device__ inline Chunk load_lane_chunk(__amdgpu_buffer_rsrc_t r, int L, int lane) {
  const int hdr = L + L / 2;
  Chunk c;
  const auto lo = __builtin_amdgcn_raw_buffer_load_b64(r, 8 * lane + 512 * K, 0, 0);
  c.lo = (uint64_t)lo[0] | ((uint64_t)lo[1] << 32);
  c.cd = __builtin_amdgcn_raw_buffer_load_b32(r, L + 4 * lane + 256 * K, 0, 0);
  c.base = __builtin_amdgcn_raw_buffer_load_b8(r, hdr + (lane >> 3) + 8 * K, 0, 0);
  c.mask = __builtin_amdgcn_raw_buffer_load_b32(r, hdr + align_up(L / 64, 4) + 4 * (K / 4), 0,
                                                0);
  return c;
}

// Four exponent codes (nibbles of c, low first) as exponent bytes: base +
// code, and 0 for code 15.  Bytes never carry: a code-15 byte is cleared
// before the add and base + code <= 255 for the others.
__device__ inline uint32_t exponents4(uint32_t c, uint32_t base) {
  uint32_t x = (c | (c << 8)) & 0x00FF00FFu;
  x = (x | (x << 4)) & 0x0F0F0F0Fu;                        // one code a byte
  const uint32_t z = (((x + 0x01010101u) >> 4) & 0x01010101u) * 0xFFu;  // code 15
  return ((x & ~z) + base * 0x01010101u) & ~z;
}

// Two bf16 values from their lo bytes (bits 0-15 of l) and exponent bytes
// (bits 0-15 of e): value 0 in the low half.
__device__ inline uint32_t join2(uint32_t l, uint32_t e) {
  const uint32_t l2 = (l & 0xFFu) | ((l & 0xFF00u) << 8);  // a byte per half
  const uint32_t e2 = (e & 0xFFu) | ((e & 0xFF00u) << 8);
  return ((l2 & 0x00800080u) << 8) | (e2 << 7) | (l2 & 0x007F007Fu);
}

// The chunk's 8 bf16 values when its block is not an exception.
__device__ inline uint4 unpack_plain(const Chunk& c) {
  const uint32_t e0 = exponents4(c.cd & 0xFFFFu, c.base), e1 = exponents4(c.cd >> 16, c.base);
  const uint32_t l0 = (uint32_t)c.lo, l1 = (uint32_t)(c.lo >> 32);
  return make_uint4(join2(l0, e0), join2(l0 >> 16, e0 >> 16), join2(l1, e1),
                    join2(l1 >> 16, e1 >> 16));
}

// Whether chunk q's block is an exception.
__device__ inline bool is_exception(const Chunk& c, int q) { return (c.mask >> ((q >> 3) & 31)) & 1u; }

// The chunk's 8 bf16 values as one 16-byte word (value 0 in the low half
// of word 0).  An exception block's exponents come from the exception area
// `exc` of the row's expert (a dependent load, on the rare blocks only).
__device__ inline uint4 unpack_chunk(const Chunk& c, const char* __restrict__ row, int L, int q,
                                     const char* __restrict__ exc) {
  const int b = q >> 3;
  uint32_t e0, e1;  // exponent bytes of values 0-3 and 4-7
  if ((c.mask >> (b & 31)) & 1u) {
    const char* mw = row + L + L / 2 + align_up(L / 64, 4);
    const int nw = (L / 64 + 31) / 32;
    uint32_t idx = *reinterpret_cast<const uint32_t*>(mw + 4 * nw) +
                   __builtin_popcount(c.mask & ((1u << (b & 31)) - 1u));
    for (int w = 0; w < (b >> 5); ++w)
      idx += __builtin_popcount(*reinterpret_cast<const uint32_t*>(mw + 4 * w));
    const uint64_t ex = *reinterpret_cast<const uint64_t*>(exc + 64 * (size_t)idx + 8 * (q & 7));
    e0 = (uint32_t)ex;
    e1 = (uint32_t)(ex >> 32);
  } else {
    e0 = exponents4(c.cd & 0xFFFFu, c.base);
    e1 = exponents4(c.cd >> 16, c.base);
  }
  const uint32_t l0 = (uint32_t)c.lo, l1 = (uint32_t)(c.lo >> 32);
  return make_uint4(join2(l0, e0), join2(l0 >> 16, e0 >> 16), join2(l1, e1),
                    join2(l1 >> 16, e1 >> 16));
}

}  // namespace packed
}  // namespace wisp
