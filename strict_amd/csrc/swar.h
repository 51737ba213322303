// Byte-lane arithmetic on packed 32-bit words (4 x u8), shared by the image
// kernels. Plain C++ so the same functions also build on the host, where a
// test checks them exhaustively against scalar clamp arithmetic.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define SH_HD __host__ __device__ __forceinline__
#else
#define SH_HD static inline
#endif

namespace sh {

// Per byte: min(a + b, 255).
SH_HD uint32_t sat_add_u8x4(uint32_t a, uint32_t b) {
  uint32_t low = (a & 0x7f7f7f7fu) + (b & 0x7f7f7f7fu);  // bit 7 = carry out of the low 7 bits
  uint32_t sum = low ^ ((a ^ b) & 0x80808080u);          // byte-wise sum mod 256
  uint32_t carry = ((a & b) | ((a | b) & ~sum)) & 0x80808080u;
  return sum | ((carry >> 7) * 0xffu);
}

// Per byte: max(a - b, 0).
SH_HD uint32_t sat_sub_u8x4(uint32_t a, uint32_t b) {
  uint32_t low = (a | 0x80808080u) - (b & 0x7f7f7f7fu);  // bit 7 = no borrow out of the low 7 bits
  uint32_t diff = low ^ (~(a ^ b) & 0x80808080u);        // byte-wise difference mod 256
  uint32_t borrow = ((~a & b) | (~(a ^ b) & diff)) & 0x80808080u;
  return diff & ~((borrow >> 7) * 0xffu);
}

// clamp(p + delta, 0, 255) on the bytes selected by `mask` (0xff per byte),
// the other bytes unchanged. `mag` = |delta| replicated into every byte.
SH_HD uint32_t brighten_u8x4(uint32_t p, uint32_t mag, bool negative, uint32_t mask) {
  uint32_t m = mag & mask;
  return negative ? sat_sub_u8x4(p, m) : sat_add_u8x4(p, m);
}

// floor(x / 25) for 0 <= x < 2^13 (exact: 5243 / 2^17 overestimates 1/25 by
// less than 1 / (25 * 2^13)).
SH_HD uint32_t div25(uint32_t x) { return (x * 5243u) >> 17; }

}  // namespace sh
