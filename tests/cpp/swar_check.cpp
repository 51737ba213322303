// Exhaustive host check of the byte-lane helpers the image kernels use
// (strict_amd/csrc/swar.h) against scalar clamp arithmetic.
#include <cstdio>
#include <cstdint>

#include "swar.h"

int main() {
  long long failures = 0;
  // every (a, b) byte pair in every lane position, with varied neighbours
  const uint32_t neighbours[] = {0x00000000u, 0xffffffffu, 0x7f80017fu, 0x80ff7f01u};
  for (uint32_t nb : neighbours)
    for (int lane = 0; lane < 4; lane++)
      for (uint32_t a = 0; a < 256; a++)
        for (uint32_t b = 0; b < 256; b++) {
          const uint32_t shift = 8u * lane, keep = ~(0xffu << shift);
          const uint32_t A = (nb & keep) | (a << shift);
          const uint32_t B = (~nb & keep) | (b << shift);
          const uint32_t add = sh::sat_add_u8x4(A, B), sub = sh::sat_sub_u8x4(A, B);
          for (int l = 0; l < 4; l++) {
            const uint32_t x = (A >> (8 * l)) & 0xff, y = (B >> (8 * l)) & 0xff;
            const uint32_t e_add = x + y > 255 ? 255 : x + y;
            const uint32_t e_sub = x < y ? 0 : x - y;
            if (((add >> (8 * l)) & 0xff) != e_add || ((sub >> (8 * l)) & 0xff) != e_sub) failures++;
          }
        }
  // brighten: delta in [-255, 255], RGBA mask keeps alpha
  for (int delta = -255; delta <= 255; delta++)
    for (uint32_t p = 0; p < 256; p++) {
      const uint32_t mag = (uint32_t)(delta < 0 ? -delta : delta) * 0x01010101u;
      const uint32_t px = p * 0x01010101u;
      const uint32_t r = sh::brighten_u8x4(px, mag, delta < 0, 0x00ffffffu);
      int e = (int)p + delta;
      e = e < 0 ? 0 : (e > 255 ? 255 : e);
      for (int l = 0; l < 3; l++)
        if ((int)((r >> (8 * l)) & 0xff) != e) failures++;
      if ((r >> 24) != p) failures++;
    }
  // div25 over its whole documented domain
  for (uint32_t x = 0; x < 8192; x++)
    if (sh::div25(x) != x / 25) failures++;
  std::printf("failures=%lld\n", failures);
  return failures == 0 ? 0 : 1;
}
