// Host harness for the register transposes and the LDS swizzle of
// tile_common.h: reads nothing, prints "OK" or the first mismatch.
#include <cstdio>
#include <cstdlib>
#include <set>

#include "backend/mi355x/tile_common.h"

using namespace txk;

int main() {
  srand(7);
  for (int trial = 0; trial < 200; ++trial) {
    u32x4 in[16], out[16];
    uint8_t bytes[16][16];
    for (int r = 0; r < 16; ++r)
      for (int c = 0; c < 16; ++c)
        bytes[r][c] = (uint8_t)rand();
    for (int r = 0; r < 16; ++r)
      for (int d = 0; d < 4; ++d)
        set(in[r], d, bytes[r][4 * d] | bytes[r][4 * d + 1] << 8 | bytes[r][4 * d + 2] << 16 |
                          (uint32_t)bytes[r][4 * d + 3] << 24);
    transpose16x16_b8(in, out);
    for (int c = 0; c < 16; ++c)
      for (int r = 0; r < 16; ++r) {
        uint8_t got = (get(out[c], r / 4) >> (8 * (r % 4))) & 0xff;
        if (got != bytes[r][c]) { printf("b8 mismatch c=%d r=%d\n", c, r); return 1; }
      }
    // 16-bit 8x8
    uint16_t h[8][8];
    for (int r = 0; r < 8; ++r)
      for (int c = 0; c < 8; ++c)
        h[r][c] = (uint16_t)rand();
    for (int r = 0; r < 8; ++r)
      for (int d = 0; d < 4; ++d)
        set(in[r], d, h[r][2 * d] | (uint32_t)h[r][2 * d + 1] << 16);
    transpose8x8_b16(in, out);
    for (int c = 0; c < 8; ++c)
      for (int r = 0; r < 8; ++r) {
        uint16_t got = (get(out[c], r / 2) >> (16 * (r % 2))) & 0xffff;
        if (got != h[r][c]) { printf("b16 mismatch c=%d r=%d\n", c, r); return 1; }
      }
  }
  // swizzle: a bijection within each row, for 4- and 8-chunk rows
  for (uint32_t nch : {4u, 8u}) {
    for (uint32_t row = 0; row < 512; ++row) {
      std::set<uint32_t> seen;
      for (uint32_t ch = 0; ch < nch; ++ch) {
        uint32_t off = lds_off(row, ch, nch);
        if (off / (nch * 16) != row || off % 16) { printf("swizzle leaves row\n"); return 1; }
        seen.insert(off);
      }
      if (seen.size() != nch) { printf("swizzle not a bijection\n"); return 1; }
    }
  }
  // bf16 RNE spot checks (ties to even, NaN stays NaN)
  float one_plus_half_ulp;  // 1 + 2^-8: tie between 1 and 1+2^-7 -> 1
  uint32_t u = 0x3f808000u;
  memcpy(&one_plus_half_ulp, &u, 4);
  if (f32_to_bf16_rne(one_plus_half_ulp) != 0x3f80) { printf("bf16 tie\n"); return 1; }
  u = 0x3f818000u;  // tie between 0x3f81 and 0x3f82 -> 0x3f82
  float t2; memcpy(&t2, &u, 4);
  if (f32_to_bf16_rne(t2) != 0x3f82) { printf("bf16 tie2\n"); return 1; }
  u = 0x7fc00001u; float nan; memcpy(&nan, &u, 4);
  if ((f32_to_bf16_rne(nan) & 0x7fc0) != 0x7fc0) { printf("bf16 nan\n"); return 1; }
  printf("OK\n");
  return 0;
}
