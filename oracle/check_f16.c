/*
 * check_f16.c -- pins the oracle's scalar converters (TEST INFRASTRUCTURE).
 *
 * Walks all 2^32 fp32 bit patterns and compares orc_f32_to_f16 with the x86
 * F16C instruction vcvtps2ph under round-to-nearest-even (the `half` crate's
 * hardware path), NaN payloads compared only as "is NaN".  Also checks that
 * orc_f16_to_f32 inverts every one of the 2^16 halfs exactly, and that
 * orc_f32_to_bf16 agrees with an independent integer formulation of RNE.
 * Exit status 0 = all agree.  Optional argv[1] = stride (1 = exhaustive).
 */
#include <immintrin.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "it_oracle.h"

static int is_nan16(uint16_t h) { return (h & 0x7C00u) == 0x7C00u && (h & 0x3FFu); }

int main(int argc, char** argv) {
  uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
  uint64_t bad = 0, checked = 0;
  for (uint64_t u = 0; u <= 0xFFFFFFFFull; u += stride) {
    uint32_t x = (uint32_t)u;
    float f;
    memcpy(&f, &x, 4);
    uint16_t mine = orc_f32_to_f16(f);
    uint16_t hw = _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
    int ok = (is_nan16(mine) && is_nan16(hw)) || mine == hw;
    /* bf16 RNE, independent formulation: compare remainder to half. */
    uint16_t b = orc_f32_to_bf16(f);
    uint32_t hi = x >> 16, lo = x & 0xFFFFu;
    uint16_t want;
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) want = 0; /* NaN: checked below */
    else want = (uint16_t)(hi + (lo > 0x8000u || (lo == 0x8000u && (hi & 1u))));
    int okb = ((x & 0x7FFFFFFFu) > 0x7F800000u) ? (((b & 0x7F80u) == 0x7F80u) && (b & 0x7Fu)) : (b == want);
    if (!ok || !okb) {
      if (bad < 10) fprintf(stderr, "mismatch x=%08x f16 mine=%04x hw=%04x bf16=%04x want=%04x\n", x, mine, hw, b, want);
      ++bad;
    }
    ++checked;
  }
  for (uint32_t h = 0; h < 0x10000u; ++h) {
    float f = orc_f16_to_f32((uint16_t)h);
    float hw = _cvtsh_ss((unsigned short)h);
    uint32_t a, c;
    memcpy(&a, &f, 4);
    memcpy(&c, &hw, 4);
    if (is_nan16((uint16_t)h) ? !(f != f) : a != c) {
      if (bad < 10) fprintf(stderr, "f16->f32 mismatch h=%04x\n", h);
      ++bad;
    }
  }
  printf("checked=%llu bad=%llu\n", (unsigned long long)checked, (unsigned long long)bad);
  return bad ? 1 : 0;
}
