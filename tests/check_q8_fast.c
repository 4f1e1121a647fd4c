/*
 * check_q8_fast.c -- pins two identities the Q8_0 quantise-append kernels
 * use in place of IEEE divisions (built and run by
 * test_oracle.py::test_q8_fast_quotient_identities; plain C, no GPU).
 *
 * 1. scale = amax / 127 for every positive normal float amax equals
 *      y = RN(amax * RN(1/127)); scale = fma(fma(-127, y, amax), RN(1/127), y)
 *    (a faithful quotient plus one exact-remainder correction), checked
 *    over all 2,130,706,432 of them.
 * 2. For x with |x| <= 127 scale and any rs within one ulp of 1 / scale
 *    (the GPU's v_rcp_f32 bound): f = fma(x, rs, 1.5 2^23) holds
 *    n = rint(x rs) in its low byte, and whenever
 *    |fma(x, rs, 1.5 2^23 - f)| < 0.4999 that byte equals
 *    round_half_away(fl(x / scale)) as an int8.  Checked on random scales
 *    with inputs placed within a few ulps of half-integers and integers,
 *    for rs = RN(1/scale) and its two neighbours.
 * Exit status 0 = both hold.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static uint64_t st = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) {
  uint64_t z = (st += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

int main(void) {
  const float r127 = 1.0f / 127.0f;
  long bad1 = 0;
#pragma omp parallel for reduction(+ : bad1) schedule(dynamic, 1 << 20)
  for (int64_t u = 0x00800000; u < 0x7F800000; ++u) {
    const float a = u2f((uint32_t)u);
    const float y = a * r127;
    const float q = fmaf(fmaf(-127.0f, y, a), r127, y);
    if (f2u(q) != f2u(a / 127.0f)) ++bad1;
  }
  long bad2 = 0, fast = 0, n2 = 0;
  const float magic = 12582912.0f;
  for (int i = 0; i < 60000; ++i) {
    const float amax = (float)ldexp(1.0 + (double)(next() >> 11) * 0x1p-53, (int)(next() % 200) - 100);
    const float scale = amax / 127.0f;
    const float r0 = 1.0f / scale;
    const float rss[3] = {nextafterf(r0, 0.0f), r0, nextafterf(r0, INFINITY)};
    for (int j = 0; j < 40; ++j) {
      const int k = (int)(next() % 255) - 127;
      const double t = (j & 1) ? k + 0.5 : k;  /* ties and integers */
      float x = (float)(t * (double)scale);
      const int nudge = (int)(next() % 9) - 4;
      for (int s = 0; s < (nudge < 0 ? -nudge : nudge); ++s) x = nextafterf(x, nudge < 0 ? -INFINITY : INFINITY);
      if (fabsf(x) > amax) continue;
      float r = roundf(x / scale);
      if (r < -128.0f) r = -128.0f;
      if (r > 127.0f) r = 127.0f;
      const int8_t want = (int8_t)(int)r;
      for (int c = 0; c < 3; ++c) {
        const float f = fmaf(x, rss[c], magic);
        const float res = fmaf(x, rss[c], magic - f);
        ++n2;
        if (fabsf(res) < 0.4999f) {
          ++fast;
          if ((int8_t)(f2u(f) & 0xFFu) != want) ++bad2;
        }
      }
    }
  }
  printf("scale identity: %ld mismatches over all positive normal floats\n", bad1);
  printf("fast quotient: %ld mismatches in %ld fast-path cases of %ld near-tie trials\n", bad2, fast, n2);
  return (bad1 || bad2 || fast == 0) ? 1 : 0;
}
