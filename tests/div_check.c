/* CPU check of the kernels' division by a per-row divisor b (kk_div in
 * kk_internal.h): with rb = 1 / b correctly rounded, q0 = a * rb,
 * r = fma(-q0, b, a), q = fma(r, rb, q0) equals the IEEE quotient a / b for
 * 2^-60 <= b <= 2^60 and 2^-60 < |a| < 2^60 (Markstein's theorem).
 * Usage: div_check GUARD; prints "n=<cases> bad=<mismatches>".  GUARD 1 uses
 * the kernels' range; GUARD 0 drops the lower bound on |a| (then tiny
 * dividends, whose remainder underflows, must show mismatches). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t s = 88172645463325252ull;
static uint32_t rnd(void) {
  s ^= s << 13;
  s ^= s >> 7;
  s ^= s << 17;
  return (uint32_t)s;
}
static float f_of(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static int guard;
static long n, bad;
static void one(float a, float b, float rb) {
  const float m = fabsf(a);
  const int in_range = (guard ? m > 0x1p-60f : m > 0.0f) && m < 0x1p60f;
  if (!in_range) return; /* the kernels divide these */
  const float q0 = a * rb;
  const float q = fmaf(fmaf(-q0, b, a), rb, q0);
  const float ref = a / b;
  ++n;
  if (memcmp(&q, &ref, 4) != 0) ++bad;
}
int main(int argc, char** argv) {
  guard = argc > 1 ? atoi(argv[1]) : 1;
  volatile float one_ = 1.0f;
  /* every mantissa of a in [1, 2) against divisors with awkward mantissas */
  const uint32_t bs[] = {0x3f800001u, 0x3fffffffu, 0x3fb504f3u, 0x3eaaaaabu};
  for (int k = 0; k < 4; ++k) {
    const float b = f_of(bs[k]), rb = one_ / b;
    for (uint32_t mnt = 0; mnt < (1u << 23); mnt += guard ? 1 : 64) one(f_of(0x3f800000u | mnt), b, rb);
  }
  /* random divisors in [2^-60, 2^60], random dividends of every exponent */
  for (int bi = 0; bi < 4000; ++bi) {
    const float b = f_of(((uint32_t)(67 + rnd() % 121) << 23) | (rnd() & 0x7fffffu)), rb = one_ / b;
    for (int ai = 0; ai < 1000; ++ai) {
      uint32_t ua = rnd();
      if ((ua >> 23 & 0xffu) == 0xffu) continue;
      one(f_of(ua), b, rb);
    }
  }
  printf("n=%ld bad=%ld\n", n, bad);
  return 0;
}
