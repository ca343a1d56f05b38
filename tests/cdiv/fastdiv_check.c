/* Checks the sampler's fast division (qsampler.hip div_fast / div_fast_ok)
 * against the correctly rounded fp32 division on the host.
 *   mode 0: every bf16 z (all 65536 patterns) x the divisors given;
 *   mode 1: n random (z, b) pairs, z any fp32 bit pattern, b log-uniform in
 *           [2^-120, 2^120].
 * Prints the number of (fast-path) mismatches. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static float f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t bits(float x) { uint32_t v; memcpy(&v, &x, 4); return v; }
static uint64_t mix(uint64_t x) {
  x ^= x >> 33; x *= 0xff51afd7ed558ccdULL; x ^= x >> 33; x *= 0xc4ceb9fe1a85ec53ULL; x ^= x >> 33;
  return x;
}
static int ok(float z, float r) {
  const uint32_t aq = bits(z * r) & 0x7fffffffu, az = bits(z) & 0x7fffffffu;
  return (aq - 0x0d800000u) < (0x71800000u - 0x0d800000u) && (az - 0x0d800000u) < (0x71800000u - 0x0d800000u);
}
static long check(float z, float b, float r, long* fast) {
  if (z != z || isinf(z) || !ok(z, r)) return 0;
  ++*fast;
  const float q0 = z * r;
  const float e = fmaf(-q0, b, z);
  const float q1 = fmaf(e, r, q0);
  return bits(q1) != bits(z / b);
}
int main(int argc, char** argv) {
  long bad = 0, fast = 0;
  if (atoi(argv[1]) == 0) {
    for (int i = 2; i < argc; ++i) {
      const float b = strtof(argv[i], 0);
      volatile float one = 1.0f;
      const float r = one / b;
      for (uint32_t h = 0; h < 65536u; ++h) bad += check(f(h << 16), b, r, &fast);
    }
  } else {
    const long n = atol(argv[2]);
    for (long i = 0; i < n; ++i) {
      const uint64_t hb = mix(0x51ed27ULL + (uint64_t)i);
      const float b = ldexpf(1.0f + (float)(hb & 0xffffff) / 16777216.0f, (int)((hb >> 32) % 241) - 120);
      volatile float one = 1.0f;
      const float r = one / b;
      bad += check(f((uint32_t)mix(hb ^ 0x9E3779B97F4A7C15ULL)), b, r, &fast);
    }
  }
  printf("%ld %ld\n", bad, fast);
  return 0;
}
