// Host check of the 16-bit keys of bf16 logits that the kernels compare two to
// a register (qs_device.hpp hkey2, key_of_h; qs_kernels.hpp bf16_of_h), over
// every pair of bf16 bit patterns in a register's low and high halves:
//   - the h key orders like the values (NaN below everything, -0 just below
//     +0), both halves independently;
//   - every NaN maps below kHNegInf, -inf to kHNegInf, the rest above;
//   - key_of_h(h) is the order key of the value (sign-magnitude bits made
//     unsigned, -0 kept apart from +0), 0 for NaN;
//   - bf16_of_h inverts hkey2 for every non-NaN pattern;
//   - the greedy key h - 0xfe (mod 2^16) puts every NaN above +inf.
// Prints the number of failures.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>
#include <math.h>
#include "qs_kernels.hpp"

using qs::u32;
static float f_of_bf16(u32 x) { u32 u = x << 16; float f; memcpy(&f, &u, 4); return f; }
static u32 order_key(float z) {  // orderable bits, -0 below +0 (no fold)
  u32 u; memcpy(&u, &z, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
int main() {
  long bad = 0;
  // every pattern in both halves, against a fixed partner in the other half
  for (u32 x = 0; x < 65536; ++x) {
    const u32 partner = (x * 2654435761u) >> 16;
    const u32 hw_lo = qs::hkey2(x | (partner << 16)), hw_hi = qs::hkey2(partner | (x << 16));
    const u32 h = hw_lo & 0xffffu;
    if ((hw_hi >> 16) != h) ++bad;                      // the halves are independent
    if ((hw_lo >> 16) != (qs::hkey2(partner) & 0xffffu)) ++bad;
    const float z = f_of_bf16(x);
    if (isnan(z)) {
      if (h >= qs::kHNegInf) ++bad;
      if (qs::key_of_h(h) != 0u) ++bad;
      if (((h + 0xff02u) & 0xffffu) < 0xff02u) ++bad;  // greedy: NaN above +inf
      continue;
    }
    if (h < qs::kHNegInf) ++bad;
    if (isinf(z) && z < 0 && h != qs::kHNegInf) ++bad;
    if (qs::key_of_h(h) != order_key(z)) ++bad;
    if (qs::bf16_of_h(h) != x) ++bad;
    const u32 g = (h + 0xff02u) & 0xffffu;
    if (g > 0xff01u) ++bad;
  }
  // order: h(a) < h(b) iff a < b (or a is -0 and b is +0), for non-NaN pairs
  for (u32 a = 0; a < 65536; a += 7) {
    const float za = f_of_bf16(a);
    if (isnan(za)) continue;
    const u32 ha = qs::hkey2(a) & 0xffffu;
    for (u32 b = 0; b < 65536; b += 13) {
      const float zb = f_of_bf16(b);
      if (isnan(zb)) continue;
      const u32 hb = qs::hkey2(b) & 0xffffu;
      const bool lt = za < zb || (za == zb && za == 0.0f && signbit(za) && !signbit(zb));
      if ((ha < hb) != lt) ++bad;
    }
  }
  printf("%ld\n", bad);
  return 0;
}
