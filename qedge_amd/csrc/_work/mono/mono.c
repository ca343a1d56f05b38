#include <math.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>
static float p2(float f) {
  float p = 0x1.c54640p-13f;
  p = fmaf(p, f, 0x1.46d326p-10f); p = fmaf(p, f, 0x1.3d0c40p-7f); p = fmaf(p, f, 0x1.c688f0p-5f);
  p = fmaf(p, f, 0x1.ebfd5ap-3f); p = fmaf(p, f, 0x1.62e42cp-1f); p = fmaf(p, f, 1.0f);
  return p;
}
static uint32_t m24(float p) { if (!(p >= 1.0f)) p = 1.0f; if (p >= 2.0f) { uint32_t u = 0x3fffffffu; memcpy(&p, &u, 4);} uint32_t u; memcpy(&u, &p, 4); return 0x800000u | (u & 0x7fffffu); }
int main(void) {
  uint32_t prev = 0, bad = 0; float pf = 0;
  for (uint32_t u = 0; u <= 0x3f800000u; ++u) {  /* all floats in [0, 1] */
    float f; memcpy(&f, &u, 4);
    uint32_t m = m24(p2(f));
    if (m < prev) { if (bad < 10) printf("non-monotone at f=%a (prev f=%a): %x < %x\n", f, pf, m, prev); ++bad; }
    prev = m; pf = f;
  }
  printf("checked, %u decreases; M(0)=%x M(1)=%x\n", bad, m24(p2(0.0f)), m24(p2(1.0f)));
  return bad != 0;
}
