// Bit-exactness check of the sampler kernel's division by a row-uniform
// divisor (ns::div_rn in csrc/ns_device.h): q0 = RN(x*r), rem = fma(-q0, t, x),
// q = fma(rem, r, q0) with r = RN(1/t), IEEE x/t outside 2^-100..2^100.
// Compared bit for bit with IEEE float division.  Argument: number of random
// divisors (default 64); exit status 1 on any mismatch.
#include <stdio.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>
#include <math.h>
static float u2f(uint32_t u){float f; memcpy(&f,&u,4); return f;}
static uint32_t f2u(float f){uint32_t u; memcpy(&u,&f,4); return u;}
static float div_rn(float x, float t, float r) {
  float q0 = x * r;
  float rem = fmaf(-q0, t, x);
  float q = fmaf(rem, r, q0);
  float aq = fabsf(q0);
  if (!(aq >= 0x1.0p-100f && aq <= 0x1.0p+100f)) q = x / t;
  return q;
}
int main(int argc, char** argv) {
  int nrand = argc > 1 ? atoi(argv[1]) : 64;
  float ts[] = {0.7f, 0.8f, 1.2f, 1.3f, 1.1f, 1e-6f, 0.5f, 3.0f, 1.0000001f, 0.99999994f, 1.9999999f, 1.5f, 7.0f, 1000.0f, 12345.678f, 0.3f};
  int nt = sizeof(ts)/sizeof(ts[0]);
  long bad = 0, tot = 0;
  for (int ti = 0; ti < nt + nrand; ++ti) {
    float t;
    if (ti < nt) t = ts[ti]; else { uint32_t m = (uint32_t)(ti - nt) * 0x1F3D5B7u; t = u2f(0x3f800000u | (m & 0x7fffffu)); if (ti % 2) t *= 3.7f; }
    float r = 1.0f / t;
    for (int e = -30; e <= 30; e += 3) {
      for (uint32_t m = 0; m < (1u << 23); m += (e == 0 ? 1 : 7)) {
        float x = ldexpf(u2f(0x3f800000u | m), e);
        for (int s = 0; s < 2; ++s) {
          float xx = s ? -x : x;
          float a = div_rn(xx, t, r), b = xx / t;
          ++tot;
          if (f2u(a) != f2u(b)) { if (bad < 10) printf("mismatch t=%a x=%a got %a want %a\n", t, xx, a, b); ++bad; }
        }
      }
    }
  }
  printf("checked %ld, mismatches %ld\n", tot, bad);
  return bad != 0;
}
