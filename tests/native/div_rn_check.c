// Bit-exactness check of the sampler kernel's division by a row-uniform
// divisor (ns::div_rn in csrc/ns_device.h): q0 = RN(x*r), rem = fma(-q0, t, x),
// q = fma(rem, r, q0) with r = RN(1/t), and IEEE x/t unless t lies in
// [2^-100, 2^100] and |q0| in [lo, 2^100], lo = max(2^-100, 2^-99 * r) (so that
// |x| >= 2^-100 too: the remainder rem is then a multiple of at least 2^-149, an
// exact float, and q0 and q are normal).  Compared bit for bit with IEEE float
// division.  Arguments: number of random divisors (default 64); "old" to run the
// earlier rule (|q0| in [2^-100, 2^100] only), which must fail.  Exit status 1 on
// any mismatch.
#include <stdio.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>
#include <math.h>
static float u2f(uint32_t u){float f; memcpy(&f,&u,4); return f;}
static uint32_t f2u(float f){uint32_t u; memcpy(&u,&f,4); return u;}
static int old_rule = 0;
static float div_lo(float t, float r) {
  return (t >= 0x1.0p-100f && t <= 0x1.0p+100f) ? fmaxf(0x1.0p-100f, 0x1.0p-99f * r) : INFINITY;
}
static float div_rn(float x, float t, float r, float lo) {
  float q0 = x * r;
  float rem = fmaf(-q0, t, x);
  float q = fmaf(rem, r, q0);
  float aq = fabsf(q0);
  if (old_rule) lo = 0x1.0p-100f;
  if (!(aq >= lo && aq <= 0x1.0p+100f)) q = x / t;
  return q;
}
static long bad = 0, tot = 0;
static void check(float xx, float t, float r, float lo) {
  float a = div_rn(xx, t, r, lo), b = xx / t;
  ++tot;
  if (f2u(a) != f2u(b) && !(isnan(a) && isnan(b))) {
    if (bad < 10) printf("mismatch t=%a x=%a got %a want %a\n", t, xx, a, b);
    ++bad;
    if (old_rule) { printf("checked %ld, mismatches %ld\n", tot, bad); exit(1); }   // the first suffices
  }
}
int main(int argc, char** argv) {
  int nrand = argc > 1 ? atoi(argv[1]) : 64;
  old_rule = argc > 2 && strcmp(argv[2], "old") == 0;
  // the workloads' penalties and temperatures, the temperature clamp (1e-6), divisors
  // near 1 and the powers of two, and extreme penalties on either side of the range
  float ts[] = {0.7f, 0.8f, 1.2f, 1.3f, 1.1f, 1e-6f, 0.5f, 3.0f, 1.0000001f, 0.99999994f, 1.9999999f, 1.5f,
                7.0f, 1000.0f, 12345.678f, 0.3f, 1e-3f, 3e-6f, 7.0e5f, 1e20f, 1e30f, 0x1.0p-100f, 0x1.0p+100f,
                0x1.fffffep-101f, 0x1.000002p+100f, 1e-35f, 3e38f, 0x1.0p-140f};
  int nt = sizeof(ts)/sizeof(ts[0]);
  for (int ti = 0; ti < nt + nrand; ++ti) {
    float t;
    if (ti < nt) t = ts[ti];
    else {
      uint32_t m = (uint32_t)(ti - nt) * 0x1F3D5B7u;
      t = u2f(0x3f800000u | (m & 0x7fffffu));
      if (ti % 2) t *= 3.7f;
      if (ti % 3 == 0) t = ldexpf(t, (int)(m % 61) - 30);
    }
    float r = 1.0f / t;
    float lo = div_lo(t, r);
    // every binade of the float range (subnormals by their bit patterns), a mantissa stride
    // per binade, and every mantissa of a few binades
    for (int e = -126; e <= 127; ++e) {
      const uint32_t step = (e == 0 || e == -118 || e == 20) ? 1u : 997u;
      for (uint32_t m = 0; m < (1u << 23); m += step) {
        float x = ldexpf(u2f(0x3f800000u | m), e);
        check(x, t, r, lo);
        check(-x, t, r, lo);
      }
    }
    for (uint32_t b = 0; b < (1u << 23); b += 331u) { check(u2f(b), t, r, lo); check(-u2f(b), t, r, lo); }
    check(0.0f, t, r, lo); check(-0.0f, t, r, lo);
    check(INFINITY, t, r, lo); check(-INFINITY, t, r, lo); check(NAN, t, r, lo);
  }
  printf("checked %ld, mismatches %ld\n", tot, bad);
  return bad != 0;
}
