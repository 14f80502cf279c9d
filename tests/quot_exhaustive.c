/*
 * Exhaustive check of the corrected reciprocal quotient used by the vector
 * quantizers (dsl_tool_amd/csrc/common.h, quot):
 *
 *     q = x * r,  e = fma(q, s, -x),  q' = fma(-e, r, q)
 *
 * The quantization contract encodes RN(x / s) (IEEE fp32 division, then RNE
 * to E4M3 or E2M1; oracle/quant.py).  For every bf16 input this program
 * shows that code(q') == code(RN(x / s)) whenever r is RN(1/s) or one ulp
 * either side of it (the hardware reciprocal is within 1 ulp), over every
 * scale the quantizers can produce:
 *
 *   (1) constants: RN(a / b) == q' (as fp32) with r = RN(1/b) for every
 *       positive finite bf16 a and b = 448, 6, 2688 (the E4M3 scale, the
 *       NVFP4 amax/6 step and the NVFP4 global scale);
 *   (2) E4M3: every pair of positive finite bf16 amax >= x, with
 *       s = max(RN(amax / 448), 1e-12);
 *   (3) NVFP4 block scale: every bf16 tensor amax (global scale
 *       sg = max(RN(amax_t / 2688), 1e-12)) and bf16 block amax m <= amax_t,
 *       E4M3 code of RN(RN(m / 6) / sg);
 *   (4) NVFP4 elements: every sg as in (3), every finite nonzero E4M3 block
 *       code b (d = RN(e4m3(b) * sg)) and every bf16 x in [d/8, 8d] (below
 *       d/8 both quotients encode to 0; above 6.4d no block amax reaches).
 * Negative x mirror positive x (RN and fma are odd functions), and a zero x
 * gives a zero of the same sign under both forms.
 *
 * Prints one line per part and exits 0 only if every count is zero.
 * Build: cc -O2 -fopenmp -ffp-contract=off quot_exhaustive.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bf(uint32_t b) { return u2f(b << 16); }

/* E4M3FN magnitude code of x >= 0, RNE (0x7f for > 464). */
static int e4m3_code(float x) {
  uint32_t mag = f2u(x) & 0x7fffffffu;
  int c;
  if (x >= 0x1p-6f) c = (int)(((int64_t)mag + 0x7ffff + ((mag >> 20) & 1)) >> 20) - (120 << 3);
  else c = (int)rint((double)x * 512.0);
  return (!isfinite(x) || c >= 0x7f) ? 0x7f : c;
}
static float e4m3_val(int c) {
  int e = (c >> 3) & 15, m = c & 7;
  return e ? ldexpf(1.0f + m / 8.0f, e - 7) : m * 0x1p-9f;
}
/* E2M1 magnitude code of a >= 0, RNE with saturation. */
static int e2m1_code(float a) {
  return 7 - (a <= 5.0f) - (a < 3.5f) - (a <= 2.5f) - (a < 1.75f) - (a <= 1.25f) - (a < 0.75f) -
         (a <= 0.25f);
}
static float quot(float x, float s, float r) {
  float q = x * r;
  float e = fmaf(q, s, -x);
  return fmaf(-e, r, q);
}
static float nudge(float r, int k) { return u2f(f2u(r) + (uint32_t)k); }

#define NBF 0x7f80u /* positive finite bf16 patterns: 0x0001 .. 0x7f7f */

int main(void) {
  long bad1 = 0, bad2 = 0, bad3 = 0, bad4 = 0, n2 = 0, n3 = 0, n4 = 0;
  const float cb[3] = {448.0f, 6.0f, 2688.0f};
  for (int i = 0; i < 3; ++i) {
    const float r = 1.0f / cb[i];
    for (uint32_t a = 1; a < NBF; ++a)
      if (f2u(quot(bf(a), cb[i], r)) != f2u(bf(a) / cb[i])) ++bad1;
  }
  printf("(1) constant divisions: %ld mismatches\n", bad1);

#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad2, n2)
  for (uint32_t a = 1; a < NBF; ++a) {
    float s = bf(a) / 448.0f;
    if (s < 1e-12f) s = 1e-12f;
    const float r0 = 1.0f / s;
    for (uint32_t xb = 0; xb <= a; ++xb) {
      const float x = bf(xb);
      const int want = e4m3_code(x / s);
      for (int k = -1; k <= 1; ++k) bad2 += e4m3_code(quot(x, s, nudge(r0, k))) != want;
      ++n2;
    }
  }
  printf("(2) E4M3 element codes: %ld pairs, %ld mismatches\n", n2, bad2);

#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad3, n3)
  for (uint32_t a = 1; a < NBF; ++a) {
    float sg = bf(a) / 2688.0f;
    if (sg < 1e-12f) sg = 1e-12f;
    const float r0 = 1.0f / sg;
    for (uint32_t mb = 1; mb <= a; ++mb) {
      const float t = bf(mb) / 6.0f;
      const int want = e4m3_code(t / sg);
      for (int k = -1; k <= 1; ++k) bad3 += e4m3_code(quot(t, sg, nudge(r0, k))) != want;
      ++n3;
    }
  }
  printf("(3) NVFP4 block scale codes: %ld pairs, %ld mismatches\n", n3, bad3);

#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad4, n4)
  for (uint32_t a = 0; a < NBF; ++a) {   /* a == 0: the all-zero tensor (floor) */
    float sg = bf(a) / 2688.0f;
    if (sg < 1e-12f) sg = 1e-12f;
    for (int b = 1; b < 0x7f; ++b) {
      const float d = e4m3_val(b) * sg;
      const float r0 = 1.0f / d;
      const uint32_t lo = f2u(d * 0.125f) >> 16, hi0 = (f2u(d * 8.0f) >> 16) + 1;
      const uint32_t hi = hi0 < NBF ? hi0 : NBF;
      for (uint32_t xb = lo; xb < hi; ++xb) {
        const float x = bf(xb);
        const int want = e2m1_code(x / d);
        for (int k = -1; k <= 1; ++k) bad4 += e2m1_code(quot(x, d, nudge(r0, k))) != want;
        ++n4;
      }
    }
  }
  printf("(4) NVFP4 element codes: %ld triples, %ld mismatches\n", n4, bad4);
  return (bad1 || bad2 || bad3 || bad4) ? 1 : 0;
}
