/*
 * Exhaustive / sampled checks of two identities the quantize kernel relies on
 * (atlasinfer_amd/csrc/aq_common.h h_div_fast, aq_quantize.hip outlier_cut),
 * against the literal arithmetic of the reference (f32 op, one rounding).
 *
 *   1. fp16(x * r + fma corrections) == fp16(RN32(x / s)) for the code of x,
 *      i.e. the int8 code clamp(rne(.), +-127) and the E4M3 code agree, for
 *      every fp16 x and the given set of fp16 scales s.
 *   2. |fp16(a / den)| > thr  <=>  a > cut(den, thr) for every fp16 a >= 0.
 *
 * Usage: c_kernel_math_check <n_scales_step> <n_den_samples>
 *   n_scales_step 1 checks all 31743 positive finite fp16 scales.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

float aqo_h2f(uint16_t h);
uint16_t aqo_f2h(float f);
uint8_t aqo_e4m3_encode(double v);

static uint16_t hdiv_lit(uint16_t a, uint16_t b) { return aqo_f2h(aqo_h2f(a) / aqo_h2f(b)); }

static uint16_t hdiv_fast(uint16_t xb, uint16_t sb) {
  float x = aqo_h2f(xb), s = aqo_h2f(sb);
  volatile float r = 1.0f / s;
  float q0 = x * r;
  float e = fmaf(-q0, s, x);
  float q = fmaf(e, r, q0);
  return aqo_f2h(copysignf(q, x));
}

static uint8_t code_int8(uint16_t q16) {
  float r = nearbyintf(aqo_h2f(q16));
  if (r > 127.f) r = 127.f;
  if (r < -127.f) r = -127.f;
  return (uint8_t)(int8_t)r;
}

static uint8_t e4m3_tab[65536];

static int pred(uint16_t a, uint16_t den, uint16_t thr) {
  return fabsf(aqo_h2f(hdiv_lit(a, den))) > aqo_h2f(thr);
}

static float cut(uint16_t den, uint16_t thr) {
  float fden = aqo_h2f(den);
  if (!(fden > 0.0f) || isinf(fden)) return NAN;
  if (pred(0, den, thr)) return -1.0f;
  if (!pred(0x7C00, den, thr)) return INFINITY;
  uint32_t lo = 0, hi = 0x7C00;
  while (hi - lo > 1) {
    uint32_t mid = (lo + hi) >> 1;
    if (pred((uint16_t)mid, den, thr)) hi = mid; else lo = mid;
  }
  return aqo_h2f((uint16_t)lo);
}

int main(int argc, char** argv) {
  int step = argc > 1 ? atoi(argv[1]) : 64;
  int nden = argc > 2 ? atoi(argv[2]) : 200;
  for (int b = 0; b < 65536; b++) {
    float v = aqo_h2f((uint16_t)b);
    if (v == v) v = v > 448.f ? 448.f : (v < -448.f ? -448.f : v);
    e4m3_tab[b] = aqo_e4m3_encode(v);
  }
  long long bad_q = 0, bad_c = 0, checked = 0;
  for (uint32_t sb = 1; sb < 0x7C00; sb += step) {
    for (uint32_t xb = 0; xb < 65536; xb++) {
      if ((xb & 0x7C00) == 0x7C00) continue; /* inf/nan inputs are out of contract */
      uint16_t a = hdiv_lit((uint16_t)xb, (uint16_t)sb), f = hdiv_fast((uint16_t)xb, (uint16_t)sb);
      checked++;
      if (a != f) {
        bad_q++;
        if (code_int8(a) != code_int8(f) || e4m3_tab[a] != e4m3_tab[f]) {
          if (bad_c < 5) fprintf(stderr, "code mismatch x=%04x s=%04x lit=%04x fast=%04x\n", xb, sb, a, f);
          bad_c++;
        }
      }
    }
  }
  printf("quotient: %lld pairs, %lld fp16 quotient differences, %lld code differences\n", checked, bad_q, bad_c);
  /* identity 2 */
  srand(12345);
  long long bad_p = 0, pairs = 0;
  uint16_t thrs[] = {0x4200 /*3.0*/, 0x4300 /*3.5*/, 0x4299 /*3.3*/, 0x3C00, 0x0000, 0x0001, 0xBC00 /*-1*/,
                     0x7BFF, 0x7C00 /*inf*/};
  for (int i = 0; i < nden; i++) {
    uint16_t den = (uint16_t)(1 + rand() % 0x7BFF);
    if (i == 0) den = aqo_f2h(1e-6f);
    for (unsigned t = 0; t < sizeof(thrs) / sizeof(thrs[0]); t++) {
      float c = cut(den, thrs[t]);
      for (uint32_t a = 0; a <= 0x7C00; a++) {
        int lit = pred((uint16_t)a, den, thrs[t]);
        int fast = aqo_h2f((uint16_t)a) > c;
        pairs++;
        if (lit != fast) bad_p++;
      }
    }
  }
  printf("threshold: %lld pairs, %lld differences\n", pairs, bad_p);
  return (bad_c || bad_p) ? 1 : 0;
}
