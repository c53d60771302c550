/*
 * Exhaustive / sampled checks of the identities the quantize kernel relies on
 * (atlasinfer_amd/csrc/aq_common.h h_div_fast, aq_quantize.hip quot2 and
 * outlier_cut), against the literal arithmetic of the reference (f32 op, one
 * rounding).
 *
 *   1. fp16(x * r + fma corrections) == fp16(RN32(x / s)) for the code of x,
 *      i.e. the int8 code clamp(rne(.), +-127) and the E4M3 code agree, for
 *      every fp16 x and the given set of fp16 scales s.
 *   2. |fp16(a / den)| > thr  <=>  a > cut(den, thr) for every fp16 a >= 0.
 *   3. One fused product: fp16(x * r - 0) with r = RN32(1 / s), the product
 *      exact and rounded once to fp16 or first to f32 and then to fp16
 *      (both forms, since either is what a mixed-precision fma may do), gives
 *      the same E4M3 code as fp16(RN32(x / s)) for every fp16 x with
 *      |x / s| <= 448.25 (every non-outlier of a block scaled by amax / 448),
 *      and the same fp16 quotient wherever that quotient is an fp16 normal.
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

/* double -> fp16, round to nearest even, one rounding (|v| < 65520). */
static uint16_t d2h(double v) {
  uint16_t sign = signbit(v) ? 0x8000 : 0;
  double a = fabs(v);
  if (a == 0.0) return sign;
  int e;
  frexp(a, &e); /* a = m 2^e, m in [0.5, 1) */
  int q_exp = e - 11 < -24 ? -24 : e - 11; /* fp16 spacing at a: 2^(e - 11), at least 2^-24 */
  double q = a / ldexp(1.0, q_exp);
  double fl = floor(q), rem = q - fl;
  if (rem > 0.5 || (rem == 0.5 && fmod(fl, 2.0) != 0.0)) fl += 1.0;
  return (uint16_t)(sign | aqo_f2h((float)ldexp(fl, q_exp)));
}

/* the fused product of identity 3: x * r + (-0), exact, rounded once (mode 0)
 * or to f32 first (mode 1) */
static uint16_t quot_product(uint16_t xb, uint16_t sb, int mode) {
  float x = aqo_h2f(xb), s = aqo_h2f(sb);
  volatile float r = 1.0f / s;
  if (mode == 1) {
    volatile float p = x * r;
    return aqo_f2h(p + -0.0f);
  }
  return d2h((double)x * (double)r + -0.0);
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
  /* identity 3 */
  long long p_checked = 0, p_bad_code = 0, p_bad_normal = 0;
  for (uint32_t sb = 1; sb < 0x7C00; sb += step) {
    float s = aqo_h2f((uint16_t)sb);
    for (uint32_t xb = 0; xb < 65536; xb++) {
      if ((xb & 0x7C00) == 0x7C00) continue;
      float x = aqo_h2f((uint16_t)xb);
      if (fabsf(x) / s > 448.25f) continue; /* not a non-outlier of a block with this scale */
      uint16_t lit = hdiv_lit((uint16_t)xb, (uint16_t)sb);
      for (int mode = 0; mode < 2; mode++) {
        uint16_t f = quot_product((uint16_t)xb, (uint16_t)sb, mode);
        p_checked++;
        if (e4m3_tab[lit] != e4m3_tab[f] || code_int8(lit) != code_int8(f)) {
          if (p_bad_code < 5) fprintf(stderr, "product code mismatch x=%04x s=%04x mode %d lit=%04x f=%04x\n", xb, sb, mode, lit, f);
          p_bad_code++;
        }
        if ((lit & 0x7C00) != 0 && lit != f) p_bad_normal++;
      }
    }
  }
  printf("product: %lld pairs, %lld code differences, %lld normal-quotient differences\n", p_checked, p_bad_code,
         p_bad_normal);
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
  return (bad_c || bad_p || p_bad_code || p_bad_normal) ? 1 : 0;
}
