/*
 * aq_oracle.c -- CPU restatement of AtlasInfer's adaptive hybrid quantizer.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (atlasinfer_amd/) links,
 * loads or calls this file; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker.
 *
 * It restates, element by element, the arithmetic of
 *   /root/reference/atlasinfer_core/quant/adaptive_quantizer.py
 *     calculate_zscore_manual        :44-49
 *     quantize_tensor (per block)    :84-133
 *     dequantize_tensor (per block)  :185-245
 * with every torch fp16 op written as "compute in f32, round once to fp16"
 * (what torch's CPU half kernels do), and the two reductions written in f64:
 *   mean = fp16(f32(S / G)),  S = sum of the block in f64
 *   std  = fp16(f32(sqrt(V / (G - 1)))), V = sum (x - S/G)^2 in f64
 * Both f64 sums use a balanced pairwise tree over next_pow2(G) leaves (the
 * leaves past G are 0).  torch accumulates in another order; the order only
 * matters when a sum lands within ~1e-16 of an fp16 rounding boundary, and
 * agreement with the reference itself is pinned by the golden vectors under
 * tests/golden/ (generated from the reference's own quantize_tensor).
 *
 * Code formats:
 *   fmt 0 "int8": the reference's format, q = clamp(rne(fp16(x / s)), +-127),
 *                 s = max(fp16(amax / 127), fp16(1e-6))   (:119-126)
 *   fmt 1 "e4m3": same op sequence with 127 -> 448 and the integer rounding
 *                 replaced by round-to-nearest-even onto OCP FP8 E4M3 (fn).
 * Codes are written densely (one byte per element of the zero-padded flat
 * tensor, 0 at outlier positions); the reference's compacted stream is a
 * reordering of the same bytes done by the Python wrapper (oracle.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 */

float aqo_h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else { /* subnormal: m * 2^-24 */
      float v = (float)m * 5.9604644775390625e-08f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else if (e == 31) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* f32 -> fp16, round to nearest, ties to even (IEEE 754 convertFormat). */
uint16_t aqo_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) {
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    return (uint16_t)(sign | 0x7C00u);
  }
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 */
  if (ax < 0x38800000u) {                                    /* < 2^-14 */
    if (ax <= 0x33000000u) return sign;                      /* <= 2^-25 */
    uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;
    uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = (ax >> 13) - (112u << 10), rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

/* -------------------------------------------------------------- e4m3fn */

double aqo_e4m3_to_double(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 0xF, m = c & 7;
  double v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexp((double)m, -9);
  else v = ldexp(1.0 + m / 8.0, e - 7);
  return s ? -v : v;
}

/* Nearest E4M3 value by exhaustive search over the 127 finite magnitudes,
 * ties to the even code (even mantissa).  |v| must be <= 448 (callers clamp
 * first, as the format definition requires); NaN maps to 0x7F. */
uint8_t aqo_e4m3_encode(double v) {
  if (isnan(v)) return 0x7F;
  uint8_t sign = signbit(v) ? 0x80 : 0x00;
  double a = fabs(v);
  int best = 0;
  double bestd = INFINITY;
  for (int c = 0; c <= 0x7E; c++) {
    double d = fabs(aqo_e4m3_to_double((uint8_t)c) - a);
    if (d < bestd) {
      bestd = d;
      best = c;
    } else if (d == bestd && (best & 1) && !(c & 1)) {
      best = c; /* tie: the even code (even mantissa) wins */
    }
  }
  return (uint8_t)(sign | best);
}

/* The quantizer only ever encodes fp16 values (the fp16 quotient, clamped to
 * +-448, which is itself an fp16 value), so the exhaustive search above is
 * run once per fp16 bit pattern and memoised: same results, a table lookup
 * per element.  Built on first use, single-threaded (aqo_init). */
static uint8_t g_e4m3_of_f16[65536];
static int g_e4m3_ready = 0;

void aqo_init(void) {
  if (g_e4m3_ready) return;
  for (uint32_t b = 0; b < 65536u; b++) {
    double v = (double)aqo_h2f((uint16_t)b);
    if (v == v) {
      if (v > 448.0) v = 448.0;
      if (v < -448.0) v = -448.0;
    }
    g_e4m3_of_f16[b] = aqo_e4m3_encode(v);
  }
  g_e4m3_ready = 1;
}

/* --------------------------------------------------------- reductions */

static double tree_sum(double* v, int64_t n) { /* n is a power of two */
  for (int64_t w = n; w > 1; w >>= 1)
    for (int64_t i = 0; i < w / 2; i++) v[i] = v[2 * i] + v[2 * i + 1];
  return v[0];
}

static int64_t next_pow2(int64_t g) {
  int64_t p = 1;
  while (p < g) p <<= 1;
  return p;
}

/* Statistics of one block, as the reference's calculate_zscore_manual
 * (:44-49) sees it: mean and std are fp16 tensors; den = fp16(std + eps). */
typedef struct {
  uint16_t mean16, std16, den16;
} aqo_stats;

static aqo_stats block_stats(const uint16_t* x, int64_t G, float eps, double* scratch) {
  int64_t P = next_pow2(G);
  for (int64_t i = 0; i < P; i++) scratch[i] = i < G ? (double)aqo_h2f(x[i]) : 0.0;
  double S = tree_sum(scratch, P);
  double mu = S / (double)G;
  for (int64_t i = 0; i < P; i++) {
    if (i < G) {
      double d = (double)aqo_h2f(x[i]) - mu;
      scratch[i] = d * d;
    } else {
      scratch[i] = 0.0;
    }
  }
  double V = tree_sum(scratch, P);
  double var = V / (double)(G - 1); /* torch.std: correction = 1; G == 1 -> NaN */
  aqo_stats st;
  st.mean16 = aqo_f2h((float)mu);
  st.std16 = aqo_f2h((float)sqrt(var));
  st.den16 = aqo_f2h(aqo_h2f(st.std16) + eps);
  return st;
}

/* fp16 tensor op "a - b" and "a / b": f32 op, one rounding to fp16. */
static uint16_t hsub(uint16_t a, uint16_t b) { return aqo_f2h(aqo_h2f(a) - aqo_h2f(b)); }
static uint16_t hdiv(uint16_t a, uint16_t b) { return aqo_f2h(aqo_h2f(a) / aqo_h2f(b)); }

/* calculate_zscore_manual(data, eps) for one 1-D fp16 tensor (:44-49). */
void aqo_zscore(const uint16_t* x, int64_t n, float eps, uint16_t* z, uint16_t* stats3) {
  double* scratch = (double*)malloc(sizeof(double) * (size_t)next_pow2(n > 0 ? n : 1));
  aqo_stats st = block_stats(x, n, eps, scratch);
  for (int64_t i = 0; i < n; i++) z[i] = hdiv(hsub(x[i], st.mean16), st.den16);
  if (stats3) {
    stats3[0] = st.mean16;
    stats3[1] = st.std16;
    stats3[2] = st.den16;
  }
  free(scratch);
}

/*
 * quantize_tensor body (:84-133) over the zero-padded flat tensor.
 *   x        fp16 bits, numel elements
 *   G        block size (>= 1)
 *   thr16    fp16 bits of the threshold (torch compares |z| > thr in fp16)
 *   fmt      0 int8, 1 e4m3
 * outputs (padded = ceil(numel / G) * G):
 *   codes    [padded]  dense codes, 0 at outliers
 *   scales   [padded / G] fp16 bits
 *   outlier  [padded]  1 where the element is an outlier
 *   stats    [padded / G * 3] (mean16, std16, den16) per block, may be NULL
 * returns the number of outliers.
 */
int64_t aqo_quantize(const uint16_t* x, int64_t numel, int64_t G, uint16_t thr16, int fmt,
                     uint8_t* codes, uint16_t* scales, uint8_t* outlier, uint16_t* stats) {
  int64_t nblocks = (numel + G - 1) / G;
  aqo_init();
  double* scratch = (double*)malloc(sizeof(double) * (size_t)next_pow2(G));
  uint16_t* blk = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)G);
  const float qmax = fmt == 0 ? 127.0f : 448.0f;
  const uint16_t min_scale = aqo_f2h(1e-6f);
  const float thr = aqo_h2f(thr16);
  int64_t nnz = 0;
  for (int64_t b = 0; b < nblocks; b++) {
    int64_t base = b * G;
    for (int64_t i = 0; i < G; i++) blk[i] = base + i < numel ? x[base + i] : 0; /* :84-87 */
    aqo_stats st = block_stats(blk, G, 1e-6f, scratch);
    if (stats) {
      stats[3 * b + 0] = st.mean16;
      stats[3 * b + 1] = st.std16;
      stats[3 * b + 2] = st.den16;
    }
    /* :106-107  is_outlier = |z| > z_threshold */
    float amax = -1.0f;
    int any_inlier = 0;
    for (int64_t i = 0; i < G; i++) {
      uint16_t z = hdiv(hsub(blk[i], st.mean16), st.den16);
      float az = fabsf(aqo_h2f(z));
      int is_out = az > thr;
      outlier[base + i] = (uint8_t)is_out;
      nnz += is_out;
      if (!is_out) {
        float a = fabsf(aqo_h2f(blk[i]));
        any_inlier = 1;
        if (a > amax) amax = a;
      }
    }
    /* :119-130  scale and codes */
    uint16_t s16 = 0x3C00; /* 1.0 when every element is an outlier */
    if (any_inlier) {
      s16 = aqo_f2h(amax / qmax);
      if (aqo_h2f(s16) < 1e-6f) s16 = min_scale;
    }
    scales[b] = s16;
    for (int64_t i = 0; i < G; i++) {
      uint8_t c = 0;
      if (!outlier[base + i]) {
        float q = aqo_h2f(hdiv(blk[i], s16));
        if (fmt == 0) {
          float r = nearbyintf(q); /* torch.round: half to even */
          if (r > 127.0f) r = 127.0f;
          if (r < -127.0f) r = -127.0f;
          c = (uint8_t)(int8_t)r;
        } else {
          /* e4m3(clamp(q, +-448)) by the memoised exhaustive search */
          c = g_e4m3_of_f16[hdiv(blk[i], s16)];
        }
      }
      codes[base + i] = c;
    }
  }
  free(scratch);
  free(blk);
  return nnz;
}

/* Value of one dense code. */
static float code_value(uint8_t c, int fmt) {
  return fmt == 0 ? (float)(int8_t)c : (float)aqo_e4m3_to_double(c);
}

/*
 * dequantize_tensor (:185-245): fp16(code * scale) for inliers, outlier
 * values verbatim, trimmed to numel.  idx are flat indices into the padded
 * tensor (ascending); entries >= numel (outliers in the padding) are dropped.
 */
void aqo_dequantize(const uint8_t* codes, const uint16_t* scales, int64_t numel, int64_t G, int fmt,
                    const int64_t* idx, const uint16_t* vals, int64_t nnz, uint16_t* out) {
  for (int64_t j = 0; j < numel; j++)
    out[j] = aqo_f2h(code_value(codes[j], fmt) * aqo_h2f(scales[j / G]));
  for (int64_t p = 0; p < nnz; p++)
    if (idx[p] < numel) out[idx[p]] = vals[p];
}

/* The quotient fp16(x / s) as the reference computes it (:123-125). */
uint16_t aqo_hdiv(uint16_t a, uint16_t b) { return hdiv(a, b); }
