// aq_quantize.hip -- the quantize kernel and its outlier compaction.
//
// Replaces the per-block Python loop of quantize_tensor
// (reference: atlasinfer_core/quant/adaptive_quantizer.py:84-133) and the
// z-score helper calculate_zscore_manual (:44-49).
//
// One team of TAU threads owns one block of G elements; each thread holds E
// consecutive elements in registers, so the input is read from HBM exactly
// once.  Per block the team computes, in this order:
//   S    = sum x            (f64, balanced tree)      mean = fp16(f32(S/G))
//   V    = sum (x - S/G)^2  (f64, balanced tree)      std  = fp16(f32(sqrt(V/(G-1))))
//   den  = fp16(std + 1e-6)
//   flag = |fp16(fp16(x - mean) / den)| > thr   -- evaluated as |fp16(x - mean)| > Th
//          with Th the largest fp16 whose quotient does not pass.  The
//          literal test is monotone in |x - mean| and turns true within a
//          few fp16 steps of fp16(thr * den), so the team's lanes evaluate
//          it on 16 consecutive bit patterns there at once and a ballot
//          locates the step (bisection over all patterns if it is not in
//          that window); both forms agree on every input.
//   amax = max |x| over non-outliers (wave shuffles)
//   s    = max(fp16(amax / qmax), fp16(1e-6)), 1.0 if all are outliers
//   code = clamp(rne(fp16(x / s)), +-127)  or  e4m3(clamp(fp16(x / s), +-448))
//          (the e4m3 rounding by the hardware f32 -> fp8 conversion, which
//          equals the round-to-nearest-even encoding on every fp16 in
//          [-448, 448])
// Outliers are compacted inside the team with a prefix sum (shuffles + LDS)
// into a per-block staging slot; a scan over the per-block counts and a
// gather pass then write the ascending outlier list.
#include <math.h>

#include "aq_common.h"
#include "aq_tiles.h"

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t h2_bits(half2v h) { return __builtin_bit_cast(uint32_t, h); }

constexpr int kWG = 256;            // threads per workgroup for TAU <= 256
constexpr int kScanChunk = 1024;    // least block counts per scan workgroup (256 x 4), sizes the partials
constexpr int64_t kMaxG = 65536;

struct QuantArgs {
  const uint16_t* x;
  int64_t numel;
  int64_t G;
  int64_t nblocks;
  uint16_t thr_bits;
  int fmt;
  int vec;  // G % 16 == 0 and x 16-byte aligned: 16-byte loads/stores
  int tiled;        // codes in the tiled layout (rows of K, K % 128 == 0, N % 16 == 0)
  int64_t K;        // row length for the tiled layout
  int64_t nchunks;  // K / 128
  int64_t bpr;      // tiled layout: blocks per row, K / G
  double inv_g;     // RN64(1 / G)
  float inv_g1;     // RN32(1 / (G - 1)) (G >= 2)
  uint8_t* codes;
  uint16_t* scales;
  int32_t* block_cnt;  // block_off, holds counts until the scan
  int32_t* stage_col;
  uint16_t* stage_val;
};

// Up to kMaxQGroup weights of one block size quantized by one launch
// (aq_quantize_grouped; aq_quantize is a group of one): workgroup b takes
// unit b - first[i] of member i, first[i] <= b < first[i + 1].
constexpr int kMaxQGroup = 8;
struct QuantGroup {
  QuantArgs m[kMaxQGroup];
  int64_t first[kMaxQGroup + 1];
  int count;
  int xcd_rows;  // units taken in XCD-contiguous order (xcd_unit)
};

// Workgroup b runs on XCD b % 8 (the dispatcher deals a launch's workgroups
// round-robin over the 8 XCDs, each with its own L2).  A 128-byte line of
// tiled codes holds 16-byte pieces of 8 consecutive rows; when the units of
// 8 consecutive rows run on 8 XCDs, every L2 writes the line back with a
// 16-byte piece of it dirty.  xcd_unit gives XCD x the x-th contiguous
// eighth of the units instead, so consecutive rows meet in one L2 (a
// bijection of [0, n)).
__device__ __forceinline__ int64_t xcd_unit(int64_t b, int64_t n) {
  const int64_t per = n >> 3, rem = n & 7, x = b & 7, slot = b >> 3;
  return x < rem ? x * (per + 1) + slot : rem * (per + 1) + (x - rem) * per + slot;
}

// E fp16 elements of one thread, two per 32-bit register (element 2i in
// the low half); indices are compile-time constants after unrolling, so
// reading an element costs at most a shift.
template <int E>
struct Elems {
  uint32_t p[E / 2];
  __device__ __forceinline__ f16 operator[](int e) const {
    return bits_to_h((uint16_t)((e & 1) ? (p[e >> 1] >> 16) : (p[e >> 1] & 0xFFFFu)));
  }
  // Between passes: the compiler may no longer reuse values derived from
  // the elements in an earlier pass (it would keep E converted copies live
  // across the whole kernel); re-deriving them is a conversion each.
  __device__ __forceinline__ void fence() {
#pragma unroll
    for (int i = 0; i < E / 2; i++) asm volatile("" : "+v"(p[i]));
  }
};

// The staged copy of a workgroup's blocks in LDS: 16-byte pieces, each
// thread's E / 8 pieces (P = thread * E / 8 + j) stored at P with its low
// bits XORed with the thread's, so that a thread's reads, at a stride of
// E * 2 bytes between threads, hit distinct banks.
template <int E>
__device__ __forceinline__ int stage_swz(int P) {
  constexpr int PPT = E / 8;
  return P ^ ((P / PPT) & (PPT - 1));
}
// uint16 index of the workgroup's element i in the staged copy.
template <int E>
__device__ __forceinline__ int staged_index(int i) {
  return (stage_swz<E>(i >> 3) << 3) | (i & 7);
}

// How much of a block a thread's E elements cover: every element of every
// block (G is a power of two), all or none of a thread's elements (E
// divides G), or any prefix.  The first two cases need no per-element
// bounds tests.
enum { kAnyLen = 0, kThreadAligned = 1, kFullBlocks = 2 };

template <int MODE>
__device__ __forceinline__ bool elem_valid(int i0, int e, int64_t G) {
  if (MODE == kFullBlocks) return true;
  if (MODE == kThreadAligned) return i0 < G;
  return i0 + e < G;
}

// Balanced pairwise tree over 16 leaves.
__device__ __forceinline__ double tree16(double (&v)[16]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int w = 16; w > 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w / 2; i++) v[i] = v[2 * i] + v[2 * i + 1];
  return v[0];
}

// Balanced tree over the E leaves of one thread, E = 16 * C.
template <int E, int MODE>
__device__ __forceinline__ double thread_tree_sum(Elems<E>& xs, int i0, int64_t G, bool sq, double mu) {
#pragma clang fp contract(off)
  constexpr int C = E / 16;
  double part[C];
#pragma unroll
  for (int c = 0; c < C; c++) {
    double leaf[16];
#pragma unroll
    for (int e = 0; e < 16; e++) {
      double v = (double)(float)xs[c * 16 + e];
      if (sq) {
        double d = v - mu;
        v = d * d;
      }
      leaf[e] = elem_valid<MODE>(i0, c * 16 + e, G) ? v : 0.0;
    }
    part[c] = tree16(leaf);
    if (C > 1) xs.fence();  // one group of 16 double leaves live at a time
  }
#pragma unroll
  for (int w = C; w > 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w / 2; i++) part[i] = part[2 * i] + part[2 * i + 1];
  return part[0];
}

struct BlockStats {
  f16 mean16, std16, den16;
};

// mean / std / std + eps of one block, as calculate_zscore_manual computes
// them (the torch fp16 tensors mean, std and std + eps).
template <int TAU, int E, int MODE = kAnyLen>
__device__ __forceinline__ BlockStats block_stats(Elems<E>& xs, int i0, int64_t G, float eps,
                                                  double* lds_d) {
#pragma clang fp contract(off)
  double s_loc = thread_tree_sum<E, MODE>(xs, i0, G, false, 0.0);
  double S = team_sum_f64<TAU>(s_loc, lds_d);
  double mu = S / (double)G;
  xs.fence();
  double v_loc = thread_tree_sum<E, MODE>(xs, i0, G, true, mu);
  double V = team_sum_f64<TAU>(v_loc, lds_d);
  double var = V / (double)(G - 1);
  BlockStats st;
  st.mean16 = rn_h((float)mu);
  st.std16 = rn_h((float)sqrt(var));
  st.den16 = rn_h((float)st.std16 + eps);
  return st;
}

// The reference's outlier test for one |x - mean| value a (fp16, >= 0).
__device__ __forceinline__ bool outlier_literal(f16 a, f16 den, f16 thr) {
  return fabsf((float)h_div(a, den)) > (float)thr;
}

// Th such that  |fp16(a / den)| > thr  <=>  a > Th  for every fp16 a >= 0.
// Returns NaN when den is not a positive finite number (then the caller
// evaluates the literal test per element).
__device__ float outlier_cut(f16 den, f16 thr) {
  const float fden = (float)den;
  if (!(fden > 0.0f) || isinf(fden)) return __builtin_nanf("");
  if (outlier_literal(bits_to_h(0), den, thr)) return -1.0f;        // all are outliers
  if (!outlier_literal(bits_to_h(0x7C00), den, thr)) return INFINITY;  // none
  uint32_t lo = 0, hi = 0x7C00;  // pred(lo) false, pred(hi) true
  while (hi - lo > 1) {
    uint32_t mid = (lo + hi) >> 1;
    if (outlier_literal(bits_to_h((uint16_t)mid), den, thr))
      hi = mid;
    else
      lo = mid;
  }
  return (float)bits_to_h((uint16_t)lo);
}

// Th for a team of TAU threads (the same value in every lane): lane j of the
// team (j < 16) tests the bit pattern c0 - 8 + j, c0 = bits of fp16(thr * den).
template <int TAU>
__device__ float outlier_cut_team(f16 den, f16 thr) {
  const float fden = (float)den;
  if (!(fden > 0.0f) || isinf(fden)) return __builtin_nanf("");
  if (outlier_literal(bits_to_h(0), den, thr)) return -1.0f;        // all are outliers
  if (!outlier_literal(bits_to_h(0x7C00), den, thr)) return INFINITY;  // none
  constexpr int W = TAU < 16 ? TAU : 16;
  constexpr int TL = TAU < 64 ? TAU : 64;  // team lanes within one wave
  const int lane = threadIdx.x & 63;
  const int ts = lane & ~(TL - 1);  // the team's first lane in this wave
  const int j = lane - ts;
  const float est = (float)thr * fden;
  const int c0 = est < 65504.0f ? (int)h_to_bits(rn_h(est)) : 0x7BFF;
  const int cand = c0 - W / 2 + j;
  // below 0 the test is false (checked at 0 above), past 0x7C00 true (checked at inf)
  bool p = cand > 0x7C00 || (cand >= 0 && outlier_literal(bits_to_h((uint16_t)cand), den, thr));
  p = p && j < W;
  const uint64_t bal = __ballot(p);
  const uint32_t bits = (uint32_t)(bal >> ts) & ((1u << W) - 1u);
  if (bits != 0 && !(bits & 1u)) {
    const int first = c0 - W / 2 + __builtin_ctz(bits);  // smallest pattern that passes
    return (float)bits_to_h((uint16_t)(first - 1));
  }
  return outlier_cut(den, thr);
}

template <int E>
__device__ __forceinline__ void load_elems(Elems<E>& xs, const QuantArgs& a, int64_t base, int i0, bool gvalid) {
  const bool full = gvalid && a.vec && (i0 + E <= a.G) && (base + i0 + E <= a.numel);
  if (full) {
    // plain loads: each thread reads E / 8 consecutive 16-byte pieces, so a
    // 128-byte line is touched by several load instructions in a row, and a
    // non-temporal hint would make each of them fetch it again
    const uint4* src = reinterpret_cast<const uint4*>(a.x + base + i0);
#pragma unroll
    for (int v = 0; v < E / 8; v++) {
      uint4 u = src[v];
      xs.p[4 * v] = u.x;
      xs.p[4 * v + 1] = u.y;
      xs.p[4 * v + 2] = u.z;
      xs.p[4 * v + 3] = u.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; e += 2) {
      uint32_t pair = 0;
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int64_t i = i0 + e + h;
        const int64_t j = base + i;
        if (gvalid && i < a.G && j < a.numel) pair |= (uint32_t)a.x[j] << (16 * h);
      }
      xs.p[e / 2] = pair;
    }
  }
}

// The rest of a block after its elements are loaded, for any block length:
// per-element bounds tests, outlier flags in a 64-bit mask.
template <int TAU, int E, int MODE>
__device__ __forceinline__ void finish_block_any(const QuantArgs& a, Elems<E>& xs, int64_t g, bool gvalid,
                                                 int64_t base, int i0, int t, double* lds_d, float* lds_f,
                                                 int* lds_i) {
  const int64_t G = a.G;
  const BlockStats st = block_stats<TAU, E, MODE>(xs, i0, G, 1e-6f, lds_d);
  xs.fence();
  const f16 thr = bits_to_h(a.thr_bits);
  const float cut = outlier_cut_team<TAU>(st.den16, thr);
  const bool literal = isnan(cut);

  // outlier flags and the absmax of the rest, 16 elements at a time; the
  // literal quotient only for blocks whose std + eps is not a positive
  // finite number (a uniform branch, so the common path has no division)
  uint64_t omask = 0;
  float amax = -1.0f;
#pragma unroll
  for (int g16 = 0; g16 < E / 16; g16++) {
#pragma unroll
    for (int b = 0; b < 16; b++) {
      const int e = 16 * g16 + b;
      if (elem_valid<MODE>(i0, e, G)) {
        const f16 d = h_sub(xs[e], st.mean16);
        const f16 ad = bits_to_h(h_to_bits(d) & 0x7FFFu);
        bool o;
        if (literal)
          o = outlier_literal(ad, st.den16, thr);
        else
          o = (float)ad > cut;
        if (o)
          omask |= 1ull << e;
        else
          amax = fmaxf(amax, fabsf((float)xs[e]));
      }
    }
    if (E > 16) xs.fence();
  }
  amax = team_max_f32<TAU>(amax, lds_f);
  xs.fence();

  const float qmax = a.fmt == AQ_FMT_INT8 ? 127.0f : 448.0f;
  f16 s16 = (f16)1.0f;
  if (amax >= 0.0f) {
    s16 = rn_h(amax / qmax);
    if ((float)s16 < 1e-6f) s16 = rn_h(1e-6f);
  }
  const float s = (float)s16;
  const float r = 1.0f / s;

  // where the thread's elements sit in the [rows, K] matrix (tiled layout)
  int64_t row = 0, col0 = 0;
  if (a.tiled) {
    row = a.bpr == 1 ? g : g / a.bpr;
    col0 = (g - row * a.bpr) * G + i0;
  }

  // codes, 16 elements at a time (four words in element order)
#pragma unroll
  for (int v = 0; v < E / 16; v++) {
    uint32_t w[4];
    if (a.fmt == AQ_FMT_INT8) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const int e = 16 * v + 4 * k + b;
          uint32_t code = 0;
          if (!((omask >> e) & 1ull) && elem_valid<MODE>(i0, e, G)) {
            float rr = __builtin_rintf((float)h_div_fast((float)xs[e], s, r));
            rr = fminf(fmaxf(rr, -127.0f), 127.0f);
            code = (uint8_t)(int8_t)(int)rr;
          }
          word |= code << (8 * b);
        }
        w[k] = word;
      }
    } else {
      float qv[16];
#pragma unroll
      for (int b = 0; b < 16; b++) {
        // outliers and padding get code 0 (+0.0)
        const int e = 16 * v + b;
        const float q = (float)h_div_fast((float)xs[e], s, r);
        qv[b] = (!((omask >> e) & 1ull) && elem_valid<MODE>(i0, e, G)) ? __builtin_amdgcn_fmed3f(q, -448.0f, 448.0f)
                                                                       : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(qv[4 * k], qv[4 * k + 1], 0, false);
        w[k] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(qv[4 * k + 2], qv[4 * k + 3], lo, true);
      }
    }
    if (E > 16) xs.fence();
    if (gvalid) {
      // 16 consecutive elements of one row land in 16 consecutive bytes of either layout
      const int64_t j = base + i0 + 16 * v;
      if (a.vec && i0 + E <= G) {
        const int64_t off = a.tiled ? tiled_offset(row, col0 + 16 * v, a.nchunks) : j;
        *reinterpret_cast<uint4*>(a.codes + off) = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
#pragma unroll
        for (int b = 0; b < 16; b++)
          if (i0 + 16 * v + b < G)
            a.codes[a.tiled ? tiled_offset(row, col0 + 16 * v + b, a.nchunks) : j + b] =
                (uint8_t)(w[b / 4] >> (8 * (b % 4)));
      }
    }
  }

  // outlier compaction: team prefix sum, then the block's staging slot
  const int cnt = __builtin_popcountll(omask);
  int total;
  const int pre = team_excl_scan_i32<TAU>(cnt, lds_i, &total);
  if (gvalid) {
    int k = pre;
    uint64_t m = omask;
    while (m) {
      const int e = __builtin_ctzll(m);
      m &= m - 1;
      // the value from memory (an L2 hit): indexing the registers with a
      // run-time e would move them to scratch; padding elements are 0
      const int64_t j = base + i0 + e;
      a.stage_col[base + k] = i0 + e;
      a.stage_val[base + k] = j < a.numel ? a.x[j] : (uint16_t)0;
      k++;
    }
    if (t == 0) {
      a.scales[g] = h_to_bits(s16);
      a.block_cnt[g] = total;
    }
  }
}

// f32 fused multiply-adds with fp16 sources taken from the halves of packed
// pairs (v_fma_mix_f32: the fp16 operands enter exactly, one f32 rounding).
// Written out because the compiler splits x * 1 + y into two conversions and
// an add.
__device__ __forceinline__ float pair_sum_f32(uint32_t p) {  // lo + hi
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(p));
  return r;
}
__device__ __forceinline__ float sq_acc_lo(uint32_t p, float c) {  // lo * lo + c
  float r;
  asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel:[0,0,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(p), "v"(c));
  return r;
}
__device__ __forceinline__ float sq_acc_hi(uint32_t p, float c) {  // hi * hi + c
  float r;
  asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel:[1,1,0] op_sel_hi:[1,1,0]" : "=v"(r) : "v"(p), "v"(c));
  return r;
}

// The reference's mean of a block whose sum is S: fp16(f32(S / G)), and its
// std from V = sum (x - mean)^2: fp16(f32(sqrt(V / (G - 1)))).  Both are
// monotone non-decreasing functions (f64 operations and round-to-nearest
// conversions, each monotone).
__device__ __forceinline__ f16 mean_of_sum(double S, int64_t G) { return rn_h((float)(S / (double)G)); }
__device__ __forceinline__ f16 std_of_var(double V, int64_t G) { return rn_h((float)sqrt(V / (double)(G - 1))); }

// mean / std / std + eps as block_stats computes them, from one pass of
// single-precision sums in the common case:
//   S  = sum x   as an f32 tree (leaf pairs by one fused multiply-add of the
//        fp16 values, x0 * 1 + x1, then a balanced tree): depth d = log2(E)
//        roundings of u = 2^-24 per thread, so |S_f32 - S| <= d u sum|x|
//        (the f64 sum across the team adds under 2^-46 relative), and
//        sum|x| <= sqrt(G Q) by Cauchy-Schwarz;
//   Q  = sum x^2 (products exact in f32, four f32 chains of E / 8 per
//        thread, then f32 across the team): a sum of non-negative terms
//        with at most E / 8 + 2 + log2(TAU) roundings, within Q 2^-19.
// mean16 is a monotone function of S, so when both ends of S_f32 +- errS
// give the same mean16, that is the value the exact sum gives; std16 is a
// monotone function of V = Q - S mu, accepted when both ends of V +- errV
// (errV covers Q's error and S's) give the same std16.  The two ends are
// evaluated with cheaper arithmetic than the functions themselves, on
// arguments pushed outward by more than that arithmetic's error, so each end
// still bounds the function's value at the true argument (see the comments
// at each step).  Otherwise (a near-tie, a non-finite sum, G < 2) the team
// falls back to the exact-order f64 trees of block_stats: the sum, and the
// two-pass variance when std16 is the open one.  Every decision is the same
// in all lanes of the team (its sums are), and for teams of several waves
// sharing a workgroup's barriers it is taken by the whole workgroup.
template <int TAU, int E, int MODE>
__device__ __forceinline__ BlockStats block_stats_fast(Elems<E>& xs, int i0, const QuantArgs& a, float eps,
                                                       double* lds_d, float* lds_f) {
#pragma clang fp contract(off)
  constexpr int NT = TAU > kWG ? TAU : kWG;
  constexpr bool kSyncedTeams = TAU > 64 && NT / TAU > 1;
  constexpr int kDepth = E == 16 ? 4 : E == 32 ? 5 : 6;
  static_assert(E == 16 || E == 32 || E == 64, "tree depth");
  const int64_t G = a.G;
  // padding elements are zeros: every E elements enter the sums
  float sp[E / 2];
#pragma unroll
  for (int i = 0; i < E / 2; i++) sp[i] = pair_sum_f32(xs.p[i]);
#pragma unroll
  for (int w = E / 2; w > 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w / 2; i++) sp[i] = sp[2 * i] + sp[2 * i + 1];
  float q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < E / 2; i++) {
    q[(2 * i) & 3] = sq_acc_lo(xs.p[i], q[(2 * i) & 3]);
    q[(2 * i + 1) & 3] = sq_acc_hi(xs.p[i], q[(2 * i + 1) & 3]);
  }
  double Sf = (double)sp[0];
  float Qf = (q[0] + q[1]) + (q[2] + q[3]);
  // the block's first use of lds_d / lds_f (one block per team and workgroup)
  team_sum_f64_f32<TAU, true>(Sf, Qf, lds_d, lds_f);
  const double Q = (double)Qf;
  // sqrt(G Q) from above: (1 + 2^-14) covers Q's 2^-19 and the two f32
  // products' roundings, (1 + 2^-20) the square root's one ulp and the last
  // rounding (G Q stays below 2^47: no overflow; an inf or NaN propagates)
  const float absum = __builtin_amdgcn_sqrtf((float)G * Qf * (1.0f + 0x1p-14f)) * (1.0f + 0x1p-20f);
  const double errS = (double)(kDepth + 1) * 0x1p-24 * (double)absum + fabs(Sf) * 0x1p-50;
  // the bracket's ends as (Sf -+ errS2) * RN64(1 / G): three f64 roundings
  // move a product by at most 3.1 * 2^-53 of |Sf| + errS2, which the extra
  // |Sf| 2^-49 and errS 2^-48 exceed, so lo_t <= (Sf - errS) / G and
  // hi_t >= (Sf + errS) / G as real numbers, and the f64 quotient of the
  // exact sum (between those) rounds between fp16(f32(lo_t)) and
  // fp16(f32(hi_t))
  const double errS2 = (errS + fabs(Sf) * 0x1p-49) * (1.0 + 0x1p-48);
  const f16 m_lo = rn_h((float)((Sf - errS2) * a.inv_g)), m_hi = rn_h((float)((Sf + errS2) * a.inv_g));
  bool need_exact = !(h_to_bits(m_lo) == h_to_bits(m_hi) && !isnan((float)m_lo));
  if constexpr (kSyncedTeams) need_exact = __syncthreads_or(need_exact);
  double S = Sf, dS = errS;
  BlockStats st;
  st.mean16 = m_lo;
  if (need_exact) {
    xs.fence();
    S = team_sum_f64<TAU>(thread_tree_sum<E, MODE>(xs, i0, G, false, 0.0), lds_d);
    dS = 0.0;
    st.mean16 = mean_of_sum(S, G);
  }
  bool open = true;
  if (G >= 2) {
    // |S * mu| <= Q (Cauchy-Schwarz): every rounding below, and mu taken as
    // S * RN64(1 / G), stays far inside the Q 2^-16 term
    const double mu = S * a.inv_g;
    const double V = Q - S * mu;
    const double err = Q * 0x1p-16 + (2.0 * fabs(S) + dS) * dS * a.inv_g + fabs(V) * 0x1p-50;
    // sqrt((V -+ err) / (G - 1)) in f32 with c = RN32(1 / (G - 1)): the
    // conversions, the product and the square root (one ulp) stay within
    // 2^-22 relative, so the 2^-20 pulls put ylo below and yhi above the
    // exact roots at V - err and V + err, and below / above the f64 results
    // there (2^-52 from the exact roots); fp16 rounding of an f32 value
    // equals fp16(f32(.)) of it, so lo <= std16 <= hi.  (An f32 argument
    // small enough to be flushed has a root below 2^-63, which rounds to
    // fp16 0 either way.)
    const float ylo = __builtin_amdgcn_sqrtf((float)fmax(V - err, 0.0) * a.inv_g1) * (1.0f - 0x1p-20f);
    const float yhi = __builtin_amdgcn_sqrtf((float)(V + err) * a.inv_g1) * (1.0f + 0x1p-20f);
    const f16 lo = rn_h(ylo), hi = rn_h(yhi);
    open = !(h_to_bits(lo) == h_to_bits(hi) && !isnan((float)lo));
    st.std16 = lo;
  }
  if constexpr (kSyncedTeams) open = __syncthreads_or(open);
  if (open) {
    xs.fence();
    double Se = S;
    if (dS != 0.0) Se = team_sum_f64<TAU>(thread_tree_sum<E, MODE>(xs, i0, G, false, 0.0), lds_d);
    const double mue = Se / (double)G;
    xs.fence();
    const double v_loc = thread_tree_sum<E, MODE>(xs, i0, G, true, mue);
    st.std16 = std_of_var(team_sum_f64<TAU>(v_loc, lds_d), G);
  }
  st.den16 = rn_h((float)st.std16 + eps);
  return st;
}

// Packed 16-bit integer operations, written out because the compiler turns
// the equivalent vector expressions into per-half compares and selects.
__device__ __forceinline__ uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
  uint32_t d;
  asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
  uint32_t d;
  asm("v_pk_sub_u16 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
  uint32_t d;
  asm("v_pk_min_u16 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
  return d;
}
// gfx950 three-operand packed fp16 maximum / minimum (IEEE maximum and
// minimum per half: -0 < +0, a NaN operand gives NaN)
__device__ __forceinline__ uint32_t pk_maximum3_f16(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_pk_maximum3_f16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ uint32_t pk_minimum3_f16(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_pk_minimum3_f16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// fp16(x / s) for both halves of a pair, s > 0, r = RN32(1 / s): one mixed
// fused multiply-add per half, x * r + (-0), the fp16 x entering exactly and
// the product rounded to fp16.  Why one product suffices: a quotient x / s
// can lie near an fp16 rounding midpoint m (odd 12-bit significand) only as
// x / s = m (1 + e) with |e| > 2^-23, since m s has a significand below 2^23
// that x (11 bits) cannot equal; x * r = (x / s)(1 + d) with |d| <= 2^-24,
// and a rounding through f32 on the way adds at most another 2^-24, so the
// product rounds to the same fp16 value as RN32(x / s) wherever that value
// is an fp16 normal.  Below, in the fp16 subnormal range, the two can differ
// only on exact ties, and every such quotient (|q| < 2^-14) encodes to code
// 0 in either format.  The -0 addend keeps the sign of a zero x (x * r = -0
// for x = -0).  Checked over all fp16 x and s with |x / s| <= 448.25, under
// both rounding behaviours (tests/c_kernel_math_check.c).
__device__ __forceinline__ uint32_t quot2(uint32_t xp, float r) {
  uint32_t q;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]\n\t"
      "v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=&v"(q)
      : "v"(xp), "v"(r), "v"(-0.0f));
  return q;
}

// Code exchange of a workgroup of four 4096-element rows (per-channel
// blocks): 16-byte piece (column piece c, row r) at slot 4 c + r, the low
// four bits XORed with bits 4-7 so that both the writes (lanes 16 slots
// apart) and the reads (consecutive slots) spread over the LDS banks.
__device__ __forceinline__ int xchg_slot(int i) { return i ^ ((i >> 4) & 15); }

// The rest of a block after its elements are loaded, when a thread's E
// elements are all inside the block or all padding (E divides G).  Works on
// element pairs with packed arithmetic: d = x - mean in fp16, then, since
// non-negative fp16 values order like their bit patterns,
//   outlier <=> |d| > Th  <=>  sat(bits|d| - bits Th) != 0   (per half).
// Outliers are replaced by +0 in xs, so the absmax is a packed max over xs
// and the code pass needs no flags (a +0 gives code 0); their values are
// read again from memory for the compaction.  Flag bits: word w covers
// pairs PW w .. PW w + PW - 1, built as acc = 2 acc + m with m holding the
// pair's low / high outlier bit at bit 0 / 16.
template <int TAU, int E, int MODE>
__device__ __forceinline__ void finish_block_fast(const QuantArgs& a, Elems<E>& xs, int64_t g, bool gvalid,
                                                  int64_t base, int i0, int t, double* lds_d, float* lds_f,
                                                  int* lds_i, const uint16_t* staged, int unit_e0,
                                                  uint4* xchg) {
  constexpr int NP = E / 2;              // pairs per thread
  constexpr int PW = NP < 16 ? NP : 16;  // pairs per flag word
  constexpr int NWD = NP / PW;
  const int64_t G = a.G;
  const bool tvalid = MODE == kFullBlocks || i0 < G;

  const BlockStats st = block_stats_fast<TAU, E, MODE>(xs, i0, a, 1e-6f, lds_d, lds_f);
  xs.fence();
  const f16 thr = bits_to_h(a.thr_bits);
  const float cut = outlier_cut_team<TAU>(st.den16, thr);

  uint32_t obits[NWD];
  // packed fp16 maximum and minimum of the pairs after the outliers are
  // zeroed, two pairs per instruction; starting from +0 is harmless since
  // the absmax below is max(max, -min) >= 0
  uint32_t mx = 0, mn = 0;
  if (cut >= 0.0f) {
    // cut is an fp16 value or +inf (none are outliers)
    const uint32_t th = (uint32_t)h_to_bits((f16)cut) * 0x00010001u;
    const half2v nm = (half2v){-st.mean16, -st.mean16};
#pragma unroll
    for (int w = 0; w < NWD; w++) {
      uint32_t acc = 0;
#pragma unroll
      for (int j = 0; j < PW; j++) {
        const int i = w * PW + j;
        const uint32_t ad = h2_bits(as_h2(xs.p[i]) + nm) & 0x7FFF7FFFu;
        const uint32_t m = pk_min_u16(pk_sub_sat_u16(ad, th), 0x00010001u);
        xs.p[i] &= ~pk_sub_u16(0u, m);  // 0xFFFF in each outlier half
        acc = 2 * acc + m;
        if (j & 1) {
          mx = pk_maximum3_f16(mx, xs.p[i - 1], xs.p[i]);
          mn = pk_minimum3_f16(mn, xs.p[i - 1], xs.p[i]);
        }
      }
      obits[w] = acc;
      if (NWD > 1) xs.fence();
    }
  } else {
    // std + eps is not a positive finite number (cut NaN), or even |d| = 0
    // passes (cut -1): the reference's quotient per element
#pragma unroll
    for (int w = 0; w < NWD; w++) {
      uint32_t acc = 0;
#pragma unroll
      for (int j = 0; j < PW; j++) {
        const int i = w * PW + j;
        uint32_t m = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const f16 d = h_sub(xs[2 * i + h], st.mean16);
          if (outlier_literal(bits_to_h(h_to_bits(d) & 0x7FFFu), st.den16, thr)) m |= 1u << (16 * h);
        }
        xs.p[i] &= ~(m * 0xFFFFu);
        acc = 2 * acc + m;
        if (j & 1) {
          mx = pk_maximum3_f16(mx, xs.p[i - 1], xs.p[i]);
          mn = pk_minimum3_f16(mn, xs.p[i - 1], xs.p[i]);
        }
      }
      obits[w] = acc;
    }
  }
  int nout = 0;
#pragma unroll
  for (int w = 0; w < NWD; w++) {
    if (!tvalid) obits[w] = 0;  // padding threads hold zeros that may pass the test
    nout += __builtin_popcount(obits[w]);
  }
  // the absmax over non-outliers (NaN and, past a finite cut, infinities are
  // outliers, so the extremes are ordered values); -1 when the thread has
  // none; its team maximum travels with the outlier counts' prefix sum
  float amax = -1.0f;
  if (tvalid && nout < E) {
    const half2v hx = as_h2(mx), hn = as_h2(mn);
    amax = fmaxf(fmaxf((float)hx.x, (float)hx.y), -fminf((float)hn.x, (float)hn.y));
  }
  // outlier compaction: team prefix sum, then the block's staging slot in
  // element order (flag word w: pair PW w + j low / high at bit PW - 1 - j /
  // 16 + PW - 1 - j, so after a bit reversal L and H below hold them at bit j)
  int total;
  // the block's first use of lds_i, its counts in the first NWT words, the
  // absmax in the next NWT
  constexpr int NWT = TAU > 64 ? TAU / 64 : 1;
  const int pre = team_scan_max<TAU, true>(nout, &amax, lds_i, reinterpret_cast<float*>(lds_i + NWT), &total);
  if (gvalid) {
    int k = pre;
#pragma unroll
    for (int w = 0; w < NWD; w++) {
      const uint32_t rev = __builtin_bitreverse32(obits[w]);
      constexpr uint32_t kMask = PW == 32 ? 0xFFFFFFFFu : (1u << PW) - 1u;
      uint32_t L = (rev >> (32 - PW)) & kMask, H = (rev >> (16 - PW)) & kMask;
      while (L | H) {
        const int jl = L ? __builtin_ctz(L) : 32, jh = H ? __builtin_ctz(H) : 32;
        int e;
        if (jl <= jh) {
          e = 2 * (w * PW + jl);
          L &= L - 1;
        } else {
          e = 2 * (w * PW + jh) + 1;
          H &= H - 1;
        }
        // the value from the staged copy in LDS, else from memory (an L2
        // hit): indexing the registers with a run-time e would move them to
        // scratch
        const int64_t jj = base + i0 + e;
        a.stage_col[base + k] = i0 + e;
        a.stage_val[base + k] = staged ? staged[staged_index<E>(unit_e0 + e)] : (jj < a.numel ? a.x[jj] : (uint16_t)0);
        k++;
      }
    }
  }
  // the outlier stores go out before the code stores (see the end)
  asm volatile("" ::: "memory");

  xs.fence();

  const float qmax = a.fmt == AQ_FMT_INT8 ? 127.0f : 448.0f;
  f16 s16 = (f16)1.0f;
  if (amax >= 0.0f) {
    s16 = rn_h(amax / qmax);
    if ((float)s16 < 1e-6f) s16 = rn_h(1e-6f);
  }
  const float s = (float)s16;
  const float r = 1.0f / s;

  int64_t row = 0, col0 = 0;  // where the thread's elements sit in the [rows, K] matrix (tiled layout)
  if (a.tiled) {
    row = a.bpr == 1 ? g : g / a.bpr;
    col0 = (g - row * a.bpr) * G + i0;
  }
  // Where the thread's first 16 codes go; group v of 16 follows at v * 256
  // bytes in the tiled layout (E divides G, so col0 is a multiple of E and
  // the thread's columns col0 .. col0 + E - 1 lie in one 64-column half of a
  // tile, 16-byte piece v = ((col0 + 16 v) >> 4) & 3 of it), at v * 16 in
  // element order.
  uint8_t* const dst = a.codes + (a.tiled ? tiled_offset(row, col0, a.nchunks) : base + i0);
  const int vstep = a.tiled ? 256 : 16;
  auto store16 = [&](int v, const uint32_t (&w)[4]) {
    if (!(gvalid && tvalid)) return;
    if (xchg) {
      // the row's column piece i0 / 16 + v, beside the same piece of the
      // workgroup's other three rows
      xchg[xchg_slot((((i0 >> 4) + v) << 2) | (int)(g & 3))] = make_uint4(w[0], w[1], w[2], w[3]);
    } else if (a.vec) {
      *reinterpret_cast<uint4*>(dst + v * vstep) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      const int64_t j = base + i0 + 16 * v;
#pragma unroll
      for (int b = 0; b < 16; b++)
        a.codes[a.tiled ? tiled_offset(row, col0 + 16 * v + b, a.nchunks) : j + b] =
            (uint8_t)(w[b / 4] >> (8 * (b % 4)));
    }
  };
  // every wave of the workgroup is past its reads of the staged copy
  if (xchg) __syncthreads();
  // codes, 16 elements (8 pairs, four words) at a time; one loop per format
  if (a.fmt == AQ_FMT_INT8) {
#pragma unroll
    for (int v = 0; v < E / 16; v++) {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const f16 xe = xs[16 * v + 4 * k + b];
          float rr = __builtin_rintf((float)h_div_fast((float)xe, s, r));
          rr = fminf(fmaxf(rr, -127.0f), 127.0f);
          word |= (uint32_t)(uint8_t)(int8_t)(int)rr << (8 * b);
        }
        w[k] = word;
      }
      if (E > 16) xs.fence();
      store16(v, w);
    }
  } else {
#pragma unroll
    for (int v = 0; v < E / 16; v++) {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        // |x| <= amax and s = fp16(amax / 448) give |x / s| < 448.25, so the
        // quotient is at most 448.25, which the conversion (round to nearest
        // even) takes to 448 as the clamp to +-448 would
        typedef short short2v __attribute__((vector_size(4)));
        const uint32_t q0 = quot2(xs.p[8 * v + 2 * k], r);
        // both halves of c are written; its initial value is never seen
        short2v c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(__builtin_bit_cast(short2v, q0), as_h2(q0), 1.0f, false);
        c = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(c, as_h2(quot2(xs.p[8 * v + 2 * k + 1], r)), 1.0f, true);
        w[k] = __builtin_bit_cast(uint32_t, c);
      }
      if (E > 16) xs.fence();
      store16(v, w);
    }
  }

  if (xchg) {
    // the workgroup's four rows' codes out of LDS: lanes 4j .. 4j + 3 store
    // the four rows' 16-byte pieces of one column piece, 64 contiguous bytes
    // of the tiled layout
    __syncthreads();
    const int64_t row0 = g & ~(int64_t)3;
    const int rr = threadIdx.x & 3;
#pragma unroll
    for (int i = 0; i < E / 16; i++) {
      const int c = (threadIdx.x >> 2) + i * 64;
      *reinterpret_cast<uint4*>(a.codes + tiled_offset(row0 + rr, (int64_t)c << 4, a.nchunks)) =
          xchg[xchg_slot((c << 2) | rr)];
    }
  }
  // the block's scale and count (the same values in every lane of the team:
  // all lanes store them, no branch around the stores)
  if (gvalid) {
    a.scales[g] = h_to_bits(s16);
    a.block_cnt[g] = total;
  }
}

template <int TAU, int E, int MODE>
__global__ __launch_bounds__(TAU > kWG ? TAU : kWG) void quantize_kernel(QuantGroup q) {
  constexpr int NT = TAU > kWG ? TAU : kWG;
  const int64_t unit = q.xcd_rows ? xcd_unit(blockIdx.x, gridDim.x) : (int64_t)blockIdx.x;
  int mi = 0;  // the workgroup's member (uniform)
#pragma unroll
  for (int j = 1; j < kMaxQGroup; j++)
    if (j < q.count && unit >= q.first[j]) mi = j;
  const QuantArgs& a = q.m[mi];
  const int64_t bid = unit - q.first[mi];
  constexpr int TEAMS = NT / TAU;
  constexpr int NWT = TAU > 64 ? TAU / 64 : 1;
  __shared__ double lds_d[TEAMS * NWT];
  __shared__ float lds_f[TEAMS * NWT];
  __shared__ int lds_i[2 * TEAMS * NWT];  // per team: NWT counts, NWT maxima (finish_block_fast)

  const int team = threadIdx.x / TAU;
  const int t = threadIdx.x % TAU;
  const int64_t g = bid * TEAMS + team;
  const bool gvalid = g < a.nblocks;
  const int64_t G = a.G;
  const int64_t base = g * G;
  const int i0 = t * E;

  // Coalesced loads: a thread's E elements are consecutive, so if each
  // thread read its own, every load instruction would touch 64 different
  // 128-byte lines.  Instead the workgroup reads its blocks (TEAMS * G
  // consecutive elements) with consecutive lanes on consecutive 16-byte
  // pieces and hands them over through LDS (stage_swz).  Used when the
  // workgroup's blocks lie wholly inside x; the staged copy also serves the
  // outlier values to the compaction.
  constexpr int PPT = E / 8;  // 16-byte pieces per thread
  constexpr bool kStage = MODE != kAnyLen && NT * E * 2 <= 32768;
  __shared__ uint4 stage[kStage ? NT * PPT : 1];
  Elems<E> xs;
  bool staged = false;
  if constexpr (kStage) {
    const int64_t wg_base = bid * TEAMS * G;
    const int64_t wg_len = TEAMS * G;
    if (a.vec && (bid + 1) * TEAMS <= a.nblocks && wg_base + wg_len <= a.numel) {
      staged = true;
      const int npieces = (int)(wg_len >> 3);
      const uint4* src = reinterpret_cast<const uint4*>(a.x + wg_base);
#pragma unroll
      for (int k = 0; k < PPT; k++) {
        const int P = threadIdx.x + NT * k;
        if (MODE == kFullBlocks || P < npieces) stage[stage_swz<E>(P)] = src[P];
      }
      __syncthreads();
      const int S0 = (int)((team * G + i0) >> 3);
#pragma unroll
      for (int j = 0; j < PPT; j++) {
        // threads past the end of their block (E divides G < TAU * E) hold padding
        const uint4 u = (MODE == kFullBlocks || i0 < G) ? stage[stage_swz<E>(S0 + j)] : make_uint4(0, 0, 0, 0);
        xs.p[4 * j] = u.x;
        xs.p[4 * j + 1] = u.y;
        xs.p[4 * j + 2] = u.z;
        xs.p[4 * j + 3] = u.w;
      }
    }
  }
  if (!staged) load_elems<E>(xs, a, base, i0, gvalid);

  if constexpr (MODE == kAnyLen)
    finish_block_any<TAU, E, MODE>(a, xs, g, gvalid, base, i0, t, lds_d + team * NWT, lds_f + team * NWT,
                                   lds_i + 2 * team * NWT);
  else {
    // four one-row blocks of 4096 elements staged together, tiled codes:
    // the codes go out through the stage in 64-byte runs (a store
    // instruction of 16-byte pieces, one per lane, would otherwise touch 64
    // cache lines)
    uint4* xchg = nullptr;
    if constexpr (kStage && TAU == 64 && E == 64 && NT == 256)
      if (staged && a.tiled && a.bpr == 1) xchg = stage;
    finish_block_fast<TAU, E, MODE>(a, xs, g, gvalid, base, i0, t, lds_d + team * NWT, lds_f + team * NWT,
                                    lds_i + 2 * team * NWT, staged ? reinterpret_cast<const uint16_t*>(stage) : nullptr,
                                    (int)(team * G + i0), xchg);
  }
}

// ---- exclusive scan of the per-block counts (in place, two passes)

// PT consecutive counts per thread, 256 * PT per workgroup.  Runs of 4 keep
// a load instruction's lanes within 1 KiB; a Llama-3-8B weight quantized in
// blocks of 128 has 458 752 counts, which then take 448 workgroups (runs of
// 16: 112 workgroups, and 4.7 + 6.5 us for the two passes against 4.7 +
// 4.6).  Beyond 2048 chunks of 1024, runs of 16, so that each apply
// workgroup's sum over the partials before it stays short.
template <int PT>
__global__ __launch_bounds__(256) void scan_partials_kernel(const int32_t* cnt, int64_t n, int32_t* partial) {
  __shared__ int lds[4];
  const int64_t start = ((int64_t)blockIdx.x * 256 + threadIdx.x) * PT;
  int s = 0;
#pragma unroll
  for (int e = 0; e < PT; e++)
    if (start + e < n) s += cnt[start + e];
  int total;
  team_excl_scan_i32<256>(s, lds, &total);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

template <int PT>
__global__ __launch_bounds__(256) void scan_apply_kernel(int32_t* off, int64_t n, const int32_t* partial) {
  __shared__ int lds[4];
  __shared__ int lds_base[4];
  // sum of the partials of the chunks before this one
  int b = 0;
  for (int i = threadIdx.x; i < (int)blockIdx.x; i += 256) b += partial[i];
  int base_total;
  team_excl_scan_i32<256>(b, lds_base, &base_total);
  const int64_t start = ((int64_t)blockIdx.x * 256 + threadIdx.x) * PT;
  int v[PT];
  int s = 0;
#pragma unroll
  for (int e = 0; e < PT; e++) {
    v[e] = (start + e < n) ? off[start + e] : 0;
    s += v[e];
  }
  int total;
  int pre = team_excl_scan_i32<256>(s, lds, &total) + base_total;
#pragma unroll
  for (int e = 0; e < PT; e++) {
    if (start + e < n) off[start + e] = pre;
    pre += v[e];
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) off[n] = base_total + total;
}

// Up to kScanSmall counts (every per-channel weight of a model this size):
// one workgroup, one launch.  The counts go in rounds of 4096, each thread
// taking 4 consecutive ones with one 16-byte load, so every load and store
// instruction covers 1 KiB of contiguous memory (per-thread runs of 16 made
// the single workgroup's loads touch 64 lines each).
constexpr int kScanSmall = 1024 * 16;
// One workgroup per member of a quantize group (n[i] <= kScanSmall counts in off[i]).
struct ScanGroup {
  int32_t* off[kMaxQGroup];
  int64_t n[kMaxQGroup];
  int32_t* totals;  // [count] or null: member i's total also goes to totals[i]
};
__global__ __launch_bounds__(1024) void scan_small_kernel(ScanGroup sg) {
  int32_t* const off = sg.off[blockIdx.x];
  const int64_t n = sg.n[blockIdx.x];
  __shared__ int lds[16];
  int carry = 0;
  for (int64_t r0 = 0; r0 < n; r0 += 4096) {
    const int64_t i = r0 + 4 * (int64_t)threadIdx.x;
    int v[4];
    const bool whole = i + 4 <= n;
    if (whole) {
      const int4 u = *reinterpret_cast<const int4*>(off + i);
      v[0] = u.x;
      v[1] = u.y;
      v[2] = u.z;
      v[3] = u.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = i + e < n ? off[i + e] : 0;
    }
    int total;
    int pre = team_excl_scan_i32<1024>((v[0] + v[1]) + (v[2] + v[3]), lds, &total) + carry;
    int o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      o[e] = pre;
      pre += v[e];
    }
    if (whole) {
      *reinterpret_cast<int4*>(off + i) = make_int4(o[0], o[1], o[2], o[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (i + e < n) off[i + e] = o[e];
    }
    carry += total;
  }
  if (threadIdx.x == 0) {
    off[n] = carry;
    if (sg.totals) sg.totals[blockIdx.x] = carry;
  }
}

// ---- gather the staged outliers into the ascending list

template <int TPB>
__global__ __launch_bounds__(256) void gather_kernel(const int32_t* off, int64_t nblocks, int64_t G, int64_t K,
                                                     const int32_t* stage_col, const uint16_t* stage_val,
                                                     int64_t* flat_idx, uint16_t* vals, int32_t* cols) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t g = gid / TPB;
  const int lane = (int)(gid % TPB);
  if (g >= nblocks) return;
  const int32_t o = off[g];
  const int32_t n = off[g + 1] - o;
  const int64_t base = g * G;
  for (int j = lane; j < n; j += TPB) {
    const int64_t flat = base + stage_col[base + j];
    flat_idx[o + j] = flat;
    vals[o + j] = stage_val[base + j];
    if (cols) cols[o + j] = (int32_t)(flat % K);
  }
}

// ---- the flat list and the 16 x 64 block lists in one pass

// Entries of one tile row straight from the quantize workspace: block g's
// outliers are staged at stage_col / stage_val[g G .. g G + n_g - 1]
// (columns within the block, ascending), and its first entry's index is
// off[g].  In the counting pass each entry also goes to the flat list, as
// gather_kernel writes it.
struct WsTileSrc {
  int rs[17];            // the tile row's row starts, off[(16 rb + r) bpr]
  const int32_t* off;    // block offsets
  const int* loff;       // the tile row's 16 bpr + 1 block offsets in LDS, or null (read off)
  int64_t g0;            // the tile row's first block
  int bpr;               // blocks per row, K / G
  int64_t G;
  const int32_t* stage_col;
  const uint16_t* stage_val;
  int64_t* flat_idx;
  uint16_t* vals;
  int32_t* cols;
  __device__ __forceinline__ int block_start(int b) const { return loff ? loff[b] : off[g0 + b]; }
  __device__ __forceinline__ aq::TileEnt operator()(int i, bool first) const {
    int b, r, o;
    if (bpr == 1) {
      // the row and its start by a select chain (an index into rs would move
      // the array to scratch memory)
      r = 0;
      o = rs[0];
#pragma unroll
      for (int k = 1; k < 16; k++)
        if (i >= rs[k]) {
          r = k;
          o = rs[k];
        }
      b = r;
    } else {
      // the last block of the tile row starting at or before entry i (blocks
      // may be empty): block_start(0) <= i < block_start(16 bpr)
      int lo = 1, hi = 16 * bpr;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (block_start(mid) <= i)
          lo = mid + 1;
        else
          hi = mid;
      }
      b = lo - 1;
      r = b / bpr;
      o = block_start(b);
    }
    const int64_t g = g0 + b;
    const int64_t at = g * G + (i - o);
    const int sc = stage_col[at];
    const uint32_t v = stage_val[at];
    const int col = (b - r * bpr) * (int)G + sc;
    if (first) {
      flat_idx[i] = g * G + sc;
      vals[i] = (uint16_t)v;
      cols[i] = col;
    }
    return aq::TileEnt{r, col, v};
  }
};

// The weights of one aq_quantize_finish_tiles(_grouped) launch: they share
// the block size and the row length.  Member i takes workgroups first[i] ..
// first[i + 1] - 1: one per tile row, and a last one that writes the block
// lists' end and their 64 padding entries.
struct FinishMember {
  const int32_t* off;
  const int32_t* stage_col;
  const uint16_t* stage_val;
  int64_t* flat_idx;
  uint16_t* vals;
  int32_t* cols;
  int32_t* tile_ptr;
  uint32_t* tile_ent;
  int32_t* tile_max;
  int nrb;
};
struct FinishGroup {
  FinishMember m[kMaxQGroup];
  int first[kMaxQGroup + 1];
  int count;
  int bpr, nch, loff_lds;
  int64_t G;
};

// LDS: 33 * nch ints, and with loff_lds the tile row's block offsets after
// them.  NT threads per tile row: 128 for rows up to 128 chunks (a tile row of
// such weights holds a few hundred entries, and the small workgroups let a
// layer's tile rows all be resident at once), 256 for wider ones.
template <int NT>
__global__ __launch_bounds__(NT) void finish_tiles_kernel(FinishGroup fg) {
  extern __shared__ int sm[];
  __shared__ int part[NT / 64];
  int mi = 0;  // the workgroup's member (uniform)
#pragma unroll
  for (int j = 1; j < kMaxQGroup; j++)
    if (j < fg.count && (int)blockIdx.x >= fg.first[j]) mi = j;
  const FinishMember& m = fg.m[mi];
  const int bpr = fg.bpr, nch = fg.nch;
  const int rb = (int)blockIdx.x - fg.first[mi], t = threadIdx.x;
  if (rb == m.nrb) {
    const int end = m.off[(int64_t)m.nrb * 16 * bpr];
    if (t == 0) m.tile_ptr[(int64_t)m.nrb * nch] = end;
    if (t < 64) m.tile_ent[end + t] = 0u;
    return;
  }
  WsTileSrc src;
#pragma unroll
  for (int r = 0; r <= 16; r++) src.rs[r] = m.off[(int64_t)(rb * 16 + r) * bpr];
  src.off = m.off;
  src.loff = nullptr;
  src.g0 = (int64_t)rb * 16 * bpr;
  src.bpr = bpr;
  src.G = fg.G;
  src.stage_col = m.stage_col;
  src.stage_val = m.stage_val;
  src.flat_idx = m.flat_idx;
  src.vals = m.vals;
  src.cols = m.cols;
  if (fg.loff_lds) {
    int* l = sm + 33 * nch;
    for (int k = t; k <= 16 * bpr; k += NT) l[k] = m.off[src.g0 + k];
    __syncthreads();
    src.loff = l;
  }
  aq::tile_row_sort<NT>(src, rb, nch, src.rs[0], src.rs[16], sm, part, m.tile_ptr, m.tile_ent, m.tile_max);
}

// ---- calculate_zscore_manual of one block of n elements

template <int TAU, int E>
__global__ __launch_bounds__(TAU < 64 ? 64 : TAU) void zscore_kernel(const uint16_t* x, int64_t n, float eps,
                                                                      uint16_t* z, uint16_t* stats) {
  constexpr int NWT = TAU > 64 ? TAU / 64 : 1;
  __shared__ double lds_d[NWT];
  const int t = threadIdx.x;
  if (t >= TAU) return;  // only when TAU < 64: the rest of the single wave sits out (no barriers then)
  const int i0 = t * E;
  Elems<E> xs;
#pragma unroll
  for (int e = 0; e < E; e += 2)
    xs.p[e / 2] = (uint32_t)(i0 + e < n ? x[i0 + e] : (uint16_t)0) |
                  ((uint32_t)(i0 + e + 1 < n ? x[i0 + e + 1] : (uint16_t)0) << 16);
  const BlockStats st = block_stats<TAU, E>(xs, i0, n, eps, lds_d);
#pragma unroll
  for (int e = 0; e < E; e++)
    if (i0 + e < n) z[i0 + e] = h_to_bits(h_div(h_sub(xs[e], st.mean16), st.den16));
  if (stats && t == 0) {
    stats[0] = h_to_bits(st.mean16);
    stats[1] = h_to_bits(st.std16);
    stats[2] = h_to_bits(st.den16);
  }
}

int64_t next_pow2(int64_t g) {
  int64_t p = 1;
  while (p < g) p <<= 1;
  return p;
}

template <int TAU, int E>
hipError_t launch_quantize_t(QuantGroup q, hipStream_t stream) {
  constexpr int NT = TAU > kWG ? TAU : kWG;
  constexpr int TEAMS = NT / TAU;
  q.first[0] = 0;
  for (int i = 0; i < q.count; i++) q.first[i + 1] = q.first[i] + aq::ceil_div(q.m[i].nblocks, TEAMS);
  for (int i = q.count + 1; i <= kMaxQGroup; i++) q.first[i] = q.first[q.count];
  const int64_t grid = q.first[q.count];
  const int64_t G = q.m[0].G;  // one block size for the group
  // tiled codes from workgroups of fewer than 4 rows: XCD-contiguous units
  // (down_proj's one-row workgroups 73 -> 61 us; with four rows, whose
  // codes leave in 64-byte runs, it measured neutral to 1 % slower)
  q.xcd_rows = 1;
  for (int i = 0; i < q.count; i++) q.xcd_rows = q.xcd_rows && q.m[i].tiled && TEAMS * G < 4 * q.m[i].K;
  if (G == (int64_t)TAU * E)
    hipLaunchKernelGGL((quantize_kernel<TAU, E, kFullBlocks>), dim3((unsigned)grid), dim3(NT), 0, stream, q);
  else if (G % E == 0)
    hipLaunchKernelGGL((quantize_kernel<TAU, E, kThreadAligned>), dim3((unsigned)grid), dim3(NT), 0, stream, q);
  else
    hipLaunchKernelGGL((quantize_kernel<TAU, E, kAnyLen>), dim3((unsigned)grid), dim3(NT), 0, stream, q);
  return hipGetLastError();
}

// Team shape per padded block size P: up to 32 elements, 16 per thread;
// 64 to 2048, 32 per thread (teams of at most one wave, several per
// workgroup: a lane's fixed work per block over twice the elements of 16
// per thread, measured 11 to 25 % faster for 64 to 1024 on a 4096 x 14336
// weight); 2048 on one wave; from 4096 on, 64 per thread (one wave for 4096, a block of
// 4096 elements then needs no barrier at all), except 16384: 32 per thread
// on 8 waves ran 4 % faster than 64 on 4 for rows of 14336 such as
// down_proj's (which now take 7 waves, below), while 32 per thread at 4096
// ran 15 % slower (measured).
hipError_t launch_quantize(const QuantGroup& q, hipStream_t stream) {
  // Rows of exactly 14336 (Llama-3 / Mistral down_proj): a team of 448
  // threads (7 waves) instead of 512, whose eighth wave would hold only
  // padding; the team sums pad the eighth wave's partial with +0, the same
  // tree.  Four such workgroups fit a CU against three of 8 waves.
  if (q.m[0].G == 448 * 32) return launch_quantize_t<448, 32>(q, stream);
  const int64_t P = next_pow2(q.m[0].G);
  switch (P) {
    case 1: case 2: case 4: case 8: case 16: return launch_quantize_t<1, 16>(q, stream);
    case 32: return launch_quantize_t<2, 16>(q, stream);
    case 64: return launch_quantize_t<2, 32>(q, stream);
    case 128: return launch_quantize_t<4, 32>(q, stream);
    case 256: return launch_quantize_t<8, 32>(q, stream);
    case 512: return launch_quantize_t<16, 32>(q, stream);
    case 1024: return launch_quantize_t<32, 32>(q, stream);
    case 2048: return launch_quantize_t<64, 32>(q, stream);
    case 4096: return launch_quantize_t<64, 64>(q, stream);
    case 8192: return launch_quantize_t<128, 64>(q, stream);
    case 16384: return launch_quantize_t<512, 32>(q, stream);
    case 32768: return launch_quantize_t<512, 64>(q, stream);
    default: return launch_quantize_t<1024, 64>(q, stream);
  }
}

template <int TAU, int E>
hipError_t launch_zscore_t(const uint16_t* x, int64_t n, float eps, uint16_t* z, uint16_t* stats, hipStream_t s) {
  constexpr int NT = TAU < 64 ? 64 : TAU;
  hipLaunchKernelGGL((zscore_kernel<TAU, E>), dim3(1), dim3(NT), 0, s, x, n, eps, z, stats);
  return hipGetLastError();
}

struct Workspace {
  int32_t* stage_col;
  uint16_t* stage_val;
  int32_t* partial;
};

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

Workspace carve(void* ws, int64_t padded, int64_t nblocks) {
  char* p = (char*)ws;
  Workspace w;
  w.stage_col = (int32_t*)p;
  p += align256(padded * 4);
  w.stage_val = (uint16_t*)p;
  p += align256(padded * 2);
  w.partial = (int32_t*)p;
  (void)nblocks;
  return w;
}

int64_t workspace_bytes(int64_t padded, int64_t nblocks) {
  return align256(padded * 4) + align256(padded * 2) + align256((aq::ceil_div(nblocks, kScanChunk) + 1) * 4);
}

}  // namespace

extern "C" int64_t aq_max_block_size(void) { return kMaxG; }

extern "C" int64_t aq_quantize_workspace_size(int64_t numel, int64_t G) {
  if (numel <= 0 || G <= 0) return 0;
  const int64_t nblocks = aq::ceil_div(numel, G);
  return workspace_bytes(nblocks * G, nblocks);
}

// Checks one weight's arguments and fills its QuantArgs (aq_quantize,
// aq_quantize_grouped).
static int quantize_args(const void* x, int64_t numel, int64_t G, uint16_t z_thr_f16, int fmt, int64_t K, int layout,
                         void* codes, void* scales, int32_t* block_off, void* workspace, int64_t ws_bytes,
                         QuantArgs* out, Workspace* wout) {
  AQ_CHECK_ARG(numel > 0, "aq_quantize: numel must be > 0 (got %lld)", (long long)numel);
  AQ_CHECK_ARG(G >= 1 && G <= kMaxG, "aq_quantize: block size %lld outside [1, %lld]", (long long)G,
               (long long)kMaxG);
  AQ_CHECK_ARG(fmt == AQ_FMT_INT8 || fmt == AQ_FMT_E4M3, "aq_quantize: unknown code format %d", fmt);
  AQ_CHECK_ARG(x && codes && scales && block_off && workspace, "aq_quantize: null pointer argument");
  AQ_CHECK_ARG(layout == AQ_LAYOUT_FLAT || layout == AQ_LAYOUT_TILED, "aq_quantize: unknown layout %d", layout);
  if (layout == AQ_LAYOUT_TILED)
    AQ_CHECK_ARG(K >= 128 && K % 128 == 0 && numel % (16 * K) == 0 && G % 16 == 0 && K % G == 0,
                 "aq_quantize: the tiled layout needs K %% 128 == 0, rows %% 16 == 0 and a block dividing K "
                 "(K=%lld, numel=%lld, G=%lld)",
                 (long long)K, (long long)numel, (long long)G);
  const int64_t nblocks = aq::ceil_div(numel, G);
  const int64_t padded = nblocks * G;
  if (padded >= (int64_t)1 << 31)
    return aq::set_error(AQ_EUNSUPPORTED, "aq_quantize: %lld elements exceed the 2^31 limit", (long long)padded);
  if (ws_bytes < workspace_bytes(padded, nblocks))
    return aq::set_error(AQ_EWORKSPACE, "aq_quantize: workspace of %lld bytes, %lld needed", (long long)ws_bytes,
                         (long long)workspace_bytes(padded, nblocks));
  const Workspace w = carve(workspace, padded, nblocks);
  QuantArgs a;
  a.x = (const uint16_t*)x;
  a.numel = numel;
  a.G = G;
  a.nblocks = nblocks;
  a.thr_bits = z_thr_f16;
  a.fmt = fmt;
  a.vec = (G % 16 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)codes % 16 == 0);
  a.tiled = layout == AQ_LAYOUT_TILED;
  a.K = K;
  a.nchunks = K / 128;
  a.bpr = a.tiled ? K / G : 1;
  a.inv_g = 1.0 / (double)G;
  a.inv_g1 = G >= 2 ? (float)(1.0 / (double)(G - 1)) : 0.0f;
  a.codes = (uint8_t*)codes;
  a.scales = (uint16_t*)scales;
  a.block_cnt = block_off;
  a.stage_col = w.stage_col;
  a.stage_val = w.stage_val;
  *out = a;
  *wout = w;
  return AQ_OK;
}

extern "C" int aq_quantize(const void* x, int64_t numel, int64_t G, uint16_t z_thr_f16, int fmt, int64_t K,
                           int layout, void* codes, void* scales, int32_t* block_off, void* workspace, int64_t ws_bytes,
                           void* stream) {
  QuantGroup q{};
  Workspace w;
  const int rc =
      quantize_args(x, numel, G, z_thr_f16, fmt, K, layout, codes, scales, block_off, workspace, ws_bytes, &q.m[0], &w);
  if (rc != AQ_OK) return rc;
  q.count = 1;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nblocks = q.m[0].nblocks;
  hipError_t e = launch_quantize(q, s);
  if (e != hipSuccess) return aq::check_hip(e, "aq_quantize: quantize kernel launch");
  if (nblocks <= kScanSmall) {
    ScanGroup sg{};
    sg.off[0] = block_off;
    sg.n[0] = nblocks;
    hipLaunchKernelGGL(scan_small_kernel, dim3(1), dim3(1024), 0, s, sg);
    AQ_LAUNCH_CHECK("aq_quantize: scan launch");
    return AQ_OK;
  }
  // w.partial holds ceil(nblocks / kScanChunk) + 1 entries, enough for either run length
  if (aq::ceil_div(nblocks, kScanChunk) <= 2048) {
    const int64_t nparts = aq::ceil_div(nblocks, 256 * 4);
    hipLaunchKernelGGL(scan_partials_kernel<4>, dim3((unsigned)nparts), dim3(256), 0, s, block_off, nblocks, w.partial);
    AQ_LAUNCH_CHECK("aq_quantize: scan launch");
    hipLaunchKernelGGL(scan_apply_kernel<4>, dim3((unsigned)nparts), dim3(256), 0, s, block_off, nblocks, w.partial);
  } else {
    const int64_t nparts = aq::ceil_div(nblocks, 256 * 16);
    hipLaunchKernelGGL(scan_partials_kernel<16>, dim3((unsigned)nparts), dim3(256), 0, s, block_off, nblocks, w.partial);
    AQ_LAUNCH_CHECK("aq_quantize: scan launch");
    hipLaunchKernelGGL(scan_apply_kernel<16>, dim3((unsigned)nparts), dim3(256), 0, s, block_off, nblocks, w.partial);
  }
  AQ_LAUNCH_CHECK("aq_quantize: scan launch");
  return AQ_OK;
}

extern "C" int aq_quantize_grouped(int64_t count, const void* const* xs, const int64_t* numels, int64_t G,
                                   uint16_t z_thr_f16, int fmt, int64_t K, int layout, void* const* codes,
                                   void* const* scales, int32_t* const* block_offs, void* const* workspaces,
                                   const int64_t* ws_bytes, int32_t* totals, void* stream) {
  AQ_CHECK_ARG(count >= 1 && count <= kMaxQGroup, "aq_quantize_grouped: 1..%d weights, got %lld", kMaxQGroup,
               (long long)count);
  AQ_CHECK_ARG(xs && numels && codes && scales && block_offs && workspaces && ws_bytes,
               "aq_quantize_grouped: null pointer argument");
  QuantGroup q{};
  ScanGroup sg{};
  for (int i = 0; i < (int)count; i++) {
    Workspace w;
    const int rc = quantize_args(xs[i], numels[i], G, z_thr_f16, fmt, K, layout, codes[i], scales[i], block_offs[i],
                                 workspaces[i], ws_bytes[i], &q.m[i], &w);
    if (rc != AQ_OK) return rc;
    AQ_CHECK_ARG(q.m[i].nblocks <= kScanSmall,
                 "aq_quantize_grouped: weight %d has %lld blocks, more than %d (quantize it alone)", i,
                 (long long)q.m[i].nblocks, kScanSmall);
    sg.off[i] = block_offs[i];
    sg.n[i] = q.m[i].nblocks;
  }
  q.count = (int)count;
  sg.totals = totals;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = launch_quantize(q, s);
  if (e != hipSuccess) return aq::check_hip(e, "aq_quantize_grouped: quantize kernel launch");
  hipLaunchKernelGGL(scan_small_kernel, dim3((unsigned)count), dim3(1024), 0, s, sg);
  AQ_LAUNCH_CHECK("aq_quantize_grouped: scan launch");
  return AQ_OK;
}

extern "C" int aq_quantize_finish(int64_t numel, int64_t G, int64_t K, const int32_t* block_off, int64_t nnz,
                                  const void* workspace, int64_t ws_bytes, int64_t* flat_idx, void* vals,
                                  int32_t* cols, void* stream) {
  AQ_CHECK_ARG(numel > 0 && G >= 1 && G <= kMaxG, "aq_quantize_finish: bad numel/G");
  AQ_CHECK_ARG(K >= 1, "aq_quantize_finish: K must be >= 1");
  const int64_t nblocks = aq::ceil_div(numel, G);
  const int64_t padded = nblocks * G;
  if (ws_bytes < workspace_bytes(padded, nblocks))
    return aq::set_error(AQ_EWORKSPACE, "aq_quantize_finish: workspace too small");
  if (nnz == 0) return AQ_OK;
  AQ_CHECK_ARG(flat_idx && vals && block_off, "aq_quantize_finish: null pointer argument");
  Workspace w = carve((void*)workspace, padded, nblocks);
  hipStream_t s = (hipStream_t)stream;
  if (G >= 256) {
    const int64_t grid = aq::ceil_div(nblocks * 64, 256);
    hipLaunchKernelGGL((gather_kernel<64>), dim3((unsigned)grid), dim3(256), 0, s, block_off, nblocks, G, K,
                       w.stage_col, w.stage_val, flat_idx, (uint16_t*)vals, cols);
  } else {
    const int64_t grid = aq::ceil_div(nblocks, 256);
    hipLaunchKernelGGL((gather_kernel<1>), dim3((unsigned)grid), dim3(256), 0, s, block_off, nblocks, G, K,
                       w.stage_col, w.stage_val, flat_idx, (uint16_t*)vals, cols);
  }
  AQ_LAUNCH_CHECK("aq_quantize_finish: gather launch");
  return AQ_OK;
}

// Checks one member of aq_quantize_finish_tiles(_grouped) and fills its
// FinishMember (fg->G, bpr, nch set by the caller).
static int finish_tiles_member(const char* fn, int64_t numel, int64_t G, int64_t K, const int32_t* block_off,
                               int64_t nnz, const void* workspace, int64_t ws_bytes, int64_t* flat_idx, void* vals,
                               int32_t* cols, int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max,
                               FinishMember* out) {
  AQ_CHECK_ARG(numel > 0 && G >= 1 && G <= kMaxG, "%s: bad numel/G", fn);
  AQ_CHECK_ARG(K >= 64 && K % 64 == 0 && K % G == 0 && numel % (16 * K) == 0 && K < (1 << 30) &&
                   (numel / K / 16) * (K / 64) < ((int64_t)1 << 31),
               "%s: needs K %% 64 == 0, a block dividing K and rows %% 16 == 0 (numel=%lld K=%lld G=%lld)", fn,
               (long long)numel, (long long)K, (long long)G);
  const int64_t nblocks = numel / G;
  if (ws_bytes < workspace_bytes(numel, nblocks))
    return aq::set_error(AQ_EWORKSPACE, "%s: workspace too small", fn);
  AQ_CHECK_ARG(block_off && workspace && tile_ptr && tile_ent && (nnz == 0 || (flat_idx && vals && cols)),
               "%s: null pointer argument", fn);
  const Workspace w = carve((void*)workspace, numel, nblocks);
  FinishMember m;
  m.off = block_off;
  m.stage_col = w.stage_col;
  m.stage_val = w.stage_val;
  m.flat_idx = flat_idx;
  m.vals = (uint16_t*)vals;
  m.cols = cols;
  m.tile_ptr = tile_ptr;
  m.tile_ent = tile_ent;
  m.tile_max = tile_max;
  m.nrb = (int)(numel / K / 16);
  *out = m;
  return AQ_OK;
}

// One launch for the group's members (all of one block size G and row length K).
static int launch_finish_tiles(FinishGroup& fg, int64_t G, int64_t K, const char* fn, hipStream_t s) {
  const int64_t nch = K / 64, bpr = K / G;
  fg.G = G;
  fg.bpr = (int)bpr;
  fg.nch = (int)nch;
  fg.first[0] = 0;
  for (int i = 0; i < fg.count; i++) fg.first[i + 1] = fg.first[i] + fg.m[i].nrb + 1;
  for (int i = fg.count + 1; i <= kMaxQGroup; i++) fg.first[i] = fg.first[fg.count];
  // the tile row's block offsets go to LDS when the sort leaves room (64 KiB in all)
  const int64_t sort_ints = 33 * nch;
  fg.loff_lds = bpr > 1 && sort_ints + 16 * bpr + 1 <= 16384;
  const size_t lds = (size_t)(sort_ints + (fg.loff_lds ? 16 * bpr + 1 : 0)) * sizeof(int);
  if (nch <= 128)
    hipLaunchKernelGGL(finish_tiles_kernel<128>, dim3((unsigned)fg.first[fg.count]), dim3(128), lds, s, fg);
  else
    hipLaunchKernelGGL(finish_tiles_kernel<256>, dim3((unsigned)fg.first[fg.count]), dim3(256), lds, s, fg);
  AQ_LAUNCH_CHECK(fn);
  return AQ_OK;
}

// Rows too wide for one workgroup's LDS: the flat list, then the block lists
// from it (one thread per block), the block offsets serving as the CSR row
// pointer at a stride of K / G.
static int finish_tiles_wide(int64_t numel, int64_t G, int64_t K, const int32_t* block_off, int64_t nnz,
                             const void* workspace, int64_t ws_bytes, int64_t* flat_idx, void* vals, int32_t* cols,
                             int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max, const char* fn,
                             hipStream_t s) {
  const int rc = aq_quantize_finish(numel, G, K, block_off, nnz, workspace, ws_bytes, flat_idx, vals, cols, s);
  if (rc != AQ_OK) return rc;
  const hipError_t e = aq::launch_outlier_tiles(block_off, K / G, cols, (const uint16_t*)vals, numel / K, K,
                                                tile_ptr, tile_ent, tile_max, s);
  if (e != hipSuccess) return aq::check_hip(e, fn);
  return AQ_OK;
}

extern "C" int aq_quantize_finish_tiles(int64_t numel, int64_t G, int64_t K, const int32_t* block_off, int64_t nnz,
                                        const void* workspace, int64_t ws_bytes, int64_t* flat_idx, void* vals,
                                        int32_t* cols, int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max,
                                        void* stream) {
  static const char* fn = "aq_quantize_finish_tiles";
  FinishGroup fg{};
  int rc = finish_tiles_member(fn, numel, G, K, block_off, nnz, workspace, ws_bytes, flat_idx, vals, cols, tile_ptr,
                               tile_ent, tile_max, &fg.m[0]);
  if (rc != AQ_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  if (K / 64 > aq::kTileRowsMaxChunks)
    return finish_tiles_wide(numel, G, K, block_off, nnz, workspace, ws_bytes, flat_idx, vals, cols, tile_ptr,
                             tile_ent, tile_max, fn, s);
  fg.count = 1;
  return launch_finish_tiles(fg, G, K, fn, s);
}

extern "C" int aq_quantize_finish_tiles_grouped(int64_t count, const int64_t* numels, int64_t G, int64_t K,
                                                const int32_t* const* block_offs, const int64_t* nnzs,
                                                const void* const* workspaces, const int64_t* ws_bytes,
                                                int64_t* const* flat_idx, void* const* vals, int32_t* const* cols,
                                                int32_t* const* tile_ptrs, uint32_t* const* tile_ents,
                                                int32_t* tile_max, void* stream) {
  static const char* fn = "aq_quantize_finish_tiles_grouped";
  AQ_CHECK_ARG(count >= 1 && count <= kMaxQGroup, "%s: 1..%d weights, got %lld", fn, kMaxQGroup, (long long)count);
  AQ_CHECK_ARG(numels && block_offs && nnzs && workspaces && ws_bytes && flat_idx && vals && cols && tile_ptrs &&
                   tile_ents,
               "%s: null pointer argument", fn);
  FinishGroup fg{};
  for (int i = 0; i < (int)count; i++) {
    const int rc = finish_tiles_member(fn, numels[i], G, K, block_offs[i], nnzs[i], workspaces[i], ws_bytes[i],
                                       flat_idx[i], vals[i], cols[i], tile_ptrs[i], tile_ents[i],
                                       tile_max ? tile_max + i : nullptr, &fg.m[i]);
    if (rc != AQ_OK) return rc;
  }
  hipStream_t s = (hipStream_t)stream;
  if (K / 64 > aq::kTileRowsMaxChunks) {
    for (int i = 0; i < (int)count; i++) {
      const int rc = finish_tiles_wide(numels[i], G, K, block_offs[i], nnzs[i], workspaces[i], ws_bytes[i],
                                       flat_idx[i], vals[i], cols[i], tile_ptrs[i], tile_ents[i],
                                       tile_max ? tile_max + i : nullptr, fn, s);
      if (rc != AQ_OK) return rc;
    }
    return AQ_OK;
  }
  fg.count = (int)count;
  return launch_finish_tiles(fg, G, K, fn, s);
}

extern "C" int aq_zscore(const void* x, int64_t n, float eps, void* z, void* stats, void* stream) {
  AQ_CHECK_ARG(n >= 1 && n <= kMaxG, "aq_zscore: n = %lld outside [1, %lld]", (long long)n, (long long)kMaxG);
  AQ_CHECK_ARG(x && z, "aq_zscore: null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  uint16_t* zp = (uint16_t*)z;
  uint16_t* sp = (uint16_t*)stats;
  const int64_t P = next_pow2(n);
  hipError_t e;
  if (P <= 16384) {
    const int64_t tau = P <= 16 ? 1 : P / 16;
    switch (tau) {
      case 1: e = launch_zscore_t<1, 16>(xp, n, eps, zp, sp, s); break;
      case 2: e = launch_zscore_t<2, 16>(xp, n, eps, zp, sp, s); break;
      case 4: e = launch_zscore_t<4, 16>(xp, n, eps, zp, sp, s); break;
      case 8: e = launch_zscore_t<8, 16>(xp, n, eps, zp, sp, s); break;
      case 16: e = launch_zscore_t<16, 16>(xp, n, eps, zp, sp, s); break;
      case 32: e = launch_zscore_t<32, 16>(xp, n, eps, zp, sp, s); break;
      case 64: e = launch_zscore_t<64, 16>(xp, n, eps, zp, sp, s); break;
      case 128: e = launch_zscore_t<128, 16>(xp, n, eps, zp, sp, s); break;
      case 256: e = launch_zscore_t<256, 16>(xp, n, eps, zp, sp, s); break;
      case 512: e = launch_zscore_t<512, 16>(xp, n, eps, zp, sp, s); break;
      default: e = launch_zscore_t<1024, 16>(xp, n, eps, zp, sp, s); break;
    }
  } else if (P <= 32768) {
    e = launch_zscore_t<512, 64>(xp, n, eps, zp, sp, s);
  } else {
    e = launch_zscore_t<1024, 64>(xp, n, eps, zp, sp, s);
  }
  return aq::check_hip(e, "aq_zscore: launch");
}
