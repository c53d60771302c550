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

namespace {

constexpr int kWG = 256;            // threads per workgroup for TAU <= 256
constexpr int kScanChunk = 4096;    // block counts per scan workgroup (256 x 16)
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
  uint8_t* codes;
  uint16_t* scales;
  int32_t* block_cnt;  // block_off, holds counts until the scan
  int32_t* stage_col;
  uint16_t* stage_val;
};

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

template <int TAU, int E, int MODE>
__global__ __launch_bounds__(TAU > kWG ? TAU : kWG) void quantize_kernel(QuantArgs a) {
  constexpr int NT = TAU > kWG ? TAU : kWG;
  constexpr int TEAMS = NT / TAU;
  constexpr int NWT = TAU > 64 ? TAU / 64 : 1;
  __shared__ double lds_d[TEAMS * NWT];
  __shared__ float lds_f[TEAMS * NWT];
  __shared__ int lds_i[TEAMS * NWT];

  const int team = threadIdx.x / TAU;
  const int t = threadIdx.x % TAU;
  const int64_t g = (int64_t)blockIdx.x * TEAMS + team;
  const bool gvalid = g < a.nblocks;
  const int64_t G = a.G;
  const int64_t base = g * G;
  const int i0 = t * E;

  Elems<E> xs;
  load_elems<E>(xs, a, base, i0, gvalid);

  const BlockStats st = block_stats<TAU, E, MODE>(xs, i0, G, 1e-6f, lds_d + team * NWT);
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
  amax = team_max_f32<TAU>(amax, lds_f + team * NWT);
  xs.fence();

  const float qmax = a.fmt == AQ_FMT_INT8 ? 127.0f : 448.0f;
  f16 s16 = (f16)1.0f;
  if (amax >= 0.0f) {
    s16 = rn_h(amax / qmax);
    if ((float)s16 < 1e-6f) s16 = rn_h(1e-6f);
  }
  const float s = (float)s16;
  const float r = 1.0f / s;

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
        const int64_t off = a.tiled ? tiled_offset(j / a.K, j % a.K, a.nchunks) : j;
        *reinterpret_cast<uint4*>(a.codes + off) = make_uint4(w[0], w[1], w[2], w[3]);
      } else {
#pragma unroll
        for (int b = 0; b < 16; b++)
          if (i0 + 16 * v + b < G)
            a.codes[a.tiled ? tiled_offset((j + b) / a.K, (j + b) % a.K, a.nchunks) : j + b] =
                (uint8_t)(w[b / 4] >> (8 * (b % 4)));
      }
    }
  }

  // outlier compaction: team prefix sum, then the block's staging slot
  const int cnt = __builtin_popcountll(omask);
  int total;
  const int pre = team_excl_scan_i32<TAU>(cnt, lds_i + team * NWT, &total);
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

// ---- exclusive scan of the per-block counts (in place, two passes)

__global__ __launch_bounds__(256) void scan_partials_kernel(const int32_t* cnt, int64_t n, int32_t* partial) {
  __shared__ int lds[4];
  const int64_t start = (int64_t)blockIdx.x * kScanChunk + threadIdx.x * 16;
  int s = 0;
#pragma unroll
  for (int e = 0; e < 16; e++)
    if (start + e < n) s += cnt[start + e];
  int total;
  team_excl_scan_i32<256>(s, lds, &total);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

__global__ __launch_bounds__(256) void scan_apply_kernel(int32_t* off, int64_t n, const int32_t* partial) {
  __shared__ int lds[4];
  __shared__ int lds_base[4];
  // sum of the partials of the chunks before this one
  int b = 0;
  for (int i = threadIdx.x; i < (int)blockIdx.x; i += 256) b += partial[i];
  int base_total;
  team_excl_scan_i32<256>(b, lds_base, &base_total);
  const int64_t start = (int64_t)blockIdx.x * kScanChunk + threadIdx.x * 16;
  int v[16];
  int s = 0;
#pragma unroll
  for (int e = 0; e < 16; e++) {
    v[e] = (start + e < n) ? off[start + e] : 0;
    s += v[e];
  }
  int total;
  int pre = team_excl_scan_i32<256>(s, lds, &total) + base_total;
#pragma unroll
  for (int e = 0; e < 16; e++) {
    if (start + e < n) off[start + e] = pre;
    pre += v[e];
  }
  if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) off[n] = base_total + total;
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
hipError_t launch_quantize_t(const QuantArgs& a, hipStream_t stream) {
  constexpr int NT = TAU > kWG ? TAU : kWG;
  constexpr int TEAMS = NT / TAU;
  const int64_t grid = aq::ceil_div(a.nblocks, TEAMS);
  if (a.G == (int64_t)TAU * E)
    hipLaunchKernelGGL((quantize_kernel<TAU, E, kFullBlocks>), dim3((unsigned)grid), dim3(NT), 0, stream, a);
  else if (a.G % E == 0)
    hipLaunchKernelGGL((quantize_kernel<TAU, E, kThreadAligned>), dim3((unsigned)grid), dim3(NT), 0, stream, a);
  else
    hipLaunchKernelGGL((quantize_kernel<TAU, E, kAnyLen>), dim3((unsigned)grid), dim3(NT), 0, stream, a);
  return hipGetLastError();
}

// Team shape per padded block size P: up to 1024 elements, 16 per thread
// (teams of at most one wave, several per workgroup); 2048, 32 per thread on
// one wave; from 4096 on, 64 per thread (one wave for 4096, a block of
// 4096 elements then needs no barrier at all).
hipError_t launch_quantize(const QuantArgs& a, hipStream_t stream) {
  const int64_t P = next_pow2(a.G);
  switch (P) {
    case 1: case 2: case 4: case 8: case 16: return launch_quantize_t<1, 16>(a, stream);
    case 32: return launch_quantize_t<2, 16>(a, stream);
    case 64: return launch_quantize_t<4, 16>(a, stream);
    case 128: return launch_quantize_t<8, 16>(a, stream);
    case 256: return launch_quantize_t<16, 16>(a, stream);
    case 512: return launch_quantize_t<32, 16>(a, stream);
    case 1024: return launch_quantize_t<64, 16>(a, stream);
    case 2048: return launch_quantize_t<64, 32>(a, stream);
    case 4096: return launch_quantize_t<64, 64>(a, stream);
    case 8192: return launch_quantize_t<128, 64>(a, stream);
    case 16384: return launch_quantize_t<256, 64>(a, stream);
    case 32768: return launch_quantize_t<512, 64>(a, stream);
    default: return launch_quantize_t<1024, 64>(a, stream);
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

extern "C" int aq_quantize(const void* x, int64_t numel, int64_t G, uint16_t z_thr_f16, int fmt, int64_t K,
                           int layout, void* codes, void* scales, int32_t* block_off, void* workspace, int64_t ws_bytes,
                           void* stream) {
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
  hipStream_t s = (hipStream_t)stream;
  Workspace w = carve(workspace, padded, nblocks);
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
  a.codes = (uint8_t*)codes;
  a.scales = (uint16_t*)scales;
  a.block_cnt = block_off;
  a.stage_col = w.stage_col;
  a.stage_val = w.stage_val;
  hipError_t e = launch_quantize(a, s);
  if (e != hipSuccess) return aq::check_hip(e, "aq_quantize: quantize kernel launch");
  const int64_t nparts = aq::ceil_div(nblocks, kScanChunk);
  hipLaunchKernelGGL(scan_partials_kernel, dim3((unsigned)nparts), dim3(256), 0, s, block_off, nblocks, w.partial);
  AQ_LAUNCH_CHECK("aq_quantize: scan launch");
  hipLaunchKernelGGL(scan_apply_kernel, dim3((unsigned)nparts), dim3(256), 0, s, block_off, nblocks, w.partial);
  AQ_LAUNCH_CHECK("aq_quantize: scan launch");
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
