// aq_common.h -- shared helpers of the gfx950 kernels: fp16/e4m3 arithmetic
// with explicit rounding, the deterministic team reductions, and the error
// reporting of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/atlasinfer_amd.h"

typedef _Float16 f16;
typedef uint16_t f16bits;

// ------------------------------------------------------------ error handling
namespace aq {

int set_error(int code, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);

#define AQ_CHECK_ARG(cond, ...)                              \
  do {                                                       \
    if (!(cond)) return ::aq::set_error(AQ_EINVAL, __VA_ARGS__); \
  } while (0)

#define AQ_LAUNCH_CHECK(what)                                         \
  do {                                                                \
    hipError_t _e = hipGetLastError();                                \
    if (_e != hipSuccess) return ::aq::check_hip(_e, what);           \
  } while (0)

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device, queried once per device (any host
// thread; the cache is atomic).
inline int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int v = 0;
    n = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0 ? v : 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace aq

// ------------------------------------------------------------ memory helpers

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load marked non-temporal (streamed once: do not keep in cache).
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ------------------------------------------------------------ tiled codes
// Code layout read by the quantized-linear kernels: W[N, K] (N % 16 == 0,
// K % 128 == 0) is cut into tiles of 16 rows x 128 columns, 2 KiB each,
// stored tile-row by tile-row.  Inside a tile, byte h*1024 + (g*16 + r)*16 + e
// holds column 64*h + 16*g + e of tile row r: a wave that loads 16 bytes per
// lane at tile + lane*16 (and + 1024) receives, in lane g*16 + r, exactly the
// 16x16x32 MFMA B-operand pieces of row r, and each load instruction reads
// 1 KiB of contiguous memory.
__host__ __device__ __forceinline__ int64_t tiled_offset(int64_t n, int64_t k, int64_t nchunks) {
  return ((((n >> 4) * nchunks + (k >> 7)) << 11) | (((k >> 6) & 1) << 10) | (((k >> 4) & 3) << 8) |
          ((n & 15) << 4) | (k & 15));
}

// ------------------------------------------------------------- fp16 helpers

__device__ __forceinline__ f16 bits_to_h(uint16_t b) { return __builtin_bit_cast(f16, b); }
__device__ __forceinline__ uint16_t h_to_bits(f16 h) { return __builtin_bit_cast(uint16_t, h); }

// f32 -> fp16, round to nearest even (v_cvt_f16_f32 under the default mode).
__device__ __forceinline__ f16 rn_h(float f) { return (f16)f; }

// fp16 tensor arithmetic as torch's CPU kernels do it: compute in f32,
// round once to fp16.
// fp16(fp16(silu(g)) u), silu(g) = g / (1 + exp(-g)) in f32 with the
// hardware reciprocal (1 ulp) for the division: the SwiGLU product of fp16
// tensors (act_fn(gate) * up).  The second product of two fp16 values is
// exact in f32, so its one rounding is the fp16 multiply's.
__device__ __forceinline__ f16 silu_mul_h(float g, float u) {
  const f16 a = rn_h(g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)));
  return rn_h((float)a * u);
}

__device__ __forceinline__ f16 h_sub(f16 a, f16 b) { return rn_h((float)a - (float)b); }
__device__ __forceinline__ f16 h_div(f16 a, f16 b) { return rn_h((float)a / (float)b); }  // IEEE f32 div

// fp16(x / s) for one scale s and many x, without a division per element.
// q0 = x * r with r = RN(1/s); e = x - q0 * s is exact (fma); q = q0 + e * r
// lies within one f32 ulp of x / s.  A normal-range fp16 quotient x / s is at
// least one f32 ulp away from every fp16 rounding midpoint (the midpoint
// times s needs 12 + 11 significant bits, x has 11), so fp16(q) equals
// fp16(RN32(x / s)); in the fp16 subnormal range the two may differ only on
// exact ties, and every such quotient encodes to code 0 in both formats.
// Checked exhaustively on the CPU against the literal division.
__device__ __forceinline__ f16 h_div_fast(float x, float s, float r) {
  float q0 = x * r;
  float e = __builtin_fmaf(-q0, s, x);
  float q = __builtin_fmaf(e, r, q0);
  return rn_h(__builtin_copysignf(q, x));  // s > 0: the sign is x's (keeps -0)
}

// ------------------------------------------------------------ e4m3 (OCP fn)

// Round an fp16 value with |v| <= 448 to the nearest E4M3 code (ties to even).
__device__ __forceinline__ uint8_t e4m3_from_h(f16 v) {
  uint32_t b = h_to_bits(v);
  uint32_t sign = (b >> 8) & 0x80u;
  uint32_t a = b & 0x7FFFu;
  uint32_t e16 = a >> 10;
  uint32_t code;
  if (e16 >= 9) {  // >= 2^-6: E4M3 normal; keep 3 of 10 mantissa bits
    uint32_t q = (a >> 7) - (8u << 3);
    uint32_t rem = a & 0x7Fu;
    code = q + ((rem > 0x40u) | ((rem == 0x40u) & (q & 1u)));
  } else {  // E4M3 subnormal: round(value * 2^9)
    uint32_t sig = e16 ? (0x400u | (a & 0x3FFu)) : (a & 0x3FFu);
    uint32_t shift = e16 ? 16u - e16 : 15u;
    uint32_t q = sig >> shift;
    uint32_t rem = sig & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    code = q + ((rem > half) | ((rem == half) & (q & 1u)));
  }
  return (uint8_t)(code | sign);
}

// Exact fp16 value of an E4M3 code (every E4M3 value is an fp16 value).
__device__ __forceinline__ f16 e4m3_to_h(uint8_t c) {
  uint32_t hb = ((uint32_t)(c & 0x7Fu) << 7) | ((uint32_t)(c & 0x80u) << 8);
  return bits_to_h((uint16_t)hb) * (f16)256.0f;  // power-of-two scaling: exact, keeps -0
}

// -------------------------------------------------------- team reductions
// A team is TAU consecutive threads (TAU a power of two) that own one block.
// Sums follow a fixed balanced binary tree: leaves in element order, pairs
// (2i, 2i+1) first.  Within a wave, level k adds to each lane's value (the
// sum of its aligned group of 2^(k-1) lanes) the value of some lane of the
// partner group, so every lane holds the tree node of its 2^k group; since
// a + b == b + a bit for bit, every lane ends with the identical value.  The
// partner lane comes from a register-to-register exchange, never through
// LDS: DPP quad permutations (partners at distance 1 and 2), half-row and
// row mirrors (the other group of 4 in 8 and of 8 in 16), and the gfx950
// row swaps (16 lanes, 32 lanes).

// Value of the partner lane at butterfly levels 1-4 (group 2^(L-1) -> 2^L).
template <int L>
__device__ __forceinline__ uint32_t xlane_partner_u32(uint32_t v) {
  if constexpr (L == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  if constexpr (L == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  if constexpr (L == 3) return __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  return __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false);                       // row_mirror
}

// Levels 5 and 6: a register swapped with itself by 16-lane rows (rows 0/1
// and 2/3) or 32-lane halves gives two registers, one holding each group's
// own value in every lane of the pair of groups and the other the partner
// group's; combining the two is the tree node, whichever is which.
template <int L>
__device__ __forceinline__ void xlane_swap_u32(uint32_t v, uint32_t& a, uint32_t& b) {
  if constexpr (L == 5) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = r[0];
    b = r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
  }
}

template <int L>
__device__ __forceinline__ double xlane_level_sum_f64(double v) {
  const uint64_t x = __builtin_bit_cast(uint64_t, v);
  if constexpr (L <= 4) {
    const uint64_t p = (uint64_t)xlane_partner_u32<L>((uint32_t)x) |
                       ((uint64_t)xlane_partner_u32<L>((uint32_t)(x >> 32)) << 32);
    return v + __builtin_bit_cast(double, p);
  } else {
    uint32_t a0, b0, a1, b1;
    xlane_swap_u32<L>((uint32_t)x, a0, b0);
    xlane_swap_u32<L>((uint32_t)(x >> 32), a1, b1);
    return __builtin_bit_cast(double, (uint64_t)a0 | ((uint64_t)a1 << 32)) +
           __builtin_bit_cast(double, (uint64_t)b0 | ((uint64_t)b1 << 32));
  }
}

template <int L>
__device__ __forceinline__ float xlane_level_sum_f32(float v) {
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  if constexpr (L <= 4) {
    return v + __builtin_bit_cast(float, xlane_partner_u32<L>(x));
  } else {
    uint32_t a, b;
    xlane_swap_u32<L>(x, a, b);
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
  }
}

template <int L>
__device__ __forceinline__ float xlane_level_max_f32(float v) {
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  if constexpr (L <= 4) {
    return fmaxf(v, __builtin_bit_cast(float, xlane_partner_u32<L>(x)));
  } else {
    uint32_t a, b;
    xlane_swap_u32<L>(x, a, b);
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
  }
}

// Sum / max over aligned groups of WL lanes (WL <= 64, a power of two).
template <int WL>
__device__ __forceinline__ double wave_group_sum_f64(double v) {
  if constexpr (WL > 1) v = xlane_level_sum_f64<1>(v);
  if constexpr (WL > 2) v = xlane_level_sum_f64<2>(v);
  if constexpr (WL > 4) v = xlane_level_sum_f64<3>(v);
  if constexpr (WL > 8) v = xlane_level_sum_f64<4>(v);
  if constexpr (WL > 16) v = xlane_level_sum_f64<5>(v);
  if constexpr (WL > 32) v = xlane_level_sum_f64<6>(v);
  return v;
}

template <int WL>
__device__ __forceinline__ float wave_group_sum_f32(float v) {
  if constexpr (WL > 1) v = xlane_level_sum_f32<1>(v);
  if constexpr (WL > 2) v = xlane_level_sum_f32<2>(v);
  if constexpr (WL > 4) v = xlane_level_sum_f32<3>(v);
  if constexpr (WL > 8) v = xlane_level_sum_f32<4>(v);
  if constexpr (WL > 16) v = xlane_level_sum_f32<5>(v);
  if constexpr (WL > 32) v = xlane_level_sum_f32<6>(v);
  return v;
}

template <int WL>
__device__ __forceinline__ float wave_group_max_f32(float v) {
  if constexpr (WL > 1) v = xlane_level_max_f32<1>(v);
  if constexpr (WL > 2) v = xlane_level_max_f32<2>(v);
  if constexpr (WL > 4) v = xlane_level_max_f32<3>(v);
  if constexpr (WL > 8) v = xlane_level_max_f32<4>(v);
  if constexpr (WL > 16) v = xlane_level_max_f32<5>(v);
  if constexpr (WL > 32) v = xlane_level_max_f32<6>(v);
  return v;
}

constexpr int pow2_ceil(int n) { return n <= 1 ? 1 : 2 * pow2_ceil((n + 1) / 2); }

template <int TAU>
__device__ __forceinline__ double team_sum_f64(double v, double* lds_team) {
  constexpr int WL = TAU < 64 ? TAU : 64;
  v = wave_group_sum_f64<WL>(v);
  if constexpr (TAU > 64) {
    constexpr int NW = TAU / 64;
    const int lane = threadIdx.x & 63;
    const int w = (threadIdx.x % TAU) >> 6;
    __syncthreads();
    if (lane == 0) lds_team[w] = v;
    __syncthreads();
    // a team of NW waves sums as one of the next power of two whose last
    // waves hold +0 (the balanced tree over next_pow2(TAU) leaves)
    constexpr int NP = pow2_ceil(NW);
    double t[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) t[i] = i < NW ? lds_team[i] : 0.0;
#pragma unroll
    for (int s = NP; s > 1; s >>= 1)
#pragma unroll
      for (int i = 0; i < s / 2; i++) t[i] = t[2 * i] + t[2 * i + 1];
    v = t[0];
  }
  return v;
}

// f32 sum over the team, the same value in every lane (the wave part is a
// butterfly, the waves' partial sums are added in a fixed tree order).
template <int TAU>
__device__ __forceinline__ float team_sum_f32(float v, float* lds_team) {
  constexpr int WL = TAU < 64 ? TAU : 64;
  v = wave_group_sum_f32<WL>(v);
  if constexpr (TAU > 64) {
    constexpr int NW = TAU / 64;
    const int lane = threadIdx.x & 63;
    const int w = (threadIdx.x % TAU) >> 6;
    __syncthreads();
    if (lane == 0) lds_team[w] = v;
    __syncthreads();
    constexpr int NP = pow2_ceil(NW);
    float t[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) t[i] = i < NW ? lds_team[i] : 0.0f;
#pragma unroll
    for (int s = NP; s > 1; s >>= 1)
#pragma unroll
      for (int i = 0; i < s / 2; i++) t[i] = t[2 * i] + t[2 * i + 1];
    v = t[0];
  }
  return v;
}

template <int TAU>
__device__ __forceinline__ float team_max_f32(float v, float* lds_team) {
  constexpr int WL = TAU < 64 ? TAU : 64;
  v = wave_group_max_f32<WL>(v);
  if constexpr (TAU > 64) {
    constexpr int NW = TAU / 64;
    const int lane = threadIdx.x & 63;
    const int w = (threadIdx.x % TAU) >> 6;
    __syncthreads();
    if (lane == 0) lds_team[w] = v;
    __syncthreads();
    v = lds_team[0];
#pragma unroll
    for (int i = 1; i < NW; i++) v = fmaxf(v, lds_team[i]);
  }
  return v;
}

// Inclusive prefix sum of v over groups of WL lanes (in lane order).
template <int WL>
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
  const int lane_in = threadIdx.x & (WL - 1);
  // inclusive scan: DPP row shifts within rows of 16 lanes (zero from
  // outside the row), then the gfx9 row broadcasts of lane 15 into rows 1
  // and 3 and of lane 31 into rows 2 and 3 (other rows receive 0)
  int inc = v;
  if constexpr (WL > 1) {
    const int t = __builtin_amdgcn_update_dpp(0, inc, 0x111, 0xF, 0xF, true);  // row_shr:1
    if (lane_in >= 1) inc += t;
  }
  if constexpr (WL > 2) {
    const int t = __builtin_amdgcn_update_dpp(0, inc, 0x112, 0xF, 0xF, true);  // row_shr:2
    if (lane_in >= 2) inc += t;
  }
  if constexpr (WL > 4) {
    const int t = __builtin_amdgcn_update_dpp(0, inc, 0x114, 0xF, 0xF, true);  // row_shr:4
    if (lane_in >= 4) inc += t;
  }
  if constexpr (WL > 8) {
    const int t = __builtin_amdgcn_update_dpp(0, inc, 0x118, 0xF, 0xF, true);  // row_shr:8
    if (lane_in >= 8) inc += t;
  }
  if constexpr (WL > 16) inc += __builtin_amdgcn_update_dpp(0, inc, 0x142, 0xA, 0xF, false);  // row_bcast:15
  if constexpr (WL > 32) inc += __builtin_amdgcn_update_dpp(0, inc, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return inc;
}

// Exclusive prefix sum of v over the team (in thread order); *total gets the
// team sum.
template <int TAU>
__device__ __forceinline__ int team_excl_scan_i32(int v, int* lds_team, int* total) {
  constexpr int WL = TAU < 64 ? TAU : 64;
  const int inc = wave_incl_scan_i32<WL>(v);
  int wave_total = __shfl(inc, WL - 1, WL);
  int excl = inc - v;
  if constexpr (TAU > 64) {
    constexpr int NW = TAU / 64;
    const int lane = threadIdx.x & 63;
    const int w = (threadIdx.x % TAU) >> 6;
    __syncthreads();
    if (lane == 63) lds_team[w] = wave_total;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) {
      int c = lds_team[i];
      before += (i < w) ? c : 0;
      all += c;
    }
    excl += before;
    *total = all;
  } else {
    *total = wave_total;
  }
  return excl;
}

// Two independent team reductions through one cross-wave exchange (one pair
// of barriers instead of two), with the same trees as the single ones:
// team_sum_f64(a) and team_sum_f32(b), in every lane of the team.  FRESH:
// no wave has read lds_d / lds_f since the last barrier every wave passed,
// so the barrier before the writes is left out.
template <int TAU, bool FRESH = false>
__device__ __forceinline__ void team_sum_f64_f32(double& a, float& b, double* lds_d, float* lds_f) {
  constexpr int WL = TAU < 64 ? TAU : 64;
  a = wave_group_sum_f64<WL>(a);
  b = wave_group_sum_f32<WL>(b);
  if constexpr (TAU > 64) {
    constexpr int NW = TAU / 64;
    constexpr int NP = pow2_ceil(NW);
    const int w = (threadIdx.x % TAU) >> 6;
    if constexpr (!FRESH) __syncthreads();
    if ((threadIdx.x & 63) == 0) {
      lds_d[w] = a;
      lds_f[w] = b;
    }
    __syncthreads();
    double t[NP];
    float u[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
      t[i] = i < NW ? lds_d[i] : 0.0;
      u[i] = i < NW ? lds_f[i] : 0.0f;
    }
#pragma unroll
    for (int s = NP; s > 1; s >>= 1)
#pragma unroll
      for (int i = 0; i < s / 2; i++) {
        t[i] = t[2 * i] + t[2 * i + 1];
        u[i] = u[2 * i] + u[2 * i + 1];
      }
    a = t[0];
    b = u[0];
  }
}

// team_excl_scan_i32(v, .., total) and team_max_f32(m) through one
// cross-wave exchange; returns the exclusive prefix, *m becomes the maximum.
// FRESH as for team_sum_f64_f32 (for lds_i / lds_f).
template <int TAU, bool FRESH = false>
__device__ __forceinline__ int team_scan_max(int v, float* m, int* lds_i, float* lds_f, int* total) {
  constexpr int WL = TAU < 64 ? TAU : 64;
  const int inc = wave_incl_scan_i32<WL>(v);
  const int wave_total = __shfl(inc, WL - 1, WL);
  int excl = inc - v;
  float mx = wave_group_max_f32<WL>(*m);
  if constexpr (TAU > 64) {
    constexpr int NW = TAU / 64;
    const int lane = threadIdx.x & 63;
    const int w = (threadIdx.x % TAU) >> 6;
    if constexpr (!FRESH) __syncthreads();
    if (lane == 63) lds_i[w] = wave_total;
    if (lane == 0) lds_f[w] = mx;
    __syncthreads();
    int before = 0, all = 0;
    mx = lds_f[0];
#pragma unroll
    for (int i = 0; i < NW; i++) {
      const int c = lds_i[i];
      before += (i < w) ? c : 0;
      all += c;
      if (i > 0) mx = fmaxf(mx, lds_f[i]);
    }
    excl += before;
    *total = all;
  } else {
    *total = wave_total;
  }
  *m = mx;
  return excl;
}
