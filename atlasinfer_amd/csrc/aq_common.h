// aq_common.h -- shared helpers of the gfx950 kernels: fp16/e4m3 arithmetic
// with explicit rounding, the deterministic team reductions, and the error
// reporting of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
// (2i, 2i+1) first.  The xor butterfly realises exactly that tree, and since
// a + b == b + a bit for bit, every lane ends with the identical value.

template <int TAU>
__device__ __forceinline__ double team_sum_f64(double v, double* lds_team) {
  constexpr int WL = TAU < 64 ? TAU : 64;
#pragma unroll
  for (int m = 1; m < WL; m <<= 1) v = v + __shfl_xor(v, m, 64);
  if constexpr (TAU > 64) {
    constexpr int NW = TAU / 64;
    const int lane = threadIdx.x & 63;
    const int w = (threadIdx.x % TAU) >> 6;
    __syncthreads();
    if (lane == 0) lds_team[w] = v;
    __syncthreads();
    double t[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) t[i] = lds_team[i];
#pragma unroll
    for (int s = NW; s > 1; s >>= 1)
#pragma unroll
      for (int i = 0; i < s / 2; i++) t[i] = t[2 * i] + t[2 * i + 1];
    v = t[0];
  }
  return v;
}

template <int TAU>
__device__ __forceinline__ float team_max_f32(float v, float* lds_team) {
  constexpr int WL = TAU < 64 ? TAU : 64;
#pragma unroll
  for (int m = 1; m < WL; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
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

// Exclusive prefix sum of v over the team (in thread order); *total gets the
// team sum.
template <int TAU>
__device__ __forceinline__ int team_excl_scan_i32(int v, int* lds_team, int* total) {
  constexpr int WL = TAU < 64 ? TAU : 64;
  const int lane_in = threadIdx.x & (WL - 1);
  int inc = v;
#pragma unroll
  for (int d = 1; d < WL; d <<= 1) {
    int t = __shfl_up(inc, d, WL);
    if (lane_in >= d) inc += t;
  }
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
