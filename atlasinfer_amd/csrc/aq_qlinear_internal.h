// aq_qlinear_internal.h -- types and decode helpers of the quantized-linear
// kernels (aq_qlinear.hip).  Not part of the C ABI.
#pragma once

#include <stdint.h>

#include "aq_common.h"

namespace aqk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kMaxGroup = 4;
// GEMV launches cut a group's matrices into up to this many pieces of equal
// tile-row count, one grid row (blockIdx.y) per piece
constexpr int kMaxPieces = 8;

struct QLMat {
  const uint8_t* codes;  // tiled
  const uint16_t* scales;
  const int32_t* row_ptr;
  const int32_t* cols;
  const uint16_t* vals;
  const int32_t* tptr;    // outliers per 16 x 64 block (GEMM, shared-x GEMV)
  const uint32_t* tent;
  const uint16_t* bias;
  uint16_t* y;
  float* part;  // GEMM split over K: this matrix's fp32 partial sums [split][M][N]
  int N;       // rows (of a GEMV piece: the rows it covers)
  int G;
  int kg;      // K / G, scale blocks per row
  int gshift;  // log2(G) when G is a power of two, else -1
  int ldy;     // row stride of y: the whole matrix's N
  // decode epilogue (decode GEMVs only; zero elsewhere): act 1 = ReLU of the
  // fp16 output, then res (fp16 [M][ldy], at this piece's first row) added
  // in fp16; act 2 (member 0 of two, shared-x GEMV): the SwiGLU pair
  const uint16_t* res;
  int act;
};

// Prologue of the decode GEMVs: what is staged in place of x (the norms on
// the M = 1 GEMV only).
enum : int { kProNone = 0, kProRms = 1, kProLayerNorm = 2, kProSwiGlu = 3 };

struct QLArgs {
  const uint16_t* x;
  int M, K, count;
  int pro;              // kPro*: 0 stages x as given
  const uint16_t* x2;   // kProSwiGlu: u (x holds the gate g)
  const uint16_t* nw;   // kProRms / kProLayerNorm: weight [K]
  const uint16_t* nb;   // kProLayerNorm: bias [K]
  float eps;
  // 256 x 256 GEMM, unsplit: the last `tail` tiles of each XCD's run of
  // `per` run as two K halves, their fp32 partial sums in tpart (0: none)
  int tail, per;
  float* tpart;
  // shared-x GEMV, aq_qlinear_decode: > 0 for a SwiGLU pair (gate, up), the
  // number of pieces of each; the product goes to gate's output
  int pair;
  int split;                 // GEMM: ways the K chunks are split (1: none)
  int first[kMaxGroup + 1];  // GEMM: first output tile of each matrix
  QLMat mat[kMaxPieces];     // GEMM: the group's matrices; GEMV: their pieces
};

// The matrix a workgroup works on (workgroup-uniform selection, no dynamic
// indexing into the argument block).
__device__ __forceinline__ QLMat pick(const QLArgs& a, int i) {
  QLMat w = a.mat[0];
#pragma unroll
  for (int j = 1; j < kMaxGroup; j++)
    if (i == j) w = a.mat[j];
  return w;
}

__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t h2_bits(half2v h) { return __builtin_bit_cast(uint32_t, h); }

// eight fp16 pairs (g, u) -> fp16(fp16(silu(g)) u)
__device__ __forceinline__ u32x4 swiglu8(u32x4 g, u32x4 u) {
  const half8 gh = __builtin_bit_cast(half8, g), uh = __builtin_bit_cast(half8, u);
  half8 o;
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = silu_mul_h((float)gh[e], (float)uh[e]);
  return __builtin_bit_cast(u32x4, o);
}

// 8 codes (two dwords) -> 8 fp16 weights value(code) * s.
template <int FMT>
__device__ __forceinline__ half8 deq8(uint32_t w0, uint32_t w1, half2v s2) {
  uint32_t r[4];
  if (FMT == AQ_FMT_E4M3) {
    // hardware E4M3 -> fp16 (exact with a unit scale), then one fp16 multiply
    r[0] = h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false) * s2);
    r[1] = h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true) * s2);
    r[2] = h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false) * s2);
    r[3] = h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true) * s2);
  } else {
    // int8: 0x6400 | (c ^ 0x80) is the fp16 1024 + (c + 128); subtract 1152
    const half2v off = (half2v){(f16)1152.0f, (f16)1152.0f};
    const uint32_t w[2] = {w0, w1};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t p = __builtin_amdgcn_perm(0u, w[i >> 1], (i & 1) ? 0x0C030C02u : 0x0C010C00u);
      r[i] = h2_bits((as_h2((p ^ 0x00800080u) | 0x64006400u) - off) * s2);
    }
  }
  return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ half2v scale2(uint16_t sbits) {
  const f16 s = bits_to_h(sbits);
  return (half2v){s, s};
}

__device__ __forceinline__ int scale_index(const QLMat& w, int n, int k) {
  return n * w.kg + (w.gshift >= 0 ? (k >> w.gshift) : (k / w.G));
}

// Byte offset of (row, 16-byte piece) in an A or B tile of the dequant-GEMMs:
// 128-byte rows, piece p stored at p ^ (row & 7) ^ ((row >> 3) & 1).
// Measured on gfx950: 16-byte LDS reads serve 16 lanes per cycle over 64
// banks, 16-byte writes 8 lanes over 128 bytes.  Reads of 16 consecutive rows
// at one piece then fall on 8 distinct pieces among the even rows and 8 among
// the odd rows, and writes of 8 consecutive rows at one piece (or of one
// row's 8 pieces) on 8 distinct pieces.
__device__ __forceinline__ uint32_t tile_off(int row, int piece) {
  return (uint32_t)(row * 128 + ((piece ^ (row & 7) ^ ((row >> 3) & 1)) << 4));
}

constexpr uint32_t kOutOfRange = 0x80000000u;  // a buffer offset past every range used here
constexpr int kBufferDword3 = 0x00020000;      // raw (untyped) buffer access on gfx9

}  // namespace aqk
