// aq_qlinear.hip -- quantized linear forward y = x W^T + b on gfx950.
//
// Replaces QuantizedLinear.forward (reference: integration/atlas_wrappers.py:
// 30-74), which dequantizes the whole weight (dequantize_tensor, :56) and
// calls F.linear on the fp16 result (:67).  Here the weight stays in its
// 1-byte code form in HBM, in the tiled layout (16 rows x 128 columns per
// 2 KiB tile, bytes in MFMA operand order, see include/atlasinfer_amd.h).
// Codes become fp16 weights in registers as fp16(value(code) * scale) -- bit
// for bit the weight dequantize_tensor produces -- and are multiplied on the
// fp16 MFMA units (16x16x32) with fp32 accumulation.  Outlier positions hold
// code 0; their fp16 values are added from the CSR lists in fp32, then the
// bias, then one rounding to fp16.
//
//  * M <= 5: dequant-GEMV.  One workgroup per 16-row tile row: NS waves
//    stream its tiles (1 KiB contiguous per load instruction, four 128-wide
//    K chunks in flight per wave) with the M rows of x as the MFMA A operand
//    (rows >= M are zero), and their partial tiles are summed through LDS in
//    a fixed order.  Wave 0 also sums the rows' CSR outliers.  NS (1, 2, 4
//    or 8) gives the launch about 1536 waves: one per tile row for a tall
//    group.  Several matrices that read the same x (q/k/v, gate/up) share
//    one launch, cut into pieces of equal tile-row count, one grid row
//    (blockIdx.y) per piece, so that a wave finds its matrix without
//    loading anything first.
//  * 6 <= M <= 64 (and from M = 2 tall groups with block-wise scales): the
//    same streaming, but 8 waves per workgroup share each chunk of x through
//    LDS (details at its kernel below), since x is then comparable to or
//    larger than the codes it multiplies.  (M = 1..5 re-read
//    x per tile row above; decode stages it in LDS once per workgroup.)
//  * M > 64: dequant-GEMM (details at its kernel below): 128 or 256 rows of
//    x by 128 output columns per workgroup, x and decoded weights staged in
//    LDS in MFMA operand order, each outlier written over its decoded zero,
//    loads two 64-wide K chunks ahead.
#include <algorithm>
#include <atomic>

#include "aq_common.h"
#include "aq_qlinear_internal.h"

namespace {

using namespace aqk;

// ------------------------------------------------------------ GEMV (M <= 64)

// The GEMV's arguments: its piece of the group (blockIdx.y, known at wave
// start) and the shared x, M, K, all read in one round of scalar loads and
// held in scalar registers (the asm below keeps the compiler from placing
// each load next to its first use, which costs a full round trip to the
// argument block per use: the first code load of a wave would wait for
// several in turn).
struct GemvIn {
  QLMat w;
  const uint16_t* x;
  int M, K;
};
__device__ __forceinline__ GemvIn gemv_in(const QLArgs& a, int off = 0) {
  GemvIn g;
  g.w = a.mat[blockIdx.y + off];
  g.x = a.x;
  g.M = a.M;
  g.K = a.K;
  asm volatile(""
               : "+s"(g.w.codes), "+s"(g.w.scales), "+s"(g.w.row_ptr), "+s"(g.w.cols), "+s"(g.w.vals),
                 "+s"(g.w.bias), "+s"(g.w.y), "+s"(g.w.N), "+s"(g.w.G), "+s"(g.w.kg), "+s"(g.w.gshift),
                 "+s"(g.w.ldy), "+s"(g.x), "+s"(g.M), "+s"(g.K));
  return g;
}

constexpr int kGemvMaxM = 64;   // larger M takes the GEMM
// From 33 rows of x on, grids of fewer than 384 tile rows take the GEMM when the
// caller passes the outlier block lists: the GEMV's x stages for 64 rows fit
// LDS only with 4 waves per tile row, which leaves half the CUs idle there
// (down_proj [4096, 14336] at M = 33..64: 78 us against 29 with the GEMM;
// q/o and k/v about equal; taller grids such as grouped q/k/v or gate+up stay
// faster on the GEMV)
constexpr int kGemvShortMaxM = 32;
constexpr int kGemvShortRows = 384;
constexpr int kGemvXMinM = 6;   // from here on the GEMV shares x through LDS (qlinear_gemv_x_kernel)
constexpr int kGemvUnroll = 2;  // 128-wide K chunks per wave with loads in flight together
constexpr int kGemvDirectMaxM = kGemvXMinM - 1;  // rows of x qlinear_gemv_kernel takes
// Outlier entries of a 16-row tile held in registers (64 * kStageBatch);
// entries beyond them (heavy-tailed weights) are read from memory.
constexpr int kStageBatch = 8;
constexpr int kGemvX1MaxK = 16384;  // decode keeps x in LDS up to this row length (32 KiB)

// s_waitcnt operand on gfx9: vmcnt(N) only (expcnt and lgkmcnt at their maxima)
template <int N>
constexpr int kVmcnt = (N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00;

// MM: the most rows of x (1 for decode, kGemvDirectMaxM otherwise)
template <int NS, int FMT, int PC, int X1, int MM>
__global__ __launch_bounds__(64 * NS) void qlinear_gemv_kernel(QLArgs a) {
  static_assert(!X1 || MM == 1, "x in LDS is for decode");
  // X1 = 2: x in LDS with aq_qlinear_decode's prologue and epilogue
  constexpr int U = kGemvUnroll;
  // X1 (M = 1): x is staged in LDS once, K fp16 followed by 64 zero bytes
  // that the lanes of rows 1..15 of the MFMA A operand read instead
  extern __shared__ __attribute__((aligned(16))) uint16_t x_lds[];
  __shared__ float red[NS][256];
  __shared__ float s_prod[MM][64 * kStageBatch];  // x * value of the tile's first entries
  __shared__ float s_osum[MM][16];                // outlier sum per (row of x, output column)

  const GemvIn in = gemv_in(a);
  const QLMat& W = in.w;
  const int rb = blockIdx.x;  // tile row in the piece
  if (rb * 16 >= W.N) return;  // the grid is as wide as the longest piece
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: chunk tests stay scalar
  const int n0 = rb * 16;
  const int M = in.M, K = in.K;
  const int nchunks = K >> 7;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int n = n0 + li;

  // Every load of the stream is a buffer load: rows of x past M, chunks past
  // K and outlier entries past the row's list lie past the end of their
  // range and read as zero without touching memory, so no load needs a
  // condition (which would make the compiler wait for all loads in flight).
  const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W.codes + ((size_t)rb * nchunks << 11)), (short)0, nchunks * 2048, kBufferDword3);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)in.x, (short)0, M * K * 2, kBufferDword3);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W.scales + (size_t)n0 * W.kg), (short)0, 16 * W.kg * 2, kBufferDword3);
  const uint32_t code_lane = lane * 16;
  const uint32_t x_lane = (uint32_t)(li * K + 16 * grp) * 2;  // x row li, columns 16 grp + ...
  const uint32_t scale_row = (uint32_t)li * W.kg;
  const uint16_t sb_row = PC == 1 ? W.scales[n] : (uint16_t)0;

  // Wave 0 also handles the rows' outliers.  Its row_ptr load goes out
  // first; the (col, val) loads of up to 64 * kStageBatch entries go out
  // right after its first code loads, and the x values at those columns
  // right before its first chunk is computed, so all of them return while
  // the codes stream in.
  int rp = 0;
  if (wave == 0 && lane <= 16) rp = W.row_ptr[n0 + lane];
  // every lane: the bias of column n0 + lane % 16 (no bias: an empty range,
  // read as zero)
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W.bias ? W.bias + n0 : W.vals), (short)0, W.bias ? 32 : 0, kBufferDword3);
  const uint32_t bias_v = __builtin_amdgcn_raw_buffer_load_b16(br, (lane & 15) * 2, 0, 0);
  // aq_qlinear_decode's residual of column n0 + lane % 16, read now for the
  // same reason (at the end it would add a round trip to the launch)
  uint32_t res_v = 0;
  if (X1 == 2) {
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(W.res ? W.res + n0 : W.vals), (short)0, W.res ? 32 : 0, kBufferDword3);
    res_v = __builtin_amdgcn_raw_buffer_load_b16(rr, (lane & 15) * 2, 0, 0);
  }
  int p0 = 0, cnt = 0;
  uint32_t scol[kStageBatch], sval[kStageBatch], sx[MM][kStageBatch];
  auto stage_first_batch = [&]() {
    // wave-uniform, so the list descriptors below live in scalar registers
    p0 = __builtin_amdgcn_readfirstlane(__shfl(rp, 0, 64));
    cnt = __builtin_amdgcn_readfirstlane(min(__shfl(rp, 16, 64) - p0, 64 * kStageBatch));
    const __amdgpu_buffer_rsrc_t colr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(W.cols + p0), (short)0, cnt * 4, kBufferDword3);
    const __amdgpu_buffer_rsrc_t valr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(W.vals + p0), (short)0, cnt * 2, kBufferDword3);
#pragma unroll
    for (int b = 0; b < kStageBatch; b++) {
      const int e = 64 * b + lane;
      scol[b] = __builtin_amdgcn_raw_buffer_load_b32(colr, e * 4, 0, 0);
      sval[b] = __builtin_amdgcn_raw_buffer_load_b16(valr, e * 2, 0, 0);
    }
  };
  auto gather_x = [&]() {
#pragma unroll
    for (int b = 0; b < kStageBatch; b++) {
      const int e = 64 * b + lane;
      if (X1) {
        sx[0][b] = x_lds[e < cnt ? scol[b] : K];
      } else {
#pragma unroll
        for (int m = 0; m < MM; m++)  // rows past M: out of range, zero
          sx[m][b] = __builtin_amdgcn_raw_buffer_load_b16(xr, e < cnt && m < M ? (m * K + scol[b]) * 2 : kOutOfRange,
                                                          0, 0);
      }
    }
  };
  // Wave 0, early in the stream so that its LDS round trips overlap the code
  // loads in flight: the products x * value of the first entries go to LDS,
  // then 4 lanes per output column r add up the column's entries (lane j:
  // entries j, j + 4, ... of the row r of W, in order; a tile with more
  // entries than the registers hold reads the rest from memory) for each
  // row of x, and two DPP levels add the 4 partial sums.
  auto outlier_sums = [&]() {
#pragma unroll
    for (int b = 0; b < kStageBatch; b++) {
      const int e = 64 * b + lane;
      const float wv = (float)bits_to_h((uint16_t)sval[b]);
#pragma unroll
      for (int m = 0; m < MM; m++)
        if (e < cnt && m < M) s_prod[m][e] = (float)bits_to_h((uint16_t)sx[m][b]) * wv;
    }
    __builtin_amdgcn_wave_barrier();  // the wave's LDS writes before its reads
    const int r = lane >> 2;
    const int e0 = __shfl(rp, r, 64) - p0, e1 = __shfl(rp, r + 1, 64) - p0;
    float v[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) v[m] = 0.0f;
    for (int e = e0 + (lane & 3); e < e1; e += 4) {
      if (e < cnt) {
#pragma unroll
        for (int m = 0; m < MM; m++)
          if (m < M) v[m] += s_prod[m][e];
      } else {
        const int col = W.cols[p0 + e];
        const float wv = (float)bits_to_h(W.vals[p0 + e]);
#pragma unroll
        for (int m = 0; m < MM; m++)
          if (m < M) v[m] += (float)bits_to_h(X1 ? x_lds[col] : in.x[(size_t)m * K + col]) * wv;
      }
    }
#pragma unroll
    for (int m = 0; m < MM; m++) {
      float t = v[m];
      t += __builtin_bit_cast(float, xlane_partner_u32<1>(__builtin_bit_cast(uint32_t, t)));
      t += __builtin_bit_cast(float, xlane_partner_u32<2>(__builtin_bit_cast(uint32_t, t)));
      if ((lane & 3) == 0 && m < M) s_osum[m][r] = t;
    }
  };

  struct Batch {
    u32x4 q[U][2];
    u32x4 x[U][4];
    uint32_t s[U][2];
  };
  // Codes are read once per call: non-temporal loads.  Launched alone, a
  // short matrix with several waves per tile row runs a few percent faster
  // with plain loads, but in a decoder layer's sequence of launches the
  // non-temporal ones win (the caches keep x and the small data instead;
  // measured on the Llama-3-8B shapes).
  constexpr int kCodePolicy = 2;  // nt
  auto load_q = [&](Batch& B, int c0) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = c0 + u * NS;
      const bool in = c < nchunks;
      const uint32_t co = in ? code_lane + (uint32_t)c * 2048 : kOutOfRange;
      B.q[u][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(cr, co, 0, kCodePolicy));
      B.q[u][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(cr, co + 1024, 0, kCodePolicy));
      if (PC == 2) {
        // blocks of 128 or more, a power of two: one scale per row and
        // chunk; the lanes of row group g load the scale of the batch's
        // chunk g (min(g, U - 1)), handed to the others in compute
        static_assert(U <= 4, "one row group per chunk of the batch");
        if (u == 0) {
          const int cg = c0 + (grp < U ? grp : U - 1) * NS;
          const uint32_t k = (uint32_t)(cg < nchunks ? cg : 0) * 128;
          B.s[0][0] = __builtin_amdgcn_raw_buffer_load_b16(sr, (scale_row + (k >> W.gshift)) * 2, 0, 0);
        }
      } else if (PC == 0) {
        const uint32_t k = (uint32_t)(in ? c : 0) * 128 + 16 * grp;
        const uint32_t k0 = W.gshift >= 0 ? k >> W.gshift : k / W.G;
        const uint32_t k1 = W.gshift >= 0 ? (k + 64) >> W.gshift : (k + 64) / W.G;
        B.s[u][0] = __builtin_amdgcn_raw_buffer_load_b16(sr, (scale_row + k0) * 2, 0, 0);
        B.s[u][1] = __builtin_amdgcn_raw_buffer_load_b16(sr, (scale_row + k1) * 2, 0, 0);
      }
    }
  };
  auto load_x = [&](Batch& B, int c0) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = c0 + u * NS;
      const bool in = c < nchunks;
      if (X1) {
        // rows 1..15 and chunks past K read the zeros after x
        const uint16_t* xp = x_lds + (li == 0 && in ? 128 * c + 16 * grp : K);
        B.x[u][0] = *reinterpret_cast<const u32x4*>(xp);
        B.x[u][1] = *reinterpret_cast<const u32x4*>(xp + (li == 0 && in ? 8 : 0));
        B.x[u][2] = *reinterpret_cast<const u32x4*>(xp + (li == 0 && in ? 64 : 0));  // + 64 columns
        B.x[u][3] = *reinterpret_cast<const u32x4*>(xp + (li == 0 && in ? 72 : 0));
      } else {
        const uint32_t xo = in ? x_lane + (uint32_t)c * 256 : kOutOfRange;
        B.x[u][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0));
        B.x[u][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + 16, 0, 0));
        B.x[u][2] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + 128, 0, 0));  // + 64 columns
        B.x[u][3] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo + 144, 0, 0));
      }
    }
  };
  auto load = [&](Batch& B, int c0) {
    load_q(B, c0);
    load_x(B, c0);
  };
  float4v acc = (float4v){0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Batch& B) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const half2v s0 = scale2(PC == 1   ? sb_row
                               : PC == 2 ? (uint16_t)__shfl((int)B.s[0][0], 16 * u + li)
                                         : (uint16_t)B.s[u][0]);
      const half2v s1 = PC == 0 ? scale2((uint16_t)B.s[u][1]) : s0;
      const half8 w0 = deq8<FMT>(B.q[u][0].x, B.q[u][0].y, s0);
      const half8 w1 = deq8<FMT>(B.q[u][0].z, B.q[u][0].w, s0);
      const half8 w2 = deq8<FMT>(B.q[u][1].x, B.q[u][1].y, s1);
      const half8 w3 = deq8<FMT>(B.q[u][1].z, B.q[u][1].w, s1);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, B.x[u][0]), w0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, B.x[u][1]), w1, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, B.x[u][2]), w2, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, B.x[u][3]), w3, acc, 0, 0, 0);
    }
  };

  // Two batches of U chunks in flight: the loads of the next batch go out
  // before the current one is computed.  Past the last chunk the loads are
  // out of range (no memory traffic) and the products zero.
  const int step = U * NS;
  Batch B0, B1;
  if (X1) {
    {
      // x in 16-byte pieces (K / 8 of x, then 4 of zeros: pieces past x are
      // out of range and read as zero), XB pieces per thread at a time,
      // enough for a row of 4096 with 64 threads, 10208 with 256 and 16352
      // with 512.
      // They go out ahead of the first two batches of codes, so their wait
      // (x comes from L2) leaves the codes in flight; longer rows take
      // further rounds.  Each thread issues only the loads its share needs
      // (a uniform test): every load instruction costs the CU's address unit
      // the same time, in range or not.
      constexpr int XB = NS >= 4 ? 5 : 9;
      const int nxp = (K >> 3) + 4;
      const int per = min(XB, (nxp + 64 * NS - 1) / (64 * NS));  // pieces per thread and round
      const __amdgpu_buffer_rsrc_t xr1 = __builtin_amdgcn_make_buffer_rsrc((void*)in.x, (short)0, K * 2, kBufferDword3);
      // Prologue (decode launches of aq_qlinear_decode): what LDS receives
      // in place of x.  kProSwiGlu: fp16(fp16(silu(x)) u) from x and a.x2,
      // piece by piece.  kProRms / kProLayerNorm: x itself first, its sum
      // (of squares) gathered on the way; after a workgroup reduction each
      // thread rewrites its own pieces as the normalised row.  The norm
      // weight (and bias) pieces of the first round load with x, ahead of
      // the codes, so the code loads stay in flight through all of this.
      // The zero pieces after x stay zero.
      const int pro = X1 == 2 ? a.pro : kProNone;  // uniform; instances without a prologue drop its code
      const __amdgpu_buffer_rsrc_t ur = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(pro == kProSwiGlu ? a.x2 : pro != kProNone ? a.nw : in.x), (short)0, pro != kProNone ? K * 2 : 0,
          kBufferDword3);
      const __amdgpu_buffer_rsrc_t br1 = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(pro == kProLayerNorm ? a.nb : in.x), (short)0, pro == kProLayerNorm ? K * 2 : 0, kBufferDword3);
      u32x4 xv[XB], uv[XB], bv[XB];
      float stat = 0.0f;  // this thread's sum (LayerNorm) or sum of squares (RMSNorm)
      auto x_round = [&](int i0) {
#pragma unroll
        for (int j = 0; j < XB; j++) {
          const int i = i0 + 64 * NS * j;
          const uint32_t off = i < (K >> 3) ? (uint32_t)i * 16 : kOutOfRange;
          if (j < per) {
            xv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr1, off, 0, 0));
            if (pro != kProNone) uv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, 0));
            if (pro == kProLayerNorm)
              bv[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(br1, off, 0, 0));
          }
        }
      };
      auto x_store = [&](int i0) {
#pragma unroll
        for (int j = 0; j < XB; j++) {
          const int i = i0 + 64 * NS * j;
          if (j < per && i < nxp) {
            u32x4 v = xv[j];
            if (pro == kProSwiGlu) {
              v = swiglu8(xv[j], uv[j]);
            } else if (pro != kProNone) {
              const half8 h = __builtin_bit_cast(half8, xv[j]);
#pragma unroll
              for (int e = 0; e < 8; e++) stat += pro == kProRms ? (float)h[e] * (float)h[e] : (float)h[e];
            }
            *reinterpret_cast<u32x4*>(x_lds + 8 * i) = v;
          }
        }
      };
      x_round(threadIdx.x);
      __builtin_amdgcn_sched_barrier(0);  // keep the issue order
      load_q(B0, wave);
      load_q(B1, wave + step);
      __builtin_amdgcn_sched_barrier(0);
      // x arrived, the codes may not have: the loads after x are 2 U code
      // pieces per batch, + 2 U scales with block-wise scales (one with one
      // scale per chunk) (the compiler's own count gives up on the
      // conditional loads above)
      if (PC == 1)
        __builtin_amdgcn_s_waitcnt(kVmcnt<4 * U>);
      else if (PC == 2)
        __builtin_amdgcn_s_waitcnt(kVmcnt<4 * U + 2>);
      else
        __builtin_amdgcn_s_waitcnt(kVmcnt<8 * U>);
      x_store(threadIdx.x);
      for (int i0 = threadIdx.x + 64 * NS * per; i0 < nxp; i0 += 64 * NS * per) {
        x_round(i0);
        x_store(i0);
      }
      // wave 0: the tile row's outlier entries load while the codes stream
      if (wave == 0) stage_first_batch();
      if (pro == kProRms || pro == kProLayerNorm) {
        // the row's statistics: waves' sums in a fixed order
        const float sw = wave_group_sum_f32<64>(stat);
        if (lane == 0) red[wave][0] = sw;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < NS; w++) tot += red[w][0];
        float mean = 0.0f, r;
        if (pro == kProRms) {
          r = 1.0f / sqrtf(tot / (float)K + a.eps);
        } else {
          mean = tot / (float)K;
          float q = 0.0f;
          for (int i = threadIdx.x; i < (K >> 3); i += 64 * NS) {
            const half8 h = *reinterpret_cast<const half8*>(x_lds + 8 * i);
#pragma unroll
            for (int e = 0; e < 8; e++) q += ((float)h[e] - mean) * ((float)h[e] - mean);
          }
          const float qw = wave_group_sum_f32<64>(q);
          if (lane == 0) red[wave][1] = qw;
          __syncthreads();
          float qt = 0.0f;
#pragma unroll
          for (int w = 0; w < NS; w++) qt += red[w][1];
          r = 1.0f / sqrtf(qt / (float)K + a.eps);
        }
        // each thread rewrites the pieces it stored (with one round, the
        // weights are still in registers; with more, the later rounds
        // replaced them and every round loads its own again)
        const bool one_round = 64 * NS * per >= nxp;
        for (int i0 = threadIdx.x; i0 < (K >> 3); i0 += 64 * NS * per) {
          if (!one_round) x_round(i0);
#pragma unroll
          for (int j = 0; j < XB; j++) {
            const int i = i0 + 64 * NS * j;
            if (j < per && i < (K >> 3)) {
              const half8 h = *reinterpret_cast<const half8*>(x_lds + 8 * i);
              const half8 wh = __builtin_bit_cast(half8, uv[j]);
              const half8 bh = __builtin_bit_cast(half8, bv[j]);
              half8 o;
              if (pro == kProRms) {
                // fp16(w fp16(x r)): the outer product of two fp16 values
                // rounds as the fp16 multiply (packed)
                half8 t;
#pragma unroll
                for (int e = 0; e < 8; e++) t[e] = rn_h((float)h[e] * r);
                o = wh * t;
              } else {
#pragma unroll
                for (int e = 0; e < 8; e++) o[e] = rn_h(((float)h[e] - mean) * r * (float)wh[e] + (float)bh[e]);
              }
              *reinterpret_cast<half8*>(x_lds + 8 * i) = o;
            }
          }
        }
      }
      __syncthreads();
    }
    load_x(B0, wave);
    load_x(B1, wave + step);
    // wave 0 sums the outliers' products in its third pass of the loop (or
    // its last, if sooner): by then their entries have arrived, and the
    // loads of the passes before went out without waiting for them (summed
    // in the first pass, their round trips held up the stream; after the
    // last, they added a tail)
    const int c_out = wave + 2 * step * min(2, (nchunks - 1 - wave) / (2 * step));
    for (int c0 = wave; c0 < nchunks; c0 += 2 * step) {
      __builtin_amdgcn_sched_barrier(0);
      if (wave == 0 && c0 == c_out) gather_x();
      compute(B0);
      __builtin_amdgcn_sched_barrier(0);
      load(B0, c0 + 2 * step);
      __builtin_amdgcn_sched_barrier(0);
      if (wave == 0 && c0 == c_out) outlier_sums();
      __builtin_amdgcn_sched_barrier(0);
      compute(B1);
      __builtin_amdgcn_sched_barrier(0);
      load(B1, c0 + 3 * step);
    }
  } else {
    load(B0, wave);
    if (wave == 0) stage_first_batch();
    for (int c0 = wave; c0 < nchunks; c0 += 2 * step) {
      load(B1, c0 + step);
      __builtin_amdgcn_sched_barrier(0);
      if (wave == 0 && c0 == 0) gather_x();
      compute(B0);
      __builtin_amdgcn_sched_barrier(0);
      load(B0, c0 + 2 * step);
      __builtin_amdgcn_sched_barrier(0);
      if (wave == 0 && c0 == 0) outlier_sums();
      __builtin_amdgcn_sched_barrier(0);
      compute(B1);
    }
  }
  // C layout: lane l, element i -> m = 4 (l / 16) + i, column l % 16
#pragma unroll
  for (int i = 0; i < 4; i++) red[wave][lane * 4 + i] = acc[i];
  __syncthreads();
  if (MM == 1) {
    // decode: C element (m = 0, column nl) sits in lane nl, slot 0
    if (wave == 0 && lane < 16) {
      float dense = 0.0f;
#pragma unroll
      for (int w = 0; w < NS; w++) dense += red[w][lane * 4];
      const float v = dense + s_osum[0][lane] + (float)bits_to_h((uint16_t)bias_v);
      f16 o = rn_h(v);
      if (X1 == 2) {
        if (W.act == 1 && (float)o < 0.0f) o = (f16)0.0f;                   // ReLU
        if (W.res) o = rn_h((float)bits_to_h((uint16_t)res_v) + (float)o);  // residual add
      }
      W.y[n0 + lane] = h_to_bits(o);
    }
    return;
  }
  // output (m, column nl): dense part (C element in lane 16 (m / 4) + nl,
  // slot m % 4 of each wave) + outlier sum + bias (nl = lane % 16)
  for (int o = threadIdx.x; o < 16 * M; o += 64 * NS) {
    const int m = o >> 4, nl = o & 15;
    float dense = 0.0f;
#pragma unroll
    for (int w = 0; w < NS; w++) dense += red[w][(16 * (m >> 2) + nl) * 4 + (m & 3)];
    const float v = dense + s_osum[m][nl] + (float)bits_to_h((uint16_t)bias_v);
    W.y[(size_t)m * W.ldy + n0 + nl] = h_to_bits(rn_h(v));
  }
}

// ------------------------------------------- GEMV with x in LDS (6 <= M <= 64)
//
// With 6 or more rows of x, re-reading x per 16-row tile row costs more
// than sharing it (2 M bytes per weight column against 1 of codes).  Here a
// workgroup of 8 waves takes TR = 8 / S tile rows with S waves each; wave
// (tr, s) streams the codes of tile row tr over the chunks c = S j + s.  For
// each chunk group j the workgroup stages x[16 MG rows][S chunks] in LDS
// once, for all TR tile rows, and each wave feeds each decoded fragment to
// one MFMA per 16-row group of x.  All loads are buffer loads: a workgroup
// barrier does not wait for them, so the loads of groups j + 1 and j + 2 stay
// in flight while group j is computed, and the zero that an out-of-range
// buffer load returns stands in for the rows of x past M, the chunks past K
// and the tile rows past the piece (no memory is read for them).  The S partial
// sums meet in LDS.
//
// Outliers (OT = 1, from the block lists of aq_outlier_tiles): each wave
// adds the outliers of its own chunk with one more MFMA per 16-row group of
// x.  The chunk's entries (its two 16 x 64 blocks, contiguous in the lists)
// are taken 32 at a time as the MFMA's k slots (as many slots per lane as
// the batch needs): the A operand gathers the x
// column of each entry from LDS, the B operand holds the entry's value in the
// column of its row and zero elsewhere, so the product adds x[m][col] * value
// to output (m, row) for every row m of x.  The entry ranges of a wave's
// chunks are loaded once, one chunk group per lane (64 groups at a time),
// and each chunk's first 64 entries travel with its codes.  Without the
// lists (OT = 0) one wave per tile row adds its rows' outliers from the CSR
// lists (see stage_outliers), the rest in the epilogue, where a lane owns
// one output column and 4 MG of its rows.

constexpr int kXWaves = 8;
constexpr int kXPad = 8;  // halves of padding per LDS row of x
constexpr int kXCsrCap = 512;  // outlier entries of a tile row staged in LDS (the rest: epilogue)

// XH: rows of x staged, 16 MG, or 8 for M <= 8 with one row group (the MFMA
// rows 8..15 then read rows 0..7 again; their outputs are never stored)
template <int FMT, int PC, int MG, int S, int OT, int XH>
__global__ __launch_bounds__(64 * kXWaves) void qlinear_gemv_x_kernel(QLArgs a) {
  constexpr int TR = kXWaves / S;
  constexpr int XR = XH;                   // staged rows of x
  static_assert(XH == 16 * MG || (XH == 8 && MG == 1), "staged rows");
  constexpr int XW = S * 128 + kXPad;      // LDS row pitch (halves)
  constexpr int XP = XR * S * 16 / (64 * kXWaves);  // 16-byte x pieces per thread and group
  static_assert(XP >= 1 && XR * S * 16 % (64 * kXWaves) == 0, "x pieces");
  // the staged row an MFMA row (16 gi + r) reads
  auto xrow = [](int r) { return XR == 8 ? (r & 7) : r; };
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][XR * XW];
  __shared__ uint32_t x_ent[TR][kXCsrCap];  // (value << 16) | column of the tile row's first outliers

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int tr = wave % TR, sp = wave / TR;  // tr: the wave's tile-row slot
  // SwiGLU pairs (a.pair > 0: a group of gate and up, a.pair pieces each,
  // TR >= 2): slots TR / 2 and up take up's pieces (grid row blockIdx.y +
  // a.pair), the same tile rows as the gate slots below them
  const bool pair = a.pair > 0;
  const int TRW = pair ? TR / 2 : TR;  // tile rows of a matrix per workgroup
  const bool upper = pair && tr >= TRW;
  const int trr = upper ? tr - TRW : tr;  // the wave's tile row in the workgroup
  const GemvIn in = gemv_in(a, upper ? a.pair : 0);
  const QLMat& W = in.w;
  const int M = in.M, K = in.K;
  const int nchunks = K >> 7;
  const int nrb = W.N / 16;
  const int rb0 = blockIdx.x * TRW;  // in the piece
  if (rb0 >= nrb) return;  // the grid is as wide as the longest piece (uniform over the workgroup)
  const int rows_here = min(TRW, nrb - rb0);  // tile rows of this workgroup inside the piece
  const int grp = lane >> 4, li = lane & 15;
  const int ngroups = (nchunks + S - 1) / S;
  const int nsteps = (ngroups + 1) & ~1;    // even: the loop body handles two groups

  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)in.x, (short)0, M * K * 2, kBufferDword3);
  const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W.codes + ((size_t)rb0 * nchunks << 11)), (short)0, rows_here * nchunks * 2048, kBufferDword3);
  const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(W.scales + (size_t)rb0 * 16 * W.kg), (short)0, rows_here * 16 * W.kg * 2, kBufferDword3);
  // tile rows past the piece: every code load of the wave is out of range (zero)
  const uint32_t code_base = trr < rows_here ? (uint32_t)(trr * nchunks * 2048 + lane * 16) : kOutOfRange;
  const uint32_t scale_row = (uint32_t)(trr * 16 + li) * W.kg;
  uint16_t sb_row = 0;
  if (PC == 1) sb_row = trr < rows_here ? W.scales[(size_t)(rb0 + trr) * 16 + li] : (uint16_t)0;

  // OT: the block lists (tile_ptr offset to the piece's first tile row;
  // tile_ent holds 64 entries of read padding past the last)
  const int nb64 = K >> 6;
  const __amdgpu_buffer_rsrc_t tpr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)W.tptr, (short)0, OT ? (nrb * nb64 + 1) * 4 : 0, kBufferDword3);
  const __amdgpu_buffer_rsrc_t ter =
      __builtin_amdgcn_make_buffer_rsrc((void*)W.tent, (short)0, OT ? 0x7FFFFFFF : 0, kBufferDword3);
  // lane i: first entry, first entry of the second block and end of chunk
  // group g0 + i of this wave (chunk S (g0 + i) + sp); zero past the piece
  uint32_t rg_s = 0, rg_m = 0, rg_e = 0;
  auto load_ranges = [&](int g0) {
    const int c = (g0 + lane) * S + sp;
    const uint32_t off =
        trr < rows_here && c < nchunks ? (uint32_t)((rb0 + trr) * nb64 + 2 * c) * 4 : kOutOfRange;
    rg_s = __builtin_amdgcn_raw_buffer_load_b32(tpr, off, 0, 0);
    rg_m = __builtin_amdgcn_raw_buffer_load_b32(tpr, off + 4, 0, 0);
    rg_e = __builtin_amdgcn_raw_buffer_load_b32(tpr, off + 8, 0, 0);
  };
  struct Slot {
    u32x4 q0, q1;
    uint32_t s0, s1;
    u32x4 x[XP];
    uint32_t ent;          // OT: entry `lane` of the chunk (0 past its end)
    int e_start, e_mid, e_cnt;  // OT: the chunk's entries (wave-uniform)
  };
  auto load = [&](Slot& sl, int j) {
    const int c = j * S + sp;
    const uint32_t co = c < nchunks ? code_base + (uint32_t)c * 2048 : kOutOfRange;
    // codes are read once per call: non-temporal
    sl.q0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(cr, co, 0, 2));
    sl.q1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(cr, co + 1024, 0, 2));
    if (PC == 2) {
      // blocks of 128 or more, a power of two: one scale per row and chunk
      const uint32_t k = (uint32_t)(c < nchunks ? c : 0) * 128;
      sl.s0 = __builtin_amdgcn_raw_buffer_load_b16(sr, (scale_row + (k >> W.gshift)) * 2, 0, 0);
    } else if (PC == 0) {
      const uint32_t k = (uint32_t)(c < nchunks ? c : 0) * 128 + 16 * grp;
      const uint32_t k0 = W.gshift >= 0 ? k >> W.gshift : k / W.G;
      const uint32_t k1 = W.gshift >= 0 ? (k + 64) >> W.gshift : (k + 64) / W.G;
      sl.s0 = __builtin_amdgcn_raw_buffer_load_b16(sr, (scale_row + k0) * 2, 0, 0);
      sl.s1 = __builtin_amdgcn_raw_buffer_load_b16(sr, (scale_row + k1) * 2, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < XP; i++) {
      const int p = t + 64 * kXWaves * i;
      const int row = p / (S * 16), col = (p % (S * 16)) * 8 + j * S * 128;
      // rows past M fall past the end of the range by themselves
      const uint32_t xo = col < K ? (uint32_t)(row * K + col) * 2 : kOutOfRange;
      sl.x[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0));
    }
    if (OT) {
      const int gl = j & 63;
      const int e0 = __builtin_amdgcn_readlane((int)rg_s, gl);
      sl.e_start = e0;
      sl.e_mid = __builtin_amdgcn_readlane((int)rg_m, gl) - e0;
      sl.e_cnt = __builtin_amdgcn_readlane((int)rg_e, gl) - e0;
      sl.ent = __builtin_amdgcn_raw_buffer_load_b32(ter, lane < sl.e_cnt ? (uint32_t)(e0 + lane) * 4 : kOutOfRange, 0,
                                                    0);
    }
  };

  float4v acc[MG];
#pragma unroll
  for (int gi = 0; gi < MG; gi++) acc[gi] = (float4v){0.f, 0.f, 0.f, 0.f};

  // the entries of the current chunk 32 at a time as one MFMA's k slots:
  // slot (grp, b) holds entry base + 4 b + grp, so that a batch of n entries
  // fills the first ceil(n / 4) slots of each lane and the rest stay zero
  // (a chunk typically holds a few entries)
  auto add_block_outliers = [&](uint32_t ent_lane, int e_start, int e_mid, int e_cnt, const uint16_t* xb) {
    for (int base = 0; base < e_cnt; base += 32) {
      const int nb = min(8, (e_cnt - base + 3) >> 2);  // slots in use per lane (wave-uniform)
      half8 bv = {};
      half8 av[MG];
#pragma unroll
      for (int gi = 0; gi < MG; gi++) av[gi] = (half8){};
#pragma unroll
      for (int b = 0; b < 8; b++) {
        if (b >= nb) break;
        const int e = base + 4 * b + grp;
        const bool valid = e < e_cnt;
        // the first 64 entries came with the codes; later ones (blocks this
        // crowded are rare) are read here
        const uint32_t ent = base < 64 ? (uint32_t)__shfl((int)ent_lane, (base + 4 * b + grp) & 63, 64)
                                       : __builtin_amdgcn_raw_buffer_load_b32(
                                             ter, valid ? (uint32_t)(e_start + e) * 4 : kOutOfRange, 0, 0);
        const int k = (int)(ent & 63u) + (e >= e_mid ? 64 : 0);
        bv[b] = valid && (int)((ent >> 6) & 15u) == li ? bits_to_h((uint16_t)(ent >> 16)) : (f16)0.0f;
#pragma unroll
        for (int gi = 0; gi < MG; gi++) {
          const f16 xv = bits_to_h(xb[xrow(16 * gi + li) * XW + sp * 128 + k]);
          av[gi][b] = valid ? xv : (f16)0.0f;
        }
      }
#pragma unroll
      for (int gi = 0; gi < MG; gi++) acc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[gi], bv, acc[gi], 0, 0, 0);
    }
  };

  auto step = [&](Slot& sl, int j, uint16_t* xb) {
    const half2v s0 = scale2(PC == 1 ? sb_row : (uint16_t)sl.s0);
    const half2v s1 = PC == 0 ? scale2((uint16_t)sl.s1) : s0;
    const half8 w0 = deq8<FMT>(sl.q0.x, sl.q0.y, s0);
    const half8 w1 = deq8<FMT>(sl.q0.z, sl.q0.w, s0);
    const half8 w2 = deq8<FMT>(sl.q1.x, sl.q1.y, s1);
    const half8 w3 = deq8<FMT>(sl.q1.z, sl.q1.w, s1);
    // this chunk's entries, read before the slot is reloaded
    const uint32_t ent = sl.ent;
    const int e_start = sl.e_start, e_mid = sl.e_mid, e_cnt = sl.e_cnt;
#pragma unroll
    for (int i = 0; i < XP; i++) {
      const int p = t + 64 * kXWaves * i;
      *reinterpret_cast<u32x4*>(xb + (p / (S * 16)) * XW + (p % (S * 16)) * 8) = sl.x[i];
    }
    __syncthreads();
    // unconditional: past the last group every offset is out of range, so the
    // loads read nothing, and the compiler keeps its partial waits
    __builtin_amdgcn_sched_barrier(0);
    load(sl, j + 2);
    __builtin_amdgcn_sched_barrier(0);  // the next group's decode stays below these loads
    const uint16_t* xw = xb + sp * 128 + 16 * grp;
#pragma unroll
    for (int gi = 0; gi < MG; gi++) {
      // A operand: x row 16 gi + li at columns 16 grp + {0, 8, 64, 72} of this wave's chunk
      const uint16_t* xp = xw + xrow(16 * gi + li) * XW;
      acc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(xp), w0, acc[gi], 0, 0, 0);
      acc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(xp + 8), w1, acc[gi], 0, 0, 0);
      acc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(xp + 64), w2, acc[gi], 0, 0, 0);
      acc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8*>(xp + 72), w3, acc[gi], 0, 0, 0);
    }
    if (OT) add_block_outliers(ent, e_start, e_mid, e_cnt, xb);
  };

  // Outliers (OT = 0): wave sp = 0 of each tile row copies the tile row's first
  // kXCsrCap entries (from the CSR lists, fetched behind the first code
  // loads) into LDS for itself, and in each chunk group adds, per lane, the
  // products of its row's entries in the group's columns with the x values
  // staged there (rows 4 grp + i of each 16-row group).  Entries past the
  // cap, and all of them when K >= 65536 (the column does not fit 16 bits),
  // are added in the epilogue.  (Sharing the rows among the S waves of the
  // tile row measured slower.)
  int op = 0, oend = 0;  // this lane's row: next staged entry and end of its staged entries
  int staged_row = 0;    // how many of the row's entries are staged
  auto stage_outliers = [&]() {
    const bool fits = sp == 0 && trr < rows_here && K < 65536;
    const int n0r = (rb0 + trr) * 16;
    int rpv = 0;
    if (fits && lane <= 16) rpv = W.row_ptr[n0r + lane];
    const int p0 = __shfl(rpv, 0, 64);
    const int cnt = fits ? min(__shfl(rpv, 16, 64) - p0, kXCsrCap) : 0;
    for (int e0 = 0; e0 < cnt; e0 += 64 * 8) {
      uint32_t ent[8];
#pragma unroll
      for (int b = 0; b < 8; b++) {
        const int e = min(e0 + 64 * b + lane, cnt - 1);  // loads stay unconditional
        ent[b] = ((uint32_t)W.vals[p0 + e] << 16) | (uint32_t)W.cols[p0 + e];
      }
#pragma unroll
      for (int b = 0; b < 8; b++)
        if (e0 + 64 * b + lane < cnt) x_ent[tr][e0 + 64 * b + lane] = ent[b];
    }
    op = min(__shfl(rpv, li, 64) - p0, cnt);
    oend = min(__shfl(rpv, li + 1, 64) - p0, cnt);
    if (!fits) op = oend = 0;
    staged_row = oend - op;
    // the wave's own LDS writes precede its reads in the loop
    __builtin_amdgcn_wave_barrier();
  };
  auto add_outliers = [&](int j, const uint16_t* xb) {
    const int gstart = j * S * 128, gend = gstart + S * 128;
    while (op < oend) {
      const uint32_t ent = x_ent[tr][op];
      const int col = (int)(ent & 0xFFFFu);
      if (col >= gend) break;
      const float wv = (float)bits_to_h((uint16_t)(ent >> 16));
      const uint16_t* xc = xb + (col - gstart);
#pragma unroll
      for (int gi = 0; gi < MG; gi++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          acc[gi][i] = __builtin_fmaf((float)bits_to_h(xc[xrow(16 * gi + 4 * grp + i) * XW]), wv, acc[gi][i]);
      op++;
    }
  };

  // the epilogue's bias and residual (aq_qlinear_decode), read now so that
  // their latency passes under the stream (at the end it would add a full
  // round trip to the launch)
  const bool active = sp == 0 && trr < rows_here;
  const int n = (rb0 + trr) * 16 + li;  // the lane's output column (C layout below)
  const float bv = active && W.bias ? (float)bits_to_h(W.bias[n]) : 0.0f;
  uint16_t rv[MG][4];
#pragma unroll
  for (int gi = 0; gi < MG; gi++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 16 * gi + 4 * grp + i;
      rv[gi][i] = active && W.res && m < M ? W.res[(size_t)m * W.ldy + n] : (uint16_t)0;
    }

  Slot sa, sb;
  if (OT) load_ranges(0);
  load(sa, 0);
  load(sb, 1);
  if (!OT && sp == 0) stage_outliers();
  for (int j = 0; j < nsteps; j += 2) {
    // the next 64 chunk groups' entry ranges, before load(j + 2) reads them
    if (OT && ((j + 2) & 63) == 0) load_ranges(j + 2);
    step(sa, j, xs[0]);
    if (!OT && sp == 0) add_outliers(j, xs[0]);
    step(sb, j + 1, xs[1]);
    if (!OT && sp == 0) add_outliers(j + 1, xs[1]);
  }

  // the S partial sums of each tile row meet in LDS (x is no longer read)
  float* red = reinterpret_cast<float*>(&xs[0][0]);
  if (S > 1) {
    __syncthreads();
    if (sp > 0)
#pragma unroll
      for (int gi = 0; gi < MG; gi++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[(((sp - 1) * TR + tr) * MG + gi) * 256 + i * 64 + lane] = acc[gi][i];
    __syncthreads();
    if (sp == 0)
      for (int s2 = 1; s2 < S; s2++)
#pragma unroll
        for (int gi = 0; gi < MG; gi++)
#pragma unroll
          for (int i = 0; i < 4; i++) acc[gi][i] += red[(((s2 - 1) * TR + tr) * MG + gi) * 256 + i * 64 + lane];
  }
  if (!pair && !active) return;  // no barrier follows (pairs meet at one below)

  // C layout: lane l, element i -> row m = 16 gi + 4 (l / 16) + i, column n = n0 + l % 16.
  // Outliers of row n, eight entries at a time: their loads, then all the x
  // loads they need, then the FMAs.
  const int p_end = OT || !active ? 0 : W.row_ptr[n + 1];
  // the row's entries past the staged ones
  for (int p = OT || !active ? 0 : W.row_ptr[n] + staged_row; p < p_end; p += 8) {
    int col[8];
    float wv[8];
#pragma unroll
    for (int b = 0; b < 8; b++) {
      const int e = min(p + b, p_end - 1);  // loads stay unconditional
      col[b] = W.cols[e];
      wv[b] = p + b < p_end ? (float)bits_to_h(W.vals[e]) : 0.0f;
    }
#pragma unroll
    for (int gi = 0; gi < MG; gi++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = min(16 * gi + 4 * grp + i, M - 1);
        float xg[8];
#pragma unroll
        for (int b = 0; b < 8; b++) xg[b] = (float)bits_to_h(in.x[(size_t)m * K + col[b]]);
#pragma unroll
        for (int b = 0; b < 8; b++) acc[gi][i] = __builtin_fmaf(xg[b], wv[b], acc[gi][i]);
      }
  }
  if (pair) {
    // up's outputs (fp16, bias added) to LDS (x is no longer read, the
    // partial sums sit in xs[0]); gate's waves write fp16(fp16(silu(g)) u)
    uint16_t* pu = &xs[1][0];
    if (active && upper)
#pragma unroll
      for (int gi = 0; gi < MG; gi++)
#pragma unroll
        for (int i = 0; i < 4; i++) pu[((trr * MG + gi) * 4 + i) * 64 + lane] = h_to_bits(rn_h(acc[gi][i] + bv));
    __syncthreads();
    if (active && !upper)
#pragma unroll
      for (int gi = 0; gi < MG; gi++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int m = 16 * gi + 4 * grp + i;
          const float u = (float)bits_to_h(pu[((trr * MG + gi) * 4 + i) * 64 + lane]);
          if (m < M) W.y[(size_t)m * W.ldy + n] = h_to_bits(silu_mul_h((float)rn_h(acc[gi][i] + bv), u));
        }
    return;
  }
#pragma unroll
  for (int gi = 0; gi < MG; gi++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 16 * gi + 4 * grp + i;
      if (m < M) {
        f16 o = rn_h(acc[gi][i] + bv);
        // aq_qlinear_decode's epilogue (zero / null for other calls)
        if (W.act == 1 && (float)o < 0.0f) o = (f16)0.0f;                                 // ReLU
        if (W.res) o = rn_h((float)bits_to_h(rv[gi][i]) + (float)o);  // residual add
        W.y[(size_t)m * W.ldy + n] = h_to_bits(o);
      }
    }
}

// ------------------------------------------------------------ GEMM (M > 64)
//
// Workgroup tile BM x 128 (BM = 256 or 128 rows of x by 128 output
// columns), K in chunks of 64, 12 waves in two roles:
//   * waves 0-7 (consumers, two per SIMD) own a 4 x 2 layout of (BM / 4) x 64
//     output tiles of 32x32x16 MFMAs.  Per chunk they only read fragments
//     from LDS and issue MFMAs, fragments two k-steps ahead of their use.
//     Eight of them: on gfx950 a wave's LDS reads are latency-bound (about
//     100 B/clk per CU with four reading waves, 195 with eight, measured),
//     and the fragments of a chunk take 128 KiB;
//   * waves 8-11 (producers) do all global loads, decode the weight codes,
//     write the x pieces and the decoded weights into LDS, and write each
//     outlier's fp16 value over the zero its code decoded to (the outliers
//     of a 16 x 64 weight block come as one short list from aq_outlier_tiles;
//     producer wave p owns weight block rows 2p and 2p + 1, so these writes
//     follow its own bulk writes of the same block in program order).
// LDS holds three chunk stages, each an A tile (x, BM rows x 64 fp16) and a
// B tile (decoded weights, 128 rows x 64 fp16), rows of 128 bytes whose
// 16-byte pieces are permuted by the row (tile_off) so that fragment reads
// and staging writes are free of bank conflicts.  In chunk c the consumers
// multiply chunk c (and read the first two k-steps of chunk c + 1, already
// complete) while the producers stage chunk c + 2 into the stage chunk c - 1
// used, from registers loaded two chunks earlier, and issue the loads of
// chunk c + 4; the workgroup meets once per chunk at a barrier.  The B tile
// holds exactly dequantize_tensor's weights, outliers included, so the MFMAs
// need no correction pass.  Every load in the K loop is a buffer load: the
// barrier's release fence would wait for global-pointer loads.

constexpr int kGemmBN = 128, kGemmBK = 64;

template <int BM>
struct GemmCfg {
  static constexpr int WM = BM / 4;            // consumer wave tile rows
  static constexpr int MI = WM / 32;           // 32-row MFMA tiles per consumer wave
  static constexpr int XP = BM * 128 / 16 / 256;  // 16-byte x pieces per producer thread and chunk
  static constexpr int A_BYTES = BM * 128;     // BM rows x 64 fp16
  static constexpr int B_BYTES = kGemmBN * 128;
  static constexpr int STAGE = A_BYTES + B_BYTES;
};

// A producer thread's share of one chunk: XP x pieces, and for each of its
// wave's two weight block rows 16 codes (one row, 16 consecutive k), their
// scale and the block's outlier list.
template <int BM>
struct GemmRegs {
  u32x4 a[GemmCfg<BM>::XP];
  u32x4 q[2];
  uint32_t s[2];   // block-wise scales only
  int e0[2], e1[2];  // outlier entries of each block: [e0, e1)
  uint32_t ent[2];   // entry e0 + lane of each block
};

// Loop-invariant part of a producer thread's global loads: buffer
// descriptors over this workgroup's x rows, code rows, block pointers,
// entries and scales, and each piece's byte offset in chunk 0 (a chunk adds
// a scalar offset).
template <int BM>
struct GemmSrc {
  __amdgpu_buffer_rsrc_t xr, cr, tr, er, sr;
  int xo[GemmCfg<BM>::XP];
  int co[2];  // code pieces
  int to[2];  // block pointer of chunk 0 of each block row
  int so[2];  // scale row of each code piece
};

// pt: producer thread 0..255
template <int BM>
__device__ __forceinline__ void gemm_src_init(GemmSrc<BM>& S, const QLMat& W, const uint16_t* x, int M, int K,
                                              int m_first, int nbase, int nch128, int pt) {
  const int l = pt & 63, pw = pt >> 6;
  const int rows = min(M - m_first, BM);  // this workgroup's x rows; the rest clamp to the last
  S.xr = __builtin_amdgcn_make_buffer_rsrc((void*)(x + (size_t)m_first * K), (short)0, rows * K * 2, kBufferDword3);
#pragma unroll
  for (int i = 0; i < GemmCfg<BM>::XP; i++) {
    const int row = min(32 * i + (pt >> 3), rows - 1);
    S.xo[i] = (row * K + 8 * (pt & 7)) * 2;
  }
  const int rb0 = nbase / 16, rb_last = W.N / 16 - 1;
  const int nrb = min(rb_last - rb0 + 1, kGemmBN / 16);  // this workgroup's block rows
  const int nch64 = nch128 * 2;
  S.cr = __builtin_amdgcn_make_buffer_rsrc((void*)(W.codes + ((size_t)rb0 * nch128 << 11)), (short)0,
                                           nrb * nch128 * 2048, kBufferDword3);
  S.tr = __builtin_amdgcn_make_buffer_rsrc((void*)(W.tptr + (size_t)rb0 * nch64), (short)0, (nrb * nch64 + 1) * 4,
                                           kBufferDword3);
  // entries: e0 + lane stays inside the list and its 64 slots of padding
  S.er = __builtin_amdgcn_make_buffer_rsrc((void*)W.tent, (short)0, 0x7fffffff, kBufferDword3);
  S.sr = __builtin_amdgcn_make_buffer_rsrc((void*)(W.scales + (size_t)rb0 * 16 * W.kg), (short)0,
                                           nrb * 16 * W.kg * 2, kBufferDword3);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    // block rows past N clamp to the last one and feed only outputs never stored
    const int rb = min(rb0 + 2 * pw + i, rb_last) - rb0;
    S.co[i] = rb * nch128 * 2048 + l * 16;
    S.to[i] = rb * nch64 * 4;
    S.so[i] = (rb * 16 + (l & 15)) * W.kg * 2;
  }
}

// Block pointers and bulk loads (x, codes, scales) of chunk c.
template <int BM, int PC>
__device__ __forceinline__ void gemm_load(GemmRegs<BM>& R, const GemmSrc<BM>& S, const QLMat& W, int c, int l) {
  typedef int int2v __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int2v p = __builtin_bit_cast(int2v, __builtin_amdgcn_raw_buffer_load_b64(S.tr, S.to[i], c * 4, 0));
    R.e0[i] = p.x;
    R.e1[i] = p.y;
  }
  __builtin_amdgcn_sched_barrier(0);  // block pointers ahead of the bulk loads: the entries wait only for them
  const int k0 = c * kGemmBK;
#pragma unroll
  for (int i = 0; i < GemmCfg<BM>::XP; i++)
    R.a[i] = __builtin_amdgcn_raw_buffer_load_b128(S.xr, S.xo[i], k0 * 2, 0);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    R.q[i] = __builtin_amdgcn_raw_buffer_load_b128(S.cr, S.co[i], ((c >> 1) << 11) + ((c & 1) << 10), 0);
    if (!PC) {
      const int k = k0 + 16 * (l >> 4);
      const int kb = W.gshift >= 0 ? (k >> W.gshift) : k / W.G;
      R.s[i] = __builtin_amdgcn_raw_buffer_load_b16(S.sr, S.so[i] + kb * 2, 0, 0);
    }
  }
}

// Outlier entries of the chunk whose block pointers R holds: lane j takes
// entry e0 + j of each block (lanes past the block's count ignore what they
// read).  Not earlier than called: the wait for the block pointers would also
// wait for the bulk loads issued after them (the empty asm keeps the first
// use of e0 behind the barrier that precedes this call).
template <int BM>
__device__ __forceinline__ void gemm_load_ent(GemmRegs<BM>& R, const GemmSrc<BM>& S, int l) {
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    int e0 = R.e0[i];
    asm volatile("" : "+v"(e0));
    R.ent[i] = __builtin_amdgcn_raw_buffer_load_b32(S.er, l * 4, __builtin_amdgcn_readfirstlane(e0) * 4, 0);
  }
  __builtin_amdgcn_sched_barrier(0);  // ahead of the next bulk loads: loads complete in issue order
}

// R -> one LDS stage: x pieces into the A tile, decoded weights into the B
// tile, then the outliers over them.  Lanes past a block's count write to the
// spare slot instead of branching.
template <int BM, int FMT, int PC, int DENSE>
__device__ __forceinline__ void gemm_stage(const GemmRegs<BM>& R, const GemmSrc<BM>& S, uint8_t* stage,
                                           uint8_t* spare, const half2v (&srow)[2], int pt) {
  uint8_t* As = stage;
  uint8_t* Bs = stage + GemmCfg<BM>::A_BYTES;
  const int l = pt & 63, pw = pt >> 6;
  const uint32_t xo = tile_off(pt >> 3, pt & 7);  // rows 32 i + pt / 8 share the permutation
#pragma unroll
  for (int i = 0; i < GemmCfg<BM>::XP; i++) *reinterpret_cast<u32x4*>(As + xo + i * 32 * 128) = R.a[i];
  const int g = l >> 4;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int n = 16 * (2 * pw + i) + (l & 15);
    const half2v s2 = PC ? srow[i] : scale2((uint16_t)R.s[i]);
    *reinterpret_cast<half8*>(Bs + tile_off(n, 2 * g)) = deq8<FMT>(R.q[i].x, R.q[i].y, s2);
    *reinterpret_cast<half8*>(Bs + tile_off(n, 2 * g + 1)) = deq8<FMT>(R.q[i].z, R.q[i].w, s2);
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    // entry: (fp16 value << 16) | r << 6 | k for row r of the block, column k of the chunk
    const int rbl = 2 * pw + i;
    auto at = [&](uint32_t e) {
      const int r = (int)((e >> 6) & 15), k = (int)(e & 63);
      return tile_off(16 * rbl + r, k >> 3) + ((k & 7) << 1);
    };
    const int cnt = R.e1[i] - R.e0[i];
    *reinterpret_cast<uint16_t*>(l < cnt ? Bs + at(R.ent[i]) : spare + 2 * l) = (uint16_t)(R.ent[i] >> 16);
    // blocks of more than 64 outliers (DENSE launches only): the rest from
    // memory, 64 per round.  Kept out of the common kernel: loads in a
    // data-dependent loop make every later wait in the chunk a full drain.
    if (DENSE) {
      const int e0 = __builtin_amdgcn_readfirstlane(R.e0[i]);
      const int ne = __builtin_amdgcn_readfirstlane(cnt);
      for (int j = 64 + l; j - l < ne; j += 64)
        if (j < ne) {
          const uint32_t e = __builtin_amdgcn_raw_buffer_load_b32(S.er, (e0 + j) * 4, 0, 0);
          *reinterpret_cast<uint16_t*>(Bs + at(e)) = (uint16_t)(e >> 16);
        }
    }
  }
}

template <int BM>
struct GemmFrags {
  half8 a[GemmCfg<BM>::MI];
  half8 b[2];
};

constexpr int kGemmConsumers = 8, kGemmThreads = 64 * (kGemmConsumers + 4);

template <int BM, int FMT, int PC, int DENSE>
__global__ __launch_bounds__(kGemmThreads, 1) void qlinear_gemm_kernel(QLArgs a) {
  typedef GemmCfg<BM> C;
  constexpr int MI = C::MI;
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * C::STAGE + 128];  // + the spare slot of gemm_stage
  uint8_t* const spare = lds + 3 * C::STAGE;

  // Output tiles of all matrices of the launch in one list (a.first[i]:
  // first tile of matrix i; within a matrix, tile = split part, then n-tile,
  // then M-band).  Workgroups go to the 8 XCDs in turn, so workgroup id
  // takes tile (id % 8) * per + id / 8: each XCD works through its own
  // contiguous run, all M-bands of a few n-tiles at a time, and their codes
  // and x rows stay in that XCD's L2.
  const int ntiles = a.first[a.count];
  const int per = (ntiles + 7) / 8;
  const int tile = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
  if (tile >= ntiles) return;
  int mi = 0;
#pragma unroll
  for (int j = 1; j < kMaxGroup; j++)
    if (j < a.count && tile >= a.first[j]) mi = j;
  const QLMat W = pick(a, mi);
  const int N = W.N;
  const int M = a.M, K = a.K;
  const int mbands = (M + BM - 1) / BM;
  const int per_split = ((N + kGemmBN - 1) / kGemmBN) * mbands;
  const int ks = (tile - a.first[mi]) / per_split;
  const int local = (tile - a.first[mi]) % per_split;
  const int nbase = (local / mbands) * kGemmBN;
  const int m_first = (local % mbands) * BM;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nch128 = K >> 7;
  const int nch_split = (K / kGemmBK) / a.split;  // even (the host checks)
  const int c_first = ks * nch_split, c_end = c_first + nch_split;
  auto next_stage = [](uint32_t s) { return s == 2 * C::STAGE ? 0u : s + C::STAGE; };

  if (wave >= kGemmConsumers) {
    // ---------------- producers
    const int pt = t - 64 * kGemmConsumers;
    GemmSrc<BM> S;
    gemm_src_init<BM>(S, W, a.x, M, K, m_first, nbase, nch128, pt);
    half2v srow[2];  // per-channel scales of this thread's code rows
#pragma unroll
    for (int i = 0; i < 2; i++)
      srow[i] = scale2(PC ? (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(S.sr, S.so[i], 0, 0) : (uint16_t)0);
    // prologue: chunks c_first, c_first + 1 staged; their successors loading
    GemmRegs<BM> R0, R1;
    gemm_load<BM, PC>(R0, S, W, c_first, lane);
    gemm_load<BM, PC>(R1, S, W, c_first + 1, lane);
    gemm_load_ent<BM>(R0, S, lane);
    gemm_load_ent<BM>(R1, S, lane);
    gemm_stage<BM, FMT, PC, DENSE>(R0, S, lds, spare, srow, pt);
    gemm_load<BM, PC>(R0, S, W, min(c_first + 2, c_end - 1), lane);
    gemm_stage<BM, FMT, PC, DENSE>(R1, S, lds + C::STAGE, spare, srow, pt);
    gemm_load<BM, PC>(R1, S, W, min(c_first + 3, c_end - 1), lane);
    gemm_load_ent<BM>(R0, S, lane);
    __syncthreads();
    uint32_t cur = 0;  // stage of chunk c, in bytes
    // chunk c: R holds chunk c + 2 (to stage), Ro chunk c + 3 (entries to
    // load).  Staging is unconditional: past the last chunk it rewrites a
    // stage no later k-step reads, with the clamped chunk's data.
    auto body = [&](int c, GemmRegs<BM>& R, GemmRegs<BM>& Ro) {
      const uint32_t stg = next_stage(next_stage(cur));
      gemm_load_ent<BM>(Ro, S, lane);
      gemm_stage<BM, FMT, PC, DENSE>(R, S, lds + stg, spare, srow, pt);
      gemm_load<BM, PC>(R, S, W, min(c + 4, c_end - 1), lane);
      __syncthreads();
      cur = next_stage(cur);
    };
    for (int c = c_first; c < c_end; c += 2) {
      body(c, R0, R1);
      body(c + 1, R1, R0);
    }
    return;
  }

  // ---------------- consumers
  const int wm = wave >> 1, wn = wave & 1;
  // fragment addresses: lane l reads row (l % 32) of a 32-row group, piece
  // 2 s + l / 32 for k-step s; the permutation depends on the row only
  // through (l % 32), so one offset per k-step serves every fragment
  uint32_t foff[4];
#pragma unroll
  for (int s = 0; s < 4; s++) foff[s] = tile_off(lane & 31, 2 * s + (lane >> 5));
  const uint32_t a_row0 = (uint32_t)(wm * C::WM) * 128, b_row0 = C::A_BYTES + (uint32_t)(wn * 64) * 128;

  float16v acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (float16v)0.0f;

  auto read_frags = [&](GemmFrags<BM>& F, uint32_t stage, int s) {
    const uint8_t* p = lds + stage + foff[s];
#pragma unroll
    for (int i = 0; i < MI; i++) F.a[i] = *reinterpret_cast<const half8*>(p + a_row0 + i * 32 * 128);
#pragma unroll
    for (int j = 0; j < 2; j++) F.b[j] = *reinterpret_cast<const half8*>(p + b_row0 + j * 32 * 128);
  };
  auto mma = [&](const GemmFrags<BM>& F) {
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(F.a[i], F.b[j], acc[i][j], 0, 0, 0);
  };

  __syncthreads();  // the producers' prologue
  // F[s] holds k-step s of a chunk: read two k-steps ahead; the first two
  // k-steps of chunk c + 1 are read during chunk c, whose last barrier made
  // them visible
  GemmFrags<BM> F[4];
  read_frags(F[0], 0, 0);
  read_frags(F[1], 0, 1);
  uint32_t cur = 0;
  // (the scheduling barriers keep each read group two k-steps ahead of its
  // MFMAs; left alone, the compiler sinks the reads next to their use)
  for (int c = c_first; c < c_end; c++) {
    const uint32_t nxt = next_stage(cur);
    read_frags(F[2], cur, 2);
    __builtin_amdgcn_sched_barrier(0);
    mma(F[0]);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(F[3], cur, 3);
    __builtin_amdgcn_sched_barrier(0);
    mma(F[1]);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(F[0], nxt, 0);
    __builtin_amdgcn_sched_barrier(0);
    mma(F[2]);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(F[1], nxt, 1);
    __builtin_amdgcn_sched_barrier(0);
    mma(F[3]);
    // The barrier needs this chunk's reads done (the producers overwrite
    // its stage next), not the reads of chunk c + 1 just issued: wait for
    // all but the newest 2 (MI + 2) LDS operations, instead of the full
    // drain a fenced barrier would do.  The memory clobber keeps every LDS
    // access on its side of the barrier.
    static_assert(2 * (MI + 2) <= 15, "lgkmcnt field");
    asm volatile("s_waitcnt lgkmcnt(%0)\n\ts_barrier" ::"n"(2 * (MI + 2)) : "memory");
    cur = nxt;
  }

  // C layout (32x32): lane l, element e -> row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
  const int hi = lane >> 5, lc = lane & 31;
  if (a.split > 1) {
    // partial sums of this part of K, no bias
    float* part = W.part + (size_t)ks * M * N;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = nbase + wn * 64 + j * 32 + lc;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int m = m_first + wm * C::WM + i * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
          if (m < M) part[(size_t)m * N + n] = acc[i][j][e];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = nbase + wn * 64 + j * 32 + lc;
    if (n >= N) continue;
    const float bv = W.bias ? (float)bits_to_h(W.bias[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m_first + wm * C::WM + i * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
        if (m < M) W.y[(size_t)m * N + n] = h_to_bits(rn_h(acc[i][j][e] + bv));
      }
  }
}

// ------------------------------------------------ GEMM, 256 x 256 tiles
//
// For grids with at least one 256 x 256 output tile per CU (the MLP
// projections of a prefill): half the LDS traffic per flop of the 256 x 128
// kernel above, which is what bounds it.  8 waves, each computing a 128 x 64
// tile (2 x 4 layout) and each also staging a share of the next chunk; two
// LDS stages, one barrier per chunk.  Per chunk c a wave reads the fragments
// of chunk c one k-step ahead of its MFMAs and fills its share of the other
// stage with chunk c + 1: the x pieces by direct-to-LDS loads (buffer_load
// ... lds, 1 KiB per wave and instruction, each lane's source piece chosen so
// the data lands in tile_off's layout: no registers, no LDS write
// instructions), the decoded weights and their outlier patches from
// registers loaded a chunk earlier; it then reloads those registers with
// chunk c + 2, loads that stay in flight across the barrier.  With two
// stages the first fragments of a chunk are read after its barrier; each
// wave then has 32 MFMAs (1024 cycles of the SIMD's matrix unit per wave
// pair) to hide them.

struct WideRegs {
  u32x4 q[2];      // codes of the wave's two block rows
  uint32_t s[2];   // their scales (block-wise scales only)
  int e0[2], e1[2];
  uint32_t ent[2];
};

struct WideSrc {
  __amdgpu_buffer_rsrc_t xr, cr, tr, er, sr;
  uint32_t xo[4];  // byte offsets of this lane's 4 x pieces of chunk 0 (direct-to-LDS loads)
  int co[2], to[2], so[2];
};

constexpr int kWideBM = 256, kWideBN = 256;
constexpr int kWideA = kWideBM * 128, kWideStage = kWideA + kWideBN * 128;

__device__ __forceinline__ void wide_src_init(WideSrc& S, const QLMat& W, const uint16_t* x, int M, int K,
                                              int m_first, int nbase, int nch128, int t) {
  const int l = t & 63, w = t >> 6;
  const int rows = min(M - m_first, kWideBM);
  // x rows past M lie past the end of this range: their pieces read as zero
  S.xr = __builtin_amdgcn_make_buffer_rsrc((void*)(x + (size_t)m_first * K), (short)0, rows * K * 2, kBufferDword3);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // direct load i of wave w fills A-tile bytes (4 w + i) KiB + 16 l: row
    // 8 (4 w + i) + l / 8, stored piece l % 8, which tile_off assigns the
    // logical piece (l % 8) ^ (row & 7) ^ ((row >> 3) & 1)
    const int row = 8 * (4 * w + i) + (l >> 3);
    const int piece = (l & 7) ^ (row & 7) ^ ((row >> 3) & 1);
    S.xo[i] = (uint32_t)(row * K + 8 * piece) * 2;
  }
  const int rb0 = nbase / 16, rb_last = W.N / 16 - 1;
  const int nrb = min(rb_last - rb0 + 1, kWideBN / 16);
  const int nch64 = nch128 * 2;
  S.cr = __builtin_amdgcn_make_buffer_rsrc((void*)(W.codes + ((size_t)rb0 * nch128 << 11)), (short)0,
                                           nrb * nch128 * 2048, kBufferDword3);
  S.tr = __builtin_amdgcn_make_buffer_rsrc((void*)(W.tptr + (size_t)rb0 * nch64), (short)0, (nrb * nch64 + 1) * 4,
                                           kBufferDword3);
  S.er = __builtin_amdgcn_make_buffer_rsrc((void*)W.tent, (short)0, 0x7fffffff, kBufferDword3);
  S.sr = __builtin_amdgcn_make_buffer_rsrc((void*)(W.scales + (size_t)rb0 * 16 * W.kg), (short)0,
                                           nrb * 16 * W.kg * 2, kBufferDword3);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int rb = min(rb0 + 2 * w + i, rb_last) - rb0;
    S.co[i] = rb * nch128 * 2048 + l * 16;
    S.to[i] = rb * nch64 * 4;
    S.so[i] = (rb * 16 + (l & 15)) * W.kg * 2;
  }
}

template <int PC>
__device__ __forceinline__ void wide_load(WideRegs& R, const WideSrc& S, const QLMat& W, int c, int l) {
  typedef int int2v __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int2v p = __builtin_bit_cast(int2v, __builtin_amdgcn_raw_buffer_load_b64(S.tr, S.to[i], c * 4, 0));
    R.e0[i] = p.x;
    R.e1[i] = p.y;
  }
  __builtin_amdgcn_sched_barrier(0);
  const int k0 = c * kGemmBK;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    R.q[i] = __builtin_amdgcn_raw_buffer_load_b128(S.cr, S.co[i], ((c >> 1) << 11) + ((c & 1) << 10), 0);
    if (!PC) {
      const int k = k0 + 16 * (l >> 4);
      const int kb = W.gshift >= 0 ? (k >> W.gshift) : k / W.G;
      R.s[i] = __builtin_amdgcn_raw_buffer_load_b16(S.sr, S.so[i] + kb * 2, 0, 0);
    }
  }
}

// Chunk c's x straight into a stage's A tile: 4 direct-to-LDS loads of 1 KiB
// per wave, no registers and no LDS write instructions.
__device__ __forceinline__ void wide_load_x(const WideSrc& S, uint8_t* stage, int c, int w) {
#pragma unroll
  for (int i = 0; i < 4; i++)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(S.xr, (void*)(stage + (4 * w + i) * 1024), 16, S.xo[i], c * kGemmBK * 2,
                                             0, 0);
}

__device__ __forceinline__ void wide_load_ent(WideRegs& R, const WideSrc& S, int l) {
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    int e0 = R.e0[i];
    asm volatile("" : "+v"(e0));
    R.ent[i] = __builtin_amdgcn_raw_buffer_load_b32(S.er, l * 4, __builtin_amdgcn_readfirstlane(e0) * 4, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int FMT, int PC, int DENSE>
__device__ __forceinline__ void wide_stage(const WideRegs& R, const WideSrc& S, uint8_t* stage, uint8_t* spare,
                                           const half2v (&srow)[2], int t) {
  uint8_t* Bs = stage + kWideA;
  const int l = t & 63, w = t >> 6, g = l >> 4;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int n = 16 * (2 * w + i) + (l & 15);
    const half2v s2 = PC ? srow[i] : scale2((uint16_t)R.s[i]);
    *reinterpret_cast<half8*>(Bs + tile_off(n, 2 * g)) = deq8<FMT>(R.q[i].x, R.q[i].y, s2);
    *reinterpret_cast<half8*>(Bs + tile_off(n, 2 * g + 1)) = deq8<FMT>(R.q[i].z, R.q[i].w, s2);
  }
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int rbl = 2 * w + i;
    auto at = [&](uint32_t e) {
      const int r = (int)((e >> 6) & 15), k = (int)(e & 63);
      return tile_off(16 * rbl + r, k >> 3) + ((k & 7) << 1);
    };
    const int cnt = R.e1[i] - R.e0[i];
    *reinterpret_cast<uint16_t*>(l < cnt ? Bs + at(R.ent[i]) : spare + 2 * l) = (uint16_t)(R.ent[i] >> 16);
    if (DENSE) {
      const int e0 = __builtin_amdgcn_readfirstlane(R.e0[i]);
      const int ne = __builtin_amdgcn_readfirstlane(cnt);
      for (int j = 64 + l; j - l < ne; j += 64)
        if (j < ne) {
          const uint32_t e = __builtin_amdgcn_raw_buffer_load_b32(S.er, (e0 + j) * 4, 0, 0);
          *reinterpret_cast<uint16_t*>(Bs + at(e)) = (uint16_t)(e >> 16);
        }
    }
  }
}

template <int FMT, int PC, int DENSE>
__global__ __launch_bounds__(512, 1) void qlinear_gemm_wide_kernel(QLArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kWideStage + 128];
  uint8_t* const spare = lds + 2 * kWideStage;

  // tiles: as in qlinear_gemm_kernel, with 256-column n-tiles.  With a tail
  // (unsplit grids only), the last `tail` tiles of each XCD's run come as
  // two work units each, one per half of K (a work unit past the others:
  // `half` 0 or 1, partial sums into a.tpart slot `tslot`)
  const int ntiles = a.first[a.count];
  const int per = a.tail ? a.per : (ntiles + 7) / 8;
  const int xcd = (int)(blockIdx.x % 8), unit = (int)(blockIdx.x / 8);
  int tile = xcd * per + unit, half = -1, tslot = 0;
  if (a.tail && unit >= per - a.tail) {
    const int v = unit - (per - a.tail);
    tile = xcd * per + per - a.tail + (v >> 1);
    half = v & 1;
    tslot = xcd * a.tail + (v >> 1);
  }
  if (tile >= ntiles) return;
  int mi = 0;
#pragma unroll
  for (int j = 1; j < kMaxGroup; j++)
    if (j < a.count && tile >= a.first[j]) mi = j;
  const QLMat W = pick(a, mi);
  const int N = W.N;
  const int M = a.M, K = a.K;
  const int mbands = (M + kWideBM - 1) / kWideBM;
  const int per_split = ((N + kWideBN - 1) / kWideBN) * mbands;
  const int ks = (tile - a.first[mi]) / per_split;
  const int local = (tile - a.first[mi]) % per_split;
  const int nbase = (local / mbands) * kWideBN;
  const int m_first = (local % mbands) * kWideBM;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int nch128 = K >> 7;
  int nch_split = (K / kGemmBK) / a.split;
  int c_first = ks * nch_split, c_end = c_first + nch_split;
  if (half >= 0) {  // a tail unit: one half of K
    nch_split = (K / kGemmBK) / 2;
    c_first = half * nch_split;
    c_end = c_first + nch_split;
  }

  WideSrc S;
  wide_src_init(S, W, a.x, M, K, m_first, nbase, nch128, t);
  half2v srow[2];
#pragma unroll
  for (int i = 0; i < 2; i++)
    srow[i] = scale2(PC ? (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(S.sr, S.so[i], 0, 0) : (uint16_t)0);

  const int wm = wave >> 2, wn = wave & 3;
  uint32_t foff[4];
#pragma unroll
  for (int s = 0; s < 4; s++) foff[s] = tile_off(lane & 31, 2 * s + (lane >> 5));
  const uint32_t a_row0 = (uint32_t)(wm * 128) * 128, b_row0 = kWideA + (uint32_t)(wn * 64) * 128;

  float16v acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (float16v)0.0f;
  struct Frags {
    half8 a[4];
    half8 b[2];
  };
  auto read_frags = [&](Frags& F, uint32_t stage, int s) {
    const uint8_t* p = lds + stage + foff[s];
#pragma unroll
    for (int i = 0; i < 4; i++) F.a[i] = *reinterpret_cast<const half8*>(p + a_row0 + i * 32 * 128);
#pragma unroll
    for (int j = 0; j < 2; j++) F.b[j] = *reinterpret_cast<const half8*>(p + b_row0 + j * 32 * 128);
  };
  auto mma = [&](const Frags& F) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(F.a[i], F.b[j], acc[i][j], 0, 0, 0);
  };

  // The barrier at the end of each chunk waits for the stage just written
  // (its direct x loads and this wave's LDS writes) but not for the weight
  // loads issued after them (2 block pointers + 2 code pieces, + 2 scales
  // for block-wise scales), which stay in flight into the next chunk.
#define AQ_WIDE_BARRIER() \
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(PC ? 4 : 6) : "memory")
  // prologue: chunk c_first staged, chunk c_first + 1's weights loading
  WideRegs R;
  wide_load_x(S, lds, c_first, wave);
  wide_load<PC>(R, S, W, c_first, lane);
  wide_load_ent(R, S, lane);
  wide_stage<FMT, PC, DENSE>(R, S, lds, spare, srow, t);
  wide_load<PC>(R, S, W, min(c_first + 1, c_end - 1), lane);
  AQ_WIDE_BARRIER();

  Frags F0, F1;
  uint32_t cur = 0;
  for (int c = c_first; c < c_end; c++) {
    const uint32_t oth = cur ^ kWideStage;
    // chunk c + 1's x into the other stage (its last reads were before the
    // previous barrier); past the last chunk, a harmless reload
    wide_load_x(S, lds + oth, min(c + 1, c_end - 1), wave);
    wide_load_ent(R, S, lane);  // entries of chunk c + 1
    read_frags(F0, cur, 0);
    read_frags(F1, cur, 1);
    __builtin_amdgcn_sched_barrier(0);
    mma(F0);
    __builtin_amdgcn_sched_barrier(0);
    // chunk c + 1 into the other stage (last read in chunk c - 1, before
    // the previous barrier); past the last chunk, a harmless rewrite
    wide_stage<FMT, PC, DENSE>(R, S, lds + oth, spare, srow, t);
    wide_load<PC>(R, S, W, min(c + 2, c_end - 1), lane);
    read_frags(F0, cur, 2);
    __builtin_amdgcn_sched_barrier(0);
    mma(F1);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(F1, cur, 3);
    __builtin_amdgcn_sched_barrier(0);
    mma(F0);
    __builtin_amdgcn_sched_barrier(0);
    mma(F1);
    AQ_WIDE_BARRIER();
    cur = oth;
  }
#undef AQ_WIDE_BARRIER

  const int hi = lane >> 5, lc = lane & 31;
  if (half >= 0) {
    // the tile's fp32 partial sums over this half of K: slot tslot, half,
    // row-major 256 x 256 (tail_reduce_kernel adds the halves)
    float* tp = a.tpart + ((size_t)tslot * 2 + half) * kWideBM * kWideBN;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int nl = wn * 64 + j * 32 + lc;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int ml = wm * 128 + i * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
          tp[ml * kWideBN + nl] = acc[i][j][e];
        }
    }
    return;
  }
  if (a.split > 1) {
    float* part = W.part + (size_t)ks * M * N;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int n = nbase + wn * 64 + j * 32 + lc;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int m = m_first + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
          if (m < M) part[(size_t)m * N + n] = acc[i][j][e];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = nbase + wn * 64 + j * 32 + lc;
    if (n >= N) continue;
    const float bv = W.bias ? (float)bits_to_h(W.bias[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m_first + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
        if (m < M) W.y[(size_t)m * N + n] = h_to_bits(rn_h(acc[i][j][e] + bv));
      }
  }
}

// y = fp16(sum of the split partial sums in order + bias), 4 outputs per
// thread (N is a multiple of 16).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* part, int64_t mn, int split, int N,
                                                            const uint16_t* bias, uint16_t* y) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= mn) return;
  float4v v = *reinterpret_cast<const float4v*>(part + i);
  for (int s = 1; s < split; s++) v += *reinterpret_cast<const float4v*>(part + (size_t)s * mn + i);
  const int n = (int)(i % N);
  uint16_t o[4];
#pragma unroll
  for (int j = 0; j < 4; j++) o[j] = h_to_bits(rn_h(v[j] + (bias ? (float)bits_to_h(bias[n + j]) : 0.0f)));
  *reinterpret_cast<uint2*>(y + i) = make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
}

// The tail tiles of a 256 x 256 GEMM (qlinear_gemm_wide_kernel with
// a.tail): y = fp16(half 0 + half 1 + bias) over each tile's rows < M and
// columns < N, the halves added in order.  Workgroup (tile slot, row band of
// 16): 256 threads x 4 columns x 4 rows.
__global__ __launch_bounds__(256) void tail_reduce_kernel(QLArgs a) {
  const int ntiles = a.first[a.count];
  const int slot = blockIdx.x, xcd = slot / a.tail, r = slot % a.tail;
  const int tile = xcd * a.per + a.per - a.tail + r;
  if (tile >= ntiles) return;
  int mi = 0;
#pragma unroll
  for (int j = 1; j < kMaxGroup; j++)
    if (j < a.count && tile >= a.first[j]) mi = j;
  const QLMat W = pick(a, mi);
  const int N = W.N, M = a.M;
  const int mbands = (M + kWideBM - 1) / kWideBM;
  const int local = tile - a.first[mi];
  const int nbase = (local / mbands) * kWideBN, m_first = (local % mbands) * kWideBM;
  const float* p0 = a.tpart + (size_t)slot * 2 * kWideBM * kWideBN;
  const float* p1 = p0 + kWideBM * kWideBN;
  const int nl = (threadIdx.x & 63) * 4;
  const int n = nbase + nl;
  if (n >= N) return;  // N is a multiple of 16: a group of 4 columns is all in or all out
  float bv[4];
#pragma unroll
  for (int c = 0; c < 4; c++) bv[c] = W.bias ? (float)bits_to_h(W.bias[n + c]) : 0.0f;
  for (int ml = (int)blockIdx.y * 16 + (threadIdx.x >> 6); ml < (int)blockIdx.y * 16 + 16; ml += 4) {
    const int m = m_first + ml;
    if (m >= M) break;
    const float4v u = *reinterpret_cast<const float4v*>(p0 + ml * kWideBN + nl);
    const float4v v = *reinterpret_cast<const float4v*>(p1 + ml * kWideBN + nl);
    uint16_t o[4];
#pragma unroll
    for (int c = 0; c < 4; c++) o[c] = h_to_bits(rn_h(u[c] + v[c] + bv[c]));
    *reinterpret_cast<uint2*>(W.y + (size_t)m * N + n) =
        make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
  }
}

// CU count of the current device, read once per device.  Any host thread
// may call this: each slot is an atomic written with the same value by
// whichever thread gets there first.
int log2_exact(int64_t g) {
  if (g <= 0 || (g & (g - 1))) return -1;
  int s = 0;
  while ((int64_t(1) << s) < g) s++;
  return s;
}

// GEMV launches take their matrix from blockIdx.y: the group's matrices are
// cut into pieces of at most P tile rows, one grid row per piece, with P a
// multiple of `unit` (the tile rows of one workgroup) chosen so that at most
// kMaxPieces pieces leave the fewest workgroups idle (the grid is as wide as
// the longest piece).  Returns the grid; *g gets the pieces.
dim3 gemv_pieces(const QLArgs& a, int unit, QLArgs* g) {
  const int64_t nch = a.K >> 7;
  int rmax = 0;
  for (int i = 0; i < a.count; i++) rmax = std::max(rmax, a.mat[i].N / 16);
  int P = 0;
  int64_t best = INT64_MAX;
  // d = 1 always fits: a group holds at most kMaxGroup <= kMaxPieces matrices
  for (int d = 1; d <= kMaxPieces; d++) {
    const int p = (int)(aq::ceil_div(aq::ceil_div(rmax, d), unit) * unit);
    int n = 0;
    for (int i = 0; i < a.count; i++) n += (int)aq::ceil_div(a.mat[i].N / 16, p);
    const int64_t idle_and_busy = aq::ceil_div(p, unit) * (int64_t)n;
    if (n <= kMaxPieces && idle_and_busy < best) {
      best = idle_and_busy;
      P = p;
    }
  }
  *g = a;
  int n = 0;
  for (int i = 0; i < a.count; i++) {
    const QLMat& w = a.mat[i];
    for (int r0 = 0; r0 < w.N / 16; r0 += P) {
      QLMat& q = g->mat[n++];
      const int row0 = 16 * r0;
      q = w;
      q.codes = w.codes + ((size_t)r0 * nch << 11);
      q.scales = w.scales + (size_t)row0 * w.kg;
      q.row_ptr = w.row_ptr + row0;
      q.bias = w.bias ? w.bias + row0 : nullptr;
      q.res = w.res ? w.res + row0 : nullptr;
      q.tptr = w.tptr ? w.tptr + (size_t)r0 * (nch * 2) : nullptr;  // blocks of 16 x 64: 2 per chunk
      q.y = w.y + row0;
      q.N = 16 * std::min(P, w.N / 16 - r0);
      q.ldy = w.N;
    }
  }
  g->count = n;
  return dim3((unsigned)aq::ceil_div(P, unit), (unsigned)n);
}

// Block-wise scales with blocks of a power of two of at least 128: a
// 128-column chunk lies inside one block, so the GEMVs load one scale per
// row and chunk (scale mode 2) instead of one per 64 columns.
bool chunk_scales(const QLArgs& a) {
  for (int i = 0; i < a.count; i++)
    if (a.mat[i].kg == 1 || a.mat[i].gshift < 7) return false;
  return true;
}

template <int NS, int FMT>
hipError_t launch_gemv(const QLArgs& a, bool per_channel, hipStream_t s) {
  // decode (M = 1) with x small enough: x in LDS (dynamic size), read by
  // every wave from there instead of by 4 loads per chunk and lane of which
  // 60 of 64 lanes are out of range (each load instruction occupies the
  // CU's address unit the same time: on short matrices, whose 8 waves per
  // tile row issue all their loads at once, those loads were the start-up
  // queue).  Decode gets instances for one row of x (no registers or loads
  // for more).
  const bool x1 = a.M == 1 && a.K <= kGemvX1MaxK;
  const size_t lds = x1 ? (size_t)a.K * 2 + 64 : 0;
  constexpr int R = kGemvDirectMaxM;
  QLArgs p;
  const dim3 g = gemv_pieces(a, 1, &p), b(64 * NS);
  bool fused = a.pro != kProNone;
  for (int i = 0; i < a.count; i++) fused = fused || a.mat[i].res || a.mat[i].act;
  if (fused) {  // aq_qlinear_decode: M = 1 and K within the x-in-LDS limit, checked there
    if (per_channel)
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 1, 2, 1>), g, b, lds, s, p);
    else
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 0, 2, 1>), g, b, lds, s, p);
    return hipGetLastError();
  }
  if (per_channel) {
    if (x1)
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 1, 1, 1>), g, b, lds, s, p);
    else if (a.M == 1)
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 1, 0, 1>), g, b, 0, s, p);
    else
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 1, 0, R>), g, b, 0, s, p);
  } else if (chunk_scales(a)) {
    if (x1)
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 2, 1, 1>), g, b, lds, s, p);
    else if (a.M == 1)
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 2, 0, 1>), g, b, 0, s, p);
    else
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 2, 0, R>), g, b, 0, s, p);
  } else {
    if (x1)
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 0, 1, 1>), g, b, lds, s, p);
    else if (a.M == 1)
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 0, 0, 1>), g, b, 0, s, p);
    else
      hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 0, 0, R>), g, b, 0, s, p);
  }
  return hipGetLastError();
}

template <int NS>
hipError_t launch_gemv(const QLArgs& a, int fmt, bool per_channel, hipStream_t s) {
  return fmt == AQ_FMT_E4M3 ? launch_gemv<NS, AQ_FMT_E4M3>(a, per_channel, s)
                            : launch_gemv<NS, AQ_FMT_INT8>(a, per_channel, s);
}

template <int FMT, int MG, int S, int XH>
hipError_t launch_gemv_x(const QLArgs& a, bool per_channel, hipStream_t s) {
  QLArgs p;
  // workgroups of 8 / S tile rows; a SwiGLU pair: 4 / S of each member, and
  // the grid's rows over gate's pieces only (up's follow them in p.mat)
  const bool pair = a.mat[0].act == 2;
  dim3 g = gemv_pieces(a, pair ? kXWaves / S / 2 : kXWaves / S, &p);
  p.pair = 0;
  if (pair) {
    p.pair = (int)g.y / 2;
    g.y = (unsigned)p.pair;
    for (int i = 0; i < p.count; i++) p.mat[i].act = 0;
  }
  // Every member's block lists given: the MFMA outlier path, except with 3
  // or 4 row groups of x at S = 2, where the gathers (one per row group and
  // entry) cost more than the CSR walk of a wave shared by only two
  // (measured on the Mistral-7B / Llama-3-8B shapes: gate+up at M = 64 52 against 43 us;
  // down at M = 8 18 against 31 us, q/k/v 10 against 12 us)
  if constexpr (S >= 4 || MG <= 2) {
    bool lists = true;
    for (int i = 0; i < a.count; i++) lists = lists && a.mat[i].tptr && a.mat[i].tent;
    if (lists) {
      if (per_channel)
        hipLaunchKernelGGL((qlinear_gemv_x_kernel<FMT, 1, MG, S, 1, XH>), g, dim3(64 * kXWaves), 0, s, p);
      else if (chunk_scales(a))
        hipLaunchKernelGGL((qlinear_gemv_x_kernel<FMT, 2, MG, S, 1, XH>), g, dim3(64 * kXWaves), 0, s, p);
      else
        hipLaunchKernelGGL((qlinear_gemv_x_kernel<FMT, 0, MG, S, 1, XH>), g, dim3(64 * kXWaves), 0, s, p);
      return hipGetLastError();
    }
  }
  if (per_channel)
    hipLaunchKernelGGL((qlinear_gemv_x_kernel<FMT, 1, MG, S, 0, XH>), g, dim3(64 * kXWaves), 0, s, p);
  else if (chunk_scales(a))
    hipLaunchKernelGGL((qlinear_gemv_x_kernel<FMT, 2, MG, S, 0, XH>), g, dim3(64 * kXWaves), 0, s, p);
  else
    hipLaunchKernelGGL((qlinear_gemv_x_kernel<FMT, 0, MG, S, 0, XH>), g, dim3(64 * kXWaves), 0, s, p);
  return hipGetLastError();
}

template <int MG, int S, int XH = 16 * MG>
hipError_t launch_gemv_x(const QLArgs& a, int fmt, bool per_channel, hipStream_t s) {
  return fmt == AQ_FMT_E4M3 ? launch_gemv_x<AQ_FMT_E4M3, MG, S, XH>(a, per_channel, s)
                            : launch_gemv_x<AQ_FMT_INT8, MG, S, XH>(a, per_channel, s);
}

// 6 <= M <= 64: x row groups of 16 per MFMA (MG = 1, 2, 3 or 4 for M up to 16, 32, 48, 64),
// S = 2 or 4 waves per tile row
hipError_t launch_gemv_x(const QLArgs& a, int fmt, bool per_channel, int S, hipStream_t s) {
  // up to 8 rows with 4 or 8 waves per tile row: 8 staged rows of x, half
  // the x loads and LDS stores of a 16-row group
  if (a.M <= 8 && S >= 4)
    return S == 4 ? launch_gemv_x<1, 4, 8>(a, fmt, per_channel, s) : launch_gemv_x<1, 8, 8>(a, fmt, per_channel, s);
  if (a.M <= 16)
    return S == 2 ? launch_gemv_x<1, 2>(a, fmt, per_channel, s)
           : S == 4 ? launch_gemv_x<1, 4>(a, fmt, per_channel, s) : launch_gemv_x<1, 8>(a, fmt, per_channel, s);
  if (a.M <= 32)
    return S == 2 ? launch_gemv_x<2, 2>(a, fmt, per_channel, s)
           : S == 4 ? launch_gemv_x<2, 4>(a, fmt, per_channel, s) : launch_gemv_x<2, 8>(a, fmt, per_channel, s);
  if (a.M <= 48)
    return S == 2 ? launch_gemv_x<3, 2>(a, fmt, per_channel, s) : launch_gemv_x<3, 4>(a, fmt, per_channel, s);
  return S == 2 ? launch_gemv_x<4, 2>(a, fmt, per_channel, s) : launch_gemv_x<4, 4>(a, fmt, per_channel, s);
}

template <int BM, int FMT, int DENSE>
hipError_t launch_gemm(QLArgs a, bool per_channel, hipStream_t s) {
  // a.first: first output tile of each matrix (see the kernel)
  const int mbands = (int)aq::ceil_div(a.M, BM);
  int ntiles = 0;
  for (int i = 0; i < a.count; i++) {
    a.first[i] = ntiles;
    ntiles += (int)aq::ceil_div(a.mat[i].N, kGemmBN) * mbands * a.split;
  }
  for (int i = a.count; i <= kMaxGroup; i++) a.first[i] = ntiles;
  const dim3 grid((unsigned)(8 * aq::ceil_div(ntiles, 8)));
  if (per_channel)
    hipLaunchKernelGGL((qlinear_gemm_kernel<BM, FMT, 1, DENSE>), grid, dim3(kGemmThreads), 0, s, a);
  else
    hipLaunchKernelGGL((qlinear_gemm_kernel<BM, FMT, 0, DENSE>), grid, dim3(kGemmThreads), 0, s, a);
  return hipGetLastError();
}

template <int BM>
hipError_t launch_gemm(const QLArgs& a, int fmt, bool per_channel, bool dense, hipStream_t s) {
  if (dense)
    return fmt == AQ_FMT_E4M3 ? launch_gemm<BM, AQ_FMT_E4M3, 1>(a, per_channel, s)
                              : launch_gemm<BM, AQ_FMT_INT8, 1>(a, per_channel, s);
  return fmt == AQ_FMT_E4M3 ? launch_gemm<BM, AQ_FMT_E4M3, 0>(a, per_channel, s)
                            : launch_gemm<BM, AQ_FMT_INT8, 0>(a, per_channel, s);
}

// GEMM shapes: 256 x 256 tiles (qlinear_gemm_wide_kernel, one workgroup of
// 8 waves per CU), 256 x 128 or 128 x 128 tiles (qlinear_gemm_kernel, one
// workgroup per CU: three LDS stages of 144 or 96 KiB).
enum { kTile256x128 = 0, kTile128x128 = 1, kTile256x256 = 2 };
struct GemmPlan {
  int tile;
  int split;
};

// The tile shape and K split of a GEMM launch, chosen by an estimate of its
// time in microseconds: a fixed cost per launch, the rounds of the grid over
// the CUs times the 64-wide K chunks per work unit times the time one CU
// takes for one chunk of that tile (measured with every CU busy on the
// Llama-3-8B shapes at M = 512 and 2048: 1.8 us for 256 x 256, 1.17 for
// 256 x 128, 0.74 for 128 x 128), plus the split-K reduction's traffic
// (4 split + 2 bytes per output at an effective 4 TB/s, launch included).
// On those shapes (single and grouped, M = 512 and 2048) its pick comes
// within 4 % of the fastest of all 24 tile / split combinations measured;
// e.g. down_proj at M = 2048 takes 256 x 256 tiles split two ways (235 us
// against 265 unsplit with 256 x 128 tiles) and grouped q/k/v at M = 2048
// 256 x 256 tiles unsplit on 192 of the CUs (110 against 153 us with 384
// tiles of 256 x 128).  Splits need an even number of chunks per part and at
// least 4; max_split bounds the split (the caller's workspace).
GemmPlan plan_gemm(int64_t M, const int64_t* Ns, int64_t count, int64_t K, int max_split) {
  struct Shape {
    int tile, bm, bn;
    double chunk_us;
  };
  static constexpr Shape kShapes[] = {{kTile256x256, kWideBM, kWideBN, 1.8},
                                      {kTile256x128, 256, kGemmBN, 1.17},
                                      {kTile128x128, 128, kGemmBN, 0.74}};
  const int64_t slots = aq::cu_count();
  const int64_t nch = K / kGemmBK;
  int64_t outs = 0;
  for (int i = 0; i < count; i++) outs += M * Ns[i];
  GemmPlan best{kTile256x256, 1};
  double best_us = 0.0;
  for (const Shape& sh : kShapes) {
    int64_t tiles = 0;
    for (int i = 0; i < count; i++) tiles += aq::ceil_div(M, sh.bm) * aq::ceil_div(Ns[i], sh.bn);
    for (int sp = 1; sp <= 8 && sp <= max_split; sp *= 2) {
      if (sp > 1 && (nch % (2 * sp) != 0 || nch / sp < 4)) break;
      const double us = 15.0 + (double)aq::ceil_div(tiles * sp, slots) * (double)(nch / sp) * sh.chunk_us +
                        (sp > 1 ? (double)(4 * sp + 2) * (double)outs / 4e6 : 0.0);
      if (best_us == 0.0 || us < best_us) {
        best = GemmPlan{sh.tile, sp};
        best_us = us;
      }
    }
  }
  return best;
}

// The tail of an unsplit 256 x 256 grid (tiles dealt to the 8 XCDs in runs
// of `per`): when each XCD's last round holds at most half its CUs' worth of
// tiles, those tiles run as two K halves each, so that round has twice the
// work units at half the length.  Returns the tail tiles per XCD (0: none)
// and their partial sums' bytes.
int wide_tail(int64_t ntiles, int64_t K, int64_t* bytes) {
  const int64_t per = aq::ceil_div(ntiles, 8), cpx = std::max(1, aq::cu_count() / 8);
  const int64_t tail = per % cpx, nch = K / kGemmBK;
  *bytes = 0;
  if (tail == 0 || 2 * tail > cpx || nch % 2 != 0 || nch < 8) return 0;
  *bytes = 8 * tail * 2 * (int64_t)kWideBM * kWideBN * 4;
  return (int)tail;
}

template <int FMT, int DENSE>
hipError_t launch_gemm_wide(QLArgs a, bool per_channel, void* ws, int64_t ws_bytes, hipStream_t s) {
  const int mbands = (int)aq::ceil_div(a.M, kWideBM);
  int ntiles = 0;
  for (int i = 0; i < a.count; i++) {
    a.first[i] = ntiles;
    ntiles += (int)aq::ceil_div(a.mat[i].N, kWideBN) * mbands * a.split;
  }
  for (int i = a.count; i <= kMaxGroup; i++) a.first[i] = ntiles;
  a.tail = 0;
  a.per = (int)aq::ceil_div(ntiles, 8);
  a.tpart = nullptr;
  if (a.split == 1 && ws && (uintptr_t)ws % 16 == 0) {
    int64_t need = 0;
    const int tail = wide_tail(ntiles, a.K, &need);
    if (tail > 0 && ws_bytes >= need) {
      a.tail = tail;
      a.tpart = (float*)ws;
    }
  }
  const dim3 grid((unsigned)(8 * (a.per + a.tail)));
  if (per_channel)
    hipLaunchKernelGGL((qlinear_gemm_wide_kernel<FMT, 1, DENSE>), grid, dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((qlinear_gemm_wide_kernel<FMT, 0, DENSE>), grid, dim3(512), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && a.tail) {
    hipLaunchKernelGGL(tail_reduce_kernel, dim3((unsigned)(8 * a.tail), kWideBM / 16), dim3(256), 0, s, a);
    e = hipGetLastError();
  }
  return e;
}

hipError_t launch_gemm_wide(const QLArgs& a, int fmt, bool per_channel, bool dense, void* ws, int64_t ws_bytes,
                            hipStream_t s) {
  if (dense)
    return fmt == AQ_FMT_E4M3 ? launch_gemm_wide<AQ_FMT_E4M3, 1>(a, per_channel, ws, ws_bytes, s)
                              : launch_gemm_wide<AQ_FMT_INT8, 1>(a, per_channel, ws, ws_bytes, s);
  return fmt == AQ_FMT_E4M3 ? launch_gemm_wide<AQ_FMT_E4M3, 0>(a, per_channel, ws, ws_bytes, s)
                            : launch_gemm_wide<AQ_FMT_INT8, 0>(a, per_channel, ws, ws_bytes, s);
}

}  // namespace

extern "C" int64_t aq_qlinear_workspace_size(int64_t M, int64_t N, int64_t K) {
  // the GEMM's fp32 partial sums when it would split K for this shape on the
  // current device (0 for the GEMV and for unsplit grids; for 33 <= M <= 64
  // on short grids the GEMM takes the call if given the block lists)
  if (N <= 0 || K < 128 || K % 128) return 0;
  if (M <= kGemvShortMaxM || (M <= kGemvMaxM && N / 16 >= kGemvShortRows)) return 0;
  const GemmPlan p = plan_gemm(M, &N, 1, K, 8);
  if (p.split > 1) return p.split * M * N * 4;
  int64_t tail_bytes = 0;  // an unsplit 256 x 256 grid's tail tiles, run as two K halves
  if (p.tile == kTile256x256) wide_tail(aq::ceil_div(N, kWideBN) * aq::ceil_div(M, kWideBM), K, &tail_bytes);
  return tail_bytes;
}



// aq_qlinear_decode's additions to a grouped launch
struct DecodeFuse {
  int pro;
  const void* x2;
  const void* nw;
  const void* nb;
  float eps;
  const void* const* res;
  const int32_t* act;
};

static int qlinear_grouped_impl(const void* x, int64_t M, int64_t K, int fmt, int64_t count, const int64_t* Ns,
                                const void* const* codes, const void* const* scales, const int64_t* Gs,
                                const int32_t* const* row_ptrs, const int32_t* const* cols, const void* const* vals,
                                const int32_t* const* tile_ptrs, const uint32_t* const* tile_ents,
                                const int64_t* tile_maxes, const void* const* biases, void* const* ys,
                                void* workspace, int64_t workspace_bytes, void* stream, const DecodeFuse* fz) {
  AQ_CHECK_ARG(count >= 1 && count <= kMaxGroup, "aq_qlinear: 1..%d matrices per call (got %lld)", kMaxGroup,
               (long long)count);
  AQ_CHECK_ARG(M >= 0 && M < (1 << 30) && K >= 128 && K % 128 == 0,
               "aq_qlinear: K must be a multiple of 128 (M=%lld K=%lld)", (long long)M, (long long)K);
  // the kernels address x and a workgroup's codes with 32-bit buffer offsets
  AQ_CHECK_ARG(K <= (1 << 22), "aq_qlinear: K=%lld too large (at most 4194304)", (long long)K);
  AQ_CHECK_ARG(fmt == AQ_FMT_INT8 || fmt == AQ_FMT_E4M3, "aq_qlinear: unknown code format %d", fmt);
  AQ_CHECK_ARG(x && Ns && codes && scales && Gs && row_ptrs && cols && vals && ys, "aq_qlinear: null pointer argument");
  AQ_CHECK_ARG((uintptr_t)x % 16 == 0, "aq_qlinear: x must be 16-byte aligned");
  QLArgs a{};
  a.x = (const uint16_t*)x;
  a.M = (int)M;
  a.K = (int)K;
  a.count = (int)count;
  int64_t blocks = 0;
  for (int i = 0; i < kMaxGroup; i++) {
    const int j = i < count ? i : 0;
    const int64_t N = Ns[j], G = Gs[j];
    if (i < count) {
      AQ_CHECK_ARG(N >= 16 && N % 16 == 0 && N < (1 << 30) && N * K < ((int64_t)1 << 40),
                   "aq_qlinear: N must be a positive multiple of 16 (N=%lld)", (long long)N);
      AQ_CHECK_ARG(G >= 32 && G % 32 == 0 && K % G == 0,
                   "aq_qlinear: block size %lld must be a multiple of 32 that divides K=%lld", (long long)G,
                   (long long)K);
      AQ_CHECK_ARG(codes[j] && scales[j] && row_ptrs[j] && ys[j] && (uintptr_t)codes[j] % 16 == 0,
                   "aq_qlinear: null or unaligned pointer for matrix %d", i);
      AQ_CHECK_ARG(M <= kGemvMaxM || (tile_ptrs && tile_ents && tile_maxes && tile_ptrs[j] && tile_ents[j]),
                   "aq_qlinear: M > 64 needs the outlier tile lists (aq_outlier_tiles) for matrix %d", i);
      a.first[i] = (int)blocks;
      blocks += N / 16;
    }
    QLMat& w = a.mat[i];
    w.codes = (const uint8_t*)codes[j];
    w.scales = (const uint16_t*)scales[j];
    w.row_ptr = row_ptrs[j];
    w.cols = cols[j];
    w.vals = (const uint16_t*)vals[j];
    w.tptr = tile_ptrs ? tile_ptrs[j] : nullptr;
    w.tent = tile_ents ? tile_ents[j] : nullptr;
    w.bias = biases ? (const uint16_t*)biases[j] : nullptr;
    w.y = (uint16_t*)ys[j];
    w.part = nullptr;
    w.N = (int)N;
    w.ldy = (int)N;
    w.G = (int)G;
    w.kg = (int)(K / G);
    w.gshift = log2_exact(G);
  }
  for (int i = (int)count; i <= kMaxGroup; i++) a.first[i] = (int)blocks;
  a.split = 1;
  if (fz) {
    // decode: the M = 1 GEMV with x in LDS (every prologue) or the shared-x
    // GEMV for 6 <= M <= 64 (epilogue only: each of its workgroups stages all
    // of x, so a prologue there would be computed once per workgroup)
    AQ_CHECK_ARG((M == 1 && K <= kGemvX1MaxK) || (M >= kGemvXMinM && M <= kGemvMaxM),
                 "aq_qlinear_decode: M = 1 with K <= %d, or 6 <= M <= 64 (M=%lld K=%lld)", kGemvX1MaxK, (long long)M,
                 (long long)K);
    AQ_CHECK_ARG(fz->pro >= kProNone && fz->pro <= kProSwiGlu, "aq_qlinear_decode: unknown prologue %d", fz->pro);
    AQ_CHECK_ARG(M == 1 || fz->pro == kProNone, "aq_qlinear_decode: prologues take one row (M=%lld)",
                 (long long)M);
    AQ_CHECK_ARG(fz->pro != kProSwiGlu || (fz->x2 && (uintptr_t)fz->x2 % 16 == 0),
                 "aq_qlinear_decode: SwiGLU needs u (16-byte aligned)");
    AQ_CHECK_ARG((fz->pro != kProRms && fz->pro != kProLayerNorm) || (fz->nw && (uintptr_t)fz->nw % 16 == 0),
                 "aq_qlinear_decode: the norm needs its weight (16-byte aligned)");
    AQ_CHECK_ARG(fz->pro != kProLayerNorm || (fz->nb && (uintptr_t)fz->nb % 16 == 0),
                 "aq_qlinear_decode: LayerNorm needs its bias (16-byte aligned)");
    a.pro = fz->pro;
    a.x2 = (const uint16_t*)fz->x2;
    a.nw = (const uint16_t*)fz->nw;
    a.nb = (const uint16_t*)fz->nb;
    a.eps = fz->eps;
    for (int i = 0; i < count; i++) {
      a.mat[i].res = fz->res ? (const uint16_t*)fz->res[i] : nullptr;
      a.mat[i].act = fz->act ? fz->act[i] : 0;
      AQ_CHECK_ARG(a.mat[i].act == 0 || a.mat[i].act == 1 || (i == 0 && a.mat[i].act == 2),
                   "aq_qlinear_decode: activation %d of member %d (0 none, 1 ReLU, 2 SwiGLU pair: member 0)",
                   a.mat[i].act, i);
      AQ_CHECK_ARG(a.mat[i].res != ys[i], "aq_qlinear_decode: the residual must not be the output");
    }
    if (a.mat[0].act == 2) {
      AQ_CHECK_ARG(count == 2 && Ns[0] == Ns[1] && M >= kGemvXMinM && a.pro == kProNone && a.mat[1].act == 0 &&
                       !a.mat[0].res && !a.mat[1].res,
                   "aq_qlinear_decode: a SwiGLU pair is two members of equal N (gate, up), 6 <= M <= 64, no "
                   "prologue, activation or residual besides");
    }
  }
  if (M == 0) return AQ_OK;
  hipStream_t s = (hipStream_t)stream;
  bool per_channel = true;
  for (int i = 0; i < count; i++) per_channel = per_channel && a.mat[i].kg == 1;
  bool have_lists = tile_ptrs && tile_ents && tile_maxes;
  for (int i = 0; i < count && have_lists; i++) have_lists = tile_ptrs[i] && tile_ents[i];
  const bool gemv = M <= kGemvShortMaxM || (M <= kGemvMaxM && (blocks >= kGemvShortRows || !have_lists));
  // From M = 2 the shared-x GEMV also takes tall groups with block-wise
  // scales (block-128 gate+up at M = 4: 29.9 against 26.7 us; shorter grids
  // and per-channel scales stay faster re-reading x per tile row below)
  const bool x_tall = !per_channel && M >= 2 && blocks >= 768;
  if (gemv && (M >= kGemvXMinM || x_tall)) {
    // S = 2 waves per tile row for tall groups, 4 for short ones and 8 for
    // fewer than 384 tile rows up to M = 32 (one tile row per workgroup; at
    // M = 64 its x stages do not fit LDS) (measured on the Llama-3-8B
    // shapes: S = 1 leaves the loads' latency exposed, S = 4 on N = 4096
    // leaves half the CUs idle).
    // Per decoder layer of those shapes it beats re-reading x per tile row
    // from M = 6 on (M = 6: 76 against 78 us, M = 16: 77 against 127 us)
    int S = blocks >= 768 ? 2 : (blocks >= 384 || M > 32) ? 4 : 8;
    if (a.mat[0].act == 2) S = std::min(S, 4);  // a SwiGLU pair needs two tile-row slots per workgroup
    return aq::check_hip(launch_gemv_x(a, fmt, per_channel, S, s), "aq_qlinear: gemv launch");
  }
  if (gemv) {
    // tall groups fill the GPU with 4 streaming waves per tile row, short ones need 8
    // waves per tile row: enough for about 1536 waves in all (1.5 per SIMD),
    // at most 8; a tall group (gate+up) streams one tile row per wave
    const int64_t want = (1536 + blocks - 1) / blocks;
    const hipError_t e = want <= 1 ? launch_gemv<1>(a, fmt, per_channel, s)
                       : want <= 2 ? launch_gemv<2>(a, fmt, per_channel, s)
                       : want <= 4 ? launch_gemv<4>(a, fmt, per_channel, s)
                                   : launch_gemv<8>(a, fmt, per_channel, s);
    return aq::check_hip(e, "aq_qlinear: gemv launch");
  }
  bool dense = false;  // some 16 x 64 block holds more than 64 outliers
  for (int i = 0; i < count; i++) dense = dense || tile_maxes[i] > 64;
  // Tile shape and K split from plan_gemm, the split as far as the workspace
  // allows: each part's fp32 partial sums go there and splitk_reduce_kernel
  // adds them in a fixed order.
  int64_t outs = 0;
  for (int i = 0; i < count; i++) outs += M * Ns[i];
  int max_split = 1;  // as far as the caller's workspace holds the partial sums
  while (workspace && max_split < 8 && workspace_bytes >= 2 * max_split * outs * 4) max_split *= 2;
  const GemmPlan plan = plan_gemm(M, Ns, count, K, max_split);
  a.split = plan.split;
  if (a.split > 1) {
    AQ_CHECK_ARG((uintptr_t)workspace % 16 == 0, "aq_qlinear: workspace must be 16-byte aligned");
    float* p = (float*)workspace;
    for (int i = 0; i < count; i++) {
      a.mat[i].part = p;
      p += (size_t)a.split * M * Ns[i];
    }
  }
  hipError_t e = plan.tile == kTile256x256   ? launch_gemm_wide(a, fmt, per_channel, dense, workspace,
                                                                 workspace_bytes, s)
                 : plan.tile == kTile256x128 ? launch_gemm<256>(a, fmt, per_channel, dense, s)
                                             : launch_gemm<128>(a, fmt, per_channel, dense, s);
  if (e != hipSuccess || a.split == 1) return aq::check_hip(e, "aq_qlinear: gemm launch");
  for (int i = 0; i < count && e == hipSuccess; i++) {
    const int64_t mn = M * Ns[i];
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)aq::ceil_div(mn, 1024)), dim3(256), 0, s, a.mat[i].part, mn,
                       a.split, (int)Ns[i], a.mat[i].bias, a.mat[i].y);
    e = hipGetLastError();
  }
  return aq::check_hip(e, "aq_qlinear: split-K reduce launch");
}

extern "C" int aq_qlinear_grouped(const void* x, int64_t M, int64_t K, int fmt, int64_t count, const int64_t* Ns,
                                  const void* const* codes, const void* const* scales, const int64_t* Gs,
                                  const int32_t* const* row_ptrs, const int32_t* const* cols,
                                  const void* const* vals, const int32_t* const* tile_ptrs,
                                  const uint32_t* const* tile_ents, const int64_t* tile_maxes,
                                  const void* const* biases, void* const* ys, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  return qlinear_grouped_impl(x, M, K, fmt, count, Ns, codes, scales, Gs, row_ptrs, cols, vals, tile_ptrs, tile_ents,
                              tile_maxes, biases, ys, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int aq_qlinear_decode(const void* x, int64_t M, int64_t K, int fmt, int64_t count, const int64_t* Ns,
                                 const void* const* codes, const void* const* scales, const int64_t* Gs,
                                 const int32_t* const* row_ptrs, const int32_t* const* cols, const void* const* vals,
                                 const int32_t* const* tile_ptrs, const uint32_t* const* tile_ents,
                                 const void* const* biases, void* const* ys, int prologue, const void* x2,
                                 const void* norm_weight, const void* norm_bias, float eps,
                                 const void* const* residuals, const int32_t* relu, void* stream) {
  const DecodeFuse fz{prologue, x2, norm_weight, norm_bias, eps, residuals, relu};
  // no tile_max: the decode GEMVs never take the GEMM
  return qlinear_grouped_impl(x, M, K, fmt, count, Ns, codes, scales, Gs, row_ptrs, cols, vals, tile_ptrs, tile_ents,
                              nullptr, biases, ys, nullptr, 0, stream, &fz);
}

extern "C" int aq_qlinear(const void* x, int64_t M, int64_t K, int64_t N, const void* codes, const void* scales,
                          int64_t G, int fmt, const int32_t* row_ptr, const int32_t* cols, const void* vals,
                          const int32_t* tile_ptr, const uint32_t* tile_ent, int64_t tile_max, const void* bias,
                          void* y, void* workspace, int64_t ws_bytes, void* stream) {
  const void* b = bias;
  void* yy = y;
  return aq_qlinear_grouped(x, M, K, fmt, 1, &N, &codes, &scales, &G, &row_ptr, &cols, &vals, &tile_ptr, &tile_ent,
                            &tile_max, &b, &yy, workspace, ws_bytes, stream);
}
