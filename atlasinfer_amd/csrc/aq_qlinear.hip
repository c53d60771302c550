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
//  * M <= 16: dequant-GEMV.  One workgroup per 16-row tile row: NS waves
//    stream its tiles (1 KiB contiguous per load instruction, four 128-wide
//    K chunks in flight per wave) with the M rows of x as the MFMA A operand
//    (rows >= M are zero), and their partial tiles are summed through LDS in
//    a fixed order.  Wave 0 then stages the rows' CSR outlier lists and the
//    x values they multiply into LDS for the epilogue.  NS is 4 for tall
//    matrices (enough workgroups to fill the GPU) and 8 otherwise.  Several
//    matrices that read the same x (q/k/v, gate/up) share one launch.
//  * M > 16: dequant-GEMM.  128x128 output tile per workgroup of 4 waves
//    (64x64 each), 128-wide K steps.  The x tile goes through LDS; each wave
//    reads its four code tiles straight from HBM into registers (they are
//    already in operand order), and the next step's x tile and codes are
//    loaded while the current step is multiplied.  Outliers are applied
//    inside the K loop from the LDS x tile, for the columns of the step.
#include <algorithm>

#include "aq_common.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kMaxGroup = 4;

struct QLMat {
  const uint8_t* codes;  // tiled
  const uint16_t* scales;
  const int32_t* row_ptr;
  const int32_t* cols;
  const uint16_t* vals;
  const uint16_t* bias;
  uint16_t* y;
  int N;
  int G;
  int kg;      // K / G, scale blocks per row
  int gshift;  // log2(G) when G is a power of two, else -1
};

struct QLArgs {
  const uint16_t* x;
  int M, K, count;
  int first[kMaxGroup + 1];  // GEMV: first workgroup of each matrix
  QLMat mat[kMaxGroup];
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

// ------------------------------------------------------------ GEMV (M <= 16)

constexpr int kGemvUnroll = 4;  // 128-wide K chunks per wave with loads in flight together
// Staging capacity per workgroup (16 rows).  Kept small so that LDS does not
// limit the workgroups resident per CU; entries beyond it (heavy-tailed
// weights) are read from memory in the epilogue.
constexpr int kCsrCap = 1024;   // outlier entries
constexpr int kXvCap = 1024;    // staged x values: entries * M <= kXvCap
constexpr int kStageBatch = 8;  // entries per lane whose loads are issued together

template <int NS, int FMT, int PC>
__global__ __launch_bounds__(64 * NS) void qlinear_gemv_kernel(QLArgs a) {
  constexpr int U = kGemvUnroll;
  __shared__ float red[NS][256];
  __shared__ int s_rp[17];
  __shared__ int s_meta[3];  // p0, staged entries, entries with staged x
  __shared__ int s_col[kCsrCap];
  __shared__ uint16_t s_val[kCsrCap];
  __shared__ uint16_t s_xv[kXvCap];

  int mi = 0;
#pragma unroll
  for (int j = 1; j < kMaxGroup; j++)
    if (j < a.count && (int)blockIdx.x >= a.first[j]) mi = j;
  const QLMat W = pick(a, mi);
  const int rb = blockIdx.x - a.first[mi];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = rb * 16;
  const int M = a.M, K = a.K, N = W.N;
  const int nchunks = K >> 7;

  // Wave 0 also stages the rows' outliers.  Its row_ptr load goes out first;
  // the (col, val) loads of up to 64 * kStageBatch entries go out after its
  // first round of the stream, and for decode the x gather after the second,
  // so they return while the codes stream in.
  int rp = 0;
  if (wave == 0 && lane <= 16) rp = W.row_ptr[n0 + lane];
  int p0 = 0, cnt = 0;
  int scol[kStageBatch];
  uint16_t sval[kStageBatch];
#pragma unroll
  for (int b = 0; b < kStageBatch; b++) {
    scol[b] = 0;
    sval[b] = 0;
  }
  auto stage_first_batch = [&]() {
    p0 = __shfl(rp, 0, 64);
    cnt = min(__shfl(rp, 16, 64) - p0, kCsrCap);
#pragma unroll
    for (int b = 0; b < kStageBatch; b++) {
      const int e = 64 * b + lane;
      if (e < cnt) {
        scol[b] = W.cols[p0 + e];
        sval[b] = W.vals[p0 + e];
      }
    }
  };
  if (wave == 0 && nchunks <= wave) stage_first_batch();  // no stream share

  {
    // The code and scale loads below are unconditional, from addresses that
    // are always valid, so the compiler keeps all of them in flight (a chunk
    // past the end of K re-reads chunk c0 with its x zeroed).  x is loaded
    // only by the lanes of rows m < M (exec-masked): for decode (M = 1) that
    // is 4 lanes, 256 bytes of x per 2 KiB chunk of codes.
    const int grp = lane >> 4;
    const int li = lane & 15;
    const int n = n0 + li;
    const bool mvalid = li < M;
    const uint8_t* tiles = W.codes + ((size_t)rb * nchunks << 11) + lane * 16;
    const uint16_t* xrow = a.x + (size_t)li * K + 16 * grp;
    const uint16_t sb_row = PC ? W.scales[n] : (uint16_t)0;
    float4v acc = (float4v){0.f, 0.f, 0.f, 0.f};
    for (int c0 = wave; c0 < nchunks; c0 += U * NS) {
      uint4 q[U][2];
      uint4 xq[U][4];
      uint16_t sb[U][2];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int c = c0 + u * NS;
        const int cc = c < nchunks ? c : c0;
        const uint8_t* t = tiles + ((size_t)cc << 11);
        q[u][0] = ld_nt16(t);
        q[u][1] = ld_nt16(t + 1024);
        if (PC) {
          sb[u][0] = sb[u][1] = sb_row;
        } else {
          sb[u][0] = W.scales[scale_index(W, n, cc * 128 + 16 * grp)];
          sb[u][1] = W.scales[scale_index(W, n, cc * 128 + 64 + 16 * grp)];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) xq[u][j] = make_uint4(0, 0, 0, 0);
        if (mvalid) {
          const uint4* xp = reinterpret_cast<const uint4*>(xrow + cc * 128);
          xq[u][0] = xp[0];
          xq[u][1] = xp[1];
          xq[u][2] = xp[8];  // + 64 columns
          xq[u][3] = xp[9];
        }
      }
#pragma unroll
      for (int u = 1; u < U; u++)
        if (c0 + u * NS >= nchunks)  // wave-uniform
#pragma unroll
          for (int j = 0; j < 4; j++) xq[u][j] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < U; u++) {
        const half2v s0 = scale2(sb[u][0]), s1 = scale2(sb[u][1]);
        const half8 w0 = deq8<FMT>(q[u][0].x, q[u][0].y, s0);
        const half8 w1 = deq8<FMT>(q[u][0].z, q[u][0].w, s0);
        const half8 w2 = deq8<FMT>(q[u][1].x, q[u][1].y, s1);
        const half8 w3 = deq8<FMT>(q[u][1].z, q[u][1].w, s1);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xq[u][0]), w0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xq[u][1]), w1, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xq[u][2]), w2, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xq[u][3]), w3, acc, 0, 0, 0);
      }
      // Staging loads go out after this round's waits, so they never hold
      // up a wait for code loads (the load counter retires in order).
      if (wave == 0 && c0 == 0) stage_first_batch();
    }
    // C layout: lane l, element i -> m = 4*(l/16) + i, column l % 16
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave][lane * 4 + i] = acc[i];
  }

  if (wave == 0) {
    // Stage the CSR lists of rows n0..n0+15 and the x values they multiply
    // (the first batch of (col, val) is already in registers).
    if (lane <= 16) s_rp[lane] = rp - p0;
    const int nx = min(cnt, kXvCap / M);
    for (int base = 0; base < cnt; base += 64 * kStageBatch) {
      int col[kStageBatch];
      uint16_t val[kStageBatch];
#pragma unroll
      for (int b = 0; b < kStageBatch; b++) {
        const int e = base + 64 * b + lane;
        col[b] = scol[b];
        val[b] = sval[b];
        if (base > 0) {
          col[b] = 0;
          val[b] = 0;
          if (e < cnt) {
            col[b] = W.cols[p0 + e];
            val[b] = W.vals[p0 + e];
          }
        }
      }
#pragma unroll
      for (int b = 0; b < kStageBatch; b++) {
        const int e = base + 64 * b + lane;
        if (e < cnt) {
          s_col[e] = col[b];
          s_val[e] = val[b];
        }
      }
      for (int m = 0; m < M; m++) {
        uint16_t xv[kStageBatch];
#pragma unroll
        for (int b = 0; b < kStageBatch; b++) {
          const int e = base + 64 * b + lane;
          xv[b] = (e < nx) ? a.x[(size_t)m * K + col[b]] : (uint16_t)0;
        }
#pragma unroll
        for (int b = 0; b < kStageBatch; b++) {
          const int e = base + 64 * b + lane;
          if (e < nx) s_xv[e * M + m] = xv[b];
        }
      }
    }
    if (lane == 0) {
      s_meta[0] = p0;
      s_meta[1] = cnt;
      s_meta[2] = nx;
    }
  }
  __syncthreads();

  if (M == 1) {
    // decode: 16 threads per row split the row's outliers, then a fixed
    // 16-lane shuffle tree adds them up
    if (threadIdx.x < 256) {
      const int nl = threadIdx.x >> 4;
      const int sub = threadIdx.x & 15;
      const int p0 = s_meta[0], cnt = s_meta[1], nx = s_meta[2];
      const int e1 = s_rp[nl + 1];
      float v = 0.0f;
      for (int e = s_rp[nl] + sub; e < e1; e += 16) {
        float xv, wv;
        if (e < cnt) {
          const int col = s_col[e];
          xv = (float)bits_to_h(e < nx ? s_xv[e] : a.x[col]);
          wv = (float)bits_to_h(s_val[e]);
        } else {
          xv = (float)bits_to_h(a.x[W.cols[p0 + e]]);
          wv = (float)bits_to_h(W.vals[p0 + e]);
        }
        v = __builtin_fmaf(xv, wv, v);
      }
#pragma unroll
      for (int d = 1; d < 16; d <<= 1) v = v + __shfl_xor(v, d, 64);
      if (sub == 0) {
        // dense part: C element (m = 0, column nl) sits in lane nl, slot 0
        float dense = 0.0f;
#pragma unroll
        for (int w = 0; w < NS; w++) dense += red[w][nl * 4];
        v = dense + v;
        if (W.bias) v += (float)bits_to_h(W.bias[n0 + nl]);
        W.y[n0 + nl] = h_to_bits(rn_h(v));
      }
    }
  } else if (threadIdx.x < 256) {
    const int o = threadIdx.x;
    const int l = o >> 2;
    const int m = 4 * (l >> 4) + (o & 3);
    const int nl = l & 15;
    const int n = n0 + nl;
    if (m < M) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < NS; w++) v += red[w][o];
      const int p0 = s_meta[0], cnt = s_meta[1], nx = s_meta[2];
      const int e1 = s_rp[nl + 1];
      for (int e = s_rp[nl]; e < e1; e++) {
        float xv, wv;
        if (e < nx) {
          xv = (float)bits_to_h(s_xv[e * M + m]);
          wv = (float)bits_to_h(s_val[e]);
        } else if (e < cnt) {
          xv = (float)bits_to_h(a.x[(size_t)m * K + s_col[e]]);
          wv = (float)bits_to_h(s_val[e]);
        } else {  // more outliers than the staging holds: straight from memory
          xv = (float)bits_to_h(a.x[(size_t)m * K + W.cols[p0 + e]]);
          wv = (float)bits_to_h(W.vals[p0 + e]);
        }
        v = __builtin_fmaf(xv, wv, v);
      }
      if (W.bias) v += (float)bits_to_h(W.bias[n]);
      W.y[(size_t)m * N + n] = h_to_bits(rn_h(v));
    }
  }
}

// ------------------------------------------------------------ GEMM (M > 16)

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int APAD = 8;  // halves of padding per LDS row of the x tile
constexpr int kTileCsrCap = 4096;

// x tile of step c into registers: 128 rows x 128 columns, 8 x 16 bytes per
// thread; rows past M are clamped to row M-1 (their outputs are not stored).
__device__ __forceinline__ void gemm_load_x(u32x4 (&ra)[8], const uint16_t* x, int mbase, int m_last, int K, int c,
                                            int t) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int idx = t + 256 * i;
    const int gm = min(mbase + (idx >> 4), m_last);
    ra[i] = *reinterpret_cast<const u32x4*>(x + (size_t)gm * K + c * BK + 8 * (idx & 15));
  }
}

__device__ __forceinline__ void gemm_store_x(uint16_t (&As)[BM][BK + APAD], const u32x4 (&ra)[8], int t) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int idx = t + 256 * i;
    *reinterpret_cast<u32x4*>(&As[idx >> 4][8 * (idx & 15)]) = ra[i];
  }
}

// The wave's four code tiles of step c (already in MFMA operand order) and,
// for block-wise scales, the two scales each lane's pieces use.
template <int PC>
__device__ __forceinline__ void gemm_load_codes(u32x4 (&q)[4][2], uint16_t (&sg)[4][2], const QLMat& W,
                                                const int (&rbi)[4], int nchunks, int c, int lane, int li, int grp) {
#pragma unroll
  for (int ni = 0; ni < 4; ni++) {
    const uint8_t* tp = W.codes + (((size_t)rbi[ni] * nchunks + c) << 11) + lane * 16;
    q[ni][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tp));
    q[ni][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tp + 1024));
    if (!PC) {
      const int n = rbi[ni] * 16 + li;
      sg[ni][0] = W.scales[scale_index(W, n, c * BK + 16 * grp)];
      sg[ni][1] = W.scales[scale_index(W, n, c * BK + 64 + 16 * grp)];
    } else {
      sg[ni][0] = sg[ni][1] = 0;
    }
  }
}

template <int FMT, int PC>
__global__ __launch_bounds__(256) void qlinear_gemm_kernel(QLArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM][BK + APAD];
  __shared__ int s_rp[BN + 1];
  __shared__ int s_col[kTileCsrCap];
  __shared__ uint16_t s_val[kTileCsrCap];

  const QLMat W = pick(a, blockIdx.z);
  const int N = W.N;
  const int nbase = blockIdx.x * BN;
  if (nbase >= N) return;  // this matrix of the group is narrower than the grid
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int mbase = blockIdx.y * BM;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int M = a.M, K = a.K;
  const int nchunks = K >> 7;

  // outlier lists of this tile's 128 output columns
  if (t <= BN) s_rp[t] = W.row_ptr[min(nbase + t, N)];
  __syncthreads();
  const int p0 = s_rp[0];
  const int cnt = min(s_rp[BN] - p0, kTileCsrCap);
  for (int e = t; e < cnt; e += 256) {
    s_col[e] = W.cols[p0 + e];
    s_val[e] = W.vals[p0 + e];
  }
  int eptr[4], eend[4];
#pragma unroll
  for (int ni = 0; ni < 4; ni++) {
    const int nl = wn + 16 * ni + li;
    eptr[ni] = s_rp[nl] - p0;
    eend[ni] = min(s_rp[nl + 1] - p0, cnt);
  }

  // This wave's four tile rows (16 output columns each).  Loads are
  // unconditional so that they all stay in flight: tile rows past N and x
  // rows past M are clamped to the last valid ones, and only feed outputs
  // that are never stored.
  const int rb_last = N / 16 - 1;
  int rbi[4];
  half2v srow[4];
#pragma unroll
  for (int ni = 0; ni < 4; ni++) {
    rbi[ni] = min((nbase + wn) / 16 + ni, rb_last);
    srow[ni] = scale2(PC ? W.scales[rbi[ni] * 16 + li] : (uint16_t)0);
  }
  const int m_last = M - 1;

  float4v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

  u32x4 ra[8];     // x tile of the next step: 128 rows x 16 x 16 bytes
  u32x4 qc[4][2];  // codes of this step: [tile row][half]
  u32x4 qn[4][2];  // codes of the next step
  uint16_t sc[4][2], sn[4][2];

  gemm_load_x(ra, a.x, mbase, m_last, K, 0, t);
  gemm_load_codes<PC>(qc, sc, W, rbi, nchunks, 0, lane, li, grp);
  for (int c = 0; c < nchunks; c++) {
    __syncthreads();  // the previous step's LDS reads are done (and the CSR staging, first time)
    gemm_store_x(As, ra, t);
    __syncthreads();
    if (c + 1 < nchunks) {
      gemm_load_x(ra, a.x, mbase, m_last, K, c + 1, t);
      gemm_load_codes<PC>(qn, sn, W, rbi, nchunks, c + 1, lane, li, grp);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {  // k-steps of 32 within the 128-wide chunk
      const int h = j >> 1;
      const int kq = 64 * h + 16 * grp + 8 * (j & 1);
      half8 af[4], bf[4];
#pragma unroll
      for (int mi = 0; mi < 4; mi++) af[mi] = *reinterpret_cast<const half8*>(&As[wm + 16 * mi + li][kq]);
#pragma unroll
      for (int ni = 0; ni < 4; ni++) {
        const u32x4 q = qc[ni][h];
        const half2v s2 = PC ? srow[ni] : scale2(sc[ni][h]);
        bf[ni] = (j & 1) ? deq8<FMT>(q.z, q.w, s2) : deq8<FMT>(q.x, q.y, s2);
      }
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mi], bf[ni], acc[mi][ni], 0, 0, 0);
    }
    // outliers whose column lies in this step: x from the LDS tile
    const int k0 = c * BK;
#pragma unroll
    for (int ni = 0; ni < 4; ni++) {
      while (eptr[ni] < eend[ni] && s_col[eptr[ni]] < k0 + BK) {
        const int cc = s_col[eptr[ni]] - k0;
        const float v = (float)bits_to_h(s_val[eptr[ni]]);
#pragma unroll
        for (int mi = 0; mi < 4; mi++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            acc[mi][ni][i] = __builtin_fmaf((float)bits_to_h(As[wm + 16 * mi + 4 * grp + i][cc]), v, acc[mi][ni][i]);
        eptr[ni]++;
      }
    }
#pragma unroll
    for (int ni = 0; ni < 4; ni++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        qc[ni][h] = qn[ni][h];
        sc[ni][h] = sn[ni][h];
      }
  }

  const bool overflow = (s_rp[BN] - p0) > kTileCsrCap;
#pragma unroll
  for (int ni = 0; ni < 4; ni++) {
    const int nl = wn + 16 * ni + li;
    const int n = nbase + nl;
    if (n >= N) continue;
    const float bv = W.bias ? (float)bits_to_h(W.bias[n]) : 0.0f;
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = mbase + wm + 16 * mi + 4 * grp + i;
        if (m >= M) continue;
        float v = acc[mi][ni][i];
        if (overflow) {  // entries past the staging capacity: from memory
          for (int p = max(p0 + cnt, s_rp[nl]); p < s_rp[nl + 1]; p++)
            v = __builtin_fmaf((float)bits_to_h(a.x[(size_t)m * K + W.cols[p]]), (float)bits_to_h(W.vals[p]), v);
        }
        W.y[(size_t)m * N + n] = h_to_bits(rn_h(v + bv));
      }
  }
}

int log2_exact(int64_t g) {
  if (g <= 0 || (g & (g - 1))) return -1;
  int s = 0;
  while ((int64_t(1) << s) < g) s++;
  return s;
}

template <int NS, int FMT>
hipError_t launch_gemv(const QLArgs& a, bool per_channel, int blocks, hipStream_t s) {
  if (per_channel)
    hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 1>), dim3(blocks), dim3(64 * NS), 0, s, a);
  else
    hipLaunchKernelGGL((qlinear_gemv_kernel<NS, FMT, 0>), dim3(blocks), dim3(64 * NS), 0, s, a);
  return hipGetLastError();
}

template <int NS>
hipError_t launch_gemv(const QLArgs& a, int fmt, bool per_channel, int blocks, hipStream_t s) {
  return fmt == AQ_FMT_E4M3 ? launch_gemv<NS, AQ_FMT_E4M3>(a, per_channel, blocks, s)
                            : launch_gemv<NS, AQ_FMT_INT8>(a, per_channel, blocks, s);
}

}  // namespace

extern "C" int64_t aq_qlinear_workspace_size(int64_t M, int64_t N, int64_t K) {
  (void)M;
  (void)N;
  (void)K;
  return 0;  // the kernels need no memory beyond LDS
}

extern "C" int aq_qlinear_grouped(const void* x, int64_t M, int64_t K, int fmt, int64_t count, const int64_t* Ns,
                                  const void* const* codes, const void* const* scales, const int64_t* Gs,
                                  const int32_t* const* row_ptrs, const int32_t* const* cols,
                                  const void* const* vals, const void* const* biases, void* const* ys,
                                  void* stream) {
  AQ_CHECK_ARG(count >= 1 && count <= kMaxGroup, "aq_qlinear: 1..%d matrices per call (got %lld)", kMaxGroup,
               (long long)count);
  AQ_CHECK_ARG(M >= 0 && M < (1 << 30) && K >= 128 && K % 128 == 0 && K < (1 << 30),
               "aq_qlinear: K must be a multiple of 128 (M=%lld K=%lld)", (long long)M, (long long)K);
  AQ_CHECK_ARG(fmt == AQ_FMT_INT8 || fmt == AQ_FMT_E4M3, "aq_qlinear: unknown code format %d", fmt);
  AQ_CHECK_ARG(x && Ns && codes && scales && Gs && row_ptrs && cols && vals && ys, "aq_qlinear: null pointer argument");
  AQ_CHECK_ARG((uintptr_t)x % 16 == 0, "aq_qlinear: x must be 16-byte aligned");
  QLArgs a;
  a.x = (const uint16_t*)x;
  a.M = (int)M;
  a.K = (int)K;
  a.count = (int)count;
  int64_t blocks = 0, maxN = 0;
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
      a.first[i] = (int)blocks;
      blocks += N / 16;
      maxN = std::max(maxN, N);
    }
    QLMat& w = a.mat[i];
    w.codes = (const uint8_t*)codes[j];
    w.scales = (const uint16_t*)scales[j];
    w.row_ptr = row_ptrs[j];
    w.cols = cols[j];
    w.vals = (const uint16_t*)vals[j];
    w.bias = biases ? (const uint16_t*)biases[j] : nullptr;
    w.y = (uint16_t*)ys[j];
    w.N = (int)N;
    w.G = (int)G;
    w.kg = (int)(K / G);
    w.gshift = log2_exact(G);
  }
  for (int i = (int)count; i <= kMaxGroup; i++) a.first[i] = (int)blocks;
  if (M == 0) return AQ_OK;
  hipStream_t s = (hipStream_t)stream;
  bool per_channel = true;
  for (int i = 0; i < count; i++) per_channel = per_channel && a.mat[i].kg == 1;
  if (M <= 16) {
    // tall groups fill the GPU with 4 streaming waves per tile row, short ones need 8
    const hipError_t e = blocks >= 512 ? launch_gemv<4>(a, fmt, per_channel, (int)blocks, s)
                                       : launch_gemv<8>(a, fmt, per_channel, (int)blocks, s);
    return aq::check_hip(e, "aq_qlinear: gemv launch");
  }
  const dim3 grid((unsigned)aq::ceil_div(maxN, BN), (unsigned)aq::ceil_div(M, BM), (unsigned)count);
  if (fmt == AQ_FMT_E4M3) {
    if (per_channel)
      hipLaunchKernelGGL((qlinear_gemm_kernel<AQ_FMT_E4M3, 1>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((qlinear_gemm_kernel<AQ_FMT_E4M3, 0>), grid, dim3(256), 0, s, a);
  } else {
    if (per_channel)
      hipLaunchKernelGGL((qlinear_gemm_kernel<AQ_FMT_INT8, 1>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((qlinear_gemm_kernel<AQ_FMT_INT8, 0>), grid, dim3(256), 0, s, a);
  }
  AQ_LAUNCH_CHECK("aq_qlinear: gemm launch");
  return AQ_OK;
}

extern "C" int aq_qlinear(const void* x, int64_t M, int64_t K, int64_t N, const void* codes, const void* scales,
                          int64_t G, int fmt, const int32_t* row_ptr, const int32_t* cols, const void* vals,
                          const void* bias, void* y, void* workspace, int64_t ws_bytes, void* stream) {
  (void)workspace;
  (void)ws_bytes;
  const void* b = bias;
  void* yy = y;
  return aq_qlinear_grouped(x, M, K, fmt, 1, &N, &codes, &scales, &G, &row_ptr, &cols, &vals, &b, &yy, stream);
}
