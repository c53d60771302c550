// aq_qlinear.hip -- quantized linear forward y = x W^T + b on gfx950.
//
// Replaces QuantizedLinear.forward (reference: integration/atlas_wrappers.py:
// 30-74), which dequantizes the whole weight (dequantize_tensor, :56) and
// calls F.linear on the fp16 result (:67).  Here the weight stays in its
// 1-byte code form in HBM; codes are turned into fp16 weights in registers as
// fp16(value(code) * scale) -- bit for bit the weight dequantize_tensor would
// produce -- and multiplied on the fp16 MFMA units with fp32 accumulation.
// Outlier positions hold code 0; their fp16 values are added from the CSR
// lists in fp32, then the bias, then one rounding to fp16.
//
//  * M <= 16: dequant-GEMV.  One workgroup of 9 waves per 16 rows of W.
//    Eight waves stream the rows' codes (16-byte non-temporal loads, four
//    128-wide K chunks in flight per wave) into 16x16x32 MFMAs with the M
//    rows of x as the A operand (rows >= M are zero); their partial tiles are
//    summed through LDS in a fixed order.  The ninth wave meanwhile stages
//    the rows' CSR outlier lists and the x values they multiply into LDS, so
//    the epilogue does not wait on memory.  No cross-workgroup reduction:
//    the grid is N/16 workgroups.
//  * M > 16: dequant-GEMM.  128x128 output tile per workgroup of 4 waves
//    (64x64 each), 64-wide K steps; the x tile (fp16) and the code tile
//    (bytes) go through LDS, the next step's tiles are prefetched into
//    registers while the current one is multiplied; codes become fp16 MFMA
//    operands in registers.  Outliers are applied inside the K loop: when
//    the x tile for columns [k0, k0+64) sits in LDS, each thread adds
//    x[m, c] * v for the outliers (c, v) of its output columns that fall in
//    that window (lists staged in LDS once per tile).
#include <algorithm>

#include "aq_common.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

struct QLArgs {
  const uint16_t* x;
  int M, K, N;
  const uint8_t* codes;
  const uint16_t* scales;
  int G;
  int kg;      // K / G, scale blocks per row
  int gshift;  // log2(G) when G is a power of two, else -1
  const int32_t* row_ptr;
  const int32_t* cols;
  const uint16_t* vals;
  const uint16_t* bias;
  uint16_t* y;
};

__device__ __forceinline__ uint32_t perm(uint32_t w, uint32_t sel) { return __builtin_amdgcn_perm(0u, w, sel); }
__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t h2_bits(half2v h) { return __builtin_bit_cast(uint32_t, h); }

// Two codes (bytes 2i, 2i+1 of w) -> fp16 pair holding value(code) * s.
template <int FMT>
__device__ __forceinline__ uint32_t deq_pair(uint32_t w, int hi, half2v s2) {
  const uint32_t p = perm(w, hi ? 0x0C030C02u : 0x0C010C00u);  // [c, 0, c', 0]
  if (FMT == AQ_FMT_E4M3) {
    // fp16 bits of value * 2^-8 (E4M3 exponent/mantissa land in the fp16
    // fields); s2 carries s * 2^8
    const uint32_t b = ((p << 7) & 0x3F803F80u) | ((p << 8) & 0x80008000u);
    return h2_bits(as_h2(b) * s2);
  } else {
    // 0x6400 | (c ^ 0x80) is the fp16 1024 + (c + 128); subtract 1152
    const half2v v = as_h2((p ^ 0x00800080u) | 0x64006400u) - (half2v){(f16)1152.0f, (f16)1152.0f};
    return h2_bits(v * s2);
  }
}

// 8 codes (two dwords) -> 8 fp16 weights.
template <int FMT>
__device__ __forceinline__ half8 deq8(uint32_t w0, uint32_t w1, half2v s2) {
  uint32_t r[4];
  r[0] = deq_pair<FMT>(w0, 0, s2);
  r[1] = deq_pair<FMT>(w0, 1, s2);
  r[2] = deq_pair<FMT>(w1, 0, s2);
  r[3] = deq_pair<FMT>(w1, 1, s2);
  return __builtin_bit_cast(half8, r);
}

template <int FMT>
__device__ __forceinline__ half2v scale_pair(uint16_t sbits) {
  f16 s = bits_to_h(sbits);
  if (FMT == AQ_FMT_E4M3) s = s * (f16)256.0f;  // exact: power-of-two scaling of a value <= 147
  return (half2v){s, s};
}

__device__ __forceinline__ int scale_index(const QLArgs& a, int n, int k) {
  const int blk = a.gshift >= 0 ? (k >> a.gshift) : (k / a.G);
  return n * a.kg + blk;
}

// ------------------------------------------------------------ GEMV (M <= 16)

constexpr int kGemvStream = 8;  // streaming waves per workgroup; one more wave stages the outliers
constexpr int kGemvUnroll = 4;  // 128-wide K chunks per wave with loads in flight together
constexpr int kCsrCap = 2048;   // outlier entries staged per workgroup (16 rows)
constexpr int kXvCap = 8192;    // staged x values: entries * M <= kXvCap
constexpr int kStageBatch = 8;  // entries per lane whose loads are issued together

template <int FMT>
__global__ __launch_bounds__(64 * (kGemvStream + 1)) void qlinear_gemv_kernel(QLArgs a) {
  constexpr int NS = kGemvStream;
  constexpr int U = kGemvUnroll;
  __shared__ float red[NS][256];
  __shared__ int s_rp[17];
  __shared__ int s_meta[3];  // p0, staged entries, entries with staged x
  __shared__ int s_col[kCsrCap];
  __shared__ uint16_t s_val[kCsrCap];
  __shared__ uint16_t s_xv[kXvCap];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int M = a.M, K = a.K, N = a.N;

  if (wave == NS) {
    // Stage the CSR lists of rows n0..n0+15 and the x values they multiply.
    // Three dependent round trips: row_ptr, then every (col, val), then
    // every x[m, col]; within each step all loads are issued together.
    int rp = 0;
    if (lane <= 16) rp = a.row_ptr[min(n0 + lane, N)];
    const int p0 = __shfl(rp, 0, 64);
    const int p1 = __shfl(rp, 16, 64);
    if (lane <= 16) s_rp[lane] = rp - p0;
    const int cnt = min(p1 - p0, kCsrCap);
    const int nx = min(cnt, kXvCap / M);
    for (int base = 0; base < cnt; base += 64 * kStageBatch) {
      int col[kStageBatch];
      uint16_t val[kStageBatch];
#pragma unroll
      for (int b = 0; b < kStageBatch; b++) {
        const int e = base + 64 * b + lane;
        col[b] = 0;
        val[b] = 0;
        if (e < cnt) {
          col[b] = a.cols[p0 + e];
          val[b] = a.vals[p0 + e];
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
  } else {
    const int grp = lane >> 4;
    const int li = lane & 15;
    const int n = n0 + li;
    const bool nvalid = n < N;
    const int nchunks = (K + 127) >> 7;
    const uint8_t* crow = a.codes + (size_t)(nvalid ? n : 0) * K;
    const uint16_t* xrow = a.x + (size_t)li * K;
    const bool mvalid = li < M;
    uint16_t sb_row = 0;
    if (a.kg == 1 && nvalid) sb_row = a.scales[n];
    float4v acc = (float4v){0.f, 0.f, 0.f, 0.f};
    for (int c0 = wave; c0 < nchunks; c0 += U * NS) {
      uint4 q[U][2];
      uint4 xq[U][4];
      uint16_t sb[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int c = c0 + u * NS;
        const int kk = c * 128 + 32 * grp;
        const bool kv = (c < nchunks) && (kk < K);
        q[u][0] = q[u][1] = make_uint4(0, 0, 0, 0);
        sb[u] = sb_row;
        if (kv && nvalid) {
          q[u][0] = ld_nt16(crow + kk);
          q[u][1] = ld_nt16(crow + kk + 16);
          if (a.kg != 1) sb[u] = a.scales[scale_index(a, n, kk)];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) xq[u][j] = make_uint4(0, 0, 0, 0);
        if (kv && mvalid) {
          const uint4* xp = reinterpret_cast<const uint4*>(xrow + kk);
#pragma unroll
          for (int j = 0; j < 4; j++) xq[u][j] = xp[j];
        }
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const half2v s2 = scale_pair<FMT>(sb[u]);
        const uint32_t qw[8] = {q[u][0].x, q[u][0].y, q[u][0].z, q[u][0].w,
                                q[u][1].x, q[u][1].y, q[u][1].z, q[u][1].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const half8 wb = deq8<FMT>(qw[2 * j], qw[2 * j + 1], s2);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, xq[u][j]), wb, acc, 0, 0, 0);
        }
      }
    }
    // C layout: lane l, element i -> m = 4*(l/16) + i, column l % 16
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave][lane * 4 + i] = acc[i];
  }
  __syncthreads();

  if (threadIdx.x < 256) {
    const int o = threadIdx.x;
    const int l = o >> 2;
    const int m = 4 * (l >> 4) + (o & 3);
    const int nl = l & 15;
    const int n = n0 + nl;
    if (m < M && n < N) {
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
          xv = (float)bits_to_h(a.x[(size_t)m * K + a.cols[p0 + e]]);
          wv = (float)bits_to_h(a.vals[p0 + e]);
        }
        v = __builtin_fmaf(xv, wv, v);
      }
      if (a.bias) v += (float)bits_to_h(a.bias[n]);
      a.y[(size_t)m * N + n] = h_to_bits(rn_h(v));
    }
  }
}

// ------------------------------------------------------------ GEMM (M > 16)

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int APAD = 8;   // halves of padding per LDS row of the x tile
constexpr int BPAD = 16;  // bytes of padding per LDS row of the code tile
constexpr int kTileCsrCap = 4096;

template <int FMT>
__global__ __launch_bounds__(256) void qlinear_gemm_kernel(QLArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM][BK + APAD];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[BN][BK + BPAD];
  __shared__ int s_rp[BN + 1];
  __shared__ int s_col[kTileCsrCap];
  __shared__ uint16_t s_val[kTileCsrCap];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int bm = blockIdx.y, bn = blockIdx.x;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int M = a.M, K = a.K, N = a.N;
  const int nbase = bn * BN;

  // outlier lists of this tile's 128 output columns
  if (t <= BN) s_rp[t] = a.row_ptr[min(nbase + t, N)];
  __syncthreads();
  const int p0 = s_rp[0];
  const int cnt = min(s_rp[BN] - p0, kTileCsrCap);
  for (int e = t; e < cnt; e += 256) {
    s_col[e] = a.cols[p0 + e];
    s_val[e] = a.vals[p0 + e];
  }
  int eptr[4], eend[4];
#pragma unroll
  for (int ni = 0; ni < 4; ni++) {
    const int nl = wn + 16 * ni + li;
    eptr[ni] = s_rp[nl] - p0;
    eend[ni] = min(s_rp[nl + 1] - p0, cnt);
  }

  // per-output-channel scales are loaded once
  half2v srow[4];
#pragma unroll
  for (int ni = 0; ni < 4; ni++) {
    const int gn = nbase + wn + 16 * ni + li;
    srow[ni] = scale_pair<FMT>((a.kg == 1 && gn < N) ? a.scales[gn] : (uint16_t)0);
  }

  float4v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

  uint4 ra[4], rb[2];
  auto load_tiles = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {  // x tile: 128 rows x 8 uint4
      const int idx = t + 256 * i;
      const int row = idx >> 3, c8 = idx & 7;
      const int gm = bm * BM + row, gk = k0 + 8 * c8;
      ra[i] = make_uint4(0, 0, 0, 0);
      if (gm < M && gk < K) ra[i] = *reinterpret_cast<const uint4*>(a.x + (size_t)gm * K + gk);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {  // code tile: 128 rows x 4 uint4
      const int idx = t + 256 * i;
      const int row = idx >> 2, c16 = idx & 3;
      const int gn = nbase + row, gk = k0 + 16 * c16;
      rb[i] = make_uint4(0, 0, 0, 0);
      if (gn < N && gk < K) rb[i] = ld_nt16(a.codes + (size_t)gn * K + gk);
    }
  };
  auto store_tiles = [&]() {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int idx = t + 256 * i;
      *reinterpret_cast<uint4*>(&As[idx >> 3][8 * (idx & 7)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int idx = t + 256 * i;
      *reinterpret_cast<uint4*>(&Bs[idx >> 2][16 * (idx & 3)]) = rb[i];
    }
  };

  load_tiles(0);
  for (int k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();  // the previous step's LDS reads are done (and the CSR staging, first time)
    store_tiles();
    __syncthreads();
    if (k0 + BK < K) load_tiles(k0 + BK);  // in flight while this step computes
#pragma unroll
    for (int ks = 0; ks < BK / 32; ks++) {
      const int kq = ks * 32 + 8 * grp;
      half8 af[4], bf[4];
#pragma unroll
      for (int mi = 0; mi < 4; mi++) af[mi] = *reinterpret_cast<const half8*>(&As[wm + 16 * mi + li][kq]);
#pragma unroll
      for (int ni = 0; ni < 4; ni++) {
        const int nl = wn + 16 * ni + li;
        const uint2 cw = *reinterpret_cast<const uint2*>(&Bs[nl][kq]);
        half2v s2 = srow[ni];
        if (a.kg != 1) {
          const int gn = nbase + nl, gk = k0 + ks * 32;
          s2 = scale_pair<FMT>((gn < N && gk < K) ? a.scales[scale_index(a, gn, gk)] : (uint16_t)0);
        }
        bf[ni] = deq8<FMT>(cw.x, cw.y, s2);
      }
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mi], bf[ni], acc[mi][ni], 0, 0, 0);
    }
    // outliers whose column lies in [k0, k0 + BK): x from the LDS tile
#pragma unroll
    for (int ni = 0; ni < 4; ni++) {
      while (eptr[ni] < eend[ni] && s_col[eptr[ni]] < k0 + BK) {
        const int c = s_col[eptr[ni]] - k0;
        const float v = (float)bits_to_h(s_val[eptr[ni]]);
#pragma unroll
        for (int mi = 0; mi < 4; mi++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            acc[mi][ni][i] = __builtin_fmaf((float)bits_to_h(As[wm + 16 * mi + 4 * grp + i][c]), v, acc[mi][ni][i]);
        eptr[ni]++;
      }
    }
  }

  const bool overflow = (s_rp[BN] - p0) > kTileCsrCap;
#pragma unroll
  for (int ni = 0; ni < 4; ni++) {
    const int nl = wn + 16 * ni + li;
    const int n = nbase + nl;
    if (n >= N) continue;
    const float bv = a.bias ? (float)bits_to_h(a.bias[n]) : 0.0f;
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = bm * BM + wm + 16 * mi + 4 * grp + i;
        if (m >= M) continue;
        float v = acc[mi][ni][i];
        if (overflow) {  // entries past the staging capacity: from memory
          for (int p = max(p0 + cnt, s_rp[nl]); p < s_rp[nl + 1]; p++)
            v = __builtin_fmaf((float)bits_to_h(a.x[(size_t)m * K + a.cols[p]]), (float)bits_to_h(a.vals[p]), v);
        }
        a.y[(size_t)m * N + n] = h_to_bits(rn_h(v + bv));
      }
  }
}

int log2_exact(int64_t g) {
  if (g <= 0 || (g & (g - 1))) return -1;
  int s = 0;
  while ((int64_t(1) << s) < g) s++;
  return s;
}

}  // namespace

extern "C" int64_t aq_qlinear_workspace_size(int64_t M, int64_t N, int64_t K) {
  (void)M;
  (void)N;
  (void)K;
  return 0;  // the kernels need no memory beyond LDS
}

extern "C" int aq_qlinear(const void* x, int64_t M, int64_t K, int64_t N, const void* codes, const void* scales,
                          int64_t G, int fmt, const int32_t* row_ptr, const int32_t* cols, const void* vals,
                          const void* bias, void* y, void* workspace, int64_t ws_bytes, void* stream) {
  (void)workspace;
  (void)ws_bytes;
  AQ_CHECK_ARG(M >= 0 && K >= 1 && N >= 1, "aq_qlinear: bad sizes M=%lld K=%lld N=%lld", (long long)M,
               (long long)K, (long long)N);
  AQ_CHECK_ARG(G >= 32 && G % 32 == 0 && K % G == 0,
               "aq_qlinear: block size %lld must be a multiple of 32 that divides K=%lld", (long long)G,
               (long long)K);
  AQ_CHECK_ARG(fmt == AQ_FMT_INT8 || fmt == AQ_FMT_E4M3, "aq_qlinear: unknown code format %d", fmt);
  AQ_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && K < (1 << 30) && (int64_t)N * K < ((int64_t)1 << 40),
               "aq_qlinear: dimension too large");
  if (M == 0) return AQ_OK;
  AQ_CHECK_ARG(x && codes && scales && row_ptr && y, "aq_qlinear: null pointer argument");
  AQ_CHECK_ARG((uintptr_t)x % 16 == 0 && (uintptr_t)codes % 16 == 0, "aq_qlinear: x and codes must be 16-byte aligned");
  QLArgs a;
  a.x = (const uint16_t*)x;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.codes = (const uint8_t*)codes;
  a.scales = (const uint16_t*)scales;
  a.G = (int)G;
  a.kg = (int)(K / G);
  a.gshift = log2_exact(G);
  a.row_ptr = row_ptr;
  a.cols = cols;
  a.vals = (const uint16_t*)vals;
  a.bias = (const uint16_t*)bias;
  a.y = (uint16_t*)y;
  hipStream_t s = (hipStream_t)stream;
  if (M <= 16) {
    const dim3 grid((unsigned)aq::ceil_div(N, 16));
    if (fmt == AQ_FMT_E4M3)
      hipLaunchKernelGGL((qlinear_gemv_kernel<AQ_FMT_E4M3>), grid, dim3(64 * (kGemvStream + 1)), 0, s, a);
    else
      hipLaunchKernelGGL((qlinear_gemv_kernel<AQ_FMT_INT8>), grid, dim3(64 * (kGemvStream + 1)), 0, s, a);
    AQ_LAUNCH_CHECK("aq_qlinear: gemv launch");
    return AQ_OK;
  }
  const dim3 grid((unsigned)aq::ceil_div(N, BN), (unsigned)aq::ceil_div(M, BM));
  if (fmt == AQ_FMT_E4M3)
    hipLaunchKernelGGL((qlinear_gemm_kernel<AQ_FMT_E4M3>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((qlinear_gemm_kernel<AQ_FMT_INT8>), grid, dim3(256), 0, s, a);
  AQ_LAUNCH_CHECK("aq_qlinear: gemm launch");
  return AQ_OK;
}
