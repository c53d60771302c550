// aq_qlinear.hip -- quantized linear forward y = x W^T + b on gfx950.
//
// Replaces QuantizedLinear.forward (reference: integration/atlas_wrappers.py:
// 30-74), which dequantizes the whole weight (dequantize_tensor, :56) and
// calls F.linear on the fp16 result (:67).  Here the weight stays in its
// 1-byte code form in HBM; codes are turned into fp16 weights in registers as
// fp16(value(code) * scale) -- bit for bit the weight dequantize_tensor would
// produce -- and multiplied on the fp16 MFMA units with fp32 accumulation.
// Outlier positions hold code 0; their fp16 values are added from the CSR
// lists in the fp32 epilogue, followed by the bias and one rounding to fp16.
//
//  * M <= 16: "skinny" kernel.  One 16x16x32 MFMA per 16 rows x 32 columns of
//    W; x rows beyond M are zero.  The kernel is HBM-bound (1 byte per weight
//    against 2*M flops), so K is split across the 4 waves of a workgroup and,
//    for narrow W, across workgroups; the last workgroup of a column tile to
//    finish (atomic ticket) sums the partial tiles in a fixed order.
//  * M > 16: tiled GEMM.  128x128 output tile per workgroup, 64-wide K steps;
//    x tile (fp16) and code tile (bytes) staged in LDS, codes dequantized to
//    fp16 MFMA operands in registers.
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
  int kg;  // K / G, scale blocks per row
  const int32_t* row_ptr;
  const int32_t* cols;
  const uint16_t* vals;
  const uint16_t* bias;
  uint16_t* y;
  float* part;
  int32_t* counters;
  int SK;   // workgroups per column tile (split-K)
  int cps;  // 128-wide K chunks per split
};

__device__ __forceinline__ uint32_t perm(uint32_t w, uint32_t sel) { return __builtin_amdgcn_perm(0u, w, sel); }

__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t h2_bits(half2v h) { return __builtin_bit_cast(uint32_t, h); }

// Two codes (bytes 2i, 2i+1 of w) -> fp16 pair holding value(code) * s.
template <int FMT>
__device__ __forceinline__ uint32_t deq_pair(uint32_t w, int hi, half2v s2) {
  const uint32_t p = perm(w, hi ? 0x0C030C02u : 0x0C010C00u);  // [c, 0, c', 0]
  if (FMT == AQ_FMT_E4M3) {
    // fp16 bits of value * 2^-8; s2 carries s * 2^8
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

__device__ __forceinline__ float outlier_dot(const QLArgs& a, int m, int n) {
  float v = 0.0f;
  const int p1 = a.row_ptr[n + 1];
  for (int p = a.row_ptr[n]; p < p1; p++)
    v = __builtin_fmaf((float)bits_to_h(a.x[(size_t)m * a.K + a.cols[p]]), (float)bits_to_h(a.vals[p]), v);
  return v;
}

__device__ __forceinline__ void store_out(const QLArgs& a, int m, int n, float v) {
  v += outlier_dot(a, m, n);
  if (a.bias) v += (float)bits_to_h(a.bias[n]);
  a.y[(size_t)m * a.N + n] = h_to_bits(rn_h(v));
}

// ------------------------------------------------------------ skinny (M <= 16)

template <int R, int FMT>
__global__ __launch_bounds__(256) void qlinear_skinny_kernel(QLArgs a) {
  __shared__ float red[4][R * 256];
  __shared__ int last_flag;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = blockIdx.x / a.SK;
  const int sk = blockIdx.x % a.SK;
  const int n0 = col * 16 * R;
  const int nchunks = (a.K + 127) >> 7;
  const int c_begin = sk * a.cps;
  const int c_end = min(nchunks, c_begin + a.cps);
  const int grp = lane >> 4;
  const int li = lane & 15;

  float4v acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = (float4v){0.f, 0.f, 0.f, 0.f};

  for (int c = c_begin + wave; c < c_end; c += 4) {
    const int kk = c * 128 + 32 * grp;
    const bool kv = kk < a.K;
    uint4 xq[4];
    if (li < a.M && kv) {
      const uint4* xp = reinterpret_cast<const uint4*>(a.x + (size_t)li * a.K + kk);
#pragma unroll
      for (int j = 0; j < 4; j++) xq[j] = xp[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++) xq[j] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int n = n0 + 16 * r + li;
      uint4 q0 = make_uint4(0, 0, 0, 0), q1 = make_uint4(0, 0, 0, 0);
      uint16_t sb = 0;
      if (n < a.N && kv) {
        const uint4* cp = reinterpret_cast<const uint4*>(a.codes + (size_t)n * a.K + kk);
        q0 = ld_nt16(cp);
        q1 = ld_nt16(cp + 1);
        sb = a.scales[(size_t)n * a.kg + kk / a.G];
      }
      const half2v s2 = scale_pair<FMT>(sb);
      const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const half8 wb = deq8<FMT>(qw[2 * j], qw[2 * j + 1], s2);
        const half8 xa = __builtin_bit_cast(half8, xq[j]);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, wb, acc[r], 0, 0, 0);
      }
    }
  }

  // reduce the four waves (C layout: lane l, element i -> m = 4*(l/16)+i, n = l%16)
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave][r * 256 + lane * 4 + i] = acc[r][i];
  __syncthreads();

  float v[R];
#pragma unroll
  for (int q = 0; q < R; q++) {
    const int o = threadIdx.x + 256 * q;
    v[q] = (red[0][o] + red[1][o]) + (red[2][o] + red[3][o]);
  }

  if (a.SK > 1) {
    float* mine = a.part + ((size_t)col * a.SK + sk) * (R * 256);
#pragma unroll
    for (int q = 0; q < R; q++) mine[threadIdx.x + 256 * q] = v[q];
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last_flag = (atomicAdd(&a.counters[col], 1) == a.SK - 1);
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    const float* all = a.part + (size_t)col * a.SK * (R * 256);
#pragma unroll
    for (int q = 0; q < R; q++) {
      const int o = threadIdx.x + 256 * q;
      float s = 0.0f;
      for (int k = 0; k < a.SK; k++) s += __builtin_nontemporal_load(all + (size_t)k * (R * 256) + o);
      v[q] = s;
    }
    if (threadIdx.x == 0) a.counters[col] = 0;  // every ticket of this tile is in: reset for the next call
  }

#pragma unroll
  for (int q = 0; q < R; q++) {
    const int o = threadIdx.x + 256 * q;
    const int r = o >> 8;
    const int l = (o & 255) >> 2;
    const int i = o & 3;
    const int m = 4 * (l >> 4) + i;
    const int n = n0 + 16 * r + (l & 15);
    if (m < a.M && n < a.N) store_out(a, m, n, v[q]);
  }
}

// ------------------------------------------------------------ GEMM (M > 16)

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int APAD = 8;   // halves of padding per LDS row of the x tile
constexpr int BPAD = 16;  // bytes of padding per LDS row of the code tile

template <int FMT>
__global__ __launch_bounds__(256) void qlinear_gemm_kernel(QLArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[BM][BK + APAD];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[BN][BK + BPAD];
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int grp = lane >> 4;
  const int li = lane & 15;
  const int bm = blockIdx.y, bn = blockIdx.x;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

  float4v acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < a.K; k0 += BK) {
#pragma unroll
    for (int i = 0; i < 4; i++) {  // x tile: 128 rows x 8 uint4
      const int idx = t + 256 * i;
      const int row = idx >> 3, c8 = idx & 7;
      const int gm = bm * BM + row, gk = k0 + 8 * c8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (gm < a.M && gk < a.K) v = *reinterpret_cast<const uint4*>(a.x + (size_t)gm * a.K + gk);
      *reinterpret_cast<uint4*>(&As[row][8 * c8]) = v;
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {  // code tile: 128 rows x 4 uint4
      const int idx = t + 256 * i;
      const int row = idx >> 2, c16 = idx & 3;
      const int gn = bn * BN + row, gk = k0 + 16 * c16;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (gn < a.N && gk < a.K) v = *reinterpret_cast<const uint4*>(a.codes + (size_t)gn * a.K + gk);
      *reinterpret_cast<uint4*>(&Bs[row][16 * c16]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BK / 32; ks++) {
      const int kq = ks * 32 + 8 * grp;
      half8 af[4], bf[4];
#pragma unroll
      for (int mi = 0; mi < 4; mi++) af[mi] = *reinterpret_cast<const half8*>(&As[wm + 16 * mi + li][kq]);
      const int gk = k0 + ks * 32;
#pragma unroll
      for (int ni = 0; ni < 4; ni++) {
        const int nl = wn + 16 * ni + li;
        const int gn = bn * BN + nl;
        const uint2 cw = *reinterpret_cast<const uint2*>(&Bs[nl][kq]);
        const uint16_t sb = (gn < a.N && gk < a.K) ? a.scales[(size_t)gn * a.kg + gk / a.G] : (uint16_t)0;
        bf[ni] = deq8<FMT>(cw.x, cw.y, scale_pair<FMT>(sb));
      }
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mi], bf[ni], acc[mi][ni], 0, 0, 0);
    }
    __syncthreads();
  }

#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 4; ni++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = bm * BM + wm + 16 * mi + 4 * grp + i;
        const int n = bn * BN + wn + 16 * ni + li;
        if (m < a.M && n < a.N) store_out(a, m, n, acc[mi][ni][i]);
      }
}

constexpr int kSkinnyR = 2;
// Workspace of the skinny kernel: the split-K tickets first, at a fixed
// offset, so that every call finds them at zero whatever the previous call's
// shape was (each call resets the tickets it used); the partial tiles after.
constexpr int64_t kMaxTickets = 65536;
constexpr int64_t kTicketBytes = kMaxTickets * 4;

struct SkinnyPlan {
  int ncol, SK, cps;
};

SkinnyPlan plan_skinny(int64_t N, int64_t K) {
  SkinnyPlan p;
  p.ncol = (int)aq::ceil_div(N, 16 * kSkinnyR);
  const int nchunks = (int)aq::ceil_div(K, 128);
  // enough workgroups to cover the 256 CUs several times, each split keeping
  // at least one 128-wide chunk per wave
  int sk = (int)aq::ceil_div(1024, p.ncol);
  sk = std::min(sk, std::max(1, nchunks / 4));
  sk = std::max(sk, 1);
  if (p.ncol > kMaxTickets) sk = 1;
  p.cps = (int)aq::ceil_div(nchunks, sk);
  p.SK = (int)aq::ceil_div(nchunks, p.cps);
  return p;
}

int64_t skinny_ws_bytes(int64_t N, int64_t K) {
  SkinnyPlan p = plan_skinny(N, K);
  if (p.SK <= 1) return 256;
  return kTicketBytes + (int64_t)p.ncol * p.SK * kSkinnyR * 256 * 4;
}

}  // namespace

extern "C" int64_t aq_qlinear_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (M <= 16) return skinny_ws_bytes(N, K);
  return 256;
}

extern "C" int aq_qlinear(const void* x, int64_t M, int64_t K, int64_t N, const void* codes, const void* scales,
                          int64_t G, int fmt, const int32_t* row_ptr, const int32_t* cols, const void* vals,
                          const void* bias, void* y, void* workspace, int64_t ws_bytes, void* stream) {
  AQ_CHECK_ARG(M >= 0 && K >= 1 && N >= 1, "aq_qlinear: bad sizes M=%lld K=%lld N=%lld", (long long)M,
               (long long)K, (long long)N);
  AQ_CHECK_ARG(G >= 32 && G % 32 == 0 && K % G == 0,
               "aq_qlinear: block size %lld must be a multiple of 32 that divides K=%lld", (long long)G,
               (long long)K);
  AQ_CHECK_ARG(fmt == AQ_FMT_INT8 || fmt == AQ_FMT_E4M3, "aq_qlinear: unknown code format %d", fmt);
  AQ_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), "aq_qlinear: dimension too large");
  if (M == 0) return AQ_OK;
  AQ_CHECK_ARG(x && codes && scales && row_ptr && y, "aq_qlinear: null pointer argument");
  AQ_CHECK_ARG((uintptr_t)x % 16 == 0 && (uintptr_t)codes % 16 == 0, "aq_qlinear: x and codes must be 16-byte aligned");
  const int64_t need = aq_qlinear_workspace_size(M, N, K);
  if (ws_bytes < need)
    return aq::set_error(AQ_EWORKSPACE, "aq_qlinear: workspace of %lld bytes, %lld needed", (long long)ws_bytes,
                         (long long)need);
  QLArgs a;
  a.x = (const uint16_t*)x;
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.codes = (const uint8_t*)codes;
  a.scales = (const uint16_t*)scales;
  a.G = (int)G;
  a.kg = (int)(K / G);
  a.row_ptr = row_ptr;
  a.cols = cols;
  a.vals = (const uint16_t*)vals;
  a.bias = (const uint16_t*)bias;
  a.y = (uint16_t*)y;
  a.part = nullptr;
  a.counters = nullptr;
  a.SK = 1;
  a.cps = 0;
  hipStream_t s = (hipStream_t)stream;
  if (M <= 16) {
    SkinnyPlan p = plan_skinny(N, K);
    a.SK = p.SK;
    a.cps = p.cps;
    if (p.SK > 1) {
      AQ_CHECK_ARG(workspace, "aq_qlinear: null workspace");
      a.counters = (int32_t*)workspace;
      a.part = (float*)((char*)workspace + kTicketBytes);
    }
    const dim3 grid((unsigned)(p.ncol * p.SK));
    if (fmt == AQ_FMT_E4M3)
      hipLaunchKernelGGL((qlinear_skinny_kernel<kSkinnyR, AQ_FMT_E4M3>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((qlinear_skinny_kernel<kSkinnyR, AQ_FMT_INT8>), grid, dim3(256), 0, s, a);
    AQ_LAUNCH_CHECK("aq_qlinear: skinny launch");
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
