// aq_layout.hip -- outlier index bookkeeping, the reference's compacted code
// stream, and dequantization.
//
// Reference: atlasinfer_core/quant/adaptive_quantizer.py
//   compacted stream of non-outlier codes     :110,125-126,136 (written)
//                                             :209-212         (read back)
//   dequantize_tensor per-block loop          :185-245
// The reference finds the outliers of each block by comparing against all
// outlier indices (O(blocks * nnz)) and syncs to the host once per block
// (:194-195,234).  Here a workgroup owns a 4096-element tile, finds its slice
// of the ascending index list with two binary searches, stages it in LDS, and
// every thread walks its 16 elements against it.
#include "aq_common.h"
#include "aq_tiles.h"

namespace {

constexpr int kTile = 4096;  // elements per workgroup (256 threads x 16)

__device__ __forceinline__ int64_t lower_bound_i64(const int64_t* a, int64_t n, int64_t key) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    int64_t mid = (lo + hi) >> 1;
    if (a[mid] < key)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(256) void segment_offsets_kernel(const int64_t* idx, int64_t nnz, int64_t nseg,
                                                              int64_t seg_len, int32_t* seg_ptr) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s > nseg) return;
  seg_ptr[s] = (int32_t)lower_bound_i64(idx, nnz, s * seg_len);
}

__global__ __launch_bounds__(256) void outlier_cols_kernel(const int64_t* idx, int64_t nnz, int64_t K,
                                                           int32_t* cols) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p < nnz) cols[p] = (int32_t)(idx[p] % K);
}

// MODE 0: compact (dense -> stream); MODE 1: expand (stream -> dense).
template <int MODE>
__global__ __launch_bounds__(256) void reorder_codes_kernel(const uint8_t* src, int64_t padded, const int64_t* idx,
                                                            int64_t nnz, uint8_t* dst) {
  __shared__ int64_t lb[2];
  __shared__ int16_t local[kTile];
  const int64_t t0 = (int64_t)blockIdx.x * kTile;
  const int64_t t1 = min(padded, t0 + kTile);
  if (threadIdx.x < 2) lb[threadIdx.x] = lower_bound_i64(idx, nnz, threadIdx.x ? t1 : t0);
  __syncthreads();
  const int64_t lb0 = lb[0];
  const int cnt = (int)(lb[1] - lb0);
  for (int i = threadIdx.x; i < cnt; i += 256) local[i] = (int16_t)(idx[lb0 + i] - t0);
  __syncthreads();
  const int e0 = threadIdx.x * 16;
  // outliers of this tile before element e0
  int lo = 0, hi = cnt;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (local[mid] < e0)
      lo = mid + 1;
    else
      hi = mid;
  }
  int k = lo;
  for (int e = e0; e < e0 + 16; e++) {
    const int64_t j = t0 + e;
    if (j >= t1) break;
    const bool out = (k < cnt) && (local[k] == e);
    const int64_t cpos = j - (lb0 + k);  // position in the compacted stream
    if (MODE == 0) {
      if (!out) dst[cpos] = src[j];
    } else {
      dst[j] = out ? (uint8_t)0 : src[cpos];
    }
    k += out;
  }
}

// Flat <-> tiled: one thread moves one 16-byte piece (16 consecutive codes of
// a row occupy 16 consecutive bytes in both layouts).
template <int TO_TILED>
__global__ __launch_bounds__(256) void retile_kernel(const uint8_t* src, int64_t N, int64_t K, uint8_t* dst) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p * 16 >= N * K) return;
  const int64_t j = p * 16;
  const int64_t t = tiled_offset(j / K, j % K, K / 128);
  if (TO_TILED)
    *reinterpret_cast<uint4*>(dst + t) = *reinterpret_cast<const uint4*>(src + j);
  else
    *reinterpret_cast<uint4*>(dst + j) = *reinterpret_cast<const uint4*>(src + t);
}

template <int FMT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* codes, const uint16_t* scales, int64_t numel,
                                                      int64_t G, uint16_t* out, int vec, int tiled, int64_t K) {
  const int64_t j0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;
  if (j0 >= numel) return;
  uint8_t c[16];
  const bool full = vec && (j0 + 16 <= numel);
  if (tiled) {  // numel is a multiple of 16 K here
    uint4 u = *reinterpret_cast<const uint4*>(codes + tiled_offset(j0 / K, j0 % K, K / 128));
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 16; k++) c[k] = (uint8_t)(w[k / 4] >> (8 * (k % 4)));
  } else if (full) {
    uint4 u = *reinterpret_cast<const uint4*>(codes + j0);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 16; k++) c[k] = (uint8_t)(w[k / 4] >> (8 * (k % 4)));
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++) c[k] = (j0 + k < numel) ? codes[j0 + k] : 0;
  }
  int64_t b = j0 / G;
  int64_t next = (b + 1) * G;
  f16 s = bits_to_h(scales[b]);
  uint16_t o[16];
#pragma unroll
  for (int k = 0; k < 16; k++) {
    if (j0 + k == next) {
      b++;
      next += G;
      if (j0 + k < numel) s = bits_to_h(scales[b]);
    }
    // code value and scale are exact fp16 values: one native fp16 multiply
    // is the single rounding of the exact product (and keeps the sign of 0,
    // which a widened multiply fused with a +0 addend would not)
    const f16 v = FMT == AQ_FMT_INT8 ? (f16)(int8_t)c[k] : e4m3_to_h(c[k]);
    o[k] = h_to_bits(v * s);
  }
  if (full) {
    uint4* dst = reinterpret_cast<uint4*>(out + j0);
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; k++) w[k] = (uint32_t)o[2 * k] | ((uint32_t)o[2 * k + 1] << 16);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
  } else {
#pragma unroll
    for (int k = 0; k < 16; k++)
      if (j0 + k < numel) out[j0 + k] = o[k];
  }
}

__global__ __launch_bounds__(256) void scatter_outliers_kernel(const int64_t* idx, const uint16_t* vals, int64_t nnz,
                                                               int64_t numel, uint16_t* out) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= nnz) return;
  const int64_t j = idx[p];
  if (j >= 0 && j < numel) out[j] = vals[p];
}

using aq::block_position;
using aq::lower_bound_i32;
using aq::raise_to;

// One workgroup per tile row (aq_tiles.h); workgroup nrb writes the list's
// end and the 64 padding entries.  LDS: 33 * nch ints.
__global__ __launch_bounds__(256) void outlier_tile_rows_kernel(const int32_t* row_ptr, int64_t rstride,
                                                                const int32_t* cols, const uint16_t* vals, int nrb,
                                                                int nch, int32_t* tile_ptr, uint32_t* tile_ent,
                                                                int32_t* tile_max) {
  extern __shared__ int sm[];
  __shared__ int part[4];
  const int rb = blockIdx.x, t = threadIdx.x;
  if (rb == nrb) {
    const int end = row_ptr[(int64_t)nrb * 16 * rstride];
    if (t == 0) tile_ptr[(int64_t)nrb * nch] = end;
    if (t < 64) tile_ent[end + t] = 0u;
    return;
  }
  aq::CsrTileSrc src;
#pragma unroll
  for (int r = 0; r <= 16; r++) src.rs[r] = row_ptr[(int64_t)(rb * 16 + r) * rstride];
  src.cols = cols;
  src.vals = vals;
  aq::tile_row_sort<256>(src, rb, nch, src.rs[0], src.rs[16], sm, part, tile_ptr, tile_ent, tile_max);
}

// One thread per block of 16 rows x 64 columns (tile row rb, chunk c), for
// rows wider than outlier_tile_rows_kernel takes.  Entries are ordered by
// block, then row, then column, so a block starts after every outlier of
// the rows above it plus, in each of its own rows, the outliers left of
// column 64c.
__global__ __launch_bounds__(256) void outlier_tiles_kernel(const int32_t* row_ptr, int64_t rstride,
                                                            const int32_t* cols, const uint16_t* vals, int nrb,
                                                            int nch, int32_t* tile_ptr, uint32_t* tile_ent,
                                                            int32_t* tile_max) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nblk = (int64_t)nrb * nch;
  if (b > nblk) return;
  if (b == nblk) {
    const int end = row_ptr[(int64_t)nrb * 16 * rstride];
    tile_ptr[b] = end;
    for (int k = 0; k < 64; k++) tile_ent[end + k] = 0u;
    return;
  }
  const int rb = (int)(b / nch), c = (int)(b % nch);
  if (c == 0 && tile_max) {
    int mx = 0;
    for (int cc = 0; cc < nch; cc++) {
      int n = 0;
      for (int r = 0; r < 16; r++) {
        const int p0 = row_ptr[(int64_t)(rb * 16 + r) * rstride], p1 = row_ptr[(int64_t)(rb * 16 + r + 1) * rstride];
        n += lower_bound_i32(cols, p0, p1, cc * 64 + 64) - lower_bound_i32(cols, p0, p1, cc * 64);
      }
      mx = max(mx, n);
    }
    if (mx > 0) raise_to(tile_max, mx);
  }
  int lo[16], hi[16];
  int pos = row_ptr[(int64_t)rb * 16 * rstride];
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int p0 = row_ptr[(int64_t)(rb * 16 + r) * rstride], p1 = row_ptr[(int64_t)(rb * 16 + r + 1) * rstride];
    lo[r] = lower_bound_i32(cols, p0, p1, c * 64);
    hi[r] = lower_bound_i32(cols, lo[r], p1, c * 64 + 64);
    pos += lo[r] - p0;
  }
  tile_ptr[b] = pos;
#pragma unroll
  for (int r = 0; r < 16; r++)
    for (int p = lo[r]; p < hi[r]; p++)
      tile_ent[pos++] = ((uint32_t)vals[p] << 16) | block_position(r, cols[p] - c * 64);
}

}  // namespace

extern "C" int aq_segment_offsets(const int64_t* flat_idx, int64_t nnz, int64_t nseg, int64_t seg_len,
                                  int32_t* seg_ptr, void* stream) {
  AQ_CHECK_ARG(nnz >= 0 && nseg >= 0 && seg_len >= 1, "aq_segment_offsets: bad sizes");
  AQ_CHECK_ARG(seg_ptr && (nnz == 0 || flat_idx), "aq_segment_offsets: null pointer argument");
  AQ_CHECK_ARG(nnz < ((int64_t)1 << 31), "aq_segment_offsets: nnz exceeds int32");
  const int64_t grid = aq::ceil_div(nseg + 1, 256);
  hipLaunchKernelGGL(segment_offsets_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, flat_idx, nnz,
                     nseg, seg_len, seg_ptr);
  AQ_LAUNCH_CHECK("aq_segment_offsets: launch");
  return AQ_OK;
}

extern "C" int aq_outlier_cols(const int64_t* flat_idx, int64_t nnz, int64_t K, int32_t* cols, void* stream) {
  AQ_CHECK_ARG(nnz >= 0 && K >= 1, "aq_outlier_cols: bad sizes");
  if (nnz == 0) return AQ_OK;
  AQ_CHECK_ARG(flat_idx && cols, "aq_outlier_cols: null pointer argument");
  hipLaunchKernelGGL(outlier_cols_kernel, dim3((unsigned)aq::ceil_div(nnz, 256)), dim3(256), 0, (hipStream_t)stream,
                     flat_idx, nnz, K, cols);
  AQ_LAUNCH_CHECK("aq_outlier_cols: launch");
  return AQ_OK;
}

static int reorder(int mode, const void* src, int64_t padded, const int64_t* idx, int64_t nnz, void* dst,
                   void* stream, const char* name) {
  AQ_CHECK_ARG(padded >= 0 && nnz >= 0 && nnz <= padded, "%s: bad sizes", name);
  if (padded == 0) return AQ_OK;
  AQ_CHECK_ARG(dst && (nnz == padded || src) && (nnz == 0 || idx), "%s: null pointer argument", name);
  const int64_t grid = aq::ceil_div(padded, kTile);
  if (mode == 0)
    hipLaunchKernelGGL((reorder_codes_kernel<0>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)src, padded, idx, nnz, (uint8_t*)dst);
  else
    hipLaunchKernelGGL((reorder_codes_kernel<1>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)src, padded, idx, nnz, (uint8_t*)dst);
  AQ_LAUNCH_CHECK(name);
  return AQ_OK;
}

extern "C" int aq_compact_codes(const void* dense, int64_t padded, const int64_t* flat_idx, int64_t nnz,
                                void* compact, void* stream) {
  if (padded == nnz) return AQ_OK;  // every element is an outlier: empty stream
  return reorder(0, dense, padded, flat_idx, nnz, compact, stream, "aq_compact_codes");
}

extern "C" int aq_expand_codes(const void* compact, int64_t padded, const int64_t* flat_idx, int64_t nnz,
                               void* dense, void* stream) {
  return reorder(1, compact, padded, flat_idx, nnz, dense, stream, "aq_expand_codes");
}

static int retile(int to_tiled, const void* src, int64_t N, int64_t K, void* dst, void* stream, const char* name) {
  AQ_CHECK_ARG(N >= 0 && K >= 128 && N % 16 == 0 && K % 128 == 0,
               "%s: needs N %% 16 == 0 and K %% 128 == 0 (N=%lld, K=%lld)", name, (long long)N, (long long)K);
  if (N == 0) return AQ_OK;
  AQ_CHECK_ARG(src && dst && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0,
               "%s: null or unaligned pointer", name);
  const int64_t grid = aq::ceil_div(N * K / 16, 256);
  if (to_tiled)
    hipLaunchKernelGGL((retile_kernel<1>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)src, N, K, (uint8_t*)dst);
  else
    hipLaunchKernelGGL((retile_kernel<0>), dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)src, N, K, (uint8_t*)dst);
  AQ_LAUNCH_CHECK(name);
  return AQ_OK;
}

extern "C" int aq_tile_codes(const void* flat, int64_t N, int64_t K, void* tiled, void* stream) {
  return retile(1, flat, N, K, tiled, stream, "aq_tile_codes");
}

extern "C" int aq_untile_codes(const void* tiled, int64_t N, int64_t K, void* flat, void* stream) {
  return retile(0, tiled, N, K, flat, stream, "aq_untile_codes");
}

extern "C" int aq_dequantize(const void* codes, const void* scales, int64_t numel, int64_t G, int fmt, int64_t K,
                             int layout, const int64_t* flat_idx, const void* vals, int64_t nnz, void* out,
                             void* stream) {
  AQ_CHECK_ARG(numel >= 0 && G >= 1 && nnz >= 0, "aq_dequantize: bad sizes");
  AQ_CHECK_ARG(fmt == AQ_FMT_INT8 || fmt == AQ_FMT_E4M3, "aq_dequantize: unknown code format %d", fmt);
  AQ_CHECK_ARG(layout == AQ_LAYOUT_FLAT || layout == AQ_LAYOUT_TILED, "aq_dequantize: unknown layout %d", layout);
  if (numel == 0) return AQ_OK;
  AQ_CHECK_ARG(codes && scales && out && (nnz == 0 || (flat_idx && vals)), "aq_dequantize: null pointer argument");
  const int tiled = layout == AQ_LAYOUT_TILED;
  if (tiled)
    AQ_CHECK_ARG(K >= 128 && K % 128 == 0 && numel % (16 * K) == 0 && (uintptr_t)codes % 16 == 0,
                 "aq_dequantize: tiled codes need K %% 128 == 0 and rows %% 16 == 0");
  hipStream_t s = (hipStream_t)stream;
  const int vec = ((uintptr_t)codes % 16 == 0) && ((uintptr_t)out % 16 == 0);
  const int64_t grid = aq::ceil_div(numel, 256 * 16);
  if (fmt == AQ_FMT_INT8)
    hipLaunchKernelGGL((dequant_kernel<AQ_FMT_INT8>), dim3((unsigned)grid), dim3(256), 0, s, (const uint8_t*)codes,
                       (const uint16_t*)scales, numel, G, (uint16_t*)out, vec, tiled, K);
  else
    hipLaunchKernelGGL((dequant_kernel<AQ_FMT_E4M3>), dim3((unsigned)grid), dim3(256), 0, s, (const uint8_t*)codes,
                       (const uint16_t*)scales, numel, G, (uint16_t*)out, vec, tiled, K);
  AQ_LAUNCH_CHECK("aq_dequantize: launch");
  if (nnz > 0) {
    hipLaunchKernelGGL(scatter_outliers_kernel, dim3((unsigned)aq::ceil_div(nnz, 256)), dim3(256), 0, s, flat_idx,
                       (const uint16_t*)vals, nnz, numel, (uint16_t*)out);
    AQ_LAUNCH_CHECK("aq_dequantize: scatter launch");
  }
  return AQ_OK;
}

hipError_t aq::launch_outlier_tiles(const int32_t* row_ptr, int64_t rstride, const int32_t* cols, const uint16_t* vals,
                                   int64_t N, int64_t K, int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max,
                                   hipStream_t stream) {
  const int64_t nblk = (N / 16) * (K / 64);
  if (K / 64 <= aq::kTileRowsMaxChunks)
    hipLaunchKernelGGL(outlier_tile_rows_kernel, dim3((unsigned)(N / 16 + 1)), dim3(256),
                       (size_t)33 * (K / 64) * sizeof(int), stream, row_ptr, rstride, cols, vals, (int)(N / 16),
                       (int)(K / 64), tile_ptr, tile_ent, tile_max);
  else
    hipLaunchKernelGGL(outlier_tiles_kernel, dim3((unsigned)aq::ceil_div(nblk + 1, 256)), dim3(256), 0, stream,
                       row_ptr, rstride, cols, vals, (int)(N / 16), (int)(K / 64), tile_ptr, tile_ent, tile_max);
  return hipGetLastError();
}

extern "C" int aq_outlier_tiles(const int32_t* row_ptr, const int32_t* cols, const void* vals, int64_t N, int64_t K,
                                int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max, void* stream) {
  AQ_CHECK_ARG(N >= 16 && N % 16 == 0 && K >= 64 && K % 64 == 0 && N < (1 << 30) && K < (1 << 30) &&
                   (N / 16) * (K / 64) < ((int64_t)1 << 31),
               "aq_outlier_tiles: N must be a multiple of 16 and K of 64 (N=%lld K=%lld)", (long long)N,
               (long long)K);
  AQ_CHECK_ARG(row_ptr && tile_ptr, "aq_outlier_tiles: null pointer argument");
  const hipError_t e = aq::launch_outlier_tiles(row_ptr, 1, cols, (const uint16_t*)vals, N, K, tile_ptr, tile_ent,
                                                tile_max, (hipStream_t)stream);
  if (e != hipSuccess) return aq::check_hip(e, "aq_outlier_tiles: launch");
  return AQ_OK;
}
