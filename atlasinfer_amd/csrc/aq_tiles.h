// aq_tiles.h -- building the outlier lists per block of 16 rows x 64 columns
// (the order in which the dequant-GEMM consumes them: block, then row, then
// column), shared by aq_outlier_tiles (from a weight's CSR lists) and
// aq_quantize_finish_tiles (straight from the quantize workspace, in the
// same launch that writes the flat outlier list).
//
// A tile row is 16 rows; its entries come in row, column order (a CSR
// slice).  One workgroup (128 or 256 threads) sorts them stably by 64-column
// chunk: per (row, chunk) counts and first entries in LDS (atomic add,
// atomic min), turned into each chunk's block total and per-row offsets
// within the block; an exclusive scan of the block totals gives the block
// starts; an entry's place is its block's start, the entries of its chunk in
// the rows above, and its rank in its (row, chunk) run, which is contiguous
// in the row's sorted columns: its index minus the run's first.  A thread's
// first kTileRowsRegs entries stay in registers between the two passes.
#pragma once

#include "aq_common.h"

namespace aq {

constexpr int kTileRowsMaxChunks = 480;  // K <= 30720: 33 * 480 ints of LDS (63360 bytes)
constexpr int kTileRowsRegs = 4;

// Position of row r (0..15), column k (0..63) in a block's entry: r << 6 | k.
__device__ __forceinline__ uint32_t block_position(int r, int k) { return ((uint32_t)r << 6) | (uint32_t)k; }

__device__ __forceinline__ int lower_bound_i32(const int32_t* a, int lo, int hi, int key) {
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] < key)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

// Raise *p to at least v.  Many workgroups raise one word: a relaxed read
// first skips the atomic when the word is already that large (it only
// grows, so skipping keeps the maximum), since atomics on one address are
// serialized at the L2 (one per wave over a layer's tile rows took three
// quarters of the tile-row sort's launch).
__device__ __forceinline__ void raise_to(int32_t* p, int v) {
  if (v > __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(p, v);
}

// Row (0..15) of entry i of a tile row whose 17 row starts are rs.
__device__ __forceinline__ int tile_row_of(const int (&rs)[17], int i) {
  int r = 0;
#pragma unroll
  for (int k = 1; k < 16; k++) r += i >= rs[k];
  return r;
}

struct TileEnt {
  int r;         // row in the tile row, 0..15
  int col;       // column, 0..K-1
  uint32_t val;  // fp16 bits
};

// Entries from CSR lists: row starts rs (row_ptr of the tile row's rows),
// columns and values by entry index.
struct CsrTileSrc {
  int rs[17];
  const int32_t* cols;
  const uint16_t* vals;
  __device__ __forceinline__ TileEnt operator()(int i, bool) const {
    return TileEnt{tile_row_of(rs, i), cols[i], (uint32_t)vals[i]};
  }
};

// The counting sort of tile row rb's entries p0 .. p1 - 1 (Src(i, first)
// gives entry i; first is true in the counting pass, false when an entry
// is read again for its placement) by a workgroup of NT threads (128 or
// 256).  sm: 33 * nch ints of LDS; part: NT / 64.  Writes
// tile_ptr[rb * nch + c] for every chunk and the entries, and raises
// *tile_max (if not null) to the largest block.  Every thread of the
// workgroup calls it.
template <int NT, typename Src>
__device__ __forceinline__ void tile_row_sort(const Src& src, int rb, int nch, int p0, int p1, int* sm, int* part,
                                              int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max) {
  static_assert(NT == 128 || NT == 256, "workgroup size");
  int* cnt = sm;                // [16][nch]: counts, then offsets within the block
  int* first = sm + 16 * nch;   // [16][nch]: index of the (row, chunk) run's first entry
  int* bstart = sm + 32 * nch;  // [nch]: block totals, then block starts
  const int t = threadIdx.x;
  // this thread's first entries: their loads go out before the LDS is cleared
  TileEnt ce[kTileRowsRegs];
#pragma unroll
  for (int k = 0; k < kTileRowsRegs; k++) {
    const int i = p0 + t + NT * k;
    ce[k] = i < p1 ? src(i, true) : TileEnt{0, 0, 0u};
  }
  for (int i = t; i < 16 * nch; i += NT) {
    cnt[i] = 0;
    first[i] = 0x7FFFFFFF;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kTileRowsRegs; k++) {
    const int i = p0 + t + NT * k;
    if (i < p1) {
      const int b = ce[k].r * nch + (ce[k].col >> 6);
      atomicAdd(&cnt[b], 1);
      atomicMin(&first[b], i);
    }
  }
  for (int i = p0 + t + NT * kTileRowsRegs; i < p1; i += NT) {
    const TileEnt e = src(i, true);
    const int b = e.r * nch + (e.col >> 6);
    atomicAdd(&cnt[b], 1);
    atomicMin(&first[b], i);
  }
  __syncthreads();
  // per chunk: offsets of the rows within the block, and the block's total
  int mx = 0;
  for (int c = t; c < nch; c += NT) {
    int run = 0;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int n = cnt[r * nch + c];
      cnt[r * nch + c] = run;
      run += n;
    }
    bstart[c] = run;
    mx = max(mx, run);
  }
  // exclusive scan of the block totals: thread t takes chunks 4t..4t+3 of
  // each run of 4 NT, its sum scanned across the workgroup (wave scans, the
  // wave totals through LDS)
  int carry = 0;
  for (int c0 = 0; c0 < nch; c0 += 4 * NT) {
    __syncthreads();
    int v[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int c = c0 + 4 * t + k;
      v[k] = c < nch ? bstart[c] : 0;
      sum += v[k];
    }
    int total;
    int run = carry + team_excl_scan_i32<NT>(sum, part, &total);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int c = c0 + 4 * t + k;
      if (c < nch) {
        bstart[c] = run;
        tile_ptr[(int64_t)rb * nch + c] = p0 + run;
      }
      run += v[k];
    }
    carry += total;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kTileRowsRegs; k++) {
    const int i = p0 + t + NT * k;
    if (i < p1) {
      const int c = ce[k].col >> 6, b = ce[k].r * nch + c;
      tile_ent[p0 + bstart[c] + cnt[b] + (i - first[b])] = (ce[k].val << 16) | block_position(ce[k].r, ce[k].col - c * 64);
    }
  }
  for (int i = p0 + t + NT * kTileRowsRegs; i < p1; i += NT) {
    const TileEnt e = src(i, false);
    const int c = e.col >> 6, b = e.r * nch + c;
    tile_ent[p0 + bstart[c] + cnt[b] + (i - first[b])] = (e.val << 16) | block_position(e.r, e.col - c * 64);
  }
  // the largest block of the tile row: wave maxima through LDS (part is
  // free again after the barrier), one raise per workgroup
  for (int d = 32; d >= 1; d >>= 1) mx = max(mx, __shfl_xor(mx, d));
  if (tile_max) {
    __syncthreads();
    if ((t & 63) == 0) part[t >> 6] = mx;
    __syncthreads();
    if (t == 0) {
#pragma unroll
      for (int w = 1; w < NT / 64; w++) mx = max(mx, part[w]);
      if (mx > 0) raise_to(tile_max, mx);
    }
  }
}

// The block lists from CSR lists whose row r starts at row_ptr[r * rstride]
// (rstride 1: a CSR row pointer; K / G: the block offsets of a weight whose
// blocks tile its rows).  One workgroup per tile row up to
// kTileRowsMaxChunks chunks, one thread per block beyond.  tile_max, if
// not null, must hold 0 (or a count to raise).  Defined in aq_layout.hip.
hipError_t launch_outlier_tiles(const int32_t* row_ptr, int64_t rstride, const int32_t* cols, const uint16_t* vals,
                                int64_t N, int64_t K, int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max,
                                hipStream_t stream);

}  // namespace aq
