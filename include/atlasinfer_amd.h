/*
 * atlasinfer_amd.h -- C ABI of libatlasinfer_amd.so, the MI355X (gfx950)
 * implementation of AtlasInfer's adaptive hybrid weight quantization path.
 *
 * Conventions
 *   - extern "C", plain pointers and sizes; no C++ or torch types.
 *   - Every pointer argument is device memory owned by the caller, unless the
 *     comment says otherwise.  No call allocates device memory; scratch space
 *     comes in through a caller-owned workspace argument whose size the
 *     matching *_workspace_size() call returns, except for
 *     aq_qlinear_noalloc, whose scratch is a static device array of the
 *     library (AQ_NOALLOC_SCRATCH_BYTES per GPU, held until process exit).
 *   - Every call enqueues work on `stream` (a hipStream_t, passed as void*)
 *     and returns without synchronising.
 *   - Return value: AQ_OK (0) or a negative AQ_E* code; aq_last_error()
 *     returns a thread-local message describing the last failure.
 *   - fp16 data is passed as IEEE binary16 bit patterns (uint16_t storage).
 *   - Code formats: AQ_FMT_INT8 is the reference's int8 symmetric code
 *     (adaptive_quantizer.py:100,119-126); AQ_FMT_E4M3 is OCP FP8 E4M3 (fn).
 *
 * Data layout of a quantized weight W[N, K] (row-major, the nn.Linear layout)
 * with block size G over the flat, zero-padded tensor (padded = ceil(N*K/G)*G):
 *   codes     uint8  [padded]        one code per element, 0 at outliers, in
 *                                    the flat (element) order or tiled (below)
 *   scales    fp16   [padded / G]    one scale per block
 *   flat_idx  int64  [nnz]           ascending flat indices of outliers
 *   vals      fp16   [nnz]           outlier values (verbatim)
 *   row_ptr   int32  [N + 1]         CSR row pointer over the outliers (< N*K)
 *   cols      int32  [nnz]           column of each outlier (flat_idx % K)
 *
 * Tiled code layout (AQ_LAYOUT_TILED; needs N % 16 == 0, K % 128 == 0): W is
 * cut into tiles of 16 rows x 128 columns, 2 KiB each, tile (rb, c) at byte
 * (rb * K/128 + c) * 2048.  Inside a tile, byte h*1024 + (g*16 + r)*16 + e
 * holds the code of row 16*rb + r, column 128*c + 64*h + 16*g + e.  This is
 * the order in which a wave of 64 lanes feeds 16x16x32 MFMAs, so the
 * quantized-linear kernels read it with fully contiguous 1 KiB loads.
 */
#ifndef ATLASINFER_AMD_H
#define ATLASINFER_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AQ_ABI_VERSION 10

enum { AQ_FMT_INT8 = 0, AQ_FMT_E4M3 = 1 };
enum { AQ_LAYOUT_FLAT = 0, AQ_LAYOUT_TILED = 1 };
enum { AQ_OK = 0, AQ_EINVAL = -1, AQ_EHIP = -2, AQ_EUNSUPPORTED = -3, AQ_EWORKSPACE = -4 };

/* ABI version of the loaded library (AQ_ABI_VERSION at build time). */
int aq_abi_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* aq_last_error(void);

/* Largest block size aq_quantize accepts (65536). */
int64_t aq_max_block_size(void);

/*
 * Quantize, phase 1 of 2.  Replaces the per-block loop of quantize_tensor
 * (reference: atlasinfer_core/quant/adaptive_quantizer.py:84-133).
 * For every block of G elements of the zero-padded flat fp16 tensor x[numel]:
 * z-score statistics, outlier flags (|z| > z_thr), scale, codes; the outliers
 * of each block are staged in the workspace and counted, and the exclusive
 * prefix sum of the counts is written to block_off.
 *   x          fp16 [numel]
 *   z_thr_f16  fp16 bits of the threshold (the reference compares in fp16)
 *   K, layout  row length and code layout (AQ_LAYOUT_TILED needs K % 128 == 0,
 *              numel % (16 K) == 0, G % 16 == 0 and K % G == 0)
 *   codes      uint8 [padded]          (out)
 *   scales     fp16  [padded / G]      (out)
 *   block_off  int32 [padded / G + 1]  (out) block_off[nblocks] = total nnz
 *   workspace  >= aq_quantize_workspace_size(numel, G) bytes, kept intact
 *              until aq_quantize_finish has run.
 */
int64_t aq_quantize_workspace_size(int64_t numel, int64_t G);
int aq_quantize(const void* x, int64_t numel, int64_t G, uint16_t z_thr_f16, int fmt, int64_t K, int layout,
                void* codes, void* scales, int32_t* block_off, void* workspace, int64_t workspace_bytes,
                void* stream);

/*
 * aq_quantize for up to 8 weights of one block size G (and K, format,
 * layout) in one launch of the quantize kernel and one of the scan: per
 * member i the arguments of aq_quantize (xs[i], numels[i], codes[i],
 * scales[i], block_offs[i], workspaces[i] of ws_bytes[i]), each with at
 * most 16384 blocks.  Results are those of aq_quantize on each member, bit
 * for bit.  totals (device int32[count], or NULL) receives each member's
 * outlier count (block_offs[i][nblocks_i]) as well, so that a caller sizing
 * the outlier lists reads them all with one copy.  No counterpart of its
 * own in the reference (its quantize_tensor,
 * adaptive_quantizer.py:51-148, takes one tensor; the model swap,
 * model_modifier.py:95-143, calls it once per Linear): for callers that
 * quantize a layer's weights together, whose small members alone fill the
 * GPU for one round of waves at most.
 */
int aq_quantize_grouped(int64_t count, const void* const* xs, const int64_t* numels, int64_t G, uint16_t z_thr_f16,
                        int fmt, int64_t K, int layout, void* const* codes, void* const* scales,
                        int32_t* const* block_offs, void* const* workspaces, const int64_t* ws_bytes,
                        int32_t* totals, void* stream);

/*
 * Quantize, phase 2 of 2: write the outlier list in ascending flat order
 * (the reference's fp16_outliers / outlier_indices, adaptive_quantizer.py:
 * 109-117,137-138) plus the column of each outlier for row width K.
 *   nnz        block_off[nblocks] as read back by the caller
 *   flat_idx   int64 [nnz] (out)     vals fp16 [nnz] (out)
 *   cols       int32 [nnz] (out, may be NULL)
 */
int aq_quantize_finish(int64_t numel, int64_t G, int64_t K, const int32_t* block_off, int64_t nnz,
                       const void* workspace, int64_t workspace_bytes, int64_t* flat_idx, void* vals,
                       int32_t* cols, void* stream);

/*
 * seg_ptr[s] = number of outliers with flat index < s * seg_len, for
 * s = 0..nseg (CSR row pointer with seg_len = K, block offsets with
 * seg_len = G).  flat_idx must be ascending.
 */
int aq_segment_offsets(const int64_t* flat_idx, int64_t nnz, int64_t nseg, int64_t seg_len,
                       int32_t* seg_ptr, void* stream);

/* cols[p] = flat_idx[p] % K. */
int aq_outlier_cols(const int64_t* flat_idx, int64_t nnz, int64_t K, int32_t* cols, void* stream);

/*
 * Outlier lists per block of 16 rows x 64 columns, the order in which the
 * dequant-GEMM consumes them (no counterpart in the reference, whose
 * dequantize_tensor scans all outlier indices per block,
 * adaptive_quantizer.py:194-201).  Needs N % 16 == 0, K % 64 == 0.
 *   tile_ptr int32  [(N/16) * (K/64) + 1]   block (rb, c) = rows 16rb..16rb+15,
 *                                           columns 64c..64c+63, at index
 *                                           rb * (K/64) + c; entries
 *                                           tile_ptr[b] .. tile_ptr[b+1]-1
 *   tile_ent uint32 [nnz + 64]              (fp16 value << 16) | r << 6 | k
 *                                           for row r (0..15) and column k
 *                                           (0..63) in the block;
 *                                           ordered by block, row, column; the
 *                                           last 64 slots are padding the
 *                                           kernels may read but never use
 *                                           (written as 0)
 *   tile_max int32  [1] or NULL             raised (atomic max) to the largest
 *                                           block's count; the caller sets it
 *                                           to 0 first
 * from the CSR lists (row_ptr, cols, vals) of the same outliers.
 */
int aq_outlier_tiles(const int32_t* row_ptr, const int32_t* cols, const void* vals, int64_t N, int64_t K,
                     int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max, void* stream);

/*
 * aq_quantize_finish (with cols) and aq_outlier_tiles of the same weight in
 * one launch, read straight from the quantize workspace: the flat list and
 * the block lists, bit for bit those of the two calls.  For weights
 * quantized with blocks that tile the rows (K % G == 0) and whose [N, K]
 * view has N % 16 == 0 and K % 64 == 0 (every weight quantized into the
 * tiled layout); rows wider than 30720 take two launches inside.  Same
 * arguments as the two calls; cols is required (non-NULL when nnz > 0),
 * tile_ptr and tile_ent always, tile_max may be NULL (else the caller sets
 * it to 0 first).  Serves the reference's quantize_tensor
 * (adaptive_quantizer.py:109-117,137-138) for callers that also want the
 * block lists the dequant-GEMM reads.
 */
int aq_quantize_finish_tiles(int64_t numel, int64_t G, int64_t K, const int32_t* block_off, int64_t nnz,
                             const void* workspace, int64_t workspace_bytes, int64_t* flat_idx, void* vals,
                             int32_t* cols, int32_t* tile_ptr, uint32_t* tile_ent, int32_t* tile_max, void* stream);

/*
 * aq_quantize_finish_tiles for up to 8 weights of one block size G and row
 * length K in one launch (the members of an aq_quantize_grouped call): per
 * member i the arguments of aq_quantize_finish_tiles (numels[i],
 * block_offs[i], nnzs[i], workspaces[i] of ws_bytes[i], flat_idx[i],
 * vals[i], cols[i], tile_ptrs[i], tile_ents[i]); tile_max, if not NULL,
 * points to count zeroed counts, member i's at tile_max[i].  Results are
 * those of aq_quantize_finish_tiles on each member, bit for bit.  No
 * counterpart of its own in the reference (quantize_tensor,
 * adaptive_quantizer.py:109-117,137-138, finishes one tensor): for callers
 * that quantize a layer's weights together.
 */
int aq_quantize_finish_tiles_grouped(int64_t count, const int64_t* numels, int64_t G, int64_t K,
                                     const int32_t* const* block_offs, const int64_t* nnzs,
                                     const void* const* workspaces, const int64_t* ws_bytes,
                                     int64_t* const* flat_idx, void* const* vals, int32_t* const* cols,
                                     int32_t* const* tile_ptrs, uint32_t* const* tile_ents, int32_t* tile_max,
                                     void* stream);

/*
 * Reference layout <-> dense flat codes.  The reference stores only the codes
 * of non-outliers, in element order (adaptive_quantizer.py:110,125-126,136;
 * read back at :209-212).
 *   aq_compact_codes: dense[padded] -> compact[padded - nnz]
 *   aq_expand_codes:  compact[padded - nnz] -> dense[padded] (0 at outliers)
 */
int aq_compact_codes(const void* dense, int64_t padded, const int64_t* flat_idx, int64_t nnz,
                     void* compact, void* stream);
int aq_expand_codes(const void* compact, int64_t padded, const int64_t* flat_idx, int64_t nnz,
                    void* dense, void* stream);

/* Flat <-> tiled code layout of a [N, K] code matrix (N % 16 == 0, K % 128 == 0). */
int aq_tile_codes(const void* flat, int64_t N, int64_t K, void* tiled, void* stream);
int aq_untile_codes(const void* tiled, int64_t N, int64_t K, void* flat, void* stream);

/*
 * Dequantize (reference: dequantize_tensor, adaptive_quantizer.py:185-245):
 * out[j] = fp16(value(codes[j]) * scales[j / G]) for j < numel, then
 * out[flat_idx[p]] = vals[p] for flat_idx[p] < numel.  codes in `layout`
 * (tiled codes: rows of K).
 */
int aq_dequantize(const void* codes, const void* scales, int64_t numel, int64_t G, int fmt, int64_t K, int layout,
                  const int64_t* flat_idx, const void* vals, int64_t nnz, void* out, void* stream);

/*
 * calculate_zscore_manual (adaptive_quantizer.py:44-49) of x[n] as one
 * block: z = fp16(fp16(x - mean) / fp16(std + eps)).  stats (may be NULL)
 * receives (mean, std, std + eps) as fp16.  n <= aq_max_block_size().
 */
int aq_zscore(const void* x, int64_t n, float eps, void* z, void* stats, void* stream);

/*
 * Quantized linear forward y = x W^T + b with W given by its quantized form
 * (reference: QuantizedLinear.forward, integration/atlas_wrappers.py:30-74,
 * which computes F.linear(x, dequantize_tensor(W), b) at :56,67).
 *   x       fp16 [M, K] row-major, 16-byte aligned    y fp16 [M, N] (out)
 *   codes   tiled layout; N % 16 == 0, K % 128 == 0, K <= 4194304
 *   G       a multiple of 32 that divides K
 *   bias    fp16 [N] or NULL
 *   row_ptr, cols, vals   CSR outlier lists (aq_segment_offsets, aq_outlier_cols)
 *   tile_ptr, tile_ent    the same outliers per 16 x 64 block (aq_outlier_tiles);
 *                         required when M > 64, used when given for
 *                         6 <= M <= 64, ignored (may be NULL) for M <= 5
 *   tile_max              the largest entry count of any block (max of
 *                         tile_ptr[b+1] - tile_ptr[b]); above 64 the GEMM
 *                         takes a variant that reads the excess from memory
 * Which kernels run:
 *   M <= 5        dequant-GEMV, each 16-row tile row reading x directly;
 *   6 <= M <= 64  dequant-GEMV sharing x through LDS, except that from
 *                 M = 33 on, grids of fewer than 384 tile rows (N < 6144,
 *                 summed over a group) take the dequant-GEMM when tile_ptr
 *                 and tile_ent are given;
 *   M > 64        dequant-GEMM (tile_ptr, tile_ent required).
 * The GEMVs add the outliers from the CSR lists in fp32, except the shared-x
 * GEMV given the block lists (M <= 32, or groups under 768 tile rows), which
 * multiplies each chunk's outliers with one more MFMA (x columns gathered
 * against the outlier values); the GEMM
 * writes each outlier's fp16 value over its decoded zero in the weight tile
 * it multiplies.  Either way the result is x times the dequantized weight
 * accumulated in fp32, plus the bias, rounded once to fp16.
 * workspace: aq_qlinear_workspace_size(M, N, K) bytes, 16-byte aligned, or
 * NULL.  A nonzero size means the GEMM would split K (2, 4 or 8 ways, chosen
 * from a time estimate of the shape on the current device) and keep the fp32
 * partial sums there; a second kernel adds them in a fixed order, so results
 * are deterministic.  A smaller workspace, or NULL, only limits the split (to
 * what it holds, down to none).  0 for every GEMV call.
 */
int64_t aq_qlinear_workspace_size(int64_t M, int64_t N, int64_t K);
int aq_qlinear(const void* x, int64_t M, int64_t K, int64_t N, const void* codes, const void* scales,
               int64_t G, int fmt, const int32_t* row_ptr, const int32_t* cols, const void* vals,
               const int32_t* tile_ptr, const uint32_t* tile_ent, int64_t tile_max, const void* bias, void* y,
               void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Several quantized linears that read the same x (e.g. the q/k/v projections
 * of an attention block, or gate/up of an MLP) in one launch: for i < count,
 * ys[i] = x W_i^T + b_i, W_i given by codes[i], scales[i], Gs[i], row_ptrs[i],
 * cols[i], vals[i], tile_ptrs[i], tile_ents[i], tile_maxes[i], biases[i]
 * (entries may be NULL), Ns[i] rows.  All W_i share K and fmt.  count <= 4.
 * The arrays themselves are host memory; tile_ptrs/tile_ents/tile_maxes may
 * be NULL when M <= 64.  workspace: aq_qlinear_workspace_size(M, N, K)
 * bytes with N the sum of Ns (the group is planned over all its output
 * columns), or less, or NULL (as for aq_qlinear).  Same per-matrix
 * requirements as aq_qlinear.
 */
int aq_qlinear_grouped(const void* x, int64_t M, int64_t K, int fmt, int64_t count, const int64_t* Ns,
                       const void* const* codes, const void* const* scales, const int64_t* Gs,
                       const int32_t* const* row_ptrs, const int32_t* const* cols, const void* const* vals,
                       const int32_t* const* tile_ptrs, const uint32_t* const* tile_ents,
                       const int64_t* tile_maxes, const void* const* biases, void* const* ys, void* workspace,
                       int64_t workspace_bytes, void* stream);

/*
 * aq_qlinear without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments, kernels and results as aq_qlinear given a workspace of
 * AQ_NOALLOC_SCRATCH_BYTES: the GEMM's split-K partial sums go to a static
 * device array of that size inside the library, one per GPU, held from the
 * first use on a GPU until the process ends.  The split is planned within
 * that size (as aq_qlinear's within its workspace), so no call is too large
 * for it; the call allocates nothing (no hipMalloc, no allocating library
 * call).  Calls that overlap in time on one GPU share the array and race:
 * serialise them (one stream, or your own ordering).
 */
#define AQ_NOALLOC_SCRATCH_BYTES (64ll << 20)
int aq_qlinear_noalloc(const void* x, int64_t M, int64_t K, int64_t N, const void* codes, const void* scales,
                       int64_t G, int fmt, const int32_t* row_ptr, const int32_t* cols, const void* vals,
                       const int32_t* tile_ptr, const uint32_t* tile_ent, int64_t tile_max, const void* bias,
                       void* y, void* stream);

/*
 * One decode-step launch of up to 4 quantized linears sharing x (M rows:
 * 1 with K <= 16384, or 6 <= M <= 64), with the layer's neighbouring
 * elementwise work folded in: the GEMV paths of aq_qlinear_grouped (the
 * reference's QuantizedLinear.forward, integration/atlas_wrappers.py:56-67,
 * at decode sizes) plus
 *   prologue  what the linears read instead of x:
 *             0  x as given
 *             1  RMSNorm(x): fp16(w fp16(x / sqrt(mean(x^2) + eps)))   (norm_weight)
 *             2  LayerNorm(x): fp16((x - mean) / sqrt(var + eps) w + b) (norm_weight, norm_bias)
 *             3  fp16(fp16(silu(x)) x2)  (x the gate, x2 the up projection)
 *             (the statistics in f32 over the row; the HF modules' order;
 *             prologues need M = 1)
 *   epilogue  per member i: relu[i] = 1 applies ReLU to the fp16 output,
 *             then residuals[i] (fp16 [M, N_i], or NULL) is added in fp16;
 *             relu[0] = 2 with two members of equal N (gate, up), 6 <= M <= 64
 *             and nothing else folded: the SwiGLU pair, fp16(fp16(silu(g)) u)
 *             written to ys[0] (ys[1] is not written).
 * tile_ptrs, tile_ents: the members' outlier block lists (aq_outlier_tiles)
 * or NULL; at 6 <= M <= 64 the GEMV adds the outliers with MFMAs from them
 * (without them: from the CSR lists, slower).
 * relu and residuals may be NULL (none for every member).  The residual
 * must not be the output.  Replaces, at decode, the norm / activation /
 * residual operations of HF's decoder layers around the reference's
 * QuantizedLinear calls (no counterpart of its own in the reference).
 */
int aq_qlinear_decode(const void* x, int64_t M, int64_t K, int fmt, int64_t count, const int64_t* Ns,
                      const void* const* codes, const void* const* scales, const int64_t* Gs,
                      const int32_t* const* row_ptrs, const int32_t* const* cols, const void* const* vals,
                      const int32_t* const* tile_ptrs, const uint32_t* const* tile_ents, const void* const* biases,
                      void* const* ys, int prologue, const void* x2, const void* norm_weight, const void* norm_bias,
                      float eps, const void* const* residuals, const int32_t* relu, void* stream);

/*
 * Attention of one decode step over a static key/value cache, the position
 * read from device memory (so that a captured HIP graph replays it for
 * every token).  Replaces the attention part of a decode step's forward:
 * the reference's AtlasAttentionWrapper.forward concatenates the cached
 * history with the new key/value, rotates, and runs SDPA or a BMM softmax
 * (integration/atlas_wrappers.py:161-262); HF's own attention modules do
 * the equivalent.  For batch row b and key/value head j (query heads
 * j G .. j G + G - 1, G = H / Hkv in {1, 2, 4, 8}):
 *   k_cache[b, j, pos, :] = k_new[b, j, :];  v_cache[b, j, pos, :] = v_new[b, j, :]
 *   s_p = fp16(q . k_p) * scale, p = 0 .. pos;  w = softmax(s) in f32
 *   out[b, h, :] = fp16(sum_p w_p v_p)   (f32 accumulation, one rounding)
 * Before that, q is multiplied by q_scale (rounded to fp16; 1 skips it:
 * OPT's query scaling) and, given rope_cos / rope_sin (fp16 [L, D]), q and
 * the new key are rotated at pos in the rotate-half form of Llama/Mistral,
 * x' = fp16(fp16(x cos) + fp16(r sin)), r = (-x[D/2:], x[:D/2]); the cache
 * receives the rotated key.
 *   q      fp16 [B, H, D]          k_new, v_new fp16 [B, Hkv, D]
 *   k_cache, v_cache fp16 [B, Hkv, L, D] (16-byte aligned)
 *   pos    int64 device scalar, 0 <= pos < L
 *   out    fp16 [B, H, D]          D = 64 or 128
 *   workspace  at least aq_decode_attention_workspace(B, H, Hkv, D, L)
 *          bytes, 16-byte aligned: the cache is split into spans of
 *          positions (one workgroup each) whose partial results a second
 *          kernel on the same stream merges.  No initial contents needed;
 *          calls that overlap in time must not share one.
 * A pos outside [0, L) leaves everything untouched (callers keep it inside).
 */
int aq_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                        const int64_t* pos, int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t L, float scale,
                        float q_scale, const void* rope_cos, const void* rope_sin, void* workspace, int64_t ws_bytes,
                        void* out, void* stream);

/* Bytes of workspace aq_decode_attention needs for these sizes (-1 for
 * sizes it cannot take).  No counterpart in the reference. */
int64_t aq_decode_attention_workspace(int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t L);

/*
 * Residual add and normalisation of `rows` rows of n fp16 (n a multiple of
 * 8, at most 16384), one launch.  With delta: x = fp16(x + delta), in place
 * (the residual stream).  Then y = norm(x):
 *   mode 0  RMSNorm of Llama/Mistral: y = fp16(w fp16(x / sqrt(mean(x^2) + eps)))
 *   mode 1  LayerNorm of OPT: y = fp16((x - mean) / sqrt(var + eps) w + bias)
 * (statistics in f32).  Replaces the norm modules and `x + residual` adds of
 * HF's OPT / Llama / Mistral decoder layers in the decode steps the reference
 * drives through model.generate (examples/run_atlas_inference.py:244-264);
 * the reference's own code has no kernel of its own here.
 */
int aq_decode_norm(void* x, const void* delta, const void* weight, const void* bias, float eps, int64_t rows,
                   int64_t n, int mode, void* y, void* stream);

/*
 * out = fp16(fp16(silu(g)) u) over n fp16 (n a multiple of 8): the SwiGLU
 * activation of HF's Llama/Mistral MLPs, act_fn(gate_proj(x)) * up_proj(x),
 * between two of the reference's quantized linears (no counterpart in the
 * reference's own code).
 */
int aq_silu_mul(const void* g, const void* u, void* out, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATLASINFER_AMD_H */
