// aq_decode.hip -- the work of one decode step around the quantized linears:
// attention over a static key/value cache (the position read from device
// memory, so that a HIP graph replays it), the residual add + RMSNorm /
// LayerNorm of a row, and the SwiGLU product.
#include "aq_common.h"

namespace {

__device__ __forceinline__ float h2f(uint16_t b) { return (float)bits_to_h(b); }

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

// s + the dot product of eight fp16 pairs (v_dot2_f32_f16: the products are
// exact in f32, each pair's sum added to s in f32).
__device__ __forceinline__ float dot8(uint4 a, uint4 b, float s) {
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.x), __builtin_bit_cast(h2_t, b.x), s, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.y), __builtin_bit_cast(h2_t, b.y), s, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.z), __builtin_bit_cast(h2_t, b.z), s, false);
  s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a.w), __builtin_bit_cast(h2_t, b.w), s, false);
  return s;
}

// x * f rounded to fp16 (fp16 tensor times a Python float); f = 1 is exact.
__device__ __forceinline__ f16 scale_h(f16 x, float f) { return f == 1.0f ? x : rn_h((float)x * f); }

// One rotate-half element: partner is x[d + D/2] (negated, lo = true) or
// x[d - D/2]; fp16(fp16(x c) + fp16(r s)).
__device__ __forceinline__ f16 rope_h(f16 x, f16 partner, bool lo, uint16_t c, uint16_t s) {
  const float r = lo ? -(float)partner : (float)partner;
  const f16 a = rn_h((float)x * (float)bits_to_h(c));
  const f16 b2 = rn_h(r * (float)bits_to_h(s));
  return rn_h((float)a + (float)b2);
}

// Splitting of the cache among workgroups.  A cache of at most 16 chunks of
// 64 positions may be one span per head, its chunks dealt to nw = min(4,
// chunks) waves of one workgroup that merge their results in LDS (no
// second kernel): taken when a wave's serial share is short -- at most 4
// chunk-units of work, a chunk costing G D / 64 units (scores and value
// sums of 64 positions per lane, about 1000 vector instructions at G = 4,
// D = 128) -- or when B Hkv >= 256 workgroups keep every SIMD busy anyway.
// (Measured: OPT-1.3b batch 1, 32 heads of D = 64, 3 chunks: one span
// 1168 against 1119 tok/s; Mistral-7B batch 32, 256 heads x batch rows:
// 8116 against 7531; Mistral-7B batch 1, 8 key/value heads of G = 4,
// D = 128, 12 chunks: 398 against 439, so split.)  Otherwise the cache is
// split into spans of nt chunks, one wave each, nt the smallest power of
// two that leaves ns = ceil(L / (64 nt)) <= 64 spans per head and
// B Hkv ns <= 4096 workgroups (or one span for the whole cache);
// decode_combine_kernel merges the spans.
constexpr int kChunk = 64;
constexpr int kOneSpanChunks = 16;
constexpr int kMaxWaves = 4;  // one per SIMD: 8 would halve the registers a wave may hold (D = 128 then spills)
constexpr int64_t kMaxGroups = 4096;
constexpr int64_t kMaxSpans = 64;

struct Split {
  int64_t nt, ns, nw, part_floats, bytes;
};

// G query heads share a key/value head; a span's partial result is its
// running maximum and denominator per query head and its G x D weighted sum.
inline Split split_of(int64_t B, int64_t Hkv, int64_t G, int64_t D, int64_t L) {
  Split sp;
  const int64_t chunks = (L + kChunk - 1) / kChunk;
  sp.part_floats = G * D + 2 * G;
  const int64_t nw1 = std::min<int64_t>(kMaxWaves, chunks);
  const int64_t serial_units = (chunks + nw1 - 1) / nw1 * G * D / 64;
  if (chunks <= kOneSpanChunks && (serial_units <= 4 || B * Hkv >= 256)) {
    sp.nt = chunks;
    sp.ns = 1;
    sp.nw = nw1;
  } else {
    sp.nw = 1;
    sp.nt = 1;
    auto spans = [&](int64_t nt) { return (L + kChunk * nt - 1) / (kChunk * nt); };
    while (kChunk * sp.nt < L && (spans(sp.nt) > kMaxSpans || B * Hkv * spans(sp.nt) > kMaxGroups)) sp.nt *= 2;
    sp.ns = spans(sp.nt);
  }
  sp.bytes = B * Hkv * sp.ns * sp.part_floats * 4;
  return sp;
}

// LDS of one workgroup of nw waves: per wave a chunk's softmax numerators
// [G][64] and its merged result [G D + 2 G] (floats).
inline size_t attention_lds(int64_t G, int64_t D, int64_t nw) { return (size_t)nw * (G * kChunk + G * D + 2 * G) * 4; }

// Workgroup (j, b, z) takes key/value head j of batch row b (query heads
// j G .. j G + G - 1) and cache positions z span .. z span + span - 1
// (span = 64 nt); q [B, H, D], k_new / v_new [B, Hkv, D], k_cache and
// v_cache [B, Hkv, L, D], out [B, H, D], all fp16.  The span holding pos
// writes k_new / v_new there.  For each query head g: scores s_p = fp16(q .
// k_p) * scale for p <= pos (the product accumulated in f32 and rounded to
// fp16, as a half-precision matrix product returns it), softmax over them in
// f32 and o = sum_p softmax_p v_p accumulated in f32, rounded to fp16 once.
//
// Wave w of the workgroup takes chunks w, w + nw, ... of the span, chunk
// by chunk with a running maximum (the sums so far are rescaled by
// exp(m_old - m_new)):
//   scores  lane ln takes position t0 + ln, its key row in D / 8 loads of
//           16 bytes, the queries as 16-byte LDS broadcasts;
//   values  lane ln takes the 16-byte chunk ln % (D / 8) of rows
//           ln / (D / 8) + (64 / (D / 8)) n, all loads issued with the keys';
//   sums    each lane keeps its share of the denominator.
// Position pos's key and value come from k_new / v_new (the cache's copy is
// this kernel's own store); positions past pos read k_new / v_new and weigh
// zero.  Before use the queries are multiplied by q_scale (rounded to fp16;
// skipped for 1) and, given rcos / rsin (fp16 [L, D] tables), the queries
// and the new key are rotated at position pos in the rotate-half form:
// x' = fp16(fp16(x c) + fp16(r s)), r = (-x[D/2:], x[:D/2]) -- the order
// and roundings of fp16 tensor arithmetic.
//
// The waves' results meet in LDS (maximum M over the waves, each wave's
// sums scaled by exp(m_w - M), waves in order).  With one span holding
// positions the workgroup writes out itself; otherwise every span with
// positions writes (M, l, sum) to its slot of part and
// decode_combine_kernel, launched next on the same stream, merges them.  (A
// merge inside this kernel by the last span to arrive would need an
// agent-scope release per span, which writes back the whole L2 of the
// span's XCD; the kernel boundary orders the slots for free.)
template <int D, int G>
__global__ __launch_bounds__(64 * kMaxWaves) void decode_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, const int64_t* __restrict__ pos_p, int H, int Hkv,
    int L, float scale, float q_scale, const uint16_t* __restrict__ rcos, const uint16_t* __restrict__ rsin, int nt,
    int ns, float* __restrict__ part, uint16_t* __restrict__ out) {
  constexpr int KV = D / 8;     // 16-byte chunks of a row
  constexpr int RPW = 64 / KV;  // rows one wave-wide load covers
  constexpr int NL = KV;        // loads per lane for 64 rows
  constexpr int PF = G * D + 2 * G;
  const int j = blockIdx.x, b = blockIdx.y, z = blockIdx.z, t = threadIdx.x;
  const int nw = blockDim.x >> 6, ln = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t pos = *pos_p;
  if (pos < 0 || pos >= L) return;  // the caller guards this; no access outside the cache
  const int64_t span = (int64_t)kChunk * nt, z0 = (int64_t)z * span;
  if (z0 > pos) return;  // no cached position in this span yet
  const int nact = (int)(pos / span) + 1;
  const int64_t kv = (int64_t)b * Hkv + j;
  uint16_t* Kc = k_cache + kv * L * D;
  uint16_t* Vc = v_cache + kv * L * D;
  const uint4* kn = reinterpret_cast<const uint4*>(k_new + kv * D);
  const uint4* vn = reinterpret_cast<const uint4*>(v_new + kv * D);
  uint16_t* o = out + ((int64_t)b * H + (int64_t)j * G) * D;

  __shared__ uint4 qs[G][KV];    // the group's queries, fp16
  __shared__ uint4 krot[KV];     // position pos's key as cached (last span only)
  extern __shared__ float dyn[];
  float* w = dyn + wave * G * kChunk;     // this wave's numerators [G][64]
  float* res = dyn + nw * G * kChunk;     // the waves' results [nw][PF]

  const uint16_t* cs = rcos ? rcos + pos * D : nullptr;
  const uint16_t* sn = rsin ? rsin + pos * D : nullptr;
  const uint16_t* qb = q + ((int64_t)b * H + (int64_t)j * G) * D;
  for (int i = t; i < G * D; i += 64 * nw) {
    const int d = i % D;
    f16 v = scale_h(bits_to_h(qb[i]), q_scale);
    if (cs) v = rope_h(v, scale_h(bits_to_h(qb[i - d + (d + D / 2) % D]), q_scale), d < D / 2, cs[d], sn[d]);
    reinterpret_cast<uint16_t*>(&qs[0][0])[i] = h_to_bits(v);
  }
  const bool last = z == nact - 1;  // the span holding pos
  if (last) {
    const uint16_t* kb = k_new + kv * D;
    for (int d = t; d < D; d += 64 * nw) {
      f16 v = bits_to_h(kb[d]);
      if (cs) v = rope_h(v, bits_to_h(kb[(d + D / 2) % D]), d < D / 2, cs[d], sn[d]);
      reinterpret_cast<uint16_t*>(krot)[d] = h_to_bits(v);
    }
  }
  __syncthreads();
  if (last && t < KV) {
    reinterpret_cast<uint4*>(Kc + pos * D)[t] = krot[t];
    reinterpret_cast<uint4*>(Vc + pos * D)[t] = vn[t];
  }

  const int ch = ln % KV, rs = ln / KV;
  float acc[G][8], m[G], lt[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    lt[g] = 0.0f;
#pragma unroll
    for (int h = 0; h < 8; h++) acc[g][h] = 0.0f;
  }

  for (int it = wave; it < nt; it += nw) {
    const int64_t t0 = z0 + (int64_t)it * kChunk;
    if (t0 > pos) break;
    const int64_t p = t0 + ln;
    const bool valid = p <= pos;
    const uint4* krow = p < pos ? reinterpret_cast<const uint4*>(Kc + p * D) : kn;
    uint4 kr[KV];
#pragma unroll
    for (int i = 0; i < KV; i++) kr[i] = krow[i];
    if (p == pos) {  // one lane of the last span: the key as cached
#pragma unroll
      for (int i = 0; i < KV; i++) kr[i] = krot[i];
    }
    uint4 vr[NL];
#pragma unroll
    for (int n = 0; n < NL; n++) {
      const int64_t pr = t0 + RPW * n + rs;
      vr[n] = (pr < pos ? reinterpret_cast<const uint4*>(Vc + pr * D) : vn)[ch];
    }

    float s[G];
#pragma unroll
    for (int g = 0; g < G; g++) s[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < KV; i++) {
      // one chunk's G query reads at a time: the scheduler would otherwise
      // issue all G * D / 8 of them up front and hold them in registers
      asm volatile("" ::: "memory");
#pragma unroll
      for (int g = 0; g < G; g++) s[g] = dot8(kr[i], qs[g][i], s[g]);
    }
    float c[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float sg = valid ? (float)rn_h(s[g]) * scale : -INFINITY;
      const float mn = fmaxf(m[g], wave_group_max_f32<64>(sg));  // every lane holds the maximum
      c[g] = m[g] == -INFINITY ? 0.0f : __expf(m[g] - mn);
      const float e = valid ? __expf(sg - mn) : 0.0f;
      lt[g] = lt[g] * c[g] + e;
      w[g * kChunk + ln] = e;
      m[g] = mn;
    }
    // w is this wave's own: its LDS writes complete before its reads, in
    // order; the compiler keeps the reads after the writes (and later
    // chunks' loads out of this one)
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int n = 0; n < NL; n++) {
      const int r = RPW * n + rs;
      const uint32_t wd[4] = {vr[n].x, vr[n].y, vr[n].z, vr[n].w};
      float vf[8];
#pragma unroll
      for (int h = 0; h < 8; h++) vf[h] = h2f((uint16_t)(wd[h >> 1] >> (16 * (h & 1))));
#pragma unroll
      for (int g = 0; g < G; g++) {
        const float wg = w[g * kChunk + r];
#pragma unroll
        for (int h = 0; h < 8; h++) acc[g][h] = fmaf(wg, vf[h], n == 0 ? acc[g][h] * c[g] : acc[g][h]);
      }
    }
    __builtin_amdgcn_wave_barrier();  // this chunk's reads of w before the next chunk's writes
    asm volatile("" ::: "memory");
  }

  // the wave's sums: the lanes' denominators, the RPW row groups' outputs
#pragma unroll
  for (int g = 0; g < G; g++) {
    lt[g] = wave_group_sum_f32<64>(lt[g]);
#pragma unroll
    for (int h = 0; h < 8; h++)
#pragma unroll
      for (int off = KV; off < 64; off <<= 1) acc[g][h] += __shfl_xor(acc[g][h], off);
  }
  if (nw == 1 && nact == 1) {
    if (rs == 0) {
#pragma unroll
      for (int g = 0; g < G; g++)
#pragma unroll
        for (int h = 0; h < 8; h++) o[g * D + 8 * ch + h] = h_to_bits(rn_h(acc[g][h] / lt[g]));
    }
    return;
  }
  float* pp = nw == 1 ? part + (kv * ns + z) * PF : res + wave * PF;
  if (rs == 0) {
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int h = 0; h < 8; h++) pp[g * D + 8 * ch + h] = acc[g][h];
  }
  if (ln == 0) {
#pragma unroll
    for (int g = 0; g < G; g++) {
      pp[G * D + g] = m[g];
      pp[G * D + G + g] = lt[g];
    }
  }
  if (nw == 1) return;  // the span's partial is in part; decode_combine_kernel merges
  __syncthreads();
  // the waves' results, merged in wave order: out when one span holds every
  // position, else the span's partial (M, l, sum) into part
  float* sp = part + (kv * ns + z) * PF;
  for (int i = t; i < G * D + G; i += 64 * nw) {
    const int g = i < G * D ? i / D : i - G * D;
    float mx = -INFINITY;
    for (int v = 0; v < nw; v++) mx = fmaxf(mx, res[v * PF + G * D + g]);
    float num = 0.0f, den = 0.0f;
    for (int v = 0; v < nw; v++) {
      const float mv = res[v * PF + G * D + g];
      const float f = mv == -INFINITY ? 0.0f : __expf(mv - mx);
      den = fmaf(res[v * PF + G * D + G + g], f, den);
      if (i < G * D) num = fmaf(res[v * PF + i], f, num);
    }
    if (i < G * D) {
      if (nact == 1)
        o[i] = h_to_bits(rn_h(num / den));
      else
        sp[i] = num;
    } else if (nact > 1) {
      sp[G * D + g] = mx;
      sp[G * D + G + g] = den;
    }
  }
}

// Merges the spans' partial results of decode_attention_kernel for (b, j):
// M = max_z m_z, f_z = exp(m_z - M), out = fp16(sum_z f_z sum_z / sum_z f_z
// l_z), the spans taken in order.  Does nothing when one span held every
// position (that span wrote out).
template <int D, int G>
__global__ __launch_bounds__(256) void decode_combine_kernel(const int64_t* __restrict__ pos_p, int H, int Hkv, int L,
                                                             int nt, int ns, const float* __restrict__ part,
                                                             uint16_t* __restrict__ out) {
  constexpr int PF = G * D + 2 * G;
  const int j = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int64_t pos = *pos_p;
  if (pos < 0 || pos >= L) return;
  const int nact = (int)(pos / ((int64_t)kChunk * nt)) + 1;
  if (nact == 1) return;
  const float* pk = part + ((int64_t)b * Hkv + j) * ns * PF;
  __shared__ float f[G][kMaxSpans];
  __shared__ float ls[G][kMaxSpans];
  __shared__ float den[G];
  // every span's (m, l) read at once (a loop of dependent reads per head
  // waited out one round trip per span)
  for (int k = t; k < G * nact; k += 256) {
    const int z = k / G, g = k - z * G;
    f[g][z] = pk[z * PF + G * D + g];
    ls[g][z] = pk[z * PF + G * D + G + g];
  }
  __syncthreads();
  if (t < G) {
    float mx = -INFINITY;
    for (int z = 0; z < nact; z++) mx = fmaxf(mx, f[t][z]);
    float d = 0.0f;
    for (int z = 0; z < nact; z++) {
      const float e = __expf(f[t][z] - mx);
      f[t][z] = e;
      d = fmaf(ls[t][z], e, d);
    }
    den[t] = d;
  }
  __syncthreads();
  uint16_t* o = out + ((int64_t)b * H + (int64_t)j * G) * D;
  for (int i = t; i < G * D; i += 256) {
    const int g = i / D;
    float num = 0.0f;
    // eight spans' loads in flight, then their products in span order
    for (int z0 = 0; z0 < nact; z0 += 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) v[k] = z0 + k < nact ? pk[(z0 + k) * PF + i] : 0.0f;
#pragma unroll
      for (int k = 0; k < 8; k++)
        if (z0 + k < nact) num = fmaf(v[k], f[g][z0 + k], num);
    }
    o[i] = h_to_bits(rn_h(num / den[g]));
  }
}

}  // namespace

extern "C" int64_t aq_decode_attention_workspace(int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t L) {
  if (B <= 0 || Hkv <= 0 || H <= 0 || H % Hkv != 0 || D <= 0 || L <= 0) return -1;
  return split_of(B, Hkv, H / Hkv, D, L).bytes;
}

extern "C" int aq_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                   const int64_t* pos, int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t L,
                                   float scale, float q_scale, const void* rope_cos, const void* rope_sin,
                                   void* workspace, int64_t ws_bytes, void* out, void* stream) {
  AQ_CHECK_ARG(q && k_new && v_new && k_cache && v_cache && pos && out && workspace,
               "aq_decode_attention: null pointer");
  AQ_CHECK_ARG((rope_cos == nullptr) == (rope_sin == nullptr),
               "aq_decode_attention: rope_cos and rope_sin come together");
  AQ_CHECK_ARG(B > 0 && Hkv > 0 && H > 0 && H % Hkv == 0 &&
                   (H / Hkv == 1 || H / Hkv == 2 || H / Hkv == 4 || H / Hkv == 8),
               "aq_decode_attention: H (%lld) must be 1, 2, 4 or 8 times Hkv (%lld)", (long long)H, (long long)Hkv);
  AQ_CHECK_ARG(D == 64 || D == 128, "aq_decode_attention: head dim %lld (64 or 128 supported)", (long long)D);
  AQ_CHECK_ARG((uintptr_t)k_cache % 16 == 0 && (uintptr_t)v_cache % 16 == 0 && (uintptr_t)k_new % 16 == 0 &&
                   (uintptr_t)v_new % 16 == 0 && (uintptr_t)workspace % 16 == 0,
               "aq_decode_attention: k_new, v_new, the caches and the workspace must be 16-byte aligned");
  AQ_CHECK_ARG(L > 0 && L <= (1 << 24) && B <= 65535 && Hkv <= 65535, "aq_decode_attention: sizes out of range");
  const Split sp = split_of(B, Hkv, H / Hkv, D, L);
  AQ_CHECK_ARG(ws_bytes >= sp.bytes, "aq_decode_attention: workspace of %lld bytes, %lld needed", (long long)ws_bytes,
               (long long)sp.bytes);
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)Hkv, (unsigned)B, (unsigned)sp.ns);  // spans past pos exit at once
  const int G = (int)(H / Hkv);
  float* part = (float*)workspace;
#define AQ_DECODE_LAUNCH(DD, GG)                                                                                     \
  do {                                                                                                               \
    hipLaunchKernelGGL((decode_attention_kernel<DD, GG>), grid, dim3(64 * (unsigned)sp.nw),                       \
                       attention_lds(GG, DD, sp.nw), s, (const uint16_t*)q,                                          \
                       (const uint16_t*)k_new, (const uint16_t*)v_new, (uint16_t*)k_cache, (uint16_t*)v_cache, pos, \
                       (int)H, (int)Hkv, (int)L, scale, q_scale, (const uint16_t*)rope_cos,                        \
                       (const uint16_t*)rope_sin, (int)sp.nt, (int)sp.ns, part, (uint16_t*)out);                    \
    if (sp.ns > 1)                                                                                                   \
      hipLaunchKernelGGL((decode_combine_kernel<DD, GG>), dim3((unsigned)Hkv, (unsigned)B), dim3(256), 0, s, pos,   \
                         (int)H, (int)Hkv, (int)L, (int)sp.nt, (int)sp.ns, part, (uint16_t*)out);                  \
  } while (0)
  if (D == 64) {
    if (G == 1) AQ_DECODE_LAUNCH(64, 1);
    else if (G == 2) AQ_DECODE_LAUNCH(64, 2);
    else if (G == 4) AQ_DECODE_LAUNCH(64, 4);
    else AQ_DECODE_LAUNCH(64, 8);
  } else {
    if (G == 1) AQ_DECODE_LAUNCH(128, 1);
    else if (G == 2) AQ_DECODE_LAUNCH(128, 2);
    else if (G == 4) AQ_DECODE_LAUNCH(128, 4);
    else AQ_DECODE_LAUNCH(128, 8);
  }
#undef AQ_DECODE_LAUNCH
  AQ_LAUNCH_CHECK("aq_decode_attention");
  return AQ_OK;
}

// ------------------------------------------------------------ decode glue

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormChunks = 8;  // 8 fp16 each: rows of up to 256 * 8 * 8 = 16384

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_group_sum_f32<64>(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup per row of n fp16.  With delta: x = fp16(x + delta), stored
// back (a residual add).  Then y = norm(x):
//   MODE 0 (RMSNorm): r = 1 / sqrt(mean_f32(x^2) + eps), y = fp16(w fp16(x r))
//   MODE 1 (LayerNorm): mean and variance in f32, y = fp16((x - mean) rstd w + b)
// (the operation order of HF's Llama/Mistral RMSNorm and torch's layer_norm
// on fp16 inputs).
template <int MODE>
__global__ __launch_bounds__(kNormThreads) void decode_norm_kernel(uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ delta,
                                                                  const uint16_t* __restrict__ w,
                                                                  const uint16_t* __restrict__ bias, float eps, int n,
                                                                  uint16_t* __restrict__ y) {
  __shared__ float red[4];
  const int t = threadIdx.x;
  uint16_t* xr = x + (int64_t)blockIdx.x * n;
  const uint16_t* dr = delta ? delta + (int64_t)blockIdx.x * n : nullptr;
  uint16_t* yr = y + (int64_t)blockIdx.x * n;
  float v[kNormChunks][8];
  float s = 0.0f;
  // the weights (and bias) go out with x, ahead of the reduction
  uint4 wv[kNormChunks], bv[kNormChunks];
#pragma unroll
  for (int c = 0; c < kNormChunks; c++) {
    const int i = (c * kNormThreads + t) * 8;
    if (i < n) {
      wv[c] = *reinterpret_cast<const uint4*>(w + i);
      bv[c] = MODE == 1 ? *reinterpret_cast<const uint4*>(bias + i) : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int c = 0; c < kNormChunks; c++) {
    const int i = (c * kNormThreads + t) * 8;
    if (i < n) {
      uint4 a = *reinterpret_cast<const uint4*>(xr + i);
      if (dr) {
        const uint4 d = *reinterpret_cast<const uint4*>(dr + i);
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, dw[4] = {d.x, d.y, d.z, d.w};
        uint32_t ow[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const f16 lo = rn_h((float)bits_to_h((uint16_t)aw[k]) + (float)bits_to_h((uint16_t)dw[k]));
          const f16 hi = rn_h((float)bits_to_h((uint16_t)(aw[k] >> 16)) + (float)bits_to_h((uint16_t)(dw[k] >> 16)));
          ow[k] = (uint32_t)h_to_bits(lo) | ((uint32_t)h_to_bits(hi) << 16);
        }
        a = make_uint4(ow[0], ow[1], ow[2], ow[3]);
        *reinterpret_cast<uint4*>(xr + i) = a;
      }
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        v[c][k] = (float)bits_to_h((uint16_t)(aw[k >> 1] >> (16 * (k & 1))));
        s += MODE == 0 ? v[c][k] * v[c][k] : v[c][k];
      }
    }
  }
  const float tot = block_sum(s, red);
  float mean = 0.0f, r;
  if (MODE == 0) {
    r = 1.0f / sqrtf(tot / (float)n + eps);
  } else {
    mean = tot / (float)n;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < kNormChunks; c++)
      if ((c * kNormThreads + t) * 8 < n)
#pragma unroll
        for (int k = 0; k < 8; k++) q += (v[c][k] - mean) * (v[c][k] - mean);
    r = 1.0f / sqrtf(block_sum(q, red) / (float)n + eps);
  }
#pragma unroll
  for (int c = 0; c < kNormChunks; c++) {
    const int i = (c * kNormThreads + t) * 8;
    if (i < n) {
      const uint32_t ww[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w}, bw[4] = {bv[c].x, bv[c].y, bv[c].z, bv[c].w};
      uint32_t ow[4] = {0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float wk = (float)bits_to_h((uint16_t)(ww[k >> 1] >> (16 * (k & 1))));
        f16 o;
        if (MODE == 0) {
          o = bits_to_h((uint16_t)(ww[k >> 1] >> (16 * (k & 1)))) * rn_h(v[c][k] * r);  // fp16 multiply: same rounding
        } else {
          const float bk = (float)bits_to_h((uint16_t)(bw[k >> 1] >> (16 * (k & 1))));
          o = rn_h((v[c][k] - mean) * r * wk + bk);
        }
        ow[k >> 1] |= (uint32_t)h_to_bits(o) << (16 * (k & 1));
      }
      *reinterpret_cast<uint4*>(yr + i) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
  }
}

// out = fp16(fp16(silu(g)) u), silu(g) = g / (1 + exp(-g)) in f32: the
// gate activation and product of a SwiGLU MLP.  Eight elements a thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                                       uint16_t* __restrict__ out, int64_t n8) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const uint4 gv = reinterpret_cast<const uint4*>(g)[i];
  const uint4 uv = reinterpret_cast<const uint4*>(u)[i];
  const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t ow[4] = {0, 0, 0, 0};
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const float gk = (float)bits_to_h((uint16_t)(gw[k >> 1] >> (16 * (k & 1))));
    const float uk = (float)bits_to_h((uint16_t)(uw[k >> 1] >> (16 * (k & 1))));
    ow[k >> 1] |= (uint32_t)h_to_bits(silu_mul_h(gk, uk)) << (16 * (k & 1));
  }
  reinterpret_cast<uint4*>(out)[i] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

}  // namespace

extern "C" int aq_decode_norm(void* x, const void* delta, const void* weight, const void* bias, float eps, int64_t rows,
                              int64_t n, int mode, void* y, void* stream) {
  AQ_CHECK_ARG(x && weight && y, "aq_decode_norm: null pointer");
  AQ_CHECK_ARG(mode == 0 || (mode == 1 && bias), "aq_decode_norm: mode %d (0 RMSNorm, 1 LayerNorm with bias)", mode);
  AQ_CHECK_ARG(rows > 0 && rows <= (1 << 20) && n > 0 && n % 8 == 0 && n <= kNormThreads * kNormChunks * 8,
               "aq_decode_norm: %lld rows of %lld (a multiple of 8, at most %d)", (long long)rows, (long long)n,
               kNormThreads * kNormChunks * 8);
  AQ_CHECK_ARG((uintptr_t)x % 16 == 0 && (uintptr_t)delta % 16 == 0 && (uintptr_t)weight % 16 == 0 &&
                   (uintptr_t)bias % 16 == 0 && (uintptr_t)y % 16 == 0,
               "aq_decode_norm: buffers must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  if (mode == 0)
    hipLaunchKernelGGL(decode_norm_kernel<0>, dim3((unsigned)rows), dim3(kNormThreads), 0, s, (uint16_t*)x,
                       (const uint16_t*)delta, (const uint16_t*)weight, (const uint16_t*)bias, eps, (int)n,
                       (uint16_t*)y);
  else
    hipLaunchKernelGGL(decode_norm_kernel<1>, dim3((unsigned)rows), dim3(kNormThreads), 0, s, (uint16_t*)x,
                       (const uint16_t*)delta, (const uint16_t*)weight, (const uint16_t*)bias, eps, (int)n,
                       (uint16_t*)y);
  AQ_LAUNCH_CHECK("aq_decode_norm");
  return AQ_OK;
}

extern "C" int aq_silu_mul(const void* g, const void* u, void* out, int64_t n, void* stream) {
  AQ_CHECK_ARG(g && u && out, "aq_silu_mul: null pointer");
  AQ_CHECK_ARG(n > 0 && n % 8 == 0, "aq_silu_mul: %lld elements (a positive multiple of 8)", (long long)n);
  AQ_CHECK_ARG((uintptr_t)g % 16 == 0 && (uintptr_t)u % 16 == 0 && (uintptr_t)out % 16 == 0,
               "aq_silu_mul: buffers must be 16-byte aligned");
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)g, (const uint16_t*)u, (uint16_t*)out, n8);
  AQ_LAUNCH_CHECK("aq_silu_mul");
  return AQ_OK;
}
