// aq_decode.hip -- attention of one decode step over a static key/value cache
// (the position read from device memory, so that a HIP graph replays it).
#include "aq_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTile = kThreads;  // cache positions per pass of the loop

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

// One workgroup per (batch row b, key/value head j); G = H / Hkv query heads
// share the head.  q [B, H, D], k_new / v_new [B, Hkv, D], k_cache and
// v_cache [B, Hkv, L, D], out [B, H, D], all fp16.  Writes k_new / v_new at
// position pos, then for each query head g: scores s_p = fp16(q . k_p) *
// scale for p = 0..pos (the product accumulated in f32 and rounded to fp16,
// as a half-precision matrix product returns it), softmax over them in f32
// and o = sum_p softmax_p v_p accumulated in f32, rounded to fp16 once.
//
// One pass over the cache in tiles of 256 positions with a running maximum
// (the sums so far are rescaled by exp(m_old - m_new) at each tile):
//   scores  thread t takes position t0 + t, its key row in D / 8 loads of
//           16 bytes, the queries as 16-byte LDS broadcasts;
//   values  wave wv takes rows 64 wv .. 64 wv + 63 of the tile, lane ln the
//           16-byte chunk ln % (D / 8) of rows ln / (D / 8) + 64 / (D / 8) n,
//           all its rows' loads issued with the key loads;
//   sums    each thread keeps its own share of the softmax denominator; the
//           lanes' and waves' shares meet once, after the last tile.
// Position pos is read from k_new / v_new (the cache's copy is this
// kernel's own store), positions past pos read pos's row and weigh zero.
template <int D, int G>
__global__ __launch_bounds__(kThreads) void decode_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, const int64_t* __restrict__ pos_p, int H, int Hkv,
    int L, float scale, uint16_t* __restrict__ out) {
  constexpr int KV = D / 8;     // 16-byte chunks of a row
  constexpr int RPW = 64 / KV;  // rows one wave-wide load covers
  constexpr int NL = 64 / RPW;  // loads per lane for a wave's 64 rows
  const int j = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int64_t pos = *pos_p;
  if (pos < 0 || pos >= L) return;  // the caller guards this; no access outside the cache
  const int64_t kv = (int64_t)b * Hkv + j;
  uint16_t* Kc = k_cache + kv * L * D;
  uint16_t* Vc = v_cache + kv * L * D;
  const uint4* kn = reinterpret_cast<const uint4*>(k_new + kv * D);
  const uint4* vn = reinterpret_cast<const uint4*>(v_new + kv * D);

  __shared__ uint4 qs[G][KV];      // the group's queries, fp16
  __shared__ float w[G][kTile];    // a tile's softmax numerators
  __shared__ float red[4][G];      // per-wave maxima, then per-wave sums
  __shared__ float part[4][G][D];  // per-wave output sums

  for (int i = t; i < G * D; i += kThreads)
    reinterpret_cast<uint16_t*>(&qs[0][0])[i] = q[((int64_t)b * H + (int64_t)j * G) * D + i];
  if (t < KV) {
    reinterpret_cast<uint4*>(Kc + pos * D)[t] = kn[t];
    reinterpret_cast<uint4*>(Vc + pos * D)[t] = vn[t];
  }
  __syncthreads();

  const int wv = t >> 6, ln = t & 63, ch = ln % KV, rs = ln / KV;
  float acc[G][8], m[G], lt[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    lt[g] = 0.0f;
#pragma unroll
    for (int h = 0; h < 8; h++) acc[g][h] = 0.0f;
  }

  for (int64_t t0 = 0; t0 <= pos; t0 += kTile) {
    const int64_t p = t0 + t;
    const bool valid = p <= pos;
    const uint4* krow = p < pos ? reinterpret_cast<const uint4*>(Kc + p * D) : kn;
    uint4 kr[KV];
#pragma unroll
    for (int i = 0; i < KV; i++) kr[i] = krow[i];
    uint4 vr[NL];
#pragma unroll
    for (int n = 0; n < NL; n++) {
      const int64_t pr = t0 + 64 * wv + RPW * n + rs;
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
#pragma unroll
    for (int g = 0; g < G; g++) {
      s[g] = valid ? (float)rn_h(s[g]) * scale : -INFINITY;
      const float mw = wave_group_max_f32<64>(s[g]);
      if (ln == 0) red[wv][g] = mw;
    }
    __syncthreads();
    float c[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float mn = fmaxf(m[g], fmaxf(fmaxf(red[0][g], red[1][g]), fmaxf(red[2][g], red[3][g])));
      c[g] = m[g] == -INFINITY ? 0.0f : __expf(m[g] - mn);
      const float e = valid ? __expf(s[g] - mn) : 0.0f;
      lt[g] = lt[g] * c[g] + e;
      w[g][t] = e;
      m[g] = mn;
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < NL; n++) {
      const int r = 64 * wv + RPW * n + rs;
      const uint32_t wd[4] = {vr[n].x, vr[n].y, vr[n].z, vr[n].w};
      float vf[8];
#pragma unroll
      for (int h = 0; h < 8; h++) vf[h] = h2f((uint16_t)(wd[h >> 1] >> (16 * (h & 1))));
#pragma unroll
      for (int g = 0; g < G; g++) {
        const float wg = w[g][r];
#pragma unroll
        for (int h = 0; h < 8; h++) acc[g][h] = fmaf(wg, vf[h], n == 0 ? acc[g][h] * c[g] : acc[g][h]);
      }
    }
  }

  // the softmax denominators: lanes, then waves (no thread reads red after
  // the last tile's second barrier)
#pragma unroll
  for (int g = 0; g < G; g++) {
    const float lw = wave_group_sum_f32<64>(lt[g]);
    if (ln == 0) red[wv][g] = lw;
  }
  // the output sums: the wave's RPW row groups, then the four waves
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int h = 0; h < 8; h++)
#pragma unroll
      for (int o = KV; o < 64; o <<= 1) acc[g][h] += __shfl_xor(acc[g][h], o);
  if (rs == 0) {
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int h = 0; h < 8; h++) part[wv][g][8 * ch + h] = acc[g][h];
  }
  __syncthreads();
  for (int i = t; i < G * D; i += kThreads) {
    const int g = i / D, d = i % D;
    const float l = (red[0][g] + red[1][g]) + (red[2][g] + red[3][g]);
    const float a = (part[0][g][d] + part[1][g][d]) + (part[2][g][d] + part[3][g][d]);
    out[((int64_t)b * H + (int64_t)j * G) * D + i] = h_to_bits(rn_h(a / l));
  }
}

}  // namespace

extern "C" int aq_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                   const int64_t* pos, int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t L,
                                   float scale, void* out, void* stream) {
  AQ_CHECK_ARG(q && k_new && v_new && k_cache && v_cache && pos && out, "aq_decode_attention: null pointer");
  AQ_CHECK_ARG(B > 0 && Hkv > 0 && H > 0 && H % Hkv == 0 &&
                   (H / Hkv == 1 || H / Hkv == 2 || H / Hkv == 4 || H / Hkv == 8),
               "aq_decode_attention: H (%lld) must be 1, 2, 4 or 8 times Hkv (%lld)", (long long)H, (long long)Hkv);
  AQ_CHECK_ARG(D == 64 || D == 128, "aq_decode_attention: head dim %lld (64 or 128 supported)", (long long)D);
  AQ_CHECK_ARG((uintptr_t)k_cache % 16 == 0 && (uintptr_t)v_cache % 16 == 0 && (uintptr_t)k_new % 16 == 0 &&
                   (uintptr_t)v_new % 16 == 0,
               "aq_decode_attention: k_new, v_new and the caches must be 16-byte aligned");
  AQ_CHECK_ARG(L > 0 && L <= (1 << 24) && B <= 65535 && Hkv <= (1 << 20), "aq_decode_attention: sizes out of range");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)Hkv, (unsigned)B);
  const int G = (int)(H / Hkv);
#define AQ_DECODE_LAUNCH(DD, GG)                                                                                     \
  hipLaunchKernelGGL((decode_attention_kernel<DD, GG>), grid, dim3(kThreads), 0, s, (const uint16_t*)q,            \
                     (const uint16_t*)k_new, (const uint16_t*)v_new, (uint16_t*)k_cache, (uint16_t*)v_cache, pos,  \
                     (int)H, (int)Hkv, (int)L, scale, (uint16_t*)out)
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
