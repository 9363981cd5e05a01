// Per-head row helpers shared by the append / attention kernels and the GEMM whose epilogue
// forms the queries and appends K/V (one head row spread over the lanes of a wave or a quarter
// wave): the projection sum, the per-head RMSNorm, rotate-half RoPE, the KV store (bf16 or
// 8-bit affine group 64) and the paged pool's token index.
#pragma once

#include "common.h"

namespace dsk {

// ----------------------------------------------------------------------------- row helpers
// RoPE angle in fp32 as the reference computes it (pos * inv_freq rounded once), with the
// library's sine and cosine of that float32 angle (full argument reduction, a few ulp). A float32
// reduction to revolutions for v_sin_f32 / v_cos_f32 would be off by up to |angle| * 2^-24
// revolutions (2.5e-4 rad at position 4096 for the fastest frequency), about an eighth of a bf16
// step of the rotated values, enough to flip their rounding at long contexts.
__device__ __forceinline__ void rope_sincos(int pos, float inv_freq, float& sn, float& cs) {
  const float ang = (float)pos * inv_freq;
  sincosf(ang, &sn, &cs);
}

// One head row of HD dims spread over L consecutive lanes (L = 64: a wave; L = 16: a quarter
// wave), PER = HD / L consecutive dims per lane starting at dim PER * (lane % L).
// Sum of the projection's split-K slices in slice order, times `scale` (the row scale of a
// normed-later input; 1 otherwise), rounded to bf16.
template <int PER>
__device__ __forceinline__ void load_proj_row(const void* qkv, int splits, int64_t slice, int64_t off, int sub,
                                              float (&v)[PER], float scale = 1.0f) {
  if (splits == 0) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(qkv) + off + (int64_t)sub * PER;
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = bf16_to_f32(src[e]);
    return;
  }
  const float* src = reinterpret_cast<const float*>(qkv) + off + (int64_t)sub * PER;
#pragma unroll
  for (int e = 0; e < PER; ++e) v[e] = 0.0f;
  // two slices' loads in flight at a time, summed in slice order
  for (int sp = 0; sp < splits; sp += 2) {
    float t[2][PER];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < PER; ++e) t[u][e] = sp + u < splits ? src[(sp + u) * slice + e] : 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < PER; ++e)
        if (sp + u < splits) v[e] += t[u][e];
  }
#pragma unroll
  for (int e = 0; e < PER; ++e) v[e] = round_bf16(v[e] * scale);
}

// sum over the L lanes of a row (L a power of two, rows aligned to L lanes)
template <int L>
__device__ __forceinline__ float row_sum(float x) {
#pragma unroll
  for (int o = 1; o < L; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// The per-lane constants of norm_rope_row: the norm gains of the lane's dims (nw may be null:
// no norm) and the RoPE frequency of each dim's pair, loaded apart from the rows they apply to.
template <int HD, int L>
struct RowConsts {
  float w[HD / L];
  float inv[HD / L];
};

template <int HD, int L>
__device__ __forceinline__ RowConsts<HD, L> row_consts(int sub, const uint16_t* nw, bool rope, const float* inv_freq) {
  constexpr int PER = HD / L;
  RowConsts<HD, L> c;
  const bool first_half = sub < L / 2;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int d = sub * PER + e;
    c.w[e] = nw ? bf16_to_f32(nw[d]) : 1.0f;
    c.inv[e] = rope ? inv_freq[first_half ? d : d - HD / 2] : 0.0f;
  }
  return c;
}

// per-head RMSNorm (norm: gains c.w) and rotate-half RoPE (rope: frequencies c.inv) of one row
// held as load_proj_row leaves it
template <int HD, int L>
__device__ __forceinline__ void norm_rope_row(float (&v)[HD / L], int sub, const RowConsts<HD, L>& c, bool norm,
                                              float eps, bool rope, int pos) {
  constexpr int PER = HD / L;
  if (norm) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) ss += v[e] * v[e];
    ss = row_sum<L>(ss);
    const float r = rsqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = round_bf16((v[e] * r) * c.w[e]);
  }
  if (rope) {
    // dim d pairs with d + HD/2, which sits L/2 lanes away
    const bool first_half = sub < L / 2;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const float partner = __shfl_xor(v[e], L / 2, 64);
      float sn, cs;
      rope_sincos(pos, c.inv[e], sn, cs);
      const float x1 = first_half ? v[e] : partner, x2 = first_half ? partner : v[e];
      v[e] = round_bf16(first_half ? x1 * cs - x2 * sn : x2 * cs + x1 * sn);
    }
  }
}

template <int HD, int L>
__device__ __forceinline__ void norm_rope_row(float (&v)[HD / L], int sub, const uint16_t* nw, float eps, bool rope,
                                              const float* inv_freq, int pos) {
  norm_rope_row<HD, L>(v, sub, row_consts<HD, L>(sub, nw, rope, inv_freq), nw != nullptr, eps, rope, pos);
}

// Store one K or V row at pool token `tok` (bf16, or 8-bit affine group 64 with its scale and
// bias) and leave in v the values attention reads back for it.
template <int HD, int L>
__device__ __forceinline__ void kv_store_row(float (&v)[HD / L], int sub, int kv_dtype, void* pool, uint32_t* sbp,
                                             int64_t tok) {
  constexpr int PER = HD / L;
  if (kv_dtype == DSK_KV_BF16) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(pool) + tok * HD + sub * PER;
#pragma unroll
    for (int e = 0; e < PER; ++e) dst[e] = f32_to_bf16(v[e]);
    return;
  }
  constexpr int GL = 64 / PER;  // lanes per group of 64 dims
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int e = 1; e < PER; ++e) {
    lo = fminf(lo, v[e]);
    hi = fmaxf(hi, v[e]);
  }
#pragma unroll
  for (int o = 1; o < GL; o <<= 1) {
    lo = fminf(lo, __shfl_xor(lo, o, 64));
    hi = fmaxf(hi, __shfl_xor(hi, o, 64));
  }
  uint16_t s16 = f32_to_bf16((hi - lo) / 255.0f);
  float sf = bf16_to_f32(s16);
  if (!(sf > 0.0f)) {
    s16 = 0x3f80;
    sf = 1.0f;
  }
  const uint16_t b16 = f32_to_bf16(lo);
  const float bf = bf16_to_f32(b16);
  uint8_t* qd = reinterpret_cast<uint8_t*>(pool) + tok * HD + sub * PER;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const float q = fminf(fmaxf(rintf((v[e] - bf) / sf), 0.0f), 255.0f);
    qd[e] = (uint8_t)(int)q;
    v[e] = round_bf16(fmaf(sf, q, bf));
  }
  if ((sub % GL) == 0) sbp[tok * (HD / 64) + (sub * PER) / 64] = (uint32_t)s16 | ((uint32_t)b16 << 16);
}

__device__ __forceinline__ int64_t pool_token(const int32_t* block_table, int max_pages, int page, int nkv, int b,
                                              int kvh, int j) {
  const int pg = block_table[(int64_t)b * max_pages + j / page];
  return ((int64_t)pg * nkv + kvh) * page + (j % page);
}

}  // namespace dsk
