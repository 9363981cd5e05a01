// Paged KV cache append and split-K attention on gfx950.
//
// Pool layout (per layer): page p, kv head h, slot t holds one token's head vector
//   bf16: kv[((p * nkv + h) * page + t) * hd + d]
//   u8  : kv[((p * nkv + h) * page + t) * hd + d] and sb[((p * nkv + h) * page + t) * (hd/64) + g]
//         (u32 = bf16 scale | bf16 bias << 16; affine group 64 along head_dim).
// A row's logical token j lives in physical page block_table[b * max_pages + j / page].
//
// Attention is computed transposed so no register transposes are needed:
//   S^T[key][q] = K . Q^T  (A = K tile from LDS, B = Q from registers), then
//   O^T[d][q]  += V^T . P^T (A = V^T tile from LDS, B = P^T straight from the S^T registers:
//   the lane that holds S^T[4c + r][q] for two 16-key halves feeds exactly those 8 keys as
//   its B items, and V^T is read from LDS with the same key order).
// Every lane therefore owns one query column, which makes the online softmax lane-local.
#include "common.h"

namespace dsk {

// ----------------------------------------------------------------------------- append
__device__ __forceinline__ void kv_quant_store(float v0, float v1, int lane, int hd, uint8_t* qdst,
                                               uint32_t* sbdst) {
  // hd values spread 2 per lane over 64 lanes (hd = 128) or 4 per lane (hd = 256, called twice);
  // groups of 64 = 32 consecutive lanes.
  float lo = fminf(v0, v1), hi = fmaxf(v0, v1);
  for (int o = 1; o < 32; o <<= 1) {
    lo = fminf(lo, __shfl_xor(lo, o, 64));
    hi = fmaxf(hi, __shfl_xor(hi, o, 64));
  }
  float s = (hi - lo) / 255.0f;
  uint16_t s16 = f32_to_bf16(s);
  float sf = bf16_to_f32(s16);
  if (!(sf > 0.0f)) {
    s16 = 0x3f80;
    sf = 1.0f;
  }
  uint16_t b16 = f32_to_bf16(lo);
  float bf = bf16_to_f32(b16);
  float q0 = fminf(fmaxf(rintf((v0 - bf) / sf), 0.0f), 255.0f);
  float q1 = fminf(fmaxf(rintf((v1 - bf) / sf), 0.0f), 255.0f);
  qdst[2 * lane] = (uint8_t)(int)q0;
  qdst[2 * lane + 1] = (uint8_t)(int)q1;
  if ((lane & 31) == 0) sbdst[lane >> 5] = (uint32_t)s16 | ((uint32_t)b16 << 16);
  (void)hd;
}

// One wave per (token row, head): lane holds dims [PER*lane, PER*lane + PER) (PER = HD/64).
template <int HD>
__global__ __launch_bounds__(256) void qkv_rope_append_kernel(
    const void* __restrict__ qkv, int qkv_splits, int B, int W, int nq, int nkv, const uint16_t* __restrict__ q_norm,
    const uint16_t* __restrict__ k_norm, float eps, const float* __restrict__ inv_freq,
    const int32_t* __restrict__ seq_lens, int pos_offset, const int32_t* __restrict__ block_table, int max_pages,
    int page, int kv_dtype, void* __restrict__ k_pool, void* __restrict__ v_pool, uint32_t* __restrict__ k_sb,
    uint32_t* __restrict__ v_sb, uint16_t* __restrict__ q_out) {
  constexpr int PER = HD / 64;  // values per lane
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nheads = nq + 2 * nkv;
  const int task = blockIdx.x * 4 + wv;
  const int row = task / nheads, head = task % nheads;
  if (row >= B * W) return;
  const int b = row / W, i = row % W;
  const int pos = seq_lens[b] + i + pos_offset;
  float v[PER];
  if (qkv_splits == 0) {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(qkv) + (int64_t)row * nheads * HD + (int64_t)head * HD;
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = bf16_to_f32(src[lane * PER + e]);
  } else {
    // fp32 partial sums [splits][B*W][nheads*HD], summed in split order, rounded to bf16
    // (the projection's output dtype)
    const int64_t slice = (int64_t)B * W * nheads * HD;
    const float* src = reinterpret_cast<const float*>(qkv) + (int64_t)row * nheads * HD + (int64_t)head * HD;
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = 0.0f;
    // four slices' loads in flight at a time, summed in slice order
    for (int sp = 0; sp < qkv_splits; sp += 4) {
      float t[4][PER];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < PER; ++e) t[u][e] = sp + u < qkv_splits ? src[(sp + u) * slice + lane * PER + e] : 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < PER; ++e)
          if (sp + u < qkv_splits) v[e] += t[u][e];
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = round_bf16(v[e]);
  }

  const bool is_q = head < nq, is_k = !is_q && head < nq + nkv;
  const uint16_t* nw = is_q ? q_norm : (is_k ? k_norm : nullptr);
  if (nw) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) ss += v[e] * v[e];
    ss = wave_sum(ss);
    const float r = rsqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = round_bf16((v[e] * r) * bf16_to_f32(nw[lane * PER + e]));
  }
  if (is_q || is_k) {
    // rotate-half RoPE: dim d pairs with d + HD/2, which sits 32 lanes away
    const bool first_half = lane < 32;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const float partner = __shfl_xor(v[e], 32, 64);
      const int d = lane * PER + e;
      const int dd = first_half ? d : d - HD / 2;
      // angle in fp32 as the reference computes it, reduced to [-1/2, 1/2) revolutions for
      // v_sin_f32 / v_cos_f32 (the reduction error is below the angle's own rounding)
      const float ang = (float)pos * inv_freq[dd];
      float rev = ang * 0.15915494309189535f;
      rev -= rintf(rev);
      const float sn = __builtin_amdgcn_sinf(rev), cs = __builtin_amdgcn_cosf(rev);
      const float x1 = first_half ? v[e] : partner, x2 = first_half ? partner : v[e];
      v[e] = round_bf16(first_half ? x1 * cs - x2 * sn : x2 * cs + x1 * sn);
    }
  }
  if (is_q) {
    uint16_t* dst = q_out + (int64_t)row * nq * HD + (int64_t)head * HD;
#pragma unroll
    for (int e = 0; e < PER; ++e) dst[lane * PER + e] = f32_to_bf16(v[e]);
    return;
  }
  const int h = is_k ? head - nq : head - nq - nkv;
  if (pos < 0 || pos >= max_pages * page) return;  // beyond the row's block table: dropped
  const int pg = block_table[(int64_t)b * max_pages + pos / page];
  const int slot = pos % page;
  const int64_t tok = ((int64_t)pg * nkv + h) * page + slot;
  if (kv_dtype == DSK_KV_BF16) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(is_k ? k_pool : v_pool) + tok * HD;
#pragma unroll
    for (int e = 0; e < PER; ++e) dst[lane * PER + e] = f32_to_bf16(v[e]);
  } else {
    uint8_t* qd = reinterpret_cast<uint8_t*>(is_k ? k_pool : v_pool) + tok * HD;
    uint32_t* sd = (is_k ? k_sb : v_sb) + tok * (HD / 64);
    if (PER == 2) {
      kv_quant_store(v[0], v[1], lane, HD, qd, sd);
    } else {
      // HD = 256: lane holds 4 consecutive dims; group = 16 lanes. Reuse the 2-wide path on
      // a regrouped view: dims (4l, 4l+1) and (4l+2, 4l+3) both belong to group l / 16.
      float lo = fminf(fminf(v[0], v[1]), fminf(v[2 % PER], v[3 % PER]));
      float hi = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2 % PER], v[3 % PER]));
      for (int o = 1; o < 16; o <<= 1) {
        lo = fminf(lo, __shfl_xor(lo, o, 64));
        hi = fmaxf(hi, __shfl_xor(hi, o, 64));
      }
      float s = (hi - lo) / 255.0f;
      uint16_t s16 = f32_to_bf16(s);
      float sf = bf16_to_f32(s16);
      if (!(sf > 0.0f)) {
        s16 = 0x3f80;
        sf = 1.0f;
      }
      uint16_t b16 = f32_to_bf16(lo);
      float bf = bf16_to_f32(b16);
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        float q = fminf(fmaxf(rintf((v[e] - bf) / sf), 0.0f), 255.0f);
        qd[lane * PER + e] = (uint8_t)(int)q;
      }
      if ((lane & 15) == 0) sd[lane >> 4] = (uint32_t)s16 | ((uint32_t)b16 << 16);
    }
  }
}

// ----------------------------------------------------------------------------- attention
struct AttnArgs {
  const uint16_t* q;
  int B, W, nq, nkv, G, R;  // R = W * G query rows per (b, kv head)
  float scale, softcap;
  int causal, window;
  const int32_t* seq_lens;
  const int32_t* block_table;
  int max_pages, page, kv_dtype;
  const void* k_pool;
  const void* v_pool;
  const uint32_t* k_sb;
  const uint32_t* v_sb;
  uint16_t* out;
  int out_packed;
  int nsplit;
  float* part;  // [B][nkv][nsplit][R][HD + 4]: o (unnormalised) | m | l | 0 | 0
};

// keys per split: one workgroup loads its whole split at once
template <int HD> struct Split {
  static constexpr int KEYS = HD == 128 ? 128 : 64;
  static constexpr int KROW = HD + 8;    // K rows in LDS (bf16, padded)
  static constexpr int VROW = KEYS + 8;  // V^T rows in LDS (bf16, padded)
  static constexpr int CK = KEYS * HD / 8 / 256;        // 8-element K chunks per thread
  static constexpr int CV = (KEYS / 2) * (HD / 8) / 256;  // (2 keys x 8 dims) V chunks per thread
  static constexpr int PSTRIDE = HD + 4;
};

// output row (b, i), head h, dim d: row-major [B*W, nq*HD] or packed
__device__ __forceinline__ int64_t attn_out_index(const AttnArgs& a, int HD, int b, int i, int h, int d) {
  const int64_t m = (int64_t)b * a.W + i, k = (int64_t)h * HD + d;
  return a.out_packed ? apack_index(m, k, (int64_t)a.nq * HD / 64) : m * a.nq * HD + k;
}

__device__ __forceinline__ int64_t kv_token(const AttnArgs& a, int b, int kvh, int j) {
  const int pg = a.block_table[(int64_t)b * a.max_pages + j / a.page];
  return ((int64_t)pg * a.nkv + kvh) * a.page + (j % a.page);
}

// 8 consecutive dims of one token as bf16 (dequantised for 8-bit KV)
struct Chunk8 {
  u32x4 raw;
  uint32_t sb;
};
template <int KVT>
__device__ __forceinline__ void load_chunk(const void* pool, const uint32_t* sbp, int HD, int64_t tok, int d0,
                                           Chunk8& c) {
  if (KVT == DSK_KV_BF16) {
    c.raw = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(pool) + tok * HD + d0);
  } else {
    const uint2 r = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(pool) + tok * HD + d0);
    c.raw = u32x4{r.x, r.y, 0, 0};
    c.sb = sbp[tok * (HD / 64) + d0 / 64];
  }
}
template <int KVT>
__device__ __forceinline__ void chunk_bf16(const Chunk8& c, uint16_t (&h)[8]) {
  if (KVT == DSK_KV_BF16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(&c.raw);
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = p[e];
  } else {
    const float sc = bf16_to_f32((uint16_t)(c.sb & 0xffff)), bi = bf16_to_f32((uint16_t)(c.sb >> 16));
    const uint8_t* qb = reinterpret_cast<const uint8_t*>(&c.raw);
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = f32_to_bf16(fmaf(sc, (float)qb[e], bi));
  }
}

// One workgroup per (row b, kv head, split of KEYS keys): every K/V load of the split is
// issued at once, dequantised into LDS (K row-major, V transposed), then each wave takes
// 16-query tiles through scores, a one-pass softmax and P.V. Splits at or past the row's
// key count exit at once (the combine reads only the live ones).
template <int HD, int QT, int KVT, bool SOFTCAP>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
  using S = Split<HD>;
  constexpr int KEYS = S::KEYS, KROW = S::KROW, VROW = S::VROW;
  __shared__ __attribute__((aligned(16))) uint16_t ks[KEYS * KROW];
  __shared__ __attribute__((aligned(16))) uint32_t vt[HD * VROW / 2];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int split = blockIdx.x % a.nsplit;
  const int bk = blockIdx.x / a.nsplit;  // b * nkv + kvh
  const int b = bk / a.nkv, kvh = bk % a.nkv;
  const int off = a.seq_lens[b];
  const int Lk = min(off + a.W, a.max_pages * a.page);
  const int j_lo = split * KEYS;
  if (j_lo >= Lk) return;
  const int j_hi = min(Lk, j_lo + KEYS);
  constexpr int DT = HD / 16;  // output d tiles
  constexpr int KS = HD / 32;  // k steps of the score MFMA
  constexpr int NKT = KEYS / 16;  // key tiles

  // ---- issue every load of the split
  Chunk8 kc[S::CK], vc[S::CV][2];
#pragma unroll
  for (int ci = 0; ci < S::CK; ++ci) {
    const int c = threadIdx.x + ci * 256;
    const int key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
    const int j = min(j_lo + key, j_hi - 1);  // keys past j_hi are masked below
    load_chunk<KVT>(a.k_pool, a.k_sb, HD, kv_token(a, b, kvh, j), d0, kc[ci]);
  }
#pragma unroll
  for (int ci = 0; ci < S::CV; ++ci) {
    const int c = threadIdx.x + ci * 256;
    const int kp = c % (KEYS / 2), d0 = (c / (KEYS / 2)) * 8;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int j = min(j_lo + 2 * kp + u, j_hi - 1);
      load_chunk<KVT>(a.v_pool, a.v_sb, HD, kv_token(a, b, kvh, j), d0, vc[ci][u]);
    }
  }
  // query fragments of tile t (row r = tile * 16 + lane % 16 = i * G + hl); the first tile's
  // are loaded with the K/V, each later tile's one tile ahead
  auto load_q = [&](int t, u32x4 (&qr)[KS]) {
    const int r = (wv + 4 * t) * 16 + (lane & 15);
    const int rr = r < a.R ? r : 0;
    const uint16_t* qp = a.q + ((int64_t)(b * a.W + rr / a.G) * a.nq + kvh * a.G + rr % a.G) * HD;
#pragma unroll
    for (int s = 0; s < KS; ++s) qr[s] = *reinterpret_cast<const u32x4*>(qp + s * 32 + (lane >> 4) * 8);
  };
  u32x4 qnext[KS];
  load_q(0, qnext);

  // ---- dequantise into LDS
#pragma unroll
  for (int ci = 0; ci < S::CK; ++ci) {
    const int c = threadIdx.x + ci * 256;
    const int key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
    uint16_t h[8];
    chunk_bf16<KVT>(kc[ci], h);
    *reinterpret_cast<u32x4*>(ks + key * KROW + d0) = *reinterpret_cast<const u32x4*>(h);
  }
#pragma unroll
  for (int ci = 0; ci < S::CV; ++ci) {
    const int c = threadIdx.x + ci * 256;
    const int kp = c % (KEYS / 2), d0 = (c / (KEYS / 2)) * 8;
    uint16_t h0[8], h1[8];
    chunk_bf16<KVT>(vc[ci][0], h0);
    chunk_bf16<KVT>(vc[ci][1], h1);
#pragma unroll
    for (int e = 0; e < 8; ++e) vt[((d0 + e) * VROW) / 2 + kp] = (uint32_t)h0[e] | ((uint32_t)h1[e] << 16);
  }
  __syncthreads();

  const uint16_t* vt16 = reinterpret_cast<const uint16_t*>(vt);
#pragma unroll 1
  for (int t = 0; t < QT; ++t) {
    if (wv + 4 * t >= (a.R + 15) / 16) break;
    bf16x8 qf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = __builtin_bit_cast(bf16x8, qnext[s]);
    if (t + 1 < QT && wv + 4 * (t + 1) < (a.R + 15) / 16) load_q(t + 1, qnext);
    const int rq = (wv + 4 * t) * 16 + (lane & 15);
    const bool qvalid = rq < a.R;
    // ---- scores: lane holds S^T[key = 16h + 4*(lane/16) + r][q = lane % 16]
    f32x4 st[NKT];
#pragma unroll
    for (int h = 0; h < NKT; ++h) {
      f32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(ks + (h * 16 + (lane & 15)) * KROW + s * 32 + (lane >> 4) * 8);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[s], acc, 0, 0, 0);
      }
      st[h] = acc;
    }
    const int qpos = off + (qvalid ? rq / a.G : 0);
    float mx = -__builtin_inff();
#pragma unroll
    for (int h = 0; h < NKT; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j_lo + h * 16 + (lane >> 4) * 4 + r;
        float sc = st[h][r] * a.scale;
        if (SOFTCAP) sc = tanhf(sc / a.softcap) * a.softcap;
        bool ok = j < j_hi && qvalid;
        if (a.causal) {
          ok = ok && j <= qpos;
          if (a.window > 0) ok = ok && j > qpos - a.window;
        }
        sc = ok ? sc : -__builtin_inff();
        st[h][r] = sc;
        mx = fmaxf(mx, sc);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float lsum = 0.0f;
    bf16x8 pb[KEYS / 32];
#pragma unroll
    for (int c = 0; c < KEYS / 32; ++c)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sc = st[2 * c + hh][r];
          const float p = sc == -__builtin_inff() ? 0.0f : round_bf16(__expf(sc - mx));
          lsum += p;
          pb[c][hh * 4 + r] = (__bf16)p;
        }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    // ---- O^T[d][q] = V^T . P^T: A = V^T rows d*16 + lane%16, keys in pb's order
    f32x4 o[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      f32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < KEYS / 32; ++c) {
        const uint16_t* vr = vt16 + (d * 16 + (lane & 15)) * VROW + 32 * c + (lane >> 4) * 4;
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
        const u32x4 vv = {lo.x, lo.y, hi.x, hi.y};
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv), pb[c], acc, 0, 0, 0);
      }
      o[d] = acc;
    }
    const int r = rq;
    if (r >= a.R) continue;
    if (a.nsplit == 1) {
      const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
      const int i = r / a.G, hl = r % a.G;
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          a.out[attn_out_index(a, HD, b, i, kvh * a.G + hl, d * 16 + (lane >> 4) * 4 + rr)] = f32_to_bf16(o[d][rr] * inv);
      continue;
    }
    float* pr = a.part + (((size_t)bk * a.nsplit + split) * a.R + r) * S::PSTRIDE;
#pragma unroll
    for (int d = 0; d < DT; ++d) *reinterpret_cast<f32x4*>(pr + d * 16 + (lane >> 4) * 4) = o[d];
    if (lane < 16) *reinterpret_cast<f32x4*>(pr + HD) = f32x4{mx, lsum, 0.0f, 0.0f};
  }
}

// Combine the live splits of one (row b, kv head, query row r) per wave in two load rounds:
// lane s reads split s's (m, l) and forms its weight exp(m_s - M); then every lane reads the
// partial outputs of all splits for its dims at once (up to 64 splits per round).
template <int HD>
__global__ __launch_bounds__(256) void attention_combine_kernel(AttnArgs a) {
  using S = Split<HD>;
  constexpr int PER = HD / 64;
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= a.B * a.nkv * a.R) return;
  const int r = task % a.R, bk = task / a.R;
  const int b = bk / a.nkv, kvh = bk % a.nkv;
  const int Lk = min(a.seq_lens[b] + a.W, a.max_pages * a.page);
  const int ns = min(a.nsplit, (Lk + S::KEYS - 1) / S::KEYS);
  const float* base = a.part + ((size_t)bk * a.nsplit * a.R + r) * S::PSTRIDE;
  const size_t sstride = (size_t)a.R * S::PSTRIDE;
  float acc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) acc[e] = 0.0f;
  float M = -__builtin_inff(), den = 0.0f;
  for (int s0 = 0; s0 < ns; s0 += 64) {
    const int n = min(64, ns - s0);
    float ml[2] = {-__builtin_inff(), 0.0f};
    if (lane < n) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(base + (s0 + lane) * sstride + HD);
      ml[0] = v[0];
      ml[1] = v[1];
    }
    const float Mn = fmaxf(M, wave_max(ml[0]));
    const float rescale = M == -__builtin_inff() ? 0.0f : __expf(M - Mn);
    const float w = ml[0] == -__builtin_inff() ? 0.0f : __expf(ml[0] - Mn);
    den = den * rescale + wave_sum(w * ml[1]);
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] *= rescale;
    M = Mn;
    // all partial rows of this round in flight, 16 at a time
    for (int u0 = 0; u0 < n; u0 += 16) {
      float ov[16][PER];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int s = s0 + min(u0 + u, n - 1);
#pragma unroll
        for (int e = 0; e < PER; ++e) ov[u][e] = base[s * sstride + e * 64 + lane];
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const float wu = __shfl(w, min(u0 + u, 63), 64);
        if (u0 + u < n)
#pragma unroll
          for (int e = 0; e < PER; ++e) acc[e] += wu * ov[u][e];
      }
    }
  }
  const int i = r / a.G, hl = r % a.G;
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
#pragma unroll
  for (int e = 0; e < PER; ++e) a.out[attn_out_index(a, HD, b, i, kvh * a.G + hl, e * 64 + lane)] = f32_to_bf16(acc[e] * inv);
}

// ----------------------------------------------------------------------------- host helpers
template <int HD, int QT>
static void launch_attention(const AttnArgs& a, int kv_dtype, bool softcap, dim3 grid, hipStream_t st) {
  if (kv_dtype == DSK_KV_U8) {
    if (softcap) hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_U8, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_U8, false>), grid, dim3(256), 0, st, a);
  } else {
    if (softcap) hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_BF16, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_BF16, false>), grid, dim3(256), 0, st, a);
  }
}

static int attn_nsplit(int hd, int max_ctx) {
  const int keys = hd == 128 ? Split<128>::KEYS : Split<256>::KEYS;
  return (max_ctx + keys - 1) / keys;
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_qkv_rope_append(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                                   const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                   const float* inv_freq, const int32_t* seq_lens, int pos_offset,
                                   const int32_t* block_table, int max_pages, int page, int kv_dtype,
                                   void* k_pool, void* v_pool, uint32_t* k_sb, uint32_t* v_sb,
                                   uint16_t* q_out, dsk_stream_t stream) {
  DSK_REQUIRE(qkv && inv_freq && seq_lens && block_table && k_pool && v_pool && (q_out || nq == 0),
              "dsk_qkv_rope_append: null pointer");
  DSK_REQUIRE(hd == 128 || hd == 256, "dsk_qkv_rope_append: head_dim %d not supported (128, 256)", hd);
  DSK_REQUIRE(B > 0 && W > 0 && nq >= 0 && nkv > 0 && nq % nkv == 0, "dsk_qkv_rope_append: bad shape");
  DSK_REQUIRE(page > 0 && max_pages > 0, "dsk_qkv_rope_append: bad page geometry");
  DSK_REQUIRE(qkv_splits >= 0, "dsk_qkv_rope_append: qkv_splits=%d", qkv_splits);
  DSK_REQUIRE(kv_dtype == DSK_KV_BF16 || (kv_dtype == DSK_KV_U8 && k_sb && v_sb),
              "dsk_qkv_rope_append: u8 KV needs scale/bias buffers");
  const int tasks = B * W * (nq + 2 * nkv);
  dim3 grid((unsigned)ceil_div(tasks, 4));
  if (hd == 128)
    hipLaunchKernelGGL(qkv_rope_append_kernel<128>, grid, dim3(256), 0, as_stream(stream), qkv, qkv_splits, B, W, nq, nkv, q_norm,
                       k_norm, eps, inv_freq, seq_lens, pos_offset, block_table, max_pages, page, kv_dtype, k_pool,
                       v_pool, k_sb, v_sb, q_out);
  else
    hipLaunchKernelGGL(qkv_rope_append_kernel<256>, grid, dim3(256), 0, as_stream(stream), qkv, qkv_splits, B, W, nq, nkv, q_norm,
                       k_norm, eps, inv_freq, seq_lens, pos_offset, block_table, max_pages, page, kv_dtype, k_pool,
                       v_pool, k_sb, v_sb, q_out);
  DSK_LAUNCH_CHECK("dsk_qkv_rope_append");
  return DSK_OK;
}

extern "C" size_t dsk_attn_ws_bytes(int B, int W, int nq, int hd, int max_ctx) {
  if (B <= 0 || W <= 0 || nq <= 0 || hd <= 0 || max_ctx <= 0) return 0;
  if (hd != 128 && hd != 256) return 0;
  // rows per kv head * nkv = W * nq
  const size_t nsplit = (size_t)attn_nsplit(hd, max_ctx);
  return nsplit > 1 ? (size_t)B * W * nq * nsplit * (hd + 4) * sizeof(float) : 0;
}

extern "C" int dsk_attention(const uint16_t* q, int B, int W, int nq, int nkv, int hd, float scale, int causal,
                             int window, float softcap, const int32_t* seq_lens, int max_ctx,
                             const int32_t* block_table, int max_pages, int page, int kv_dtype, const void* k_pool,
                             const void* v_pool, const uint32_t* k_sb, const uint32_t* v_sb, uint16_t* out,
                             int out_packed, void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(q && seq_lens && block_table && k_pool && v_pool && out, "dsk_attention: null pointer");
  DSK_REQUIRE(hd == 128 || hd == 256, "dsk_attention: head_dim %d not supported (128, 256)", hd);
  DSK_REQUIRE(B > 0 && W > 0 && nq > 0 && nkv > 0 && nq % nkv == 0, "dsk_attention: bad shape");
  DSK_REQUIRE(kv_dtype == DSK_KV_BF16 || (kv_dtype == DSK_KV_U8 && k_sb && v_sb), "dsk_attention: u8 KV needs sb");
  DSK_REQUIRE(max_ctx >= W && (int64_t)max_pages * page >= max_ctx, "dsk_attention: max_ctx %d beyond block table",
              max_ctx);
  const int G = nq / nkv;
  const int R = W * G;
  const int tiles = (R + 15) / 16;
  const int QT = (tiles + 3) / 4;
  DSK_REQUIRE(QT <= (hd == 128 ? 4 : 2), "dsk_attention: W*G=%d query rows per kv head exceeds %d", R,
              (hd == 128 ? 256 : 128));
  AttnArgs a;
  a.q = q;
  a.B = B;
  a.W = W;
  a.nq = nq;
  a.nkv = nkv;
  a.G = G;
  a.R = R;
  a.scale = scale;
  a.softcap = softcap;
  a.causal = causal;
  a.window = window;
  a.seq_lens = seq_lens;
  a.block_table = block_table;
  a.max_pages = max_pages;
  a.page = page;
  a.kv_dtype = kv_dtype;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.k_sb = k_sb;
  a.v_sb = v_sb;
  a.out = out;
  a.out_packed = out_packed ? 1 : 0;
  DSK_REQUIRE(!out_packed || (B * W <= 64 && (nq * hd) % 64 == 0), "dsk_attention: packed output needs B*W <= 64");
  a.nsplit = attn_nsplit(hd, max_ctx);
  const size_t need = a.nsplit > 1 ? (size_t)B * nkv * a.nsplit * R * (hd + 4) * sizeof(float) : 0;
  DSK_REQUIRE(a.nsplit == 1 || (workspace && ws_bytes >= need), "dsk_attention: workspace %zu < %zu", ws_bytes, need);
  a.part = reinterpret_cast<float*>(workspace);
  dim3 grid((unsigned)(B * nkv * a.nsplit));
  hipStream_t st = as_stream(stream);
  const bool sc = softcap > 0.0f;
#define DSK_ATTN_CASE(hdv, qt) \
  if (hd == hdv && QT == qt) launch_attention<hdv, qt>(a, kv_dtype, sc, grid, st);
  DSK_ATTN_CASE(128, 1) DSK_ATTN_CASE(128, 2) DSK_ATTN_CASE(128, 3) DSK_ATTN_CASE(128, 4)
  DSK_ATTN_CASE(256, 1) DSK_ATTN_CASE(256, 2)
#undef DSK_ATTN_CASE
  DSK_LAUNCH_CHECK("dsk_attention");
  if (a.nsplit > 1) {
    const dim3 cgrid((unsigned)ceil_div((int64_t)B * nkv * R, 4));
    if (hd == 128) hipLaunchKernelGGL(attention_combine_kernel<128>, cgrid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(attention_combine_kernel<256>, cgrid, dim3(256), 0, st, a);
    DSK_LAUNCH_CHECK("dsk_attention (combine)");
  }
  return DSK_OK;
}
