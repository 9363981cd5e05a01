// Paged KV cache append and split-K attention on gfx950.
//
// Pool layout (per layer): page p, kv head h, slot t holds one token's head vector
//   bf16: kv[((p * nkv + h) * page + t) * hd + d]
//   u8  : kv[((p * nkv + h) * page + t) * hd + d] and sb[((p * nkv + h) * page + t) * (hd/64) + g]
//         (u32 = bf16 scale | bf16 bias << 16; affine group 64 along head_dim).
// A row's logical token j lives in physical page block_table[b * max_pages + j / page]; every
// entry of the table must name a valid page (the kernels read whole splits through it).
//
// Attention is computed transposed so no register transposes are needed:
//   S^T[key][q] = K . Q^T  (A = K tile from LDS, B = Q from registers), then
//   O^T[d][q]  += V^T . P^T (A = V^T tile from LDS, B = P^T straight from the S^T registers:
//   the lane that holds S^T[4c + r][q] for two 16-key halves feeds exactly those 8 keys as
//   its B items, and V^T is read from LDS with the same key order).
// Every lane therefore owns one query column, which makes the online softmax lane-local.
//
// The fused entry (dsk_qkv_attention) starts from the qkv projection itself: each workgroup
// forms its own queries (sum of the split-K partial slices, RMSNorm, RoPE) while its K/V loads
// are in flight, and the workgroup whose key range holds the new tokens also normalises,
// rotates and quantises their K/V, appends them to the pool and uses them straight from LDS.
#include <stdlib.h>

#include <algorithm>

#include "common.h"
#include "kvrow.h"

namespace dsk {

// ----------------------------------------------------------------------------- append
// One wave per (token row, head): lane holds dims [PER*lane, PER*lane + PER) (PER = HD/64).
// F32: the projection arrives as qkv_splits f32 split-K slices (else one bf16 row); RS: their sum
// takes the row scale of a normed-later projection input. Every independent load is issued
// first, with no branch between them (a value that is not needed reads a valid address and is
// discarded): the first two slices, the first 256 tile partials of the input's x^2, the norm gains
// and RoPE frequencies, and, once the row length is in, a K/V row's page id. The slices are summed
// as load_proj_row sums them; the row scale is the W8 GEMM's (rsqrt(sum / 16 x_tiles + x_eps),
// the partials summed in the same order).
template <int HD, bool RS, bool F32>
__global__ __launch_bounds__(256) void qkv_rope_append_kernel(
    const void* __restrict__ qkv, int qkv_splits, int B, int W, int nq, int nkv, const uint16_t* __restrict__ q_norm,
    const uint16_t* __restrict__ k_norm, const uint16_t* __restrict__ v_norm, float eps,
    const float* __restrict__ inv_freq, const int32_t* __restrict__ seq_lens, int pos_offset,
    const int32_t* __restrict__ block_table, int max_pages, int page, int kv_dtype, void* __restrict__ k_pool,
    void* __restrict__ v_pool, uint32_t* __restrict__ k_sb, uint32_t* __restrict__ v_sb,
    uint16_t* __restrict__ q_out, const float* __restrict__ x_ssq, int x_tiles, float x_k, float x_eps) {
  static_assert(F32 || !RS, "the row scale applies to split-K slices");
  constexpr int PER = HD / 64;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nheads = nq + 2 * nkv;
  const int task = blockIdx.x * 4 + wv;
  const int row = task / nheads, head = task % nheads;
  if (row >= B * W) return;
  const int b = row / W, i = row % W;
  const bool is_q = head < nq, is_k = !is_q && head < nq + nkv;
  const uint16_t* nw = is_q ? q_norm : (is_k ? k_norm : v_norm);
  const bool rope = is_q || is_k;
  const int pos = seq_lens[b] + i + pos_offset;  // first: the page id load waits for it alone

  const int64_t slice = (int64_t)B * W * nheads * HD, off = ((int64_t)row * nheads + head) * HD + lane * PER;
  float t[2][PER];
  if constexpr (F32) {
    const float* src = reinterpret_cast<const float*>(qkv) + off;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < PER; ++e) t[u][e] = src[(int64_t)min(u, qkv_splits - 1) * slice + e];
  } else {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(qkv) + off;
#pragma unroll
    for (int e = 0; e < PER; ++e) t[0][e] = bf16_to_f32(src[e]);
  }
  float xs[4];
  if constexpr (RS) {
#pragma unroll
    for (int j = 0; j < 4; ++j) xs[j] = x_ssq[(int64_t)row * x_tiles + min(lane + 64 * j, x_tiles - 1)];
  }
  RowConsts<HD, 64> rc;
  const uint16_t* wsrc = nw ? nw : reinterpret_cast<const uint16_t*>(inv_freq);  // HD / 2 floats: HD halves
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int d = lane * PER + e;
    rc.w[e] = bf16_to_f32(wsrc[d]);
    rc.inv[e] = inv_freq[lane < 32 ? d : d - HD / 2];
  }
  const int h = is_k ? head - nq : head - nq - nkv;
  const bool stored = !is_q && pos >= 0 && pos < max_pages * page;  // beyond the row's block table: dropped
  const int pg = block_table[stored ? (int64_t)b * max_pages + pos / page : 0];

  float v[PER];
  if constexpr (F32) {
    // the slices summed in slice order (two loads in flight at a time past the first two), times
    // the row scale, rounded to bf16
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      v[e] = 0.0f;
      v[e] += t[0][e];
      if (qkv_splits > 1) v[e] += t[1][e];
    }
    const float* src = reinterpret_cast<const float*>(qkv) + off;
    for (int sp = 2; sp < qkv_splits; sp += 2) {
      float n[2][PER];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < PER; ++e) n[u][e] = sp + u < qkv_splits ? src[(sp + u) * slice + e] : 0.0f;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < PER; ++e)
          if (sp + u < qkv_splits) v[e] += n[u][e];
    }
    float scale = 1.0f;
    if constexpr (RS) {
      // lane l sums the partials l, l + 64, ... in that order, then the wave sums its lanes
#pragma unroll
      for (int j = 0; j < 4; ++j) xs[j] = lane + 64 * j < x_tiles ? xs[j] : 0.0f;
      float ss = ((xs[0] + xs[1]) + xs[2]) + xs[3];
      for (int j = lane + 256; j < x_tiles; j += 64) ss += x_ssq[(int64_t)row * x_tiles + j];
      scale = rsqrtf(wave_sum(ss) / x_k + x_eps);
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = round_bf16(v[e] * scale);
  } else {
#pragma unroll
    for (int e = 0; e < PER; ++e) v[e] = t[0][e];
  }
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    if (!nw) rc.w[e] = 1.0f;
    if (!rope) rc.inv[e] = 0.0f;
  }
  norm_rope_row<HD, 64>(v, lane, rc, nw != nullptr, eps, rope, pos);
  if (is_q) {
    uint16_t* dst = q_out + (int64_t)row * nq * HD + (int64_t)head * HD;
#pragma unroll
    for (int e = 0; e < PER; ++e) dst[lane * PER + e] = f32_to_bf16(v[e]);
    return;
  }
  if (!stored) return;
  const int64_t tok = ((int64_t)pg * nkv + h) * page + pos % page;
  kv_store_row<HD, 64>(v, lane, kv_dtype, is_k ? k_pool : v_pool, is_k ? k_sb : v_sb, tok);
}

// ----------------------------------------------------------------------------- attention
struct AttnArgs {
  const uint16_t* q;  // roped queries [B*W][nq*HD] (dsk_attention)
  const void* qkv;    // the qkv projection (dsk_qkv_attention), bf16 or fp32 split-K slices
  int qkv_splits;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  float eps;
  const float* inv_freq;
  int B, W, nq, nkv, G, R;  // R = W * G query rows per (b, kv head)
  float scale, softcap;
  int causal, window;
  const int32_t* seq_lens;
  const int32_t* block_table;
  int max_pages, page, kv_dtype;
  void* k_pool;
  void* v_pool;
  uint32_t* k_sb;
  uint32_t* v_sb;
  uint16_t* out;
  int out_packed;
  int nsplit;
  int kps;           // keys per (context) split: a whole number of LDS blocks (Split<HD>::KEYS)
  int fused;         // splits 0 .. nsplit-2: cached keys; split nsplit-1: the new tokens
  float* part_o;     // [B*nkv][nsplit][R][HD] float32: the split's o / l
  float* part_ml;    // [B*nkv][nsplit][R][2]: the split's running max m and sum l
  int tgroups;       // verify kernel: groups of QT query tiles per kv head, one workgroup each
  int wrel;          // verify kernel, sliding window: split s of row b starts at split
                     // max(0, seq_lens[b] - window + 1) / kps + s (nsplit covers one window)
};

// bf16 terms that carry a float32 probability into the P.V MFMAs of the verify and split
// kernels: hi + mid + lo is within 2^-26 of p. Two terms (within 2^-17) put the full-width
// Qwen3-8B verify logits at 1.3x the noise floor's rms against the float32-softmax reference
// (1.07x with three); one term (bf16 P) moves them further.
#ifndef DSK_ATTN_P_TERMS
#define DSK_ATTN_P_TERMS 3
#endif
constexpr int kPTerms = DSK_ATTN_P_TERMS;

// page ids one split may span (kps / page + 1), held in LDS
constexpr int kAttnMaxSplitPages = 256;

// LDS capacity in keys of one block (a split streams kps / KEYS blocks through it)
template <int HD> struct Split {
  static constexpr int KEYS = HD == 128 ? 128 : (HD == 256 ? 64 : 32);
  static constexpr int KROW = HD + 8;    // K rows in LDS (bf16, padded)
  static constexpr int VROW = KEYS + 8;  // V^T rows in LDS (bf16, padded)
};

// output row (b, i), head h, dim d: row-major [B*W, nq*HD] or packed
__device__ __forceinline__ int64_t attn_out_index(const AttnArgs& a, int HD, int b, int i, int h, int d) {
  const int64_t m = (int64_t)b * a.W + i, k = (int64_t)h * HD + d;
  return a.out_packed ? apack_index(m, k, (int64_t)a.nq * HD / 64) : m * a.nq * HD + k;
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

// The queries of one 16-row tile in the score MFMA's B layout: lane holds row
// r = tile * 16 + lane % 16 (token r / G, q head kvh * G + r % G), dims 32 s + 8 (lane / 16) + e.
template <int HD, bool FUSED>
struct QTile {
  static constexpr int KS = HD / 32;
  float v[FUSED ? KS : 1][FUSED ? 8 : 1];
  u32x4 raw[FUSED ? 1 : KS];
};

template <int HD, bool FUSED>
__device__ __forceinline__ void qtile_load(const AttnArgs& a, int b, int kvh, int tile, int lane, QTile<HD, FUSED>& q) {
  constexpr int KS = HD / 32;
  const int r = tile * 16 + (lane & 15);
  const int rr = r < a.R ? r : 0;
  const int i = rr / a.G, head = kvh * a.G + rr % a.G;
  const int g8 = (lane >> 4) * 8;
  if constexpr (!FUSED) {
    const uint16_t* qp = a.q + ((int64_t)(b * a.W + i) * a.nq + head) * HD;
#pragma unroll
    for (int s = 0; s < KS; ++s) q.raw[s] = *reinterpret_cast<const u32x4*>(qp + s * 32 + g8);
  } else {
    const int nheads = a.nq + 2 * a.nkv;
    const int64_t off = ((int64_t)(b * a.W + i) * nheads + head) * HD;
    if (a.qkv_splits == 0) {
      const uint16_t* src = reinterpret_cast<const uint16_t*>(a.qkv) + off;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(src + s * 32 + g8);
        const uint16_t* h = reinterpret_cast<const uint16_t*>(&w);
#pragma unroll
        for (int e = 0; e < 8; ++e) q.v[s][e] = bf16_to_f32(h[e]);
      }
    } else {
      const int64_t slice = (int64_t)a.B * a.W * nheads * HD;
      const float* src = reinterpret_cast<const float*>(a.qkv) + off;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) q.v[s][e] = 0.0f;
      for (int sp = 0; sp < a.qkv_splits; sp += 2) {
        f32x4 t[2][KS][2];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int h = 0; h < 2; ++h)
              t[u][s][h] = sp + u < a.qkv_splits
                               ? *reinterpret_cast<const f32x4*>(src + (sp + u) * slice + s * 32 + g8 + 4 * h)
                               : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < 2; ++u)
          if (sp + u < a.qkv_splits)
#pragma unroll
            for (int s = 0; s < KS; ++s)
#pragma unroll
              for (int e = 0; e < 8; ++e) q.v[s][e] += t[u][s][e / 4][e % 4];
      }
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) q.v[s][e] = round_bf16(q.v[s][e]);
    }
  }
}

// q norm and RoPE of a loaded tile (fused), or the loaded bf16 queries as they are
template <int HD, bool FUSED>
__device__ __forceinline__ void qtile_finish(const AttnArgs& a, int off, int tile, int lane, QTile<HD, FUSED>& q,
                                             bf16x8 (&qf)[HD / 32]) {
  constexpr int KS = HD / 32;
  if constexpr (!FUSED) {
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = __builtin_bit_cast(bf16x8, q.raw[s]);
  } else {
    const int r = tile * 16 + (lane & 15);
    const int rr = r < a.R ? r : 0;
    const int pos = off + rr / a.G;
    const int g8 = (lane >> 4) * 8;
    if (a.q_norm) {
      float ss = 0.0f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += q.v[s][e] * q.v[s][e];
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      const float rn = rsqrtf(ss / (float)HD + a.eps);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(a.q_norm + s * 32 + g8);
        const uint16_t* h = reinterpret_cast<const uint16_t*>(&w);
#pragma unroll
        for (int e = 0; e < 8; ++e) q.v[s][e] = round_bf16((q.v[s][e] * rn) * bf16_to_f32(h[e]));
      }
    }
    // rotate-half: dim 32 s + ... pairs with 32 (s + KS/2) + ... in the same lane
#pragma unroll
    for (int s = 0; s < KS / 2; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float sn, cs;
        rope_sincos(pos, a.inv_freq[s * 32 + g8 + e], sn, cs);
        const float x1 = q.v[s][e], x2 = q.v[s + KS / 2][e];
        q.v[s][e] = round_bf16(x1 * cs - x2 * sn);
        q.v[s + KS / 2][e] = round_bf16(x2 * cs + x1 * sn);
      }
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] = (__bf16)q.v[s][e];
  }
}

// One workgroup per (row b, kv head, split of kps keys). A split is nblk blocks of KEYS keys
// streamed through LDS: each block's K/V chunks are dequantised into LDS (K row-major, V
// transposed) and, while the waves run scores, a one-pass online softmax and P.V on it, the
// next block's loads are already in flight. Every wave owns one 16-query tile for the whole
// split (nblk > 1 needs QT == 1), carrying its running max, sum and output across blocks.
// Splits at or past the row's key count exit before loading (the combine reads only the live
// ones).
// FUSED: splits 0 .. nsplit-2 cover the cached keys [0, seq_lens[b]) and the last split the W
// new tokens, which it forms from the projection (K RMSNorm + RoPE, append to the pool) while
// the context splits stream the cache; every workgroup forms its own queries meanwhile.
template <int HD, int QT, int KVT, bool SOFTCAP, bool FUSED, int WPT>
__global__ __launch_bounds__(256 * WPT) __attribute__((amdgpu_waves_per_eu(1, 2))) void attention_kernel(AttnArgs a) {
  using S = Split<HD>;
  static_assert(WPT == 1 || (WPT == 2 && QT == 1 && !FUSED), "two waves per tile: one tile per wave, no new-token split");
  constexpr int NTHR = 256 * WPT;                      // WPT waves per 16-query tile
  constexpr int CK = S::KEYS * HD / 8 / NTHR;          // 8-element K chunks per thread
  constexpr int CV = (S::KEYS / 2) * (HD / 8) / NTHR;  // (2 keys x 8 dims) V chunks per thread
  constexpr int KH = S::KEYS / WPT;                    // keys of a block one wave scores
  constexpr int KEYS = S::KEYS, KROW = S::KROW, VROW = S::VROW;
  constexpr int DT = HD / 16;     // output d tiles
  constexpr int KS = HD / 32;     // k steps of the score MFMA
  constexpr int NKT = KEYS / 16;  // key tiles
  constexpr int PER16 = HD / 16;  // dims per lane when a quarter wave holds a row
  __shared__ __attribute__((aligned(16))) uint16_t ks[KEYS * KROW];
  __shared__ __attribute__((aligned(16))) uint32_t vt[HD * VROW / 2];
  uint16_t* vt16 = reinterpret_cast<uint16_t*>(vt);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int split = blockIdx.x % a.nsplit;
  const int bk = blockIdx.x / a.nsplit;  // b * nkv + kvh
  const int b = bk / a.nkv, kvh = bk % a.nkv;
  const int jmax = a.max_pages * a.page;
  const bool newsplit = FUSED && split == a.nsplit - 1;
  const int ntiles = (a.R + 15) / 16;
  // keep the arguments the tile loop needs in SGPRs from here on: after the LDS barrier the
  // compiler would otherwise reload them from the kernel-argument segment (a memory round trip)
  float scale = a.scale, softcap = a.softcap;
  int causal = a.causal, window = a.window, nsplit = a.nsplit, kps = a.kps;
  float* part_o = a.part_o;
  float* part_ml = a.part_ml;
  asm volatile("" : "+s"(scale), "+s"(softcap), "+s"(causal), "+s"(window), "+s"(nsplit), "+s"(kps));
  asm volatile("" : "+s"(part_o), "+s"(part_ml));

  // page ids of the split's keys, read once into LDS (the blocks after the first then cost no
  // page-table round trip); pool tokens of the block starting at key j0, clamped into the block
  // table (keys past the split's end are loaded but zeroed in LDS)
  __shared__ int pgs[kAttnMaxSplitPages];
  const int pg0 = (split * kps) / a.page;
  int64_t ktok[CK], vtok[CV][2];
  auto tok_of = [&](int j) -> int64_t {
    j = min(j, jmax - 1);
    return ((int64_t)pgs[j / a.page - pg0] * a.nkv + kvh) * a.page + (j % a.page);
  };
  auto tokens = [&](int j0) {
#pragma unroll
    for (int ci = 0; ci < CK; ++ci) {
      const int c = threadIdx.x + ci * NTHR;
      ktok[ci] = tok_of(j0 + c / (HD / 8));
    }
#pragma unroll
    for (int ci = 0; ci < CV; ++ci) {
      const int kp = (threadIdx.x + ci * NTHR) % (KEYS / 2);
#pragma unroll
      for (int u = 0; u < 2; ++u) vtok[ci][u] = tok_of(j0 + 2 * kp + u);
    }
  };
  Chunk8 kc[CK], vc[CV][2];
  auto issue = [&]() {
#pragma unroll
    for (int ci = 0; ci < CK; ++ci) {
      const int d0 = ((threadIdx.x + ci * NTHR) % (HD / 8)) * 8;
      load_chunk<KVT>(a.k_pool, a.k_sb, HD, ktok[ci], d0, kc[ci]);
    }
#pragma unroll
    for (int ci = 0; ci < CV; ++ci) {
      const int d0 = ((threadIdx.x + ci * NTHR) / (KEYS / 2)) * 8;
#pragma unroll
      for (int u = 0; u < 2; ++u) load_chunk<KVT>(a.v_pool, a.v_sb, HD, vtok[ci][u], d0, vc[ci][u]);
    }
  };
  // dequantise the loaded block [j_lo, j_hi) into LDS (keys past j_hi are zeroed: masked, but finite)
  auto to_lds = [&](int j_lo, int j_hi) {
#pragma unroll
    for (int ci = 0; ci < CK; ++ci) {
      const int c = threadIdx.x + ci * NTHR;
      const int key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
      uint16_t h[8];
      chunk_bf16<KVT>(kc[ci], h);
      u32x4 w = *reinterpret_cast<const u32x4*>(h);
      if (j_lo + key >= j_hi) w = u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(ks + key * KROW + d0) = w;
    }
#pragma unroll
    for (int ci = 0; ci < CV; ++ci) {
      const int c = threadIdx.x + ci * NTHR;
      const int kp = c % (KEYS / 2), d0 = (c / (KEYS / 2)) * 8;
      const int j0 = j_lo + 2 * kp;
      uint16_t h0[8], h1[8];
      chunk_bf16<KVT>(vc[ci][0], h0);
      chunk_bf16<KVT>(vc[ci][1], h1);
      const bool z0 = j0 >= j_hi, z1 = j0 + 1 >= j_hi;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vt[((d0 + e) * VROW) / 2 + kp] = (uint32_t)(z0 ? 0 : h0[e]) | ((uint32_t)(z1 ? 0 : h1[e]) << 16);
    }
  };

  // ---- independent loads: the split's page ids, the first query tile, the row length
  if (!newsplit) {
    const int npg = min((split * kps + kps - 1) / a.page, a.max_pages - 1) - pg0 + 1;
    for (int t = threadIdx.x; t < npg; t += NTHR) pgs[t] = a.block_table[(int64_t)b * a.max_pages + pg0 + t];
  }
  // WPT == 2: waves w and w + 4 share tile w, key halves; blockIdx.y: groups of 4 query tiles
  // (head_dim 512, whose one-tile-per-wave kernel covers any number of query rows this way)
  const int mytile = (int)blockIdx.y * 4 + (wv & 3), half = wv >> 2;
  QTile<HD, FUSED> qt;
  if (mytile < ntiles) qtile_load<HD, FUSED>(a, b, kvh, mytile, lane, qt);
  const int off = a.seq_lens[b];
  __syncthreads();  // the page ids
  const int Lk = min(off + a.W, jmax);
  int j_beg, j_end;
  if (newsplit) {
    j_beg = off;
    j_end = Lk;
  } else {
    j_beg = split * kps;
    const int kend = FUSED ? min(off, jmax) : Lk;  // the fused context splits stop at the cache
    if (j_beg >= kend) return;
    // causal: a split past every query of this workgroup's tile group is never read (the
    // combine counts each row's splits up to its own position)
    if (causal && gridDim.y > 1) {
      const int last_row = min(a.R, ((int)blockIdx.y * 4 + 4) * 16) - 1;
      if (j_beg > off + last_row / a.G) return;
    }
    j_end = min(kend, j_beg + kps);
    // sliding window: a split wholly before the window of this workgroup's first row is never
    // read (every later row's window starts later; the combine starts each row at the first
    // split its window reaches)
    if (causal && window > 0) {
      const int first_row = gridDim.y > 1 ? (int)blockIdx.y * 4 * 16 : 0;
      if (j_end <= off + first_row / a.G - window + 1) return;
    }
  }
  const int nb = newsplit ? 1 : (j_end - j_beg + KEYS - 1) / KEYS;
  if (!newsplit) {
    tokens(j_beg);
    issue();
  }
  // the first tile's queries while the K/V loads are in flight
  bf16x8 qf[KS];
  if (mytile < ntiles) qtile_finish<HD, FUSED>(a, off, mytile, lane, qt, qf);

  if (newsplit) {
    // ---- the new tokens: zero the tile, then K normed + roped, K/V appended to the pool and
    // the values attention reads written to LDS; a quarter wave per (token, K or V) row, two
    // rows per quarter in flight
    for (int c = threadIdx.x; c < KEYS * KROW / 8; c += NTHR) reinterpret_cast<u32x4*>(ks)[c] = u32x4{0, 0, 0, 0};
    for (int c = threadIdx.x; c < HD * VROW / 8; c += NTHR) reinterpret_cast<u32x4*>(vt)[c] = u32x4{0, 0, 0, 0};
    __syncthreads();
    const int n_new = j_end - j_beg;  // <= W
    const int nheads = a.nq + 2 * a.nkv;
    const int quarter = lane >> 4, sub = lane & 15;
    for (int t0 = wv * 4; t0 < 2 * n_new; t0 += 32) {
      float v[2][PER16];
      int jj[2];
      bool kk[2], live[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int task = t0 + 16 * u + quarter;
        live[u] = task < 2 * n_new;
        const int tt = live[u] ? task : 0;
        kk[u] = tt < n_new;
        jj[u] = j_beg + (kk[u] ? tt : tt - n_new);
        const int head = a.nq + (kk[u] ? kvh : a.nkv + kvh);
        load_proj_row<PER16>(a.qkv, a.qkv_splits, (int64_t)a.B * a.W * nheads * HD,
                             ((int64_t)(b * a.W + (jj[u] - off)) * nheads + head) * HD, sub, v[u]);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (!live[u]) continue;  // a whole quarter: its shuffles stay inside it
        norm_rope_row<HD, 16>(v[u], sub, kk[u] ? a.k_norm : nullptr, a.eps, kk[u], a.inv_freq, jj[u]);
        const int64_t tok = pool_token(a.block_table, a.max_pages, a.page, a.nkv, b, kvh, jj[u]);
        kv_store_row<HD, 16>(v[u], sub, a.kv_dtype, kk[u] ? a.k_pool : a.v_pool, kk[u] ? a.k_sb : a.v_sb, tok);
        const int key = jj[u] - j_beg;
        if (kk[u]) {
          uint16_t h[PER16];
#pragma unroll
          for (int e = 0; e < PER16; ++e) h[e] = f32_to_bf16(v[u][e]);
#pragma unroll
          for (int e = 0; e < PER16; e += 8)
            *reinterpret_cast<u32x4*>(ks + key * KROW + sub * PER16 + e) = *reinterpret_cast<const u32x4*>(h + e);
        } else {
#pragma unroll
          for (int e = 0; e < PER16; ++e) vt16[(sub * PER16 + e) * VROW + key] = f32_to_bf16(v[u][e]);
        }
      }
    }
  }

  // running state of this wave's tile across the blocks (one tile per wave when nb > 1)
  float m_run = -__builtin_inff(), l_run = 0.0f;
  f32x4 o[DT];

  // scores, one-pass online softmax and P.V of one 16-query tile over the wave's KH keys of the
  // block in LDS (keys kb .. kb + KH - 1 of the block)
  constexpr int NKH = KH / 16;  // key tiles of the wave
  auto block_compute = [&](int j_lo, int j_hi, int rq, bool qvalid, int kb) {
    // ---- scores: lane holds S^T[key = 16h + 4*(lane/16) + r][q = lane % 16]
    // k-step outer, key tile inner: NKT independent accumulators per k-step keep the MFMA
    // pipe busy, and the next k-step's K fragments are read from LDS while these run
    f32x4 st[NKH];
#pragma unroll
    for (int h = 0; h < NKH; ++h) st[h] = f32x4{0, 0, 0, 0};
    {
      const uint16_t* kbase = ks + (kb + (lane & 15)) * KROW + (lane >> 4) * 8;
      bf16x8 kf[2][NKH];
#pragma unroll
      for (int h = 0; h < NKH; ++h) kf[0][h] = *reinterpret_cast<const bf16x8*>(kbase + h * 16 * KROW);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        if (s + 1 < KS)
#pragma unroll
          for (int h = 0; h < NKH; ++h)
            kf[(s + 1) & 1][h] = *reinterpret_cast<const bf16x8*>(kbase + h * 16 * KROW + (s + 1) * 32);
        __builtin_amdgcn_sched_barrier(0);  // the reads stay grouped ahead of this step's MFMAs
#pragma unroll
        for (int h = 0; h < NKH; ++h) st[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[s & 1][h], qf[s], st[h], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // visible keys of this lane's query: [k_first, k_last] (branch-free mask below)
    const int qpos = off + (qvalid ? rq / a.G : 0);
    int k_last = j_hi - 1, k_first = 0;
    if (causal) {
      k_last = min(k_last, qpos);
      if (window > 0) k_first = qpos - window + 1;
    }
    if (!qvalid) k_last = -1;
    float mx = m_run;
#pragma unroll
    for (int h = 0; h < NKH; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = j_lo + kb + h * 16 + (lane >> 4) * 4 + r;
        float sc = st[h][r] * scale;
        if (SOFTCAP) sc = tanhf(sc / softcap) * softcap;
        sc = (j >= k_first && j <= k_last) ? sc : -__builtin_inff();
        st[h][r] = sc;
        mx = fmaxf(mx, sc);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // rescale of the previous blocks' sum and output (none on the first block)
    const float alpha = m_run == -__builtin_inff() ? 0.0f : __expf(m_run - mx);
    // float32 probabilities in place of the scores (kPTerms bf16 terms each in the P.V MFMAs)
    float lsum = 0.0f;
#pragma unroll
    for (int h = 0; h < NKH; ++h)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sc = st[h][r];
        const float p = sc == -__builtin_inff() ? 0.0f : __expf(sc - mx);
        lsum += p;
        st[h][r] = p;
      }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    l_run = l_run * alpha + lsum;
    m_run = mx;
    // ---- O^T[d][q] = V^T . P^T: A = V^T rows d*16 + lane%16, keys in pb's order
    // (key chunk outer, d tile inner: DT independent accumulators, next chunk's reads ahead)
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] *= alpha;
    {
      auto vfrag = [&](int d, int c) {
        const uint16_t* vr = vt16 + (d * 16 + (lane & 15)) * VROW + kb + 32 * c + (lane >> 4) * 4;
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
        return __builtin_bit_cast(bf16x8, (u32x4{lo.x, lo.y, hi.x, hi.y}));
      };
      bf16x8 vv[2][DT];
#pragma unroll
      for (int d = 0; d < DT; ++d) vv[0][d] = vfrag(d, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < KH / 32; ++c) {
        if (c + 1 < KH / 32)
#pragma unroll
          for (int d = 0; d < DT; ++d) vv[(c + 1) & 1][d] = vfrag(d, c + 1);
        // P of the chunk's 8 keys (score tiles 2c, 2c + 1) as kPTerms bf16 terms
        uint32_t w[kPTerms][4];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int r2 = 0; r2 < 2; ++r2) {
            uint32_t tt[kPTerms];
            split_terms_bf16x2<kPTerms>(st[2 * c + hh][2 * r2], st[2 * c + hh][2 * r2 + 1], tt);
#pragma unroll
            for (int k = 0; k < kPTerms; ++k) w[k][2 * hh + r2] = tt[k];
          }
        __builtin_amdgcn_sched_barrier(0);
        bf16x8 pk[kPTerms];
#pragma unroll
        for (int k = 0; k < kPTerms; ++k) pk[k] = __builtin_bit_cast(bf16x8, (u32x4{w[k][0], w[k][1], w[k][2], w[k][3]}));
        if constexpr (DT >= 16) {
          // wide heads: a V fragment's products back to back, so it is free after them
#pragma unroll
          for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int k = 0; k < kPTerms; ++k) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv[c & 1][d], pk[k], o[d], 0, 0, 0);
        } else {
          // one term over every d tile before the next (DT independent accumulators in between)
#pragma unroll
          for (int k = 0; k < kPTerms; ++k)
#pragma unroll
            for (int d = 0; d < DT; ++d) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv[c & 1][d], pk[k], o[d], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // the tile's result: the output itself (one split) or the split's partial o / l and (m, l)
  auto store_tile = [&](int rq, bool qvalid) {
    if (!qvalid) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    if (nsplit == 1) {
      const int i = rq / a.G, hl = rq % a.G;
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          a.out[attn_out_index(a, HD, b, i, kvh * a.G + hl, d * 16 + (lane >> 4) * 4 + rr)] = f32_to_bf16(o[d][rr] * inv);
      return;
    }
    // partial: o / l in float32 (4 consecutive dims per d tile), (m, l)
    const size_t prow = ((size_t)bk * nsplit + split) * a.R + rq;
    float* po = part_o + prow * HD + (lane >> 4) * 4;
#pragma unroll
    for (int d = 0; d < DT; ++d) *reinterpret_cast<f32x4*>(po + d * 16) = o[d] * inv;
    if (lane < 16) *reinterpret_cast<float2*>(part_ml + prow * 2) = float2{m_run, l_run};
  };

  if (nb > 1 || QT == 1) {
    // ---- one tile per wave (WPT waves per tile), blocks streamed: block blk+1's loads fly
    // while blk is computed
    const int rq = mytile * 16 + (lane & 15);
    const bool qvalid = rq < a.R;
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = f32x4{0, 0, 0, 0};
#pragma unroll 1
    for (int blk = 0; blk < nb; ++blk) {
      const int j_lo = j_beg + blk * KEYS, j_hi = min(j_end, j_lo + KEYS);
      if (!newsplit) {
        if (blk > 0) __syncthreads();  // every wave is done with the previous block's LDS
        to_lds(j_lo, j_hi);
        if (blk + 1 < nb) {
          tokens(j_lo + KEYS);
          issue();
        }
      }
      __syncthreads();
      if (mytile < ntiles) block_compute(j_lo, j_hi, rq, qvalid, half * KH);
    }
    if constexpr (WPT == 2) {
      static_assert(4 * (DT * 4 + 2) * 64 * sizeof(float) <= KEYS * KROW * sizeof(uint16_t), "merge area");
      // the second key half's (m, l, o) through LDS (the K tile area) into the first half's waves
      // indexed by the tile's place in this workgroup (0..3), not its global number
      float* mb = reinterpret_cast<float*>(ks) + (wv & 3) * (DT * 4 + 2) * 64 + lane;
      __syncthreads();  // every wave is done with the last block
      if (half == 1 && mytile < ntiles) {
        mb[0] = m_run;
        mb[64] = l_run;
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
          for (int r = 0; r < 4; ++r) mb[(2 + d * 4 + r) * 64] = o[d][r];
      }
      __syncthreads();
      if (half == 1 || mytile >= ntiles) return;
      const float m1 = mb[0], l1 = mb[64];
      const float M = fmaxf(m_run, m1);
      const float a0 = m_run == -__builtin_inff() ? 0.0f : __expf(m_run - M);
      const float a1 = m1 == -__builtin_inff() ? 0.0f : __expf(m1 - M);
      l_run = l_run * a0 + l1 * a1;
      m_run = M;
#pragma unroll
      for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[d][r] = o[d][r] * a0 + mb[(2 + d * 4 + r) * 64] * a1;
    }
    if (mytile < ntiles) store_tile(rq, qvalid);
    return;
  }

  // ---- one block, QT tiles per wave (nb == 1)
  if (!newsplit) to_lds(j_beg, j_end);
  __syncthreads();
#pragma unroll 1
  for (int t = 0; t < QT; ++t) {
    const int tile = wv + 4 * t;
    if (tile >= ntiles) break;
    if (t > 0) {
      qtile_load<HD, FUSED>(a, b, kvh, tile, lane, qt);
      qtile_finish<HD, FUSED>(a, off, tile, lane, qt, qf);
    }
    const int rq = tile * 16 + (lane & 15);
    const bool qvalid = rq < a.R;
    m_run = -__builtin_inff();
    l_run = 0.0f;
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = f32x4{0, 0, 0, 0};
    block_compute(j_beg, j_end, rq, qvalid, 0);
    store_tile(rq, qvalid);
  }
}

// Combine the live splits of one (row b, kv head, query row r) per wave, 64 (hd 128) or 32
// splits per load round: lane s reads split s's (m, l) and forms its weight exp(m_s - M) * l_s while every lane
// reads the normalised partial outputs of the round's splits for its dims.
template <int HD>
__global__ __launch_bounds__(256) void attention_combine_kernel(AttnArgs a) {
  using S = Split<HD>;
  constexpr int PER = HD / 64;  // consecutive dims per lane
  const int lane = threadIdx.x & 63;
  const int task = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= a.B * a.nkv * a.R) return;
  const int r = task % a.R, bk = task / a.R;
  const int b = bk / a.nkv, kvh = bk % a.nkv;
  // live splits: the first ns; with a.fused the context splits [0, ns - 1) and the new-token
  // split (the last one)
  const int jmax = a.max_pages * a.page;
  // causal rows read the splits up to their own position (the attention kernel may skip later
  // ones for whole query-tile groups); the fused form keeps its new-token split last
  const int visible = a.causal && !a.fused ? a.seq_lens[b] + r / a.G + 1 : a.seq_lens[b] + a.W;
  const int ns = a.fused ? min((min(a.seq_lens[b], jmax) + a.kps - 1) / a.kps, a.nsplit - 1) + 1
                         : min(a.nsplit, (min(visible, jmax) + a.kps - 1) / a.kps);
  const int nlast = a.fused ? a.nsplit - 1 - (ns - 1) : 0;  // split index shift of the last live one
  // a sliding-window row starts at the split holding its window's first key (the attention
  // kernel skips the splits before every window of a workgroup)
  const int s_beg = a.causal && !a.fused && a.window > 0 ? max(0, visible - a.window) / a.kps : 0;
  const float* base_o = a.part_o + ((size_t)bk * a.nsplit * a.R + r) * HD + lane * PER;
  const float* base_ml = a.part_ml + ((size_t)bk * a.nsplit * a.R + r) * 2;
  const size_t so = (size_t)a.R * HD, sml = (size_t)a.R * 2;
  float acc[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) acc[e] = 0.0f;
  float M = -__builtin_inff(), den = 0.0f;
  // rounds of RS splits: the (m, l) and partial-output loads of a round are issued together
  constexpr int RS = PER == 2 ? 32 : 16;
  for (int s0 = s_beg; s0 < ns; s0 += RS) {
    const int n = min(RS, ns - s0);
    float m = -__builtin_inff(), l = 0.0f;
    if (lane < n) {
      const int sp = s0 + lane + (s0 + lane == ns - 1 ? nlast : 0);
      const float2 v = *reinterpret_cast<const float2*>(base_ml + sp * sml);
      m = v.x;
      l = v.y;
    }
    // loads of the live splits only, in batches of 16 (all batches issued before any use)
    float ov[RS][PER];
#pragma unroll
    for (int u0 = 0; u0 < RS; u0 += 16) {
      if (u0 >= n) break;
#pragma unroll
      for (int u = u0; u < u0 + 16; ++u) {
        int sp = s0 + min(u, n - 1);
        if (sp == ns - 1) sp += nlast;
#pragma unroll
        for (int e = 0; e < PER; e += 2) {
          const float2 x = *reinterpret_cast<const float2*>(base_o + sp * so + e);
          ov[u][e] = x.x;
          ov[u][e + 1] = x.y;
        }
      }
    }
    const float Mn = fmaxf(M, wave_max(m));
    const float rescale = M == -__builtin_inff() ? 0.0f : __expf(M - Mn);
    const float w = m == -__builtin_inff() ? 0.0f : __expf(m - Mn) * l;
    den = den * rescale + wave_sum(w);
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] *= rescale;
    M = Mn;
#pragma unroll
    for (int u0 = 0; u0 < RS; u0 += 16) {
      if (u0 >= n) break;
#pragma unroll
      for (int u = u0; u < u0 + 16; ++u) {
        const float wu = __shfl(w, u, 64);
        if (u < n)
#pragma unroll
          for (int e = 0; e < PER; ++e) acc[e] += wu * ov[u][e];
      }
    }
  }
  const int i = r / a.G, hl = r % a.G;
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
#pragma unroll
  for (int e = 0; e < PER; ++e)
    a.out[attn_out_index(a, HD, b, i, kvh * a.G + hl, lane * PER + e)] = f32_to_bf16(acc[e] * inv);
}

// ----------------------------------------------------------------------------- verify passes
// A verify pass (at most 80 query rows per kv head at head_dim 128, 64 at 256; keys already in
// the pool): one workgroup of 4 waves per (row b, kv head, split of 4 x 16 KB keys), KB 16-key
// tiles per wave (4 at head_dim 128: 256-key splits; 2 at 256: 128-key splits). Wave w owns the
// split's keys [16 KB w, 16 KB (w + 1)): it loads their K/V rows straight from the pool into
// registers, dequantises each element once (K row-major for the score MFMA, V transposed for
// the P.V MFMA), then runs the query tiles of its group (staged once in LDS) one at a time over
// its keys. After each tile the four waves' (o, m, l) meet in LDS, 8 d tiles at a time (32 KB),
// and each wave merges two d tiles of every row into the split's partial (or the output when
// there is one split). At most 256 registers and ~54 KB of LDS: two workgroups share a CU.
//  - head_dim order: lane group a = lane / 16 holds dims [DPL a, DPL a + DPL) of its key row,
//    DPL = HD / 4 (one contiguous load, inside one 64-dim quantization group), so k-step s of
//    the score MFMA takes dims DPL a + 8 s .. + 7 from both K (A operand: lane = key) and Q
//    (B operand: lane = query): S^T[key][q] summed over a permutation of head_dim.
//  - V is transposed in registers: v_mfma_f32_16x16x16_bf16 of a 16-key x 16-dim tile (lane =
//    key, dims DPL a + 4 dt .. + 3) with the identity gives lane (a, c) the keys 4 a .. 4 a + 3
//    at physical dim DPL (c / 4) + 4 dt + c % 4 (exact: bf16 in, f32 out). Two key tiles give
//    the 8 keys {4 a + r, 16 + 4 a + r} the lane also holds scores for, so P^T goes from the
//    score registers straight into the P.V MFMA.
//  - O^T[dim index][q]: lane (a, q) ends with physical dims DPL a + 4 dt + r.
// The probabilities stay float32 (kPTerms bf16 terms in the P.V MFMAs); masks and the partial
// layout are the attention kernel's; attention_verify_combine_kernel merges the splits (a split
// past a row's keys, or before every window of its rows, writes m = -inf, which the merge skips).
constexpr int kVerifyBlock = 32;   // keys per page-aligned block (the page size is a multiple)
#ifndef DSK_VERIFY_TG_MAX
#define DSK_VERIFY_TG_MAX 128      // most (b, kv head, split) workgroups that get two query-tile groups
#endif
constexpr int kVerifyWaves = 4;
// 16-key tiles per wave (KB): 4 at head_dim 128 (256-key splits), 2 at 256 (128 keys), and 2 at
// head_dim 128 for grids of at most DSK_VERIFY_KB2_MAX 256-key (b, kv head, split) workgroups
// of at most 2 query tiles: twice the splits then fill more CUs. Measured on 9 rows of a
// 16-query-head / 8-kv-head model over 768 keys: 2 us less per layer; on 16 rows of a 32 / 8
// model over 4096 keys (136 workgroups) 3 us more, so larger grids keep 256-key splits.
#ifndef DSK_VERIFY_KB2_MAX
#define DSK_VERIFY_KB2_MAX 64
#endif
template <int HD> struct VerifyShape {
  static constexpr int MAXR = HD == 128 ? 80 : 64;      // query rows per kv head (5 or 4 tiles)
};

template <int HD, int KVT>
__device__ __forceinline__ void verify_load_rows(const void* pool, const uint32_t* sbp, int64_t tok, int grp,
                                                 u32x4 (&c)[HD / 32], uint32_t& sb) {
  constexpr int DPL = HD / 4;
  if (KVT == DSK_KV_BF16) {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(pool) + tok * HD + grp * DPL);
#pragma unroll
    for (int i = 0; i < DPL / 8; ++i) c[i] = p[i];
  } else {
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(pool) + tok * HD + grp * DPL);
#pragma unroll
    for (int i = 0; i < DPL / 16; ++i) c[i] = p[i];
    sb = sbp[tok * (HD / 64) + grp * DPL / 64];
  }
}

// 8 values of a lane's DPL-dim row slice, elements e0 .. e0 + 7 (dequantised for 8-bit KV)
template <int HD, int KVT>
__device__ __forceinline__ bf16x8 verify_elems8(const u32x4 (&c)[HD / 32], uint32_t sb, int e0) {
  if (KVT == DSK_KV_BF16) {
    return __builtin_bit_cast(bf16x8, c[e0 / 8]);
  } else {
    const float s = bf16_to_f32((uint16_t)(sb & 0xffffu)), b = bf16_to_f32((uint16_t)(sb >> 16));
    const u32x4 v = c[e0 / 16];
    const uint32_t w0 = v[(e0 % 16) / 4], w1 = v[(e0 % 16) / 4 + 1];
    uint32_t o[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t w = h ? w1 : w0;
      o[2 * h] = pack_bf16x2(fmaf(s, (float)(w & 0xffu), b), fmaf(s, (float)((w >> 8) & 0xffu), b));
      o[2 * h + 1] = pack_bf16x2(fmaf(s, (float)((w >> 16) & 0xffu), b), fmaf(s, (float)(w >> 24), b));
    }
    return __builtin_bit_cast(bf16x8, (u32x4{o[0], o[1], o[2], o[3]}));
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// Workgroups: (row b, kv head, split) x tgroups query-tile groups of QT tiles. The groups of one
// split are 8 workgroup ids apart, so they run on one XCD (workgroups go to the 8 XCDs round
// robin) and the second reads the split's K/V from that XCD's L2; ids past the grid's
// (b, kv head, split) count exit at once.
template <int HD, int KVT, bool SOFTCAP, int QT, int KB>
__global__ __launch_bounds__(kVerifyWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attention_verify_kernel(AttnArgs a) {
  constexpr int QROW = HD + 8, DPL = HD / 4, DT = HD / 16;    // LDS query row, dims per lane, d tiles
  constexpr int NW = kVerifyWaves, KEYS = NW * 16 * KB;      // keys per split
  static_assert(KB == 2 || KB == 4, "key tiles per wave");
  constexpr int NC = KVT == DSK_KV_BF16 ? DPL / 8 : DPL / 16;  // 16-byte loads per lane and key row
  // TP query tiles per pass (interleaved: their MFMAs and exponentials overlap; pairs at head_dim
  // 128, single tiles at 256 where a pair's accumulators exceed the registers), merged through
  // LDS in chunks of MC d tiles: TP * MC = 8 d tiles of 4 waves' partials, 32 KB
  constexpr int TP = HD == 128 && QT >= 2 && QT != 5 ? 2 : 1, MC = 8 / TP;  // (five tiles in pairs spill)
  __shared__ f32x4 mo[NW][TP][MC][64];               // one chunk of a pass's (o) per [wave][tile][d tile][lane]
  __shared__ float2 mml[NW][TP][64];                 // and the pass's (m, l) per lane
  __shared__ __attribute__((aligned(16))) uint16_t qs[QT * 16 * QROW];  // the group's query rows
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int grp = lane >> 4, row16 = lane & 15;
  const int per = 8 * a.tgroups;
  const int tg = (int)(blockIdx.x % per) / 8;
  const int task = (int)(blockIdx.x / per) * 8 + (int)(blockIdx.x % 8);
  if (task >= a.B * a.nkv * a.nsplit) return;
  const int split = task % a.nsplit;
  const int bk = task / a.nsplit;
  const int r0 = tg * QT * 16;                       // the group's first query row
  const int b = bk / a.nkv, kvh = bk % a.nkv;
  const int jmax = a.max_pages * a.page;
  // splits relative to the window (wrel): the row length first, then the page ids
  const int off_w = a.wrel ? a.seq_lens[b] : 0;
  const int j_beg = (split + (a.wrel ? max(0, off_w - a.window + 1) / KEYS : 0)) * KEYS;
  const int j0 = j_beg + 16 * KB * wv;  // the wave's first key
  // independent loads first: the wave's page ids (in the block table for any key) and the row length
  int pg[(KB + 1) / 2];
#pragma unroll
  for (int i = 0; i < (KB + 1) / 2; ++i)
    pg[i] = a.block_table[(int64_t)b * a.max_pages + min(j0 + 32 * i, jmax - 1) / a.page];
  const int off = a.wrel ? off_w : a.seq_lens[b];
  const int j_lim = min(off + a.W, jmax);
  // past every row's keys, or (sliding window) before the window of the group's first row and
  // so of every row after it: an empty partial (m = -inf) for the combine
  const bool before_window = a.causal && a.window > 0 && j_beg + KEYS <= off + r0 / a.G - a.window + 1;
  if (j_beg >= j_lim || before_window) {
    if (a.nsplit > 1)
      for (int r = r0 + threadIdx.x; r < min(a.R, r0 + QT * 16); r += NW * 64)
        *reinterpret_cast<float2*>(a.part_ml + (((size_t)bk * a.nsplit + split) * a.R + r) * 2) =
            float2{-__builtin_inff(), 0.0f};
    return;
  }
  const int j_end = min(j_lim, j_beg + KEYS);
  const int ntiles = min(QT, ((a.R + 15) >> 4) - tg * QT);  // the group's tiles
  const bool live = j0 < j_end;  // the wave has keys (uniform)

  // ---- loads: the group's query rows (issued before the K/V loads and stored to LDS after them,
  // so that every load is in flight at once; a row past R reads row R - 1 and stores zeros),
  // then the wave's K/V rows (16-key tiles t: keys j0 + 16 t + row16)
  constexpr int NQ = QT * 16 * (HD / 8) / (NW * 64);  // 8-dim query chunks per thread
  static_assert(NQ * NW * 64 == QT * 16 * (HD / 8), "whole query chunks per thread");
  u32x4 qv[NQ];
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int c = threadIdx.x + NW * 64 * u;  // rows x HD / 8 chunks of 8 dims
    const int rq = min(r0 + c / (HD / 8), a.R - 1), ch = c % (HD / 8);
    qv[u] = *reinterpret_cast<const u32x4*>(a.q + ((int64_t)(b * a.W + rq / a.G) * a.nq + kvh * a.G + rq % a.G) * HD +
                                            ch * 8);
  }
  u32x4 kc[KB][HD / 32], vc[KB][HD / 32];
  uint32_t ksb[KB], vsb[KB];
  if (live) {
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      const int j = j0 + 16 * t;
      const int64_t tok = ((int64_t)pg[t / 2] * a.nkv + kvh) * a.page + (j % a.page) + row16;
      verify_load_rows<HD, KVT>(a.k_pool, a.k_sb, tok, grp, kc[t], ksb[t]);
      verify_load_rows<HD, KVT>(a.v_pool, a.v_sb, tok, grp, vc[t], vsb[t]);
    }
  }
  static_assert(NC <= HD / 32, "row slice registers");
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int c = threadIdx.x + NW * 64 * u;
    const int r = c / (HD / 8), ch = c % (HD / 8);
    *reinterpret_cast<u32x4*>(qs + r * QROW + ch * 8) = r0 + r < a.R ? qv[u] : u32x4{0, 0, 0, 0};
  }

  // ---- K dequantised once (the A operand of every score MFMA), V transposed once
  bf16x8 kel[KB][DPL / 8], vt[KB / 2][DT];
  if (live) {
#pragma unroll
    for (int t = 0; t < KB; ++t)
#pragma unroll
      for (int s = 0; s < DPL / 8; ++s) kel[t][s] = verify_elems8<HD, KVT>(kc[t], ksb[t], 8 * s);
    // identity B operand of the transpose MFMA: B[k][n] = (k == n), lane holds k = 4 grp + e, n = row16
    s16x4 ident;
#pragma unroll
    for (int e = 0; e < 4; ++e) ident[e] = (4 * grp + e == row16) ? (short)0x3f80 : (short)0;
#pragma unroll
    for (int cp = 0; cp < KB / 2; ++cp) {
#pragma unroll
      for (int dp = 0; dp < DPL / 8; ++dp) {
        s16x8 v8[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t = 2 * cp + u;
          // whole-vector bit casts (a bit cast of one element of a bf16 vector reads element 0);
          // keys past the split's end are zeroed (masked, but finite)
          v8[u] = __builtin_bit_cast(s16x8, verify_elems8<HD, KVT>(vc[t], vsb[t], 8 * dp));
          if (j0 + 16 * t + row16 >= j_end) v8[u] = s16x8{0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t w[4];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const s16x4 v4 = h ? __builtin_shufflevector(v8[u], v8[u], 4, 5, 6, 7)
                               : __builtin_shufflevector(v8[u], v8[u], 0, 1, 2, 3);
            const f32x4 tr = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4, ident, f32x4{0, 0, 0, 0}, 0, 0, 0);
            w[2 * u] = pack_bf16x2(tr[0], tr[1]);
            w[2 * u + 1] = pack_bf16x2(tr[2], tr[3]);
          }
          vt[cp][2 * dp + h] = __builtin_bit_cast(bf16x8, (u32x4{w[0], w[1], w[2], w[3]}));
        }
      }
    }
  }
  // exp(scale * s - m) as exp2 of one fma: c = scale * log2(e) (softcap: the capped score, c = log2(e))
  const float softcap = a.softcap;
  const float c2 = (SOFTCAP ? 1.0f : a.scale) * 1.4426950408889634f;
  const float mscale = SOFTCAP ? 1.0f : a.scale;  // the stored max is in natural-log units of scale * s
  // a block needs masks when a key may be past the split's end or past some row's position (the
  // group's rows sit at off + r0 / G .. off + W - 1), or with a sliding window
  const bool masked = j0 + 16 * KB > j_end || (a.causal && (j0 + 16 * KB - 1 > off + r0 / a.G || a.window > 0));
  __syncthreads();  // the query rows

  // ---- passes of TP query tiles over the wave's keys: scores, softmax, P.V, then the four waves'
  // (m, l, o) meet in LDS, MC d tiles of each tile at a time, and every wave merges two d tiles
  // (of one tile) for all that tile's rows. Only one pass's accumulators and one chunk of LDS are
  // ever live.
#pragma unroll
  for (int p0 = 0; p0 < QT; p0 += TP) {
    float m[TP], l[TP];
    f32x4 o[TP][DT];
#pragma unroll
    for (int u = 0; u < TP; ++u) {
      m[u] = -__builtin_inff();
      l[u] = 0.0f;
#pragma unroll
      for (int d = 0; d < DT; ++d) o[u][d] = f32x4{0, 0, 0, 0};
    }
    if (live) {
      f32x4 st[TP][KB];
#pragma unroll
      for (int u = 0; u < TP; ++u)
#pragma unroll
        for (int t = 0; t < KB; ++t) st[u][t] = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < DPL / 8; ++s) {
#pragma unroll
        for (int u = 0; u < TP; ++u) {
          if (p0 + u >= QT) break;
          const bf16x8 qf =
              *reinterpret_cast<const bf16x8*>(qs + ((p0 + u) * 16 + row16) * QROW + grp * DPL + 8 * s);
#pragma unroll
          for (int t = 0; t < KB; ++t)
            st[u][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kel[t][s], qf, st[u][t], 0, 0, 0);
        }
      }
      // ---- softmax (lane: query row16, keys j0 + 16 t + 4 grp + rr); rows past R are not
      // masked (their columns of the MFMAs touch no other row, and are not stored)
      float mx[TP];
#pragma unroll
      for (int u = 0; u < TP; ++u) {
        mx[u] = -__builtin_inff();
        if (p0 + u >= QT) break;
        if (SOFTCAP) {
#pragma unroll
          for (int t = 0; t < KB; ++t)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) st[u][t][rr] = tanhf(st[u][t][rr] * a.scale / softcap) * softcap;
        }
        if (masked) {
          const int rq = r0 + (p0 + u) * 16 + row16;
          const int qpos = off + (rq < a.R ? rq : 0) / a.G;
          int k_first = 0, k_last = j_end - 1;
          if (a.causal) {
            k_last = min(k_last, qpos);
            if (a.window > 0) k_first = qpos - a.window + 1;
          }
#pragma unroll
          for (int t = 0; t < KB; ++t)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const int j = j0 + 16 * t + 4 * grp + rr;
              if (j < k_first || j > k_last) st[u][t][rr] = -__builtin_inff();
            }
        }
#pragma unroll
        for (int t = 0; t < KB; ++t)
          mx[u] = fmaxf(mx[u], fmaxf(fmaxf(st[u][t][0], st[u][t][1]), fmaxf(st[u][t][2], st[u][t][3])));
        mx[u] = fmaxf(mx[u], __shfl_xor(mx[u], 16, 64));
        mx[u] = fmaxf(mx[u], __shfl_xor(mx[u], 32, 64));
      }
      // per tile: float32 probabilities (in place of the scores) and their sums, then O^T +=
      // V^T . P^T over the wave's keys (32 per MFMA) with P as kPTerms bf16 terms; a tile's MFMAs
      // run while the next tile's exponentials are computed. Masked keys: exp2(-inf) = 0; a row
      // with no visible key keeps m = -inf, l = 0.
#pragma unroll
      for (int u = 0; u < TP; ++u) {
        if (p0 + u >= QT) break;
        const float mb = mx[u] == -__builtin_inff() ? 0.0f : mx[u] * c2;
#pragma unroll
        for (int t = 0; t < KB; ++t)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const float pr = __builtin_amdgcn_exp2f(fmaf(st[u][t][rr], c2, -mb));
            st[u][t][rr] = pr;
            l[u] += pr;
          }
        m[u] = mx[u] * mscale;
#pragma unroll
        for (int cp = 0; cp < KB / 2; ++cp) {
          uint32_t w[kPTerms][4];
#pragma unroll
          for (int v = 0; v < 2; ++v)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const f32x4& pv = st[u][2 * cp + v];
              uint32_t tt[kPTerms];
              split_terms_bf16x2<kPTerms>(pv[2 * h], pv[2 * h + 1], tt);
#pragma unroll
              for (int k = 0; k < kPTerms; ++k) w[k][2 * v + h] = tt[k];
            }
#pragma unroll
          for (int k = 0; k < kPTerms; ++k) {
            const bf16x8 pk = __builtin_bit_cast(bf16x8, (u32x4{w[k][0], w[k][1], w[k][2], w[k][3]}));
#pragma unroll
            for (int d = 0; d < DT; ++d)
              o[u][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[cp][d], pk, o[u][d], 0, 0, 0);
          }
        }
        l[u] += __shfl_xor(l[u], 16, 64);
        l[u] += __shfl_xor(l[u], 32, 64);
      }
    }
    // ---- merge of the waves, chunk by chunk: wave w takes tile p0 + (2 w) / MC, d tiles
    // c0 + (2 w) % MC and the one after, of every row of that tile (lane: its row16 and its
    // group's 8 dims DPL grp + 4 (c0 + (2 w) % MC) .. + 7)
    const int mu = (2 * wv) / MC, md = (2 * wv) % MC;
    const int rq = r0 + (p0 + mu) * 16 + row16;
    const bool store = p0 + mu < QT && p0 + mu < ntiles && rq < a.R;
#pragma unroll
    for (int c0 = 0; c0 < DT; c0 += MC) {
      if (p0 > 0 || c0 > 0) __syncthreads();   // the previous chunk's merge has read the slots
#pragma unroll
      for (int u = 0; u < TP; ++u) {
#pragma unroll
        for (int d = 0; d < MC; ++d) mo[wv][u][d][lane] = o[u][c0 + d];
        if (c0 == 0) mml[wv][u][lane] = float2{m[u], l[u]};
      }
      __syncthreads();
      if (store) {
        float2 ml[NW];
        float M = -__builtin_inff();
#pragma unroll
        for (int q = 0; q < NW; ++q) {
          ml[q] = mml[q][mu][lane];
          M = fmaxf(M, ml[q].x);
        }
        float L = 0.0f, wq[NW];
#pragma unroll
        for (int q = 0; q < NW; ++q) {
          wq[q] = ml[q].x == -__builtin_inff() ? 0.0f : __expf(ml[q].x - M);
          L += ml[q].y * wq[q];
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        f32x4 res[2];
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
          f32x4 acc = f32x4{0, 0, 0, 0};
#pragma unroll
          for (int q = 0; q < NW; ++q) acc += mo[q][mu][md + dd][lane] * wq[q];
          res[dd] = acc * inv;
        }
        const int dim0 = grp * DPL + 4 * (c0 + md);
        if (a.nsplit == 1) {
          // 8 contiguous dims (one run in both output layouts)
          *reinterpret_cast<u32x4*>(a.out + attn_out_index(a, HD, b, rq / a.G, kvh * a.G + rq % a.G, dim0)) =
              u32x4{pack_bf16x2(res[0][0], res[0][1]), pack_bf16x2(res[0][2], res[0][3]),
                    pack_bf16x2(res[1][0], res[1][1]), pack_bf16x2(res[1][2], res[1][3])};
        } else {
          // the split's partial o / l in float32 and its (m, l)
          const size_t prow = ((size_t)bk * a.nsplit + split) * a.R + rq;
          f32x4* dst = reinterpret_cast<f32x4*>(a.part_o + prow * HD + dim0);
          dst[0] = res[0];
          dst[1] = res[1];
          if (md == 0 && grp == 0 && c0 == 0) *reinterpret_cast<float2*>(a.part_ml + prow * 2) = float2{M, L};
        }
      }
    }
  }
}

// The verify kernel's splits merged: one thread per (row b, kv head, query row, 4 dims), every
// split from the first one the row's sliding window reaches (a split past the row length holds
// m = -inf and is skipped by value), the loads of a batch of BATCH splits issued together (the
// split count rounded up to 4, at most 24: past the last split a load re-reads it and is not
// merged). Same merge as attention_combine_kernel: weights exp(m_s - M) * l_s over the splits'
// normalised float32 partial outputs.
constexpr int kVerifyCombineThreads = 64;
template <int HD, int BATCH>
__global__ __launch_bounds__(kVerifyCombineThreads) void attention_verify_combine_kernel(AttnArgs a) {
  constexpr int CH = HD / 4;
  const int64_t task = (int64_t)blockIdx.x * kVerifyCombineThreads + threadIdx.x;
  if (task >= (int64_t)a.B * a.nkv * a.R * CH) return;
  const int ch = (int)(task % CH);
  const int64_t rowt = task / CH;
  const int r = (int)(rowt % a.R);
  const int bk = (int)(rowt / a.R);
  const int b = bk / a.nkv, kvh = bk % a.nkv;
  int s_beg = 0;
  if (a.causal && a.window > 0) {  // only a sliding window needs the row length (one round trip)
    const int sl = a.seq_lens[b];
    s_beg = max(0, sl + r / a.G + 1 - a.window) / a.kps - (a.wrel ? max(0, sl - a.window + 1) / a.kps : 0);
  }
  const size_t base = (size_t)bk * a.nsplit * a.R + r;  // partial row of split 0
  float M = -__builtin_inff(), L = 0.0f;
  f32x4 acc = f32x4{0, 0, 0, 0};
  for (int s0 = s_beg; s0 < a.nsplit; s0 += BATCH) {
    float2 ml[BATCH];
    f32x4 ov[BATCH];
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int sp = min(s0 + u, a.nsplit - 1);
      const size_t prow = base + (size_t)sp * a.R;
      ml[u] = *reinterpret_cast<const float2*>(a.part_ml + prow * 2);
      ov[u] = *reinterpret_cast<const f32x4*>(a.part_o + prow * HD + ch * 4);
      if (s0 + u >= a.nsplit) ml[u].x = -__builtin_inff();
    }
    float Mn = M;
#pragma unroll
    for (int u = 0; u < BATCH; ++u) Mn = fmaxf(Mn, ml[u].x);
    if (Mn == -__builtin_inff()) continue;
    const float rescale = M == -__builtin_inff() ? 0.0f : __expf(M - Mn);
    L *= rescale;
    acc *= rescale;
    M = Mn;
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      if (ml[u].x == -__builtin_inff()) continue;  // also skips a never-written partial output
      const float wl = __expf(ml[u].x - M) * ml[u].y;
      L += wl;
      acc += wl * ov[u];
    }
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  *reinterpret_cast<uint2*>(a.out + attn_out_index(a, HD, b, r / a.G, kvh * a.G + r % a.G, ch * 4)) =
      uint2{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv)};
}

// ----------------------------------------------------------------------------- many-query pass
// A prefill (head_dim 128, more than 64 new tokens per row): one workgroup per (row b, kv head,
// block of 128 query rows), no key splits and so no combine. The row block's keys stream through
// LDS in 64-key blocks (double-buffered: block n + 1 is dequantised into the other buffer while
// block n is scored, block n + 2's loads are in flight meanwhile, one barrier per block). Each
// of the kPfWaves waves owns two 16-query tiles, so every K and V fragment it reads from LDS
// feeds two tiles' MFMAs, and each block's dequantisation is shared by all the rows. The row
// sums of P come out of the P.V MFMAs as one more V^T tile of ones. Scores S^T = K . Q^T and O^T = V^T . P^T as in the other attention kernels; masking
// runs only on blocks that straddle a wave's causal diagonal, its window edge or the last key.
// Row blocks with the most keys are launched first (the grid's y runs from the last block).
constexpr int kPfKeys = 64;                   // keys per LDS block
constexpr int kPfKRow = 128 + 8;              // K rows in LDS (bf16, padded: conflict-free reads)
constexpr int kPfVRow = kPfKeys + 8;          // V^T rows in LDS (bf16, padded)
constexpr int kPfTiles = 2;                   // 16-query tiles per wave
#ifndef DSK_PF_WAVES
#define DSK_PF_WAVES 8
#endif
constexpr int kPfWaves = DSK_PF_WAVES;
constexpr int kPfThreads = kPfWaves * 64;
constexpr int kPfRows = kPfWaves * kPfTiles * 16;  // query rows per workgroup
constexpr int kPfMaxPages = 1024;             // page ids of a row block's keys held in LDS

// At most 256 VGPRs (two waves per SIMD: one 8-wave workgroup per CU, whose waves' staging and
// MFMAs interleave). On the 4096-token Qwen3-8B layer: 436 us with 4 waves and no bound, 299 us
// with 4 waves and this bound, 239 us with 8 waves sharing each block's dequantisation.
template <int KVT>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void attention_prefill_kernel(AttnArgs a) {
  constexpr int HD = 128, KS = HD / 32, DT = HD / 16, NKT = kPfKeys / 16, TPW = kPfTiles, NTHR = kPfThreads;
  constexpr int CK = kPfKeys * (HD / 8) / NTHR;        // 8-dim K chunks per thread
  constexpr int CV = (kPfKeys / 2) * (HD / 8) / NTHR;  // (2 keys x 8 dims) V chunks per thread
  static_assert(CK * NTHR == kPfKeys * (HD / 8) && CV * NTHR == (kPfKeys / 2) * (HD / 8), "whole chunks per thread");
  __shared__ __attribute__((aligned(16))) uint16_t ks[2][kPfKeys * kPfKRow];
  __shared__ __attribute__((aligned(16))) uint32_t vt[2][HD * kPfVRow / 2];
  __shared__ int pgs[kPfMaxPages];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int bk = blockIdx.x, b = bk / a.nkv, kvh = bk % a.nkv;
  const int nrb = (a.R + kPfRows - 1) / kPfRows;
  const int rb = nrb - 1 - (int)blockIdx.y;
  float scale = a.scale;
  int causal = a.causal, window = a.window;
  asm volatile("" : "+s"(scale), "+s"(causal), "+s"(window));
  const int off = a.seq_lens[b];
  const int jmax = a.max_pages * a.page;
  const int Lk = min(off + a.W, jmax);
  const int r0 = rb * kPfRows, r_last = min(a.R, r0 + kPfRows) - 1;
  // the workgroup's keys [j_beg, j_end): up to its last row's position (causal), from its first
  // row's window start, in whole blocks from there
  int j_beg = 0, j_end = Lk;
  if (causal) {
    j_end = min(Lk, off + r_last / a.G + 1);
    if (window > 0) j_beg = max(0, off + r0 / a.G - window + 1);
  }
  const int nb = j_end > j_beg ? (j_end - j_beg + kPfKeys - 1) / kPfKeys : 0;
  const int pg0 = j_beg / a.page;
  if (nb > 0) {
    const int npg = (j_end - 1) / a.page - pg0 + 1;
    for (int t = threadIdx.x; t < npg; t += NTHR) pgs[t] = a.block_table[(int64_t)b * a.max_pages + pg0 + t];
  }
  // this wave's query tiles (rows past R load row 0 and are never stored)
  const int wr0 = r0 + wv * TPW * 16;
  bf16x8 qf[TPW][KS];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    QTile<HD, false> qt;
    qtile_load<HD, false>(a, b, kvh, wr0 / 16 + t, lane, qt);
    qtile_finish<HD, false>(a, off, wr0 / 16 + t, lane, qt, qf[t]);
  }
  // the queries and page ids retire here: the compiler's load counting cannot tell that no
  // block loads follow them when the range is empty, and would otherwise wait for the block
  // prefetch inside every block's scores
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  __syncthreads();  // the page ids

  auto tok_of = [&](int j) -> int64_t {
    j = min(j, j_end - 1);  // keys past the range load the last one and are zeroed in LDS
    return ((int64_t)pgs[j / a.page - pg0] * a.nkv + kvh) * a.page + (j % a.page);
  };
  Chunk8 kc[CK], vc[CV][2];
  auto issue = [&](int j0) {
#pragma unroll
    for (int ci = 0; ci < CK; ++ci) {
      const int c = threadIdx.x + ci * NTHR;
      load_chunk<KVT>(a.k_pool, a.k_sb, HD, tok_of(j0 + c / (HD / 8)), (c % (HD / 8)) * 8, kc[ci]);
    }
#pragma unroll
    for (int ci = 0; ci < CV; ++ci) {
      const int c = threadIdx.x + ci * NTHR;
      const int kp = c % (kPfKeys / 2), d0 = (c / (kPfKeys / 2)) * 8;
#pragma unroll
      for (int u = 0; u < 2; ++u) load_chunk<KVT>(a.v_pool, a.v_sb, HD, tok_of(j0 + 2 * kp + u), d0, vc[ci][u]);
    }
  };
  // the loaded words stay opaque until to_lds: the compiler would otherwise unpack the 8-bit
  // codes right behind their loads, waiting for the next block's loads before the barrier
  auto pin = [](Chunk8& c) {
    if constexpr (KVT == DSK_KV_BF16) asm volatile("" : "+v"(c.raw[0]), "+v"(c.raw[1]), "+v"(c.raw[2]), "+v"(c.raw[3]));
    else asm volatile("" : "+v"(c.raw[0]), "+v"(c.raw[1]), "+v"(c.sb));
  };
  // dequantise the loaded block [j_lo, j_hi) into LDS buffer buf (keys past j_hi zeroed)
  auto to_lds = [&](int buf, int j_lo, int j_hi) {
#pragma unroll
    for (int ci = 0; ci < CK; ++ci) pin(kc[ci]);
#pragma unroll
    for (int ci = 0; ci < CV; ++ci) {
      pin(vc[ci][0]);
      pin(vc[ci][1]);
    }
#pragma unroll
    for (int ci = 0; ci < CK; ++ci) {
      const int c = threadIdx.x + ci * NTHR;
      const int key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
      uint16_t h[8];
      chunk_bf16<KVT>(kc[ci], h);
      u32x4 w = *reinterpret_cast<const u32x4*>(h);
      if (j_lo + key >= j_hi) w = u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(&ks[buf][key * kPfKRow + d0]) = w;
    }
#pragma unroll
    for (int ci = 0; ci < CV; ++ci) {
      const int c = threadIdx.x + ci * NTHR;
      const int kp = c % (kPfKeys / 2), d0 = (c / (kPfKeys / 2)) * 8;
      const int j0 = j_lo + 2 * kp;
      uint16_t h0[8], h1[8];
      chunk_bf16<KVT>(vc[ci][0], h0);
      chunk_bf16<KVT>(vc[ci][1], h1);
      const bool z0 = j0 >= j_hi, z1 = j0 + 1 >= j_hi;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        vt[buf][((d0 + e) * kPfVRow) / 2 + kp] = (uint32_t)(z0 ? 0 : h0[e]) | ((uint32_t)(z1 ? 0 : h1[e]) << 16);
    }
  };

  // running state per tile: the max, O^T and the row sums of P (every element of lt[t] holds the
  // lane's query's sum: a V^T tile of ones in the P.V product)
  float m_run[TPW];
  f32x4 o[TPW][DT], lt[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    m_run[t] = -__builtin_inff();
    lt[t] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int d = 0; d < DT; ++d) o[t][d] = f32x4{0, 0, 0, 0};
  }
  const u32x4 ones_u = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const bf16x8 ones = __builtin_bit_cast(bf16x8, ones_u);
  const float c2 = scale * 1.4426950408889634f;
  const bool wave_live = wr0 < a.R;
  const bool wave_full = wr0 + TPW * 16 <= a.R;
  const int wq_lo = off + min(wr0, a.R - 1) / a.G;                // smallest position of the wave's rows
  const int wq_hi = off + min(wr0 + TPW * 16 - 1, a.R - 1) / a.G;  // largest

  auto compute = [&](int buf, int j_lo, int j_hi) {
    // ---- S^T[key][q]: k-step outer, every key tile's fragment feeding both query tiles
    f32x4 st[TPW][NKT];
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int h = 0; h < NKT; ++h) st[t][h] = f32x4{0, 0, 0, 0};
    const uint16_t* kbase = &ks[buf][(lane & 15) * kPfKRow + (lane >> 4) * 8];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 kf[NKT];
#pragma unroll
      for (int h = 0; h < NKT; ++h) kf[h] = *reinterpret_cast<const bf16x8*>(kbase + h * 16 * kPfKRow + s * 32);
#pragma unroll
      for (int h = 0; h < NKT; ++h)
#pragma unroll
        for (int t = 0; t < TPW; ++t) st[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[h], qf[t][s], st[t][h], 0, 0, 0);
    }
    // ---- mask (only a block that straddles a row's visible range), max, exp2, P
    const bool masked = !wave_full || j_hi - j_lo < kPfKeys || (causal && j_lo + kPfKeys - 1 > wq_lo) ||
                        (causal && window > 0 && j_lo < wq_hi - window + 1);
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      if (masked) {
        const int rq = wr0 + t * 16 + (lane & 15);
        const bool qvalid = rq < a.R;
        const int qpos = off + (qvalid ? rq / a.G : 0);
        int k_last = j_hi - 1, k_first = 0;
        if (causal) {
          k_last = min(k_last, qpos);
          if (window > 0) k_first = qpos - window + 1;
        }
        if (!qvalid) k_last = -1;
#pragma unroll
        for (int h = 0; h < NKT; ++h)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = j_lo + h * 16 + (lane >> 4) * 4 + r;
            if (j < k_first || j > k_last) st[t][h][r] = -__builtin_inff();
          }
      }
      float mx = m_run[t];
#pragma unroll
      for (int h = 0; h < NKT; ++h) mx = fmaxf(mx, fmaxf(fmaxf(st[t][h][0], st[t][h][1]), fmaxf(st[t][h][2], st[t][h][3])));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // masked keys: exp2(-inf) = 0; a row with no visible key yet keeps m = -inf, l = 0, o = 0
      const float mb = mx == -__builtin_inff() ? 0.0f : mx * c2;
      const float alpha = m_run[t] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f((m_run[t] - mx) * c2);
      // float32 probabilities in place of the scores
#pragma unroll
      for (int h = 0; h < NKT; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) st[t][h][r] = __builtin_amdgcn_exp2f(fmaf(st[t][h][r], c2, -mb));
      m_run[t] = mx;
      if (__any(alpha != 1.0f)) {
        lt[t] *= alpha;
#pragma unroll
        for (int d = 0; d < DT; ++d) o[t][d] *= alpha;
      }
    }
    // ---- O^T[d][q] += V^T . P^T with P as hi + lo (two MFMAs per fragment and tile; a prefill
    // is MFMA-heavy, so the third term of the verify kernels is left out: P within 2^-17):
    // each V^T fragment feeds both query tiles
    const uint16_t* vt16 = reinterpret_cast<const uint16_t*>(vt[buf]);
#pragma unroll
    for (int cp = 0; cp < NKT / 2; ++cp) {
      bf16x8 pk[TPW][2];
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        uint32_t w[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const f32x4& pv = st[t][2 * cp + u];
            split2_bf16x2(pv[2 * hh], pv[2 * hh + 1], w[0][2 * u + hh], w[1][2 * u + hh]);
          }
#pragma unroll
        for (int k = 0; k < 2; ++k) pk[t][k] = __builtin_bit_cast(bf16x8, (u32x4{w[k][0], w[k][1], w[k][2], w[k][3]}));
      }
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const uint16_t* vr = vt16 + (d * 16 + (lane & 15)) * kPfVRow + 32 * cp + (lane >> 4) * 4;
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
        const bf16x8 vf = __builtin_bit_cast(bf16x8, (u32x4{lo.x, lo.y, hi.x, hi.y}));
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
          for (int t = 0; t < TPW; ++t) o[t][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pk[t][k], o[t][d], 0, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int t = 0; t < TPW; ++t) lt[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pk[t][k], lt[t], 0, 0, 0);
    }
  };

  if (nb > 0) {
    issue(j_beg);
    to_lds(0, j_beg, min(j_end, j_beg + kPfKeys));
    if (nb > 1) issue(j_beg + kPfKeys);
  }
  __syncthreads();
#pragma unroll 1
  for (int n = 0; n < nb; ++n) {
    const int j_lo = j_beg + n * kPfKeys, j_hi = min(j_end, j_lo + kPfKeys);
    // a wave whose rows see none of the block skips it (causal: all its rows before the block;
    // window: all its rows' windows past it)
    const bool skip = !wave_live || (causal && j_lo > wq_hi) || (causal && window > 0 && j_hi - 1 < wq_lo - window + 1);
    if (!skip) compute(n & 1, j_lo, j_hi);
    if (n + 1 < nb) {
      // the other buffer was last read in block n - 1, which every wave finished before the
      // previous barrier
      to_lds((n + 1) & 1, j_lo + kPfKeys, min(j_end, j_lo + 2 * kPfKeys));
      if (n + 2 < nb) issue(j_lo + 2 * kPfKeys);
    }
    __syncthreads();
  }

  // ---- the output: o / l, 4 consecutive dims per lane and d tile
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const float l = lt[t][0];
    const int rq = wr0 + t * 16 + (lane & 15);
    if (rq >= a.R) continue;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int i = rq / a.G, hl = rq % a.G;
    uint16_t* dst = a.out + attn_out_index(a, HD, b, i, kvh * a.G + hl, (lane >> 4) * 4);
#pragma unroll
    for (int d = 0; d < DT; ++d)
      *reinterpret_cast<uint2*>(dst + d * 16) = uint2{pack_bf16x2(o[t][d][0] * inv, o[t][d][1] * inv),
                                                      pack_bf16x2(o[t][d][2] * inv, o[t][d][3] * inv)};
  }
}

// ----------------------------------------------------------------------------- host helpers
template <int HD, int QT, bool FUSED>
static void launch_attention(const AttnArgs& a, int kv_dtype, bool softcap, dim3 grid, hipStream_t st) {
  // one tile per wave and no new-token split: two waves per tile, each scoring half of a block
  // (head_dim 128: the halves' merge fits the K tile's LDS)
  constexpr int WPT = (QT == 1 && !FUSED && HD == 128) ? 2 : 1;
  const dim3 blk(256 * WPT);
  if (kv_dtype == DSK_KV_U8) {
    if (softcap) hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_U8, true, FUSED, WPT>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_U8, false, FUSED, WPT>), grid, blk, 0, st, a);
  } else {
    if (softcap) hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_BF16, true, FUSED, WPT>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((attention_kernel<HD, QT, DSK_KV_BF16, false, FUSED, WPT>), grid, blk, 0, st, a);
  }
}

// Keys of one LDS block; a split streams nblk blocks (graph-stable: the split grid depends on
// max_ctx only). One block per split gives the most splits, which sizes the workspace.
static int attn_split_keys(int hd, int) {
  return hd == 128 ? Split<128>::KEYS : (hd == 256 ? Split<256>::KEYS : Split<512>::KEYS);
}
static int attn_nsplit(int hd, int max_ctx) { return (int)ceil_div(max_ctx, attn_split_keys(hd, max_ctx)); }
// blocks per split of the streamed path: about DSK_ATTN_SPLITS splits over the keys a row
// reads (its sliding window, when it has one), at most 8 blocks; a many-query pass (more than
// 64 new tokens: a prefill) takes 8 blocks per split, its query tiles giving the parallelism
#ifndef DSK_ATTN_SPLITS
#define DSK_ATTN_SPLITS 24
#endif
constexpr int kAttnVerifyMaxW = 64;
static int attn_blocks(int hd, int span, int W = 1) {
  if (W > kAttnVerifyMaxW) return 8;
  const int64_t blocks = ceil_div(span, attn_split_keys(hd, span));
  return (int)std::min<int64_t>(8, std::max<int64_t>(1, ceil_div(blocks, DSK_ATTN_SPLITS)));
}

// partial outputs first, then (m, l) at a 256-byte boundary
static size_t attn_part_o_bytes(int B, int W, int nq, int hd, int nsplit) {
  return ((size_t)B * W * nq * nsplit * hd * sizeof(float) + 255) & ~(size_t)255;
}
static size_t attn_ws_need(int B, int W, int nq, int hd, int nsplit) {
  return nsplit > 1 ? attn_part_o_bytes(B, W, nq, hd, nsplit) + (size_t)B * W * nq * nsplit * 2 * sizeof(float) : 0;
}

// shared validation and launch of both attention entries
static int attention_run(AttnArgs& a, int hd, int max_ctx, float softcap, void* workspace, size_t ws_bytes,
                         bool fused, hipStream_t st, const char* who) {
  DSK_REQUIRE(hd == 128 || hd == 256 || (hd == 512 && !fused), "%s: head_dim %d not supported (128, 256; 512 "
              "without the fused append)", who, hd);
  DSK_REQUIRE(a.B > 0 && a.W > 0 && a.nq > 0 && a.nkv > 0 && a.nq % a.nkv == 0, "%s: bad shape", who);
  DSK_REQUIRE(a.kv_dtype == DSK_KV_BF16 || (a.kv_dtype == DSK_KV_U8 && a.k_sb && a.v_sb), "%s: u8 KV needs sb", who);
  DSK_REQUIRE(a.page > 0 && a.max_pages > 0, "%s: bad page geometry", who);
  DSK_REQUIRE(max_ctx >= a.W && (int64_t)a.max_pages * a.page >= max_ctx, "%s: max_ctx %d beyond block table", who,
              max_ctx);
  a.G = a.nq / a.nkv;
  a.R = a.W * a.G;
  const int tiles = (a.R + 15) / 16;
  // head_dim 512 and many-query passes: one tile per wave, query-tile groups on the grid's y axis
  const bool grouped = hd == 512 || a.W > kAttnVerifyMaxW;
  const int QT = grouped ? 1 : (tiles + 3) / 4;
  const int tile_groups = grouped ? (tiles + 3) / 4 : 1;
  DSK_REQUIRE(QT <= (hd == 128 ? 4 : 2), "%s: W*G=%d query rows per kv head exceeds %d", who, a.R,
              (hd == 128 ? 256 : 128));
  DSK_REQUIRE(tile_groups <= 65535, "%s: %d query rows per kv head", who, a.R);
  DSK_REQUIRE(!fused || a.W <= 64, "%s: W=%d new tokens exceeds 64", who, a.W);
  DSK_REQUIRE(!a.out_packed || (a.B * a.W <= 64 && (a.nq * hd) % 64 == 0), "%s: packed output needs B*W <= 64", who);
  a.fused = fused ? 1 : 0;
  const bool sc = softcap > 0.0f;
  if (hd == 128 && !fused && !sc && !a.out_packed && a.W > kAttnVerifyMaxW && a.max_pages <= kPfMaxPages) {
    // many-query passes (prefills): whole key ranges per query block, no splits, no combine
    a.nsplit = 1;
    a.kps = max_ctx;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    const dim3 pgrid((unsigned)(a.B * a.nkv), (unsigned)ceil_div(a.R, kPfRows));
    if (a.kv_dtype == DSK_KV_U8) hipLaunchKernelGGL(attention_prefill_kernel<DSK_KV_U8>, pgrid, dim3(kPfThreads), 0, st, a);
    else hipLaunchKernelGGL(attention_prefill_kernel<DSK_KV_BF16>, pgrid, dim3(kPfThreads), 0, st, a);
    DSK_LAUNCH_CHECK(who);
    return DSK_OK;
  }
  // a sliding-window pass reads at most window + W keys per row: its splits are sized for that
  // span (the splits before a window exit at once), not for the whole cache
  const int span = (a.causal && a.window > 0) ? std::min(max_ctx, a.window + a.W) : max_ctx;
  int nblk = (fused || QT != 1) ? 1 : attn_blocks(hd, span, a.W);
  while (nblk > 1 && attn_split_keys(hd, max_ctx) * nblk / a.page + 1 > kAttnMaxSplitPages) --nblk;
  DSK_REQUIRE(attn_split_keys(hd, max_ctx) / a.page + 1 <= kAttnMaxSplitPages, "%s: page size %d too small", who,
              a.page);
  a.kps = attn_split_keys(hd, max_ctx) * nblk;
  a.nsplit = (int)ceil_div(max_ctx, a.kps) + (fused ? 1 : 0);
  const size_t need = attn_ws_need(a.B, a.W, a.nq, hd, a.nsplit);
  DSK_REQUIRE(a.nsplit == 1 || (workspace && ws_bytes >= need), "%s: workspace %zu < %zu", who, ws_bytes, need);
  a.part_o = reinterpret_cast<float*>(workspace);
  a.part_ml = a.nsplit > 1 ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) +
                                                       attn_part_o_bytes(a.B, a.W, a.nq, hd, a.nsplit))
                           : nullptr;
  const int verify_maxr = hd == 128 ? VerifyShape<128>::MAXR : VerifyShape<256>::MAXR;
  if ((hd == 128 || hd == 256) && !fused && a.R <= verify_maxr && a.page % kVerifyBlock == 0) {
    // verify passes: 4 waves per split (256 keys at head_dim 128, 128 at 256 and for small
    // head_dim-128 grids), every query tile
    const int kb = hd == 256 || (tiles <= 2 && (int64_t)a.B * a.nkv * ceil_div(span, 256) <= DSK_VERIFY_KB2_MAX) ? 2 : 4;
    a.kps = kVerifyWaves * 16 * kb;
    a.nsplit = (int)ceil_div(max_ctx, a.kps);
    // a sliding window spans at most (window + W - 2) / kps + 2 splits from the one holding the
    // first row's window start: only those are launched
    a.wrel = 0;
    if (a.causal && a.window > 0) {
      const int nw = (a.window + a.W - 2) / a.kps + 2;
      if (nw < a.nsplit) {
        a.nsplit = nw;
        a.wrel = 1;
      }
    }
    const size_t need_v = attn_ws_need(a.B, a.W, a.nq, hd, a.nsplit);
    DSK_REQUIRE(a.nsplit == 1 || (workspace && ws_bytes >= need_v), "%s: workspace %zu < %zu", who, ws_bytes, need_v);
    a.part_o = reinterpret_cast<float*>(workspace);
    a.part_ml = a.nsplit > 1 ? reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) +
                                                        attn_part_o_bytes(a.B, a.W, a.nq, hd, a.nsplit))
                             : nullptr;
    // two query-tile groups per split when the (b, kv head, split) workgroups leave most CUs
    // free: each group dequantises the split's K/V again but runs half the softmax, P.V and
    // merge, and twice the waves run at once
    const int tasks = a.B * a.nkv * a.nsplit;
    a.tgroups = ((tiles == 2 || tiles == 4) && tasks <= DSK_VERIFY_TG_MAX) ? 2 : 1;
    const int qt = tiles / a.tgroups;
    const dim3 vgrid((unsigned)(ceil_div(tasks, 8) * 8 * a.tgroups)), vblk(kVerifyWaves * 64);
#define DSK_VERIFY_QT(kvt, scv)                                                                              \
  if (hd == 256) {                                                                                           \
    switch (qt) {                                                                                            \
      case 1: hipLaunchKernelGGL((attention_verify_kernel<256, kvt, scv, 1, 2>), vgrid, vblk, 0, st, a); break; \
      case 2: hipLaunchKernelGGL((attention_verify_kernel<256, kvt, scv, 2, 2>), vgrid, vblk, 0, st, a); break; \
      case 3: hipLaunchKernelGGL((attention_verify_kernel<256, kvt, scv, 3, 2>), vgrid, vblk, 0, st, a); break; \
      default: hipLaunchKernelGGL((attention_verify_kernel<256, kvt, scv, 4, 2>), vgrid, vblk, 0, st, a); break; \
    }                                                                                                        \
  } else if (kb == 2) {                                                                                      \
    if (qt == 1) hipLaunchKernelGGL((attention_verify_kernel<128, kvt, scv, 1, 2>), vgrid, vblk, 0, st, a);  \
    else hipLaunchKernelGGL((attention_verify_kernel<128, kvt, scv, 2, 2>), vgrid, vblk, 0, st, a);          \
  } else {                                                                                                   \
    switch (qt) {                                                                                            \
      case 1: hipLaunchKernelGGL((attention_verify_kernel<128, kvt, scv, 1, 4>), vgrid, vblk, 0, st, a); break; \
      case 2: hipLaunchKernelGGL((attention_verify_kernel<128, kvt, scv, 2, 4>), vgrid, vblk, 0, st, a); break; \
      case 3: hipLaunchKernelGGL((attention_verify_kernel<128, kvt, scv, 3, 4>), vgrid, vblk, 0, st, a); break; \
      case 4: hipLaunchKernelGGL((attention_verify_kernel<128, kvt, scv, 4, 4>), vgrid, vblk, 0, st, a); break; \
      default: hipLaunchKernelGGL((attention_verify_kernel<128, kvt, scv, 5, 4>), vgrid, vblk, 0, st, a); break; \
    }                                                                                                        \
  }
    if (a.kv_dtype == DSK_KV_U8) {
      if (sc) { DSK_VERIFY_QT(DSK_KV_U8, true) } else { DSK_VERIFY_QT(DSK_KV_U8, false) }
    } else {
      if (sc) { DSK_VERIFY_QT(DSK_KV_BF16, true) } else { DSK_VERIFY_QT(DSK_KV_BF16, false) }
    }
#undef DSK_VERIFY_QT
    DSK_LAUNCH_CHECK(who);
    if (a.nsplit > 1) {
      const dim3 cgrid((unsigned)ceil_div((int64_t)a.B * a.nkv * a.R * (hd / 4), kVerifyCombineThreads));
      // splits per batch of loads: the split count rounded up to 4, at most 24
      const int batch = std::min(24, (a.nsplit + 3) / 4 * 4);
#define DSK_COMBINE(HDV, BV) \
  hipLaunchKernelGGL((attention_verify_combine_kernel<HDV, BV>), cgrid, dim3(kVerifyCombineThreads), 0, st, a)
#define DSK_COMBINE_B(HDV)                                                                          \
  switch (batch) {                                                                                  \
    case 4: DSK_COMBINE(HDV, 4); break;                                                             \
    case 8: DSK_COMBINE(HDV, 8); break;                                                             \
    case 12: DSK_COMBINE(HDV, 12); break;                                                           \
    case 16: DSK_COMBINE(HDV, 16); break;                                                           \
    case 20: DSK_COMBINE(HDV, 20); break;                                                           \
    default: DSK_COMBINE(HDV, 24); break;                                                           \
  }
      if (hd == 256) { DSK_COMBINE_B(256) } else { DSK_COMBINE_B(128) }
#undef DSK_COMBINE_B
#undef DSK_COMBINE
      DSK_LAUNCH_CHECK(who);
    }
    return DSK_OK;
  }
  dim3 grid((unsigned)(a.B * a.nkv * a.nsplit), (unsigned)tile_groups);
#define DSK_ATTN_CASE(hdv, qt)                                      \
  if (hd == hdv && QT == qt) {                                      \
    if (fused) launch_attention<hdv, qt, true>(a, a.kv_dtype, sc, grid, st); \
    else launch_attention<hdv, qt, false>(a, a.kv_dtype, sc, grid, st);      \
  }
  DSK_ATTN_CASE(128, 1) DSK_ATTN_CASE(128, 2) DSK_ATTN_CASE(128, 3) DSK_ATTN_CASE(128, 4)
  DSK_ATTN_CASE(256, 1) DSK_ATTN_CASE(256, 2)
#undef DSK_ATTN_CASE
  if (hd == 512) launch_attention<512, 1, false>(a, a.kv_dtype, sc, grid, st);
  DSK_LAUNCH_CHECK(who);
  if (a.nsplit > 1) {
    const dim3 cgrid((unsigned)ceil_div((int64_t)a.B * a.nkv * a.R, 4));
    if (hd == 128) hipLaunchKernelGGL(attention_combine_kernel<128>, cgrid, dim3(256), 0, st, a);
    else if (hd == 256) hipLaunchKernelGGL(attention_combine_kernel<256>, cgrid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL(attention_combine_kernel<512>, cgrid, dim3(256), 0, st, a);
    DSK_LAUNCH_CHECK(who);
  }
  return DSK_OK;
}

}  // namespace dsk

using namespace dsk;

static int qkv_append_entry(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                            const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* v_norm, float eps,
                            const float* inv_freq, const int32_t* seq_lens, int pos_offset, const int32_t* block_table,
                            int max_pages, int page, int kv_dtype, void* k_pool, void* v_pool, uint32_t* k_sb,
                            uint32_t* v_sb, uint16_t* q_out, const float* x_ssq, int x_tiles, float x_eps,
                            dsk_stream_t stream);

extern "C" int dsk_qkv_norm_rope_append(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                                        const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* v_norm,
                                        float eps, const float* inv_freq, const int32_t* seq_lens, int pos_offset,
                                        const int32_t* block_table, int max_pages, int page, int kv_dtype,
                                        void* k_pool, void* v_pool, uint32_t* k_sb, uint32_t* v_sb, uint16_t* q_out,
                                        dsk_stream_t stream) {
  return qkv_append_entry(qkv, qkv_splits, B, W, nq, nkv, hd, q_norm, k_norm, v_norm, eps, inv_freq, seq_lens,
                          pos_offset, block_table, max_pages, page, kv_dtype, k_pool, v_pool, k_sb, v_sb, q_out,
                          nullptr, 0, 0.0f, stream);
}

extern "C" int dsk_qkv_rope_append_rn(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                                      const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                      const float* inv_freq, const int32_t* seq_lens, const int32_t* block_table,
                                      int max_pages, int page, int kv_dtype, void* k_pool, void* v_pool,
                                      uint32_t* k_sb, uint32_t* v_sb, uint16_t* q_out, const float* x_ssq,
                                      int x_tiles, float x_eps, dsk_stream_t stream) {
  DSK_REQUIRE(x_ssq && x_tiles > 0 && x_eps >= 0.0f, "dsk_qkv_rope_append_rn: needs the input's row-scale partials");
  return qkv_append_entry(qkv, qkv_splits, B, W, nq, nkv, hd, q_norm, k_norm, nullptr, eps, inv_freq, seq_lens, 0,
                          block_table, max_pages, page, kv_dtype, k_pool, v_pool, k_sb, v_sb, q_out, x_ssq, x_tiles,
                          x_eps, stream);
}

static int qkv_append_entry(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                            const uint16_t* q_norm, const uint16_t* k_norm, const uint16_t* v_norm, float eps,
                            const float* inv_freq, const int32_t* seq_lens, int pos_offset, const int32_t* block_table,
                            int max_pages, int page, int kv_dtype, void* k_pool, void* v_pool, uint32_t* k_sb,
                            uint32_t* v_sb, uint16_t* q_out, const float* x_ssq, int x_tiles, float x_eps,
                            dsk_stream_t stream) {
  DSK_REQUIRE(qkv && inv_freq && seq_lens && block_table && k_pool && v_pool && (q_out || nq == 0),
              "dsk_qkv_rope_append: null pointer");
  DSK_REQUIRE(hd == 128 || hd == 256 || hd == 512, "dsk_qkv_rope_append: head_dim %d not supported (128, 256, 512)",
              hd);
  DSK_REQUIRE(B > 0 && W > 0 && nq >= 0 && nkv > 0 && nq % nkv == 0, "dsk_qkv_rope_append: bad shape");
  DSK_REQUIRE(page > 0 && max_pages > 0, "dsk_qkv_rope_append: bad page geometry");
  DSK_REQUIRE(qkv_splits >= 0, "dsk_qkv_rope_append: qkv_splits=%d", qkv_splits);
  DSK_REQUIRE(!x_ssq || qkv_splits > 0, "dsk_qkv_rope_append_rn: the row scale applies to f32 split-K slices");
  DSK_REQUIRE(kv_dtype == DSK_KV_BF16 || (kv_dtype == DSK_KV_U8 && k_sb && v_sb),
              "dsk_qkv_rope_append: u8 KV needs scale/bias buffers");
  const int tasks = B * W * (nq + 2 * nkv);
  dim3 grid((unsigned)ceil_div(tasks, 4));
#define DSK_APPEND(HDV)                                                                                         \
  if (x_ssq)                                                                                                    \
    hipLaunchKernelGGL((qkv_rope_append_kernel<HDV, true, true>), grid, dim3(256), 0, as_stream(stream), qkv,   \
                       qkv_splits, B, W, nq, nkv, q_norm, k_norm, v_norm, eps, inv_freq, seq_lens, pos_offset,  \
                       block_table, max_pages, page, kv_dtype, k_pool, v_pool, k_sb, v_sb, q_out, x_ssq,       \
                       x_tiles, (float)(x_tiles * 16), x_eps);                                                  \
  else if (qkv_splits > 0)                                                                                      \
    hipLaunchKernelGGL((qkv_rope_append_kernel<HDV, false, true>), grid, dim3(256), 0, as_stream(stream), qkv,  \
                       qkv_splits, B, W, nq, nkv, q_norm, k_norm, v_norm, eps, inv_freq, seq_lens, pos_offset,  \
                       block_table, max_pages, page, kv_dtype, k_pool, v_pool, k_sb, v_sb, q_out, nullptr, 0,  \
                       0.0f, 0.0f);                                                                             \
  else                                                                                                          \
    hipLaunchKernelGGL((qkv_rope_append_kernel<HDV, false, false>), grid, dim3(256), 0, as_stream(stream), qkv, \
                       qkv_splits, B, W, nq, nkv, q_norm, k_norm, v_norm, eps, inv_freq, seq_lens, pos_offset,  \
                       block_table, max_pages, page, kv_dtype, k_pool, v_pool, k_sb, v_sb, q_out, nullptr, 0,  \
                       0.0f, 0.0f)
  if (hd == 128) {
    DSK_APPEND(128);
  } else if (hd == 256) {
    DSK_APPEND(256);
  } else {
    DSK_APPEND(512);
  }
#undef DSK_APPEND
  DSK_LAUNCH_CHECK("dsk_qkv_rope_append");
  return DSK_OK;
}

extern "C" int dsk_qkv_rope_append(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                                   const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                                   const float* inv_freq, const int32_t* seq_lens, int pos_offset,
                                   const int32_t* block_table, int max_pages, int page, int kv_dtype,
                                   void* k_pool, void* v_pool, uint32_t* k_sb, uint32_t* v_sb,
                                   uint16_t* q_out, dsk_stream_t stream) {
  return dsk_qkv_norm_rope_append(qkv, qkv_splits, B, W, nq, nkv, hd, q_norm, k_norm, nullptr, eps, inv_freq,
                                  seq_lens, pos_offset, block_table, max_pages, page, kv_dtype, k_pool, v_pool, k_sb,
                                  v_sb, q_out, stream);
}

extern "C" size_t dsk_attn_ws_bytes(int B, int W, int nq, int hd, int max_ctx) {
  if (B <= 0 || W <= 0 || nq <= 0 || hd <= 0 || max_ctx <= 0) return 0;
  if (hd != 128 && hd != 256 && hd != 512) return 0;
  if (W > kAttnVerifyMaxW)  // many-query passes: splits of 8 blocks
    return attn_ws_need(B, W, nq, hd, (int)ceil_div(max_ctx, attn_split_keys(hd, max_ctx) * 8));
  // + the fused new-token split (also covers the verify kernel's splits of 128 keys and more)
  return attn_ws_need(B, W, nq, hd, attn_nsplit(hd, max_ctx) + 1);
}

extern "C" int dsk_attention(const uint16_t* q, int B, int W, int nq, int nkv, int hd, float scale, int causal,
                             int window, float softcap, const int32_t* seq_lens, int max_ctx,
                             const int32_t* block_table, int max_pages, int page, int kv_dtype, const void* k_pool,
                             const void* v_pool, const uint32_t* k_sb, const uint32_t* v_sb, uint16_t* out,
                             int out_packed, void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(q && seq_lens && block_table && k_pool && v_pool && out, "dsk_attention: null pointer");
  AttnArgs a = {};
  a.q = q;
  a.B = B;
  a.W = W;
  a.nq = nq;
  a.nkv = nkv;
  a.scale = scale;
  a.softcap = softcap;
  a.causal = causal;
  a.window = window;
  a.seq_lens = seq_lens;
  a.block_table = block_table;
  a.max_pages = max_pages;
  a.page = page;
  a.kv_dtype = kv_dtype;
  a.k_pool = const_cast<void*>(k_pool);
  a.v_pool = const_cast<void*>(v_pool);
  a.k_sb = const_cast<uint32_t*>(k_sb);
  a.v_sb = const_cast<uint32_t*>(v_sb);
  a.out = out;
  a.out_packed = out_packed ? 1 : 0;
  return attention_run(a, hd, max_ctx, softcap, workspace, ws_bytes, false, as_stream(stream), "dsk_attention");
}

extern "C" int dsk_qkv_attention(const void* qkv, int qkv_splits, int B, int W, int nq, int nkv, int hd,
                                 const uint16_t* q_norm, const uint16_t* k_norm, float eps, const float* inv_freq,
                                 float scale, int causal, int window, float softcap, const int32_t* seq_lens,
                                 int max_ctx, const int32_t* block_table, int max_pages, int page, int kv_dtype,
                                 void* k_pool, void* v_pool, uint32_t* k_sb, uint32_t* v_sb, uint16_t* out,
                                 int out_packed, void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(qkv && inv_freq && seq_lens && block_table && k_pool && v_pool && out,
              "dsk_qkv_attention: null pointer");
  DSK_REQUIRE(qkv_splits >= 0, "dsk_qkv_attention: qkv_splits=%d", qkv_splits);
  DSK_REQUIRE(((uintptr_t)q_norm | (uintptr_t)qkv) % 16 == 0, "dsk_qkv_attention: q_norm and qkv must be 16-byte aligned");
  AttnArgs a = {};
  a.qkv = qkv;
  a.qkv_splits = qkv_splits;
  a.q_norm = q_norm;
  a.k_norm = k_norm;
  a.eps = eps;
  a.inv_freq = inv_freq;
  a.B = B;
  a.W = W;
  a.nq = nq;
  a.nkv = nkv;
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
  return attention_run(a, hd, max_ctx, softcap, workspace, ws_bytes, true, as_stream(stream), "dsk_qkv_attention");
}
