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
    const uint16_t* __restrict__ qkv, int B, int W, int nq, int nkv, const uint16_t* __restrict__ q_norm,
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
  const uint16_t* src = qkv + (int64_t)row * nheads * HD + (int64_t)head * HD;
  float v[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) v[e] = bf16_to_f32(src[lane * PER + e]);

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
      const float ang = (float)pos * inv_freq[dd];
      float sn, cs;
      sincosf(ang, &sn, &cs);
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
  int nsplit, split_tokens;
  float* part;  // [B][nkv][nsplit][R][HD + 2]
  int* cnt;     // [B * nkv]
};

constexpr int kKeyTile = 32;
template <int HD> struct Lds { static constexpr int KROW = HD + 8, VROW = kKeyTile + 8; };

// K/V tile staging, split into a global->register load (issued one tile ahead) and a
// register->LDS store (dequantising 8-bit KV to bf16).
template <int HD>
struct KVRegs {
  static constexpr int CPT = kKeyTile * HD / 8 / 256;  // 8-element chunks per thread
  u32x4 k[CPT], v[CPT];
  uint32_t ksb[CPT], vsb[CPT];
  bool valid[CPT];
};

template <int HD>
__device__ __forceinline__ void load_kv(const AttnArgs& a, int b, int kvh, int j0, int Lk, KVRegs<HD>& r) {
#pragma unroll
  for (int ci = 0; ci < KVRegs<HD>::CPT; ++ci) {
    const int c = threadIdx.x + ci * 256;
    const int key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
    const int j = j0 + key;
    r.valid[ci] = j < Lk;
    if (!r.valid[ci]) continue;
    const int pg = a.block_table[(int64_t)b * a.max_pages + j / a.page];
    const int64_t tok = ((int64_t)pg * a.nkv + kvh) * a.page + (j % a.page);
    if (a.kv_dtype == DSK_KV_BF16) {
      r.k[ci] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.k_pool) + tok * HD + d0);
      r.v[ci] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.v_pool) + tok * HD + d0);
    } else {
      const uint2 kr = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(a.k_pool) + tok * HD + d0);
      const uint2 vr = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(a.v_pool) + tok * HD + d0);
      r.k[ci] = u32x4{kr.x, kr.y, 0, 0};
      r.v[ci] = u32x4{vr.x, vr.y, 0, 0};
      r.ksb[ci] = a.k_sb[tok * (HD / 64) + d0 / 64];
      r.vsb[ci] = a.v_sb[tok * (HD / 64) + d0 / 64];
    }
  }
}

template <int HD>
__device__ __forceinline__ void store_kv(const AttnArgs& a, const KVRegs<HD>& r, uint16_t* ks, uint16_t* vt) {
  // ks: [32 keys][KROW] bf16 row-major; vt: [HD][VROW] bf16 (transposed V), rows padded.
#pragma unroll
  for (int ci = 0; ci < KVRegs<HD>::CPT; ++ci) {
    const int c = threadIdx.x + ci * 256;
    const int key = c / (HD / 8), d0 = (c % (HD / 8)) * 8;
    uint16_t kh[8], vh[8];
    if (!r.valid[ci]) {
#pragma unroll
      for (int e = 0; e < 8; ++e) kh[e] = vh[e] = 0;
    } else if (a.kv_dtype == DSK_KV_BF16) {
      const uint16_t* kk = reinterpret_cast<const uint16_t*>(&r.k[ci]);
      const uint16_t* vv = reinterpret_cast<const uint16_t*>(&r.v[ci]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kh[e] = kk[e];
        vh[e] = vv[e];
      }
    } else {
      const float ksc = bf16_to_f32((uint16_t)(r.ksb[ci] & 0xffff)), kbi = bf16_to_f32((uint16_t)(r.ksb[ci] >> 16));
      const float vsc = bf16_to_f32((uint16_t)(r.vsb[ci] & 0xffff)), vbi = bf16_to_f32((uint16_t)(r.vsb[ci] >> 16));
      const uint8_t* kb = reinterpret_cast<const uint8_t*>(&r.k[ci]);
      const uint8_t* vb = reinterpret_cast<const uint8_t*>(&r.v[ci]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kh[e] = f32_to_bf16(fmaf(ksc, (float)kb[e], kbi));
        vh[e] = f32_to_bf16(fmaf(vsc, (float)vb[e], vbi));
      }
    }
    *reinterpret_cast<u32x4*>(ks + key * Lds<HD>::KROW + d0) = *reinterpret_cast<const u32x4*>(kh);
#pragma unroll
    for (int e = 0; e < 8; ++e) vt[(d0 + e) * Lds<HD>::VROW + key] = vh[e];
  }
}

template <int HD, int QT>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[kKeyTile * Lds<HD>::KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt[HD * Lds<HD>::VROW];
  __shared__ int last;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int split = blockIdx.x % a.nsplit;
  const int bk = blockIdx.x / a.nsplit;  // b * nkv + kvh
  const int b = bk / a.nkv, kvh = bk % a.nkv;
  const int off = a.seq_lens[b];
  const int Lk = off + a.W;
  const int j_lo = split * a.split_tokens;
  const int j_hi = min(min(Lk, j_lo + a.split_tokens), a.max_pages * a.page);
  constexpr int DT = HD / 16;  // d tiles of the output
  constexpr int KS = HD / 32;  // k steps of the score MFMA

  // query rows handled by this wave: tiles wv, wv + 4, ... ; row r = i * G + hl
  f32x4 o[QT][DT];
  float mrow[QT], lrow[QT];
  bf16x8 qf[QT][KS];
  int qi[QT];
  bool qvalid[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int r = (wv + 4 * t) * 16 + (lane & 15);
    qvalid[t] = r < a.R;
    const int i = qvalid[t] ? r / a.G : 0, hl = qvalid[t] ? r % a.G : 0;
    qi[t] = i;
    const uint16_t* qp = a.q + ((int64_t)(b * a.W + i) * a.nq + kvh * a.G + hl) * HD;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 raw = qvalid[t] ? *reinterpret_cast<const u32x4*>(qp + s * 32 + (lane >> 4) * 8) : u32x4{0, 0, 0, 0};
      qf[t][s] = __builtin_bit_cast(bf16x8, raw);
    }
#pragma unroll
    for (int d = 0; d < DT; ++d) o[t][d] = f32x4{0, 0, 0, 0};
    mrow[t] = -__builtin_inff();
    lrow[t] = 0.0f;
  }

  KVRegs<HD> kvr;
  if (j_lo < j_hi) load_kv<HD>(a, b, kvh, j_lo, j_hi, kvr);
  for (int j0 = j_lo; j0 < j_hi; j0 += kKeyTile) {
    __syncthreads();
    store_kv<HD>(a, kvr, ks, vt);
    if (j0 + kKeyTile < j_hi) load_kv<HD>(a, b, kvh, j0 + kKeyTile, j_hi, kvr);  // next tile in flight
    __syncthreads();
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      if (wv + 4 * t >= (a.R + 15) / 16) continue;
      // scores for keys j0 + {0..15} (h = 0) and j0 + {16..31} (h = 1)
      f32x4 st[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4 acc = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(ks + (h * 16 + (lane & 15)) * Lds<HD>::KROW + s * 32 + (lane >> 4) * 8);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[t][s], acc, 0, 0, 0);
        }
        st[h] = acc;
      }
      // lane holds S^T[key = h*16 + 4*(lane/16) + r][q = lane % 16]
      const int qpos = off + qi[t];
      float smax = -__builtin_inff();
      float sv[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = j0 + h * 16 + (lane >> 4) * 4 + r;
          float s = st[h][r] * a.scale;
          if (a.softcap > 0.0f) s = tanhf(s / a.softcap) * a.softcap;
          bool ok = j < j_hi && qvalid[t];
          if (a.causal) {
            ok = ok && j <= qpos;
            if (a.window > 0) ok = ok && j > qpos - a.window;
          }
          s = ok ? s : -__builtin_inff();
          sv[h][r] = s;
          smax = fmaxf(smax, s);
        }
      smax = fmaxf(smax, __shfl_xor(smax, 16, 64));
      smax = fmaxf(smax, __shfl_xor(smax, 32, 64));
      const float mnew = fmaxf(mrow[t], smax);
      const float alpha = (mnew == -__builtin_inff()) ? 1.0f : __expf(mrow[t] - mnew);
      float psum = 0.0f;
      float pv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = (sv[h][r] == -__builtin_inff()) ? 0.0f : __expf(sv[h][r] - mnew);
          const float pr = round_bf16(p);
          pv[h * 4 + r] = pr;
          psum += pr;
        }
      psum += __shfl_xor(psum, 16, 64);
      psum += __shfl_xor(psum, 32, 64);
      lrow[t] = lrow[t] * alpha + psum;
      mrow[t] = mnew;
      bf16x8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = (__bf16)pv[e];
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        // A = V^T rows d*16 + lane%16, keys in the same order as pb: {4c..4c+3, 16+4c..16+4c+3}
        const uint16_t* vr = vt + (d * 16 + (lane & 15)) * Lds<HD>::VROW + (lane >> 4) * 4;
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16);
        u32x4 vv = {lo.x, lo.y, hi.x, hi.y};
        f32x4 acc = o[t][d];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] *= alpha;
        o[t][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv), pb, acc, 0, 0, 0);
      }
    }
  }

  // publish this split's partial: rows r, [o(HD) | m | l]
  const size_t rstride = HD + 2;
  float* pbase = a.part + (((size_t)bk * a.nsplit + split) * a.R) * rstride;
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int r = (wv + 4 * t) * 16 + (lane & 15);
    if (wv + 4 * t >= (a.R + 15) / 16 || r >= a.R) continue;
    float* pr = pbase + (size_t)r * rstride;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) pr[d * 16 + (lane >> 4) * 4 + rr] = o[t][d][rr];
    if (lane < 16) {
      pr[HD] = mrow[t];
      pr[HD + 1] = lrow[t];
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    int prev = atomicAdd(&a.cnt[bk], 1);
    last = (prev == a.nsplit - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  // combine the splits: lanes own splits for the max / denominator, then dims for the sum
  const float* base = a.part + ((size_t)bk * a.nsplit * a.R) * rstride;
  for (int r = wv; r < a.R; r += 4) {
    float M = -__builtin_inff();
    for (int s = lane; s < a.nsplit; s += 64)
      M = fmaxf(M, __builtin_nontemporal_load(base + ((size_t)s * a.R + r) * rstride + HD));
    M = wave_max(M);
    float den = 0.0f;
    for (int s = lane; s < a.nsplit; s += 64) {
      const float* pr = base + ((size_t)s * a.R + r) * rstride;
      const float ms = __builtin_nontemporal_load(pr + HD);
      if (ms != -__builtin_inff()) den += __expf(ms - M) * __builtin_nontemporal_load(pr + HD + 1);
    }
    den = wave_sum(den);
    float acc[HD / 64];
#pragma unroll
    for (int e = 0; e < HD / 64; ++e) acc[e] = 0.0f;
    int s = 0;
    for (; s + 8 <= a.nsplit; s += 8) {
      float ms[8], ov[8][HD / 64];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float* pr = base + ((size_t)(s + u) * a.R + r) * rstride;
        ms[u] = __builtin_nontemporal_load(pr + HD);
#pragma unroll
        for (int e = 0; e < HD / 64; ++e) ov[u][e] = __builtin_nontemporal_load(pr + e * 64 + lane);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float w = ms[u] == -__builtin_inff() ? 0.0f : __expf(ms[u] - M);
#pragma unroll
        for (int e = 0; e < HD / 64; ++e) acc[e] += w * ov[u][e];
      }
    }
    for (; s < a.nsplit; ++s) {
      const float* pr = base + ((size_t)s * a.R + r) * rstride;
      const float ms = __builtin_nontemporal_load(pr + HD);
      const float w = ms == -__builtin_inff() ? 0.0f : __expf(ms - M);
#pragma unroll
      for (int e = 0; e < HD / 64; ++e) acc[e] += w * __builtin_nontemporal_load(pr + e * 64 + lane);
    }
    const int i = r / a.G, hl = r % a.G;
    uint16_t* op = a.out + ((int64_t)(b * a.W + i) * a.nq + kvh * a.G + hl) * HD;
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
#pragma unroll
    for (int e = 0; e < HD / 64; ++e) op[e * 64 + lane] = f32_to_bf16(acc[e] * inv);
  }
  if (threadIdx.x == 0) a.cnt[bk] = 0;
}

// ----------------------------------------------------------------------------- host helpers
static int attn_split_tokens(int B, int nkv, int max_ctx) {
  // aim for ~256 blocks, never splits shorter than 128 tokens
  int st = 2048;
  while (st > 128 && (int64_t)B * nkv * ((max_ctx + st - 1) / st) < 256) st >>= 1;
  return st;
}

constexpr size_t kAttnCounterBytes = 16384;

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_qkv_rope_append(const uint16_t* qkv, int B, int W, int nq, int nkv, int hd,
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
  DSK_REQUIRE(kv_dtype == DSK_KV_BF16 || (kv_dtype == DSK_KV_U8 && k_sb && v_sb),
              "dsk_qkv_rope_append: u8 KV needs scale/bias buffers");
  const int tasks = B * W * (nq + 2 * nkv);
  dim3 grid((unsigned)ceil_div(tasks, 4));
  if (hd == 128)
    hipLaunchKernelGGL(qkv_rope_append_kernel<128>, grid, dim3(256), 0, as_stream(stream), qkv, B, W, nq, nkv, q_norm,
                       k_norm, eps, inv_freq, seq_lens, pos_offset, block_table, max_pages, page, kv_dtype, k_pool,
                       v_pool, k_sb, v_sb, q_out);
  else
    hipLaunchKernelGGL(qkv_rope_append_kernel<256>, grid, dim3(256), 0, as_stream(stream), qkv, B, W, nq, nkv, q_norm,
                       k_norm, eps, inv_freq, seq_lens, pos_offset, block_table, max_pages, page, kv_dtype, k_pool,
                       v_pool, k_sb, v_sb, q_out);
  DSK_LAUNCH_CHECK("dsk_qkv_rope_append");
  return DSK_OK;
}

extern "C" size_t dsk_attn_ws_bytes(int B, int W, int nq, int hd, int max_ctx) {
  if (B <= 0 || W <= 0 || nq <= 0 || hd <= 0 || max_ctx <= 0) return 0;
  // worst case over nkv: rows per kv head * nkv = W * nq
  const int st = 128;  // smallest split => most splits
  const size_t nsplit = (size_t)((max_ctx + st - 1) / st);
  return kAttnCounterBytes + (size_t)B * W * nq * nsplit * (hd + 2) * sizeof(float);
}

extern "C" int dsk_attn_ws_init(void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(workspace && ws_bytes >= kAttnCounterBytes, "dsk_attn_ws_init: workspace too small");
  hipError_t e = hipMemsetAsync(workspace, 0, kAttnCounterBytes, as_stream(stream));
  if (e != hipSuccess) {
    set_error("dsk_attn_ws_init: %s", hipGetErrorString(e));
    return DSK_ELAUNCH;
  }
  return DSK_OK;
}

extern "C" int dsk_attention(const uint16_t* q, int B, int W, int nq, int nkv, int hd, float scale, int causal,
                             int window, float softcap, const int32_t* seq_lens, int max_ctx,
                             const int32_t* block_table, int max_pages, int page, int kv_dtype, const void* k_pool,
                             const void* v_pool, const uint32_t* k_sb, const uint32_t* v_sb, uint16_t* out,
                             void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(q && seq_lens && block_table && k_pool && v_pool && out && workspace, "dsk_attention: null pointer");
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
  DSK_REQUIRE(B * nkv <= (int)(kAttnCounterBytes / sizeof(int)), "dsk_attention: too many (row, kv head) pairs");
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
  a.split_tokens = attn_split_tokens(B, nkv, max_ctx);
  a.nsplit = (max_ctx + a.split_tokens - 1) / a.split_tokens;
  const size_t need = kAttnCounterBytes + (size_t)B * nkv * a.nsplit * R * (hd + 2) * sizeof(float);
  DSK_REQUIRE(ws_bytes >= need, "dsk_attention: workspace %zu < %zu", ws_bytes, need);
  a.cnt = reinterpret_cast<int*>(workspace);
  a.part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + kAttnCounterBytes);
  dim3 grid((unsigned)(B * nkv * a.nsplit));
  hipStream_t st = as_stream(stream);
#define DSK_ATTN_CASE(hdv, qt) \
  if (hd == hdv && QT == qt) hipLaunchKernelGGL((attention_kernel<hdv, qt>), grid, dim3(256), 0, st, a);
  DSK_ATTN_CASE(128, 1) DSK_ATTN_CASE(128, 2) DSK_ATTN_CASE(128, 3) DSK_ATTN_CASE(128, 4)
  DSK_ATTN_CASE(256, 1) DSK_ATTN_CASE(256, 2)
#undef DSK_ATTN_CASE
  DSK_LAUNCH_CHECK("dsk_attention");
  return DSK_OK;
}
