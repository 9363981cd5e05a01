// Fused acceptance on gfx950: greedy argmax-compare and speculative-sampling acceptance
// (min(1, p/q) with residual resampling) after temperature / top-k / top-p, plus the KV
// rollback to the accepted length. One canonical arithmetic is shared with the CPU oracle
// so decisions, sampled indices and rollback lengths are bit-identical:
//   - exp: dsk_expf (Cody-Waite reduction by ln 2 with a two-word constant, Taylor
//     polynomial to r^7 evaluated with explicit fmaf, inputs below -86 flush to zero);
//   - probability sums: integers of fx(p) = floor(p * 2^44) (order-independent);
//   - uniforms: Philox4x32-10 word 0, u = (w >> 8) * 2^-24;
//   - categorical draws: inverse CDF over the fixed-point masses.
// Floating-point contraction is off in this file: every fma is written out.
#pragma clang fp contract(off)

#include <mutex>

#include "common.h"

namespace dsk {

// ----------------------------------------------------------------------------- math
__device__ __forceinline__ float dsk_expf(float x) {
  if (x < -86.0f) return 0.0f;
  if (x != x) return x;
  if (x > 88.7f) return __builtin_inff();
  float t = x * 1.44269504f;
  float k = rintf(t);
  float r = __builtin_fmaf(-k, 0.693145751953125f, x);
  r = __builtin_fmaf(-k, 1.428606765330187e-06f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ki = (int)k;
  if (ki > 127) {
    p = p * 0x1p127f;
    ki -= 127;
  }
  return p * bits_f32((uint32_t)(ki + 127) << 23);
}

__device__ __forceinline__ uint64_t fx(float p) { return (uint64_t)(p * 0x1p44f); }
__device__ __forceinline__ float fx_to_float(uint64_t s) { return (float)((double)s * 0x1p-44); }

__device__ __forceinline__ uint32_t philox_word(uint64_t seed, uint32_t c0, uint32_t c1, uint32_t c2,
                                                uint32_t c3) {
  const uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += W0;
      k1 += W1;
    }
    uint32_t hi0 = __umulhi(M0, c0), lo0 = M0 * c0;
    uint32_t hi1 = __umulhi(M1, c2), lo1 = M1 * c2;
    uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  return c0;
}

__device__ __forceinline__ float u24_to_float(uint32_t w) { return (float)(w >> 8) * 0x1p-24f; }

// ----------------------------------------------------------------------------- block helpers
constexpr int kNT = 512;  // threads per row block
constexpr int kNW = kNT / 64;

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  uint32_t lo = __shfl((uint32_t)v, src, 64), hi = __shfl((uint32_t)(v >> 32), src, 64);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int d) {
  uint32_t lo = __shfl_up((uint32_t)v, d, 64), hi = __shfl_up((uint32_t)(v >> 32), d, 64);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t lo = __shfl_xor((uint32_t)v, o, 64), hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}
// inclusive prefix sum across a wave
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  const int lane = threadIdx.x & 63;
  for (int d = 1; d < 64; d <<= 1) {
    uint64_t o = shfl_up_u64(v, d);
    if (lane >= d) v += o;
  }
  return v;
}

struct RowSmem {
  uint64_t hist[2048];
  uint64_t wsum[kNW];
  float wmax[kNW];
  uint64_t bc64[4];
  uint32_t bc32[4];
};

__device__ uint64_t block_sum_u64(uint64_t v, RowSmem& sm) {
  v = wave_sum_u64(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm.wsum[w] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int i = 0; i < kNW; ++i) t += sm.wsum[i];
  return t;
}

__device__ float block_max(float v, RowSmem& sm) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm.wmax[w] = v;
  __syncthreads();
  float t = sm.wmax[0];
#pragma unroll
  for (int i = 1; i < kNW; ++i) t = fmaxf(t, sm.wmax[i]);
  return t;
}

// Radix select over the keys of p (fp32 bits of non-negative values are ordered like the
// values). Keys below `floor_key` count as key 0 with weight 0 (they were zeroed by an
// earlier truncation). count_mode: weight 1 per element, else weight fx(p).
// Returns the key K with weight(> K) < target <= weight(>= K); returns 0 when the total
// weight stays below target.
__device__ uint32_t radix_select(const float* __restrict__ p, int64_t V, uint32_t floor_key, int count_mode,
                                 uint64_t target, RowSmem& sm) {
  const int shifts[3] = {21, 10, 0};
  const int widths[3] = {11, 11, 10};
  uint32_t prefix = 0;
  uint64_t above = 0;
  for (int lv = 0; lv < 3; ++lv) {
    const int sh = shifts[lv], wd = widths[lv];
    const int nb = 1 << wd;
    const int hi_sh = sh + wd;
    __syncthreads();
    for (int i = threadIdx.x; i < 2048; i += kNT) sm.hist[i] = 0;
    __syncthreads();
    for (int64_t j = threadIdx.x; j < V; j += kNT) {
      float v = p[j];
      uint32_t key = f32_bits(v);
      uint64_t wgt;
      if (key < floor_key) {
        key = 0;
        wgt = count_mode ? 1 : 0;
      } else {
        wgt = count_mode ? 1 : fx(v);
      }
      if (lv == 0 || (hi_sh >= 32 ? true : ((key >> hi_sh) == (prefix >> hi_sh)))) {
        if (wgt) atomicAdd((unsigned long long*)&sm.hist[(key >> sh) & (nb - 1)], (unsigned long long)wgt);
      }
    }
    __syncthreads();
    // descending scan over the nb buckets: thread t owns buckets nb-1-4t .. nb-4-4t
    const int per = 4;
    const int nthr = nb / per;  // 512 or 256
    uint64_t loc[4] = {0, 0, 0, 0};
    uint64_t tsum = 0;
    if ((int)threadIdx.x < nthr) {
#pragma unroll
      for (int q = 0; q < per; ++q) {
        loc[q] = sm.hist[nb - 1 - (int)threadIdx.x * per - q];
        tsum += loc[q];
      }
    }
    // block exclusive scan of tsum in thread order
    uint64_t incl = wave_incl_scan_u64(tsum);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 63) sm.wsum[w] = incl;
    if (threadIdx.x == 0) {
      sm.bc32[0] = 0xFFFFFFFFu;
      sm.bc64[0] = 0;
    }
    __syncthreads();
    uint64_t wbefore = 0;
    for (int i = 0; i < w; ++i) wbefore += sm.wsum[i];
    uint64_t run = above + wbefore + incl - tsum;
    if ((int)threadIdx.x < nthr) {
#pragma unroll
      for (int q = 0; q < per; ++q) {
        const uint64_t nrun = run + loc[q];
        if (run < target && nrun >= target) {
          sm.bc32[0] = (uint32_t)(nb - 1 - (int)threadIdx.x * per - q);
          sm.bc64[0] = run;  // weight above this bucket
        }
        run = nrun;
      }
    }
    __syncthreads();
    const uint32_t d = sm.bc32[0];
    if (d == 0xFFFFFFFFu) return 0;  // never reached: everything qualifies
    above = sm.bc64[0];
    prefix |= d << sh;
  }
  return prefix;
}

// Softmax with temperature and truncation for one row. Leaves p = e / Z in `scratch` and
// returns the cut key and the renormalisation denominator: the final probability of j is
// trunc ? (key(p_j) >= cut ? p_j / den : 0) : p_j.
struct RowProbs {
  uint32_t cut;
  int trunc;
  float den;
};

__device__ __forceinline__ float final_prob(const RowProbs& rp, float pj) {
  if (!rp.trunc) return pj;
  return f32_bits(pj) >= rp.cut ? pj / rp.den : 0.0f;
}

__device__ RowProbs row_probs(const float* __restrict__ logits, int64_t V, float T, int mul_inv, float top_p,
                              int top_k, float* __restrict__ scratch, RowSmem& sm) {
  const float inv_t = 1.0f / T;
  float m = -__builtin_inff();
  for (int64_t j = threadIdx.x; j < V; j += kNT) {
    float y = mul_inv ? logits[j] * inv_t : logits[j] / T;
    m = fmaxf(m, y);
  }
  m = block_max(m, sm);
  uint64_t z = 0;
  for (int64_t j = threadIdx.x; j < V; j += kNT) {
    float y = mul_inv ? logits[j] * inv_t : logits[j] / T;
    float e = dsk_expf(y - m);
    scratch[j] = e;
    z += fx(e);
  }
  const uint64_t Z = block_sum_u64(z, sm);
  const float Zf = fx_to_float(Z);
  for (int64_t j = threadIdx.x; j < V; j += kNT) scratch[j] = scratch[j] / Zf;
  __syncthreads();

  RowProbs rp;
  rp.trunc = 0;
  rp.cut = 0;
  rp.den = 1.0f;
  const int do_k = (top_k > 0 && (int64_t)top_k < V);
  const int do_p = (top_p < 1.0f);
  if (!do_k && !do_p) return rp;
  rp.trunc = 1;
  uint32_t kk = 0;
  if (do_k) kk = radix_select(scratch, V, 0, 1, (uint64_t)top_k, sm);
  uint32_t cut = kk;
  if (do_p) {
    const uint64_t TP = (uint64_t)floor((double)top_p * 0x1p44);
    if (TP == 0) {
      cut = 0xFFFFFFFFu;  // empty nucleus: every probability becomes 0
    } else {
      uint32_t c = radix_select(scratch, V, kk, 0, TP, sm);
      if (c > 0) cut = c;
    }
  }
  rp.cut = cut;
  uint64_t s = 0;
  for (int64_t j = threadIdx.x; j < V; j += kNT) {
    float pj = scratch[j];
    if (f32_bits(pj) >= cut) s += fx(pj);
  }
  const uint64_t S = block_sum_u64(s, sm);
  const float Sf = fx_to_float(S);
  rp.den = Sf > 1e-12f ? Sf : 1e-12f;
  return rp;
}

// Inverse-CDF draw; weight(j) is a device lambda giving the float weight of element j.
// Each wave owns a contiguous slice of the index range so prefix order is index order.
template <typename WF>
__device__ int64_t block_categorical(int64_t V, uint32_t word, WF weight, RowSmem& sm) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t per_wave = ((V + kNW - 1) / kNW + 63) / 64 * 64;
  const int64_t lo = (int64_t)w * per_wave, hi = min(V, lo + per_wave);
  uint64_t tot = 0;
  for (int64_t j = lo + lane; j < hi; j += 64) tot += fx(weight(j));
  tot = wave_sum_u64(tot);
  __syncthreads();
  if (lane == 0) sm.wsum[w] = tot;
  if (threadIdx.x == 0) sm.bc64[1] = (uint64_t)-1;
  __syncthreads();
  uint64_t W = 0, before = 0;
#pragma unroll
  for (int i = 0; i < kNW; ++i) {
    if (i < w) before += sm.wsum[i];
    W += sm.wsum[i];
  }
  const uint64_t u = word >> 8;
  if (W == 0) return (int64_t)((u * (uint64_t)V) >> 24);
  const uint64_t t = (W >> 24) * u + (((W & 0xFFFFFFull) * u) >> 24);
  if (t >= before && t < before + sm.wsum[w]) {
    uint64_t run = before;
    for (int64_t j0 = lo; j0 < hi; j0 += 64) {
      const int64_t j = j0 + lane;
      uint64_t c = (j < hi) ? fx(weight(j)) : 0;
      uint64_t incl = wave_incl_scan_u64(c) + run;
      // first lane whose inclusive prefix exceeds t
      unsigned long long hit = __ballot(j < hi && incl > t);
      if (hit) {
        int first = __ffsll(hit) - 1;
        if (lane == first) sm.bc64[1] = (uint64_t)j;
        break;
      }
      run = shfl_u64(incl, 63);
    }
  }
  __syncthreads();
  return (int64_t)sm.bc64[1];
}

// ----------------------------------------------------------------------------- workspace
struct AcceptWs {
  int* cnt;         // [B] arrival counters (zero between calls)
  float* gval;      // [B*W*S] greedy slice maxima
  int* gidx;        // [B*W*S]
  int* acc;         // [B*(L+1)]
  int* samp;        // [B*(L+1)]
  float* scratch;   // [B*(L+1)][2][V]
};

constexpr int kGreedySlices = 64;  // slices per row: one per lane of the merging wave
constexpr size_t kAcceptCounterBytes = 4096;

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__host__ __device__ inline AcceptWs accept_ws(void* base, int B, int W, int64_t V) {
  AcceptWs ws;
  uint8_t* p = reinterpret_cast<uint8_t*>(base);
  size_t off = 0;
  ws.cnt = reinterpret_cast<int*>(p + off);
  off += kAcceptCounterBytes;
  const size_t rows = (size_t)B * W;
  ws.gval = reinterpret_cast<float*>(p + off);
  off += align256(rows * kGreedySlices * 4);
  ws.gidx = reinterpret_cast<int*>(p + off);
  off += align256(rows * kGreedySlices * 4);
  ws.acc = reinterpret_cast<int*>(p + off);
  off += align256(rows * 4);
  ws.samp = reinterpret_cast<int*>(p + off);
  off += align256(rows * 4);
  ws.scratch = reinterpret_cast<float*>(p + off);
  return ws;
}

__host__ __device__ inline size_t accept_ws_total(int B, int W, int64_t V) {
  const size_t rows = (size_t)B * W;
  return kAcceptCounterBytes + 2 * align256(rows * kGreedySlices * 4) + 2 * align256(rows * 4) +
         rows * 2 * (size_t)V * 4;
}

// ----------------------------------------------------------------------------- greedy
// Running argmax (lowest index on ties; NaN never wins) of this thread's share of row[lo, hi),
// 256 threads. VEC: the row is 16-byte aligned and lo a multiple of 8, so whole 16-byte chunks
// (4 f32 / 8 bf16) are read with four loads in flight per thread; the scalar loop takes the tail.
template <int BF16, bool VEC>
__device__ inline void span_argmax(const void* __restrict__ row, int64_t lo, int64_t hi, float& best, int64_t& bi) {
  if constexpr (VEC) {
    constexpr int E = BF16 ? 8 : 4;
    constexpr int UN = 4;
    const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(row) + lo * (BF16 ? 2 : 4));
    const int64_t nv = hi > lo ? (hi - lo) / E : 0;
    for (int64_t c0 = threadIdx.x; c0 < nv; c0 += 256 * UN) {
      u32x4 v[UN];
#pragma unroll
      for (int u = 0; u < UN; ++u)
        if (c0 + u * 256 < nv) v[u] = __builtin_nontemporal_load(p + c0 + u * 256);
#pragma unroll
      for (int u = 0; u < UN; ++u) {
        const int64_t c = c0 + u * 256;
        if (c < nv) {
#pragma unroll
          for (int e = 0; e < E; ++e) {
            const uint32_t w = v[u][BF16 ? e / 2 : e];
            const float x = __uint_as_float(BF16 ? ((e & 1) ? (w & 0xffff0000u) : (w << 16)) : w);
            const int64_t j = lo + c * E + e;
            if (x > best || (x == best && j < bi)) {
              best = x;
              bi = j;
            }
          }
        }
      }
    }
    lo += nv * E;
  }
  for (int64_t j = lo + threadIdx.x; j < hi; j += 256) {
    const float x = BF16 ? bf16_to_f32(reinterpret_cast<const uint16_t*>(row)[j]) : reinterpret_cast<const float*>(row)[j];
    if (x > best || (x == best && j < bi)) {
      best = x;
      bi = j;
    }
  }
}

// wave-wide argmax of (best, bi), lowest index on ties; every lane ends with the result
__device__ inline void wave_argmax(float& best, int64_t& bi) {
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(best, o, 64);
    int64_t oi = (int64_t)__shfl_xor((int)bi, o, 64);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
}

// slice length: ceil(V / S) rounded up to 8 elements, so every slice starts 16-byte aligned
__host__ __device__ inline int64_t slice_len(int64_t V) { return ((V + kGreedySlices - 1) / kGreedySlices + 7) & ~(int64_t)7; }

// Pass 1 of a greedy pick: block (row, slice) writes the argmax of logits[row][slice range]
// (lowest index on ties; index V when the range is empty or all NaN) to partial slot
// row * kGreedySlices + slice. The merge runs as the next kernel: no fences or atomics.
template <int BF16, bool VEC>
__global__ __launch_bounds__(256) void slice_argmax_kernel(const void* __restrict__ logits, int64_t ldl, int64_t V,
                                                           float* __restrict__ gval, int* __restrict__ gidx) {
  const int S = kGreedySlices;
  const int slice = blockIdx.x % S;
  const int row = blockIdx.x / S;
  const int64_t per = slice_len(V);
  const int64_t lo = min(V, slice * per), hi = min(V, lo + per);
  float best = -__builtin_inff();
  int64_t bi = V;
  span_argmax<BF16, VEC>(reinterpret_cast<const uint8_t*>(logits) + (int64_t)row * ldl * (BF16 ? 2 : 4), lo, hi,
                         best, bi);
  wave_argmax(best, bi);
  __shared__ float sv[4];
  __shared__ int si[4];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = best;
    si[w] = (int)bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = sv[0];
    int bidx = si[0];
    for (int i = 1; i < 4; ++i)
      if (sv[i] > bv || (sv[i] == bv && si[i] < bidx)) {
        bv = sv[i];
        bidx = si[i];
      }
    gval[blockIdx.x] = bv;
    gidx[blockIdx.x] = bidx;
  }
}

// The calling wave's merge of row r's kGreedySlices (= 64) partials, a lane per slice; 0 for a
// row of -inf / NaN.
__device__ inline int merge_row_argmax(const float* gval, const int* gidx, int r, int64_t V) {
  const int lane = threadIdx.x & 63;
  float bv = gval[r * kGreedySlices + lane];
  int64_t bidx = gidx[r * kGreedySlices + lane];
  wave_argmax(bv, bidx);
  return bidx >= V ? 0 : (int)bidx;
}

// Pass 2 of the greedy acceptance, one block per batch row b: per-position argmax tt (a wave
// per position), then the accept length n = matching draft prefix, the next token tt[n], and
// the rollback seq_lens[b] += n + 1.
__global__ __launch_bounds__(256) void accept_greedy_finish_kernel(int W, int64_t V, const int32_t* __restrict__ draft,
                                                                   int32_t* __restrict__ tt, int32_t* __restrict__ n_out,
                                                                   int32_t* __restrict__ token_out,
                                                                   int32_t* __restrict__ seq_lens, AcceptWs ws) {
  const int b = blockIdx.x;
  __shared__ int tts[256];
  for (int i = threadIdx.x >> 6; i < W; i += 4) {
    const int id = merge_row_argmax(ws.gval, ws.gidx, b * W + i, V);
    if ((threadIdx.x & 63) == 0) {
      tts[i] = id;
      if (tt) tt[b * W + i] = id;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int n = 0;
    while (n < W - 1 && draft[b * (W - 1) + n] == tts[n]) ++n;
    n_out[b] = n;
    token_out[b] = tts[n];
    if (seq_lens) seq_lens[b] += n + 1;
  }
}

// Pass 2 of a row-wise greedy pick: token_out[r] = merged argmax of row r (one wave per row).
__global__ __launch_bounds__(64) void argmax_merge_kernel(int64_t V, const float* __restrict__ gval,
                                                          const int* __restrict__ gidx, int32_t* __restrict__ token_out) {
  const int id = merge_row_argmax(gval, gidx, blockIdx.x, V);
  if (threadIdx.x == 0) token_out[blockIdx.x] = id;
}

// ----------------------------------------------------------------------------- sampled
struct SampleArgs {
  const float* p_logits;
  const float* q_logits;
  int64_t V;
  int B, L;
  const int32_t* draft;
  float T, top_p;
  int top_k, q_mul_inv_t;
  uint64_t seed;
  uint32_t offset;
  const uint32_t* offset_dev;  // when non-null, the Philox offset is read here (graph replays)
  int32_t* n_out;
  int32_t* token_out;
  int32_t* seq_lens;
  uint8_t* accept_out;
  int32_t* sample_out;
  AcceptWs ws;
};

__global__ __launch_bounds__(kNT) void accept_sample_kernel(SampleArgs a) {
  __shared__ RowSmem sm;
  __shared__ int last;
  const int R = a.L + 1;
  const uint32_t off = a.offset_dev ? a.offset_dev[0] : a.offset;
  const int b = blockIdx.x / R, i = blockIdx.x % R;
  const int64_t V = a.V;
  float* ps = a.ws.scratch + (size_t)blockIdx.x * 2 * V;
  float* qs = ps + V;
  const RowProbs pr =
      row_probs(a.p_logits + ((int64_t)b * R + i) * V, V, a.T, 0, a.top_p, a.top_k, ps, sm);
  int acc = 0;
  int64_t samp;
  if (i < a.L) {
    const int32_t d = a.draft[(int64_t)b * a.L + i];
    RowProbs qr;
    qr.trunc = 0;
    qr.cut = 0;
    qr.den = 1.0f;
    const bool onehot = (a.q_logits == nullptr);
    if (!onehot) qr = row_probs(a.q_logits + ((int64_t)b * a.L + i) * V, V, a.T, a.q_mul_inv_t, a.top_p, a.top_k, qs, sm);
    __syncthreads();
    // a draft id outside [0, V) is rejected (probability 0 under p)
    const bool dvalid = d >= 0 && (int64_t)d < V;
    const float pd = dvalid ? final_prob(pr, ps[d]) : 0.0f;
    const float qd = !dvalid ? 1.0f : (onehot ? 1.0f : final_prob(qr, qs[d]));
    const float u = u24_to_float(philox_word(a.seed, (uint32_t)i, (uint32_t)b, 0u, off));
    float ratio = pd / (qd > 1e-9f ? qd : 1e-9f);
    if (ratio > 1.0f) ratio = 1.0f;
    acc = u < ratio;
    auto resid = [&](int64_t j) -> float {
      float pj = final_prob(pr, ps[j]);
      float qj = onehot ? (j == d ? 1.0f : 0.0f) : final_prob(qr, qs[j]);
      float t = pj - qj;
      return t > 0.0f ? t : 0.0f;
    };
    uint64_t r = 0;
    for (int64_t j = threadIdx.x; j < V; j += kNT) r += fx(resid(j));
    const uint64_t Rs = block_sum_u64(r, sm);
    const float Rf = fx_to_float(Rs);
    const float den = Rf > 1e-9f ? Rf : 1e-9f;
    samp = block_categorical(V, philox_word(a.seed, (uint32_t)i, (uint32_t)b, 1u, off),
                             [&](int64_t j) { return resid(j) / den; }, sm);
  } else {
    samp = block_categorical(V, philox_word(a.seed, (uint32_t)i, (uint32_t)b, 1u, off),
                             [&](int64_t j) { return final_prob(pr, ps[j]); }, sm);
  }
  if (threadIdx.x == 0) {
    a.ws.acc[blockIdx.x] = acc;
    a.ws.samp[blockIdx.x] = (int)samp;
    __threadfence();
    int prev = atomicAdd(&a.ws.cnt[b], 1);
    last = (prev == R - 1);
  }
  __syncthreads();
  if (!last || threadIdx.x != 0) return;
  __threadfence();
  int n = 0, token = -1;
  bool done = false;
  for (int k = 0; k < R; ++k) {
    const int ak = __builtin_nontemporal_load(&a.ws.acc[b * R + k]);
    const int sk = __builtin_nontemporal_load(&a.ws.samp[b * R + k]);
    if (a.accept_out && k < a.L) a.accept_out[(int64_t)b * a.L + k] = (uint8_t)ak;
    if (a.sample_out) a.sample_out[(int64_t)b * R + k] = sk;
    if (!done) {
      if (k < a.L && ak) {
        ++n;
      } else {
        done = true;
        token = sk;
      }
    }
  }
  a.n_out[b] = n;
  a.token_out[b] = token;
  if (a.seq_lens) a.seq_lens[b] += n + 1;
  a.ws.cnt[b] = 0;
}

// ----------------------------------------------------------------------------- row sampling
__global__ __launch_bounds__(kNT) void sample_rows_kernel(const float* __restrict__ logits, int64_t V, float T,
                                                          float top_p, int top_k, int mul_inv, uint64_t seed,
                                                          uint32_t offset, const uint32_t* __restrict__ offset_dev,
                                                          int row0, int32_t* __restrict__ token_out,
                                                          float* __restrict__ probs) {
  __shared__ RowSmem sm;
  const int r = blockIdx.x;
  if (offset_dev) offset = offset_dev[0];
  const float* l = logits + (int64_t)r * V;
  if (T <= 0.0f) {
    float best = -__builtin_inff();
    int bi = 0x7fffffff;
    for (int64_t j = threadIdx.x; j < V; j += kNT)
      if (l[j] > best || (l[j] == best && j < bi)) {
        best = l[j];
        bi = (int)j;
      }
    for (int o = 32; o > 0; o >>= 1) {
      float ov = __shfl_xor(best, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      if (ov > best || (ov == best && oi < bi)) {
        best = ov;
        bi = oi;
      }
    }
    __shared__ float sv[kNW];
    __shared__ int si[kNW];
    if ((threadIdx.x & 63) == 0) {
      sv[threadIdx.x >> 6] = best;
      si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < kNW; ++w)
        if (sv[w] > sv[0] || (sv[w] == sv[0] && si[w] < si[0])) {
          sv[0] = sv[w];
          si[0] = si[w];
        }
      token_out[r] = si[0] >= V ? 0 : si[0];
    }
    return;
  }
  float* ps = probs + (int64_t)r * V;
  const RowProbs pr = row_probs(l, V, T, mul_inv, top_p, top_k, ps, sm);
  __syncthreads();
  const int64_t tok = block_categorical(V, philox_word(seed, (uint32_t)(row0 + r), 0u, 2u, offset),
                                        [&](int64_t j) { return final_prob(pr, ps[j]); }, sm);
  __syncthreads();
  if (pr.trunc)
    for (int64_t j = threadIdx.x; j < V; j += kNT) ps[j] = final_prob(pr, ps[j]);
  if (threadIdx.x == 0) token_out[r] = (int32_t)tok;
}

}  // namespace dsk

using namespace dsk;

// Pass 1 over `rows` rows of logits into ws.gval / ws.gidx; 16-byte chunk loads when every row
// starts 16-byte aligned.
static void launch_slice_argmax(const void* logits, int dtype, int64_t ldl, int64_t V, int rows, const AcceptWs& ws,
                                hipStream_t st) {
  const int64_t esz = dtype == DSK_BF16 ? 2 : 4;
  const bool vec = ((uintptr_t)logits & 15) == 0 && (ldl * esz) % 16 == 0;
  const dim3 grid((unsigned)(rows * kGreedySlices)), blk(256);
  if (dtype == DSK_BF16) {
    if (vec) hipLaunchKernelGGL((slice_argmax_kernel<1, true>), grid, blk, 0, st, logits, ldl, V, ws.gval, ws.gidx);
    else hipLaunchKernelGGL((slice_argmax_kernel<1, false>), grid, blk, 0, st, logits, ldl, V, ws.gval, ws.gidx);
  } else {
    if (vec) hipLaunchKernelGGL((slice_argmax_kernel<0, true>), grid, blk, 0, st, logits, ldl, V, ws.gval, ws.gidx);
    else hipLaunchKernelGGL((slice_argmax_kernel<0, false>), grid, blk, 0, st, logits, ldl, V, ws.gval, ws.gidx);
  }
}

extern "C" size_t dsk_accept_ws_bytes(int B, int W, int64_t V) {
  if (B <= 0 || W <= 0 || V <= 0) return 0;
  return accept_ws_total(B, W, V);
}

extern "C" int dsk_accept_ws_init(void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(workspace && ws_bytes >= kAcceptCounterBytes, "dsk_accept_ws_init: workspace too small");
  hipError_t e = hipMemsetAsync(workspace, 0, kAcceptCounterBytes, as_stream(stream));
  if (e != hipSuccess) {
    set_error("dsk_accept_ws_init: %s", hipGetErrorString(e));
    return DSK_ELAUNCH;
  }
  return DSK_OK;
}

extern "C" int dsk_accept_greedy(const void* logits, int dtype, int64_t ldl, int B, int W, int64_t V,
                                 const int32_t* draft, int32_t* tt, int32_t* n_out, int32_t* token_out,
                                 int32_t* seq_lens, void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(logits && n_out && token_out && workspace, "dsk_accept_greedy: null pointer");
  DSK_REQUIRE(W == 1 || draft, "dsk_accept_greedy: draft is null");
  DSK_REQUIRE(B > 0 && B <= 1024 && W > 0 && W <= 256 && V > 0 && V < (1ll << 31),
              "dsk_accept_greedy: bad shape B=%d W=%d V=%lld", B, W, (long long)V);
  DSK_REQUIRE(ldl >= V, "dsk_accept_greedy: ldl < V");
  DSK_REQUIRE(dtype == DSK_F32 || dtype == DSK_BF16, "dsk_accept_greedy: dtype must be f32 or bf16");
  DSK_REQUIRE(ws_bytes >= accept_ws_total(B, W, V) - (size_t)B * W * 2 * V * 4,
              "dsk_accept_greedy: workspace too small");
  AcceptWs ws = accept_ws(workspace, B, W, V);
  const hipStream_t st = as_stream(stream);
  launch_slice_argmax(logits, dtype, ldl, V, B * W, ws, st);
  hipLaunchKernelGGL(accept_greedy_finish_kernel, dim3((unsigned)B), dim3(256), 0, st, W, V, draft, tt, n_out,
                     token_out, seq_lens, ws);
  DSK_LAUNCH_CHECK("dsk_accept_greedy");
  return DSK_OK;
}

// ----------------------------------------------------------------------------- no-allocation greedy
// dsk_accept_greedy_static: the greedy acceptance with its slice partials in a file-scope device
// array instead of a caller workspace, for callers that cannot allocate. Each device holds its
// own copy of `scratch`; its address on the current device is looked up once (the array's host
// name is only a stand-in: a kernel given it would fault) and cached per device. Every call on a
// device shares that device's array, so calls that overlap on one GPU race. The slice pass
// writes every partial the merge reads, so nothing needs clearing between calls.
constexpr int kStaticRows = 1024;
constexpr size_t kStaticSliceBytes = (size_t)kStaticRows * kGreedySlices * 4;
static __device__ __align__(256) uint8_t scratch[2 * kStaticSliceBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices];

static int static_scratch(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("%s: hipGetDevice: %s", who, hipGetErrorString(e));
    return DSK_ELAUNCH;
  }
  DSK_REQUIRE(dev >= 0 && dev < kMaxDevices, "%s: device %d beyond %d", who, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("%s: hipGetSymbolAddress(scratch): %s", who, hipGetErrorString(e));
      return DSK_ELAUNCH;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return DSK_OK;
}

extern "C" int dsk_accept_greedy_static(const void* logits, int dtype, int64_t ldl, int B, int W, int64_t V,
                                        const int32_t* draft, int32_t* tt, int32_t* n_out, int32_t* token_out,
                                        int32_t* seq_lens, dsk_stream_t stream) {
  DSK_REQUIRE(logits && n_out && token_out, "dsk_accept_greedy_static: null pointer");
  DSK_REQUIRE(W == 1 || draft, "dsk_accept_greedy_static: draft is null");
  DSK_REQUIRE(B > 0 && W > 0 && W <= 256 && V > 0 && V < (1ll << 31),
              "dsk_accept_greedy_static: bad shape B=%d W=%d V=%lld", B, W, (long long)V);
  DSK_REQUIRE(ldl >= V, "dsk_accept_greedy_static: ldl < V");
  DSK_REQUIRE(dtype == DSK_F32 || dtype == DSK_BF16, "dsk_accept_greedy_static: dtype must be f32 or bf16");
  if ((int64_t)B * W > kStaticRows) {
    set_error("dsk_accept_greedy_static: B*W = %lld rows beyond the static scratch maximum of %d",
              (long long)B * W, kStaticRows);
    return DSK_ERANGE;
  }
  void* base = nullptr;
  const int rc = static_scratch(&base, "dsk_accept_greedy_static");
  if (rc != DSK_OK) return rc;
  AcceptWs ws{};
  ws.gval = reinterpret_cast<float*>(base);
  ws.gidx = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(base) + kStaticSliceBytes);
  const hipStream_t st = as_stream(stream);
  launch_slice_argmax(logits, dtype, ldl, V, B * W, ws, st);
  hipLaunchKernelGGL(accept_greedy_finish_kernel, dim3((unsigned)B), dim3(256), 0, st, W, V, draft, tt, n_out,
                     token_out, seq_lens, ws);
  DSK_LAUNCH_CHECK("dsk_accept_greedy_static");
  return DSK_OK;
}

extern "C" size_t dsk_argmax_ws_bytes(int R) {
  if (R <= 0 || R > 1024) return 0;
  return kAcceptCounterBytes + 2 * align256((size_t)R * kGreedySlices * 4);
}

extern "C" int dsk_argmax_rows(const void* logits, int dtype, int64_t ldl, int64_t V, int R, int32_t* token_out,
                               void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(logits && token_out && workspace, "dsk_argmax_rows: null pointer");
  DSK_REQUIRE(R > 0 && R <= 1024 && V > 0 && V < (1ll << 31), "dsk_argmax_rows: bad shape R=%d V=%lld", R,
              (long long)V);
  DSK_REQUIRE(ldl >= V, "dsk_argmax_rows: ldl < V");
  DSK_REQUIRE(dtype == DSK_F32 || dtype == DSK_BF16, "dsk_argmax_rows: dtype must be f32 or bf16");
  DSK_REQUIRE(ws_bytes >= dsk_argmax_ws_bytes(R), "dsk_argmax_rows: workspace %zu < %zu", ws_bytes,
              dsk_argmax_ws_bytes(R));
  AcceptWs ws = accept_ws(workspace, R, 1, V);
  const hipStream_t st = as_stream(stream);
  launch_slice_argmax(logits, dtype, ldl, V, R, ws, st);
  hipLaunchKernelGGL(argmax_merge_kernel, dim3((unsigned)R), dim3(64), 0, st, V, ws.gval, ws.gidx, token_out);
  DSK_LAUNCH_CHECK("dsk_argmax_rows");
  return DSK_OK;
}

extern "C" int dsk_accept_sample(const float* p_logits, const float* q_logits, int64_t V, int B, int L,
                                 const int32_t* draft, float temperature, float top_p, int top_k, int q_mul_inv_t,
                                 uint64_t seed, uint32_t offset, int32_t* n_out, int32_t* token_out,
                                 int32_t* seq_lens, uint8_t* accept_out, int32_t* sample_out, void* workspace,
                                 size_t ws_bytes, const uint32_t* offset_dev, dsk_stream_t stream) {
  DSK_REQUIRE(p_logits && n_out && token_out && workspace, "dsk_accept_sample: null pointer");
  DSK_REQUIRE(L == 0 || draft, "dsk_accept_sample: draft is null");
  DSK_REQUIRE(B > 0 && B <= 1024 && L >= 0 && L < 255 && V > 0 && V < (1ll << 31),
              "dsk_accept_sample: bad shape B=%d L=%d V=%lld", B, L, (long long)V);
  DSK_REQUIRE(temperature > 0.0f, "dsk_accept_sample: temperature must be > 0");
  DSK_REQUIRE(ws_bytes >= accept_ws_total(B, L + 1, V), "dsk_accept_sample: workspace %zu < %zu", ws_bytes,
              accept_ws_total(B, L + 1, V));
  SampleArgs a;
  a.p_logits = p_logits;
  a.q_logits = q_logits;
  a.V = V;
  a.B = B;
  a.L = L;
  a.draft = draft;
  a.T = temperature;
  a.top_p = top_p;
  a.top_k = top_k;
  a.q_mul_inv_t = q_mul_inv_t;
  a.seed = seed;
  a.offset = offset;
  a.offset_dev = offset_dev;
  a.n_out = n_out;
  a.token_out = token_out;
  a.seq_lens = seq_lens;
  a.accept_out = accept_out;
  a.sample_out = sample_out;
  a.ws = accept_ws(workspace, B, L + 1, V);
  hipLaunchKernelGGL(accept_sample_kernel, dim3((unsigned)(B * (L + 1))), dim3(kNT), 0, as_stream(stream), a);
  DSK_LAUNCH_CHECK("dsk_accept_sample");
  return DSK_OK;
}

extern "C" int dsk_sample_rows(const float* logits, int64_t V, int R, float temperature, float top_p, int top_k,
                               int mul_inv_t, uint64_t seed, uint32_t offset, int row0, int32_t* token_out,
                               float* probs_out, const uint32_t* offset_dev, dsk_stream_t stream) {
  DSK_REQUIRE(logits && token_out, "dsk_sample_rows: null pointer");
  DSK_REQUIRE(R > 0 && V > 0 && V < (1ll << 31), "dsk_sample_rows: bad shape");
  DSK_REQUIRE(temperature <= 0.0f || probs_out, "dsk_sample_rows: probs_out is required when temperature > 0");
  hipLaunchKernelGGL(sample_rows_kernel, dim3((unsigned)R), dim3(kNT), 0, as_stream(stream), logits, V, temperature,
                     top_p, top_k, mul_inv_t, seed, offset, offset_dev, row0, token_out, probs_out);
  DSK_LAUNCH_CHECK("dsk_sample_rows");
  return DSK_OK;
}
