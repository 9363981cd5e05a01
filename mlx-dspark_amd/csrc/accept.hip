// Fused acceptance on gfx950: greedy argmax-compare and speculative-sampling acceptance
// (min(1, p/q) with residual resampling) after temperature / top-k / top-p, plus the KV
// rollback to the accepted length. One canonical arithmetic is shared with the CPU oracle
// (oracle/accept_oracle.c) so decisions, sampled indices and rollback lengths are identical:
//   - exp: dsk_expf_le0 (Cody-Waite reduction by ln 2 with a two-word constant, Taylor
//     polynomial to r^7 evaluated with explicit fmaf, inputs below -86 flush to zero);
//   - a row's distribution lives on the unnormalised exponentials e_j = exp(y_j - max y)
//     with fixed-point masses w_j = fx(e_j) = floor(e_j * 2^31) (integer sums: order-free);
//   - top-k keeps e_j >= the k-th largest e; top-p keeps e_j >= the largest value c whose
//     mass at or above it reaches TP = ceil(top_p * Z); both keep e_j >= max of the two
//     thresholds (the reference's top-k followed by top-p on the zeroed values); the final
//     probability of a kept element is e_j / float(S * 2^-31), S the kept mass;
//   - uniforms: Philox4x32-10 word 0, u = (w >> 8) * 2^-24;
//   - categorical draws: inverse CDF over fixed-point masses, in index order.
// Floating-point contraction is off in this file: every fma is written out.
//
// The sampled paths split every row over many workgroups and run as a chain of kernels with
// no fences or last-arriver counters (each kernel boundary is the only synchronisation):
//   1 row max per slice;
//   2 Z and a 512-bucket histogram of e's float key (count and mass per bucket), merged per
//     row with integer atomics (exact in any order);
//   3 (truncation only) the threshold buckets from the merged histogram, then every element
//     of those buckets gathered as a candidate key;
//   4 per row (a verify position: its target and draft rows): the exact thresholds by a radix
//     select over the candidates, the kept mass S, and the accept test of the drafted token;
//   5 per slice: the mass of the distribution each draw uses (residual at the first rejected
//     position, or the bonus / row distribution);
//   6 per draw: the slice holding the uniform's mass, then the element inside it.
#pragma clang fp contract(off)

#include <algorithm>
#include <mutex>

#include "common.h"

namespace dsk {

// ----------------------------------------------------------------------------- math
// exp on x <= 0 (and NaN), the only arguments used here (x = y - max y), without branches:
// Cody-Waite reduction by ln 2 with a two-word constant, Taylor polynomial to r^7 with explicit
// fmaf, arguments below -86 flush to 0 (the polynomial runs on the clamped argument, so the
// scale factor 2^k stays a normal number); the oracle's oracle_expf on the same inputs.
__device__ __forceinline__ float dsk_expf_le0(float x) {
  const bool under = x < -86.0f;
  const float xc = under ? -86.0f : x;
  float t = xc * 1.44269504f;
  float k = rintf(t);
  float r = __builtin_fmaf(-k, 0.693145751953125f, xc);
  r = __builtin_fmaf(-k, 1.428606765330187e-06f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float v = ldexpf(p, (int)k);  // k in [-124, 0]: p * 2^k exactly, as a multiply by 2^k
  return under ? 0.0f : v;
}

// p in [0, 1] (every mass here: e, p' and residuals are at most 1): p * 2^31 fits a u32 and the
// conversion truncates, i.e. floors
__device__ __forceinline__ uint64_t fx(float p) { return (uint64_t)(uint32_t)(p * 0x1p31f); }
__device__ __forceinline__ float fx_to_float(uint64_t s) { return (float)((double)s * 0x1p-31); }

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

// TP = ceil(top_p * Z) exactly: top_p = M * 2^E with an integer M < 2^24, the product an integer
// below 2^87, the ceiling a shift of a 128-bit sum. top_p <= 0 gives 0 (an empty nucleus).
__device__ inline uint64_t top_p_target(float top_p, uint64_t Z) {
  if (!(top_p > 0.0f)) return 0;
  const uint32_t bits = f32_bits(top_p);
  const uint32_t ex = (bits >> 23) & 0xFFu;
  uint64_t M = bits & 0x7FFFFFu;
  int E;
  if (ex == 0) {
    E = -149;
  } else {
    M |= 0x800000u;
    E = (int)ex - 150;
  }
  const unsigned __int128 P = (unsigned __int128)M * Z;
  if (E >= 0) return (uint64_t)(P << E);
  const int sh = -E;
  if (sh >= 128) return P ? 1 : 0;
  return (uint64_t)((P + (((unsigned __int128)1 << sh) - 1)) >> sh);
}

// ----------------------------------------------------------------------------- wave helpers
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

// ----------------------------------------------------------------------------- greedy workspace
constexpr int kGreedySlices = 64;  // slices per row: one per lane of the merging wave

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct GreedyWs {
  float* gval;  // [rows * kGreedySlices] slice maxima
  int* gidx;    // [rows * kGreedySlices] their indices
};

__host__ inline size_t greedy_ws_bytes(size_t rows) { return 2 * align256(rows * kGreedySlices * 4); }

__host__ inline GreedyWs greedy_ws(void* base, size_t rows) {
  GreedyWs ws;
  ws.gval = reinterpret_cast<float*>(base);
  ws.gidx = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(base) + align256(rows * kGreedySlices * 4));
  return ws;
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
      for (int u = 0; u < UN; ++u)  // all in flight: a chunk past nv reads chunk c0 (skipped below)
        v[u] = __builtin_nontemporal_load(p + (c0 + u * 256 < nv ? c0 + u * 256 : c0));
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
                                                                   int32_t* __restrict__ seq_lens, GreedyWs ws) {
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

// ============================================================================= sampled paths
constexpr int kST = 512;              // threads per workgroup
constexpr int kSW = kST / 64;
constexpr int kMaxSlices = 32;        // workgroups per row in the row passes
constexpr int kEPT = 32;              // elements per thread in the gather pass: slice <= 16384
constexpr int kMaxDrawSlices = 128;   // workgroups per draw in the draw passes (<= kST)
constexpr int kDrawEPT = 8;           // elements per thread in the draw pass: draw slice <= 4096
constexpr int kHistCopies = 8;        // lane-striped copies of the stats pass's LDS histogram
                                      // (rows whose probabilities fill few buckets: 2 copies took
                                      // the T = 0.6, top-k 20 stats pass from 15.8 to 39.0 us)
constexpr int kFinCap = 10240;        // candidate keys the finishing pass stages in LDS
constexpr int64_t kMaxSlice = (int64_t)kST * kEPT;
constexpr int kL1 = 512;              // first-level buckets: key >> 21 (e <= 1 keeps it <= 508)
constexpr int kL1Shift = 21;
constexpr uint32_t kNone = 0xFFFFFFFFu;
static_assert(kST == kL1, "the merged-histogram scan gives each thread one first-level bucket");

struct RowInfo {        // the threshold buckets of one row (selection pass)
  uint32_t bk, bp;      // top-k bucket (by count), top-p bucket (by mass); kNone when inactive
  uint32_t above_k;     // elements in buckets above bk
  uint32_t pad;
  uint64_t wabove_k;    // mass in buckets above bk
  uint64_t wabove_p;    // mass in buckets above bp
  uint64_t tp;          // ceil(top_p * Z)
  float wlo, whi;       // window of x = y - m holding both buckets' elements
  float vlo, vhi;       // the same window on raw values (used when T == 1)
};

struct RowParam {       // one row's final distribution: p'_j = key(e_j) >= thr ? e_j / sf : 0
  float m;              // max of y over the row
  uint32_t thr;         // 0 keeps every element, kNone keeps none
  float sf;             // float(S * 2^-31), S the kept mass
  uint32_t pad;
};

struct SampArgs {
  // rows: p rows [0, Rp), then q rows [Rp, Rp + Rq), each V floats
  const float* p;
  const float* q;
  int64_t V;
  int Rp, Rq;
  int S;                // slices per row (row passes)
  int64_t slen;         // slice length (multiple of 4)
  int Sd;               // slices per draw (draw passes)
  int64_t slen_d;       // draw slice length (multiple of 4, at most kST * kDrawEPT)
  float T, top_p;
  int top_k, p_mul, q_mul;
  int do_k, do_p;
  int vec;              // rows 16-byte aligned, V % 4 == 0: float4 loads
  // acceptance (mode 0): positions (b, i), i <= L; p row b*(L+1)+i, q row Rp + b*L + i
  int mode;             // 0 acceptance, 1 row sampling
  int B, L;
  int all_pos;          // draw at every position (sample_out requested)
  const int32_t* draft;
  uint64_t seed;
  uint32_t offset;
  const uint32_t* offset_dev;
  int32_t* n_out;
  int32_t* token_out;
  int32_t* seq_lens;
  uint8_t* accept_out;
  int32_t* sample_out;
  // row sampling (mode 1): row r draws with Philox row row0 + r
  int row0;
  int32_t* tok_rows;
  float* probs_out;
  // workspace
  float* gmax;          // [rows][kMaxSlices]
  uint64_t* zsum;       // [rows]
  uint32_t* hcnt;       // [rows][kL1]
  uint64_t* hwgt;       // [rows][kL1]
  uint32_t* ccnt;       // [rows][2] candidate counts (top-k list from the front, top-p from the back)
  RowInfo* info;        // [rows]
  RowParam* prm;        // [rows]
  int32_t* acc;         // [B][L] accept flags
  uint64_t* wsum;       // [draws][kMaxDrawSlices]
  uint32_t* cand;       // [rows][V]
};

__device__ __forceinline__ const float* samp_row(const SampArgs& a, int r) {
  return r < a.Rp ? a.p + (int64_t)r * a.V : a.q + (int64_t)(r - a.Rp) * a.V;
}
__device__ __forceinline__ int samp_mul(const SampArgs& a, int r) { return r < a.Rp ? a.p_mul : a.q_mul; }
__device__ __forceinline__ float yval(float x, int mul, float T, float inv_t) {
  if (T == 1.0f) return x;  // x / 1 == x * (1 / 1) == x exactly
  return mul ? x * inv_t : x / T;
}
// the row passes are instantiated for T == 1 (TONE: y = x) and for any T
template <bool TONE>
__device__ __forceinline__ float yv(float x, int mul, float T, float inv_t) {
  if constexpr (TONE) return x;
  else return mul ? x * inv_t : x / T;
}
__device__ __forceinline__ uint32_t samp_offset(const SampArgs& a) { return a.offset_dev ? a.offset_dev[0] : a.offset; }

__device__ __forceinline__ float row_max(const SampArgs& a, int r) {
  float m = a.gmax[r * kMaxSlices];
  for (int s = 1; s < a.S; ++s) m = fmaxf(m, a.gmax[r * kMaxSlices + s]);
  return m;
}

// final probability of element j of a row with parameters rp
__device__ __forceinline__ float final_prob(const RowParam& rp, float x, int mul, float T, float inv_t) {
  const float e = dsk_expf_le0(yval(x, mul, T, inv_t) - rp.m);
  return f32_bits(e) >= rp.thr && rp.thr != kNone ? e / rp.sf : 0.0f;
}

// A thread's share of a row slice [lo, hi) (at most kST * kEPT elements), loaded into registers
// with every load issued at once: VEC (16-byte aligned rows, lo and hi multiples of 4) as float4
// c = tid + i * kST, else element j = lo + tid + i * kST.
template <bool VEC>
struct SliceRegs {
  float v[kEPT];
  // Every load is issued without a branch, so all of them are in flight together: an index
  // past the slice reads the slice's first element instead, and every user masks such
  // elements with valid().
  __device__ __forceinline__ void load(const float* __restrict__ x, int64_t lo, int64_t hi) {
    const int n = (int)(hi - lo);
    if (n <= 0) {
#pragma unroll
      for (int k = 0; k < kEPT; ++k) v[k] = 0.0f;
      return;
    }
    if constexpr (VEC) {
      const f32x4* x4 = reinterpret_cast<const f32x4*>(x + lo);
#pragma unroll
      for (int i = 0; i < kEPT / 4; ++i) {
        const int c = i * kST + (int)threadIdx.x;
        const f32x4 t = x4[4 * c < n ? c : 0];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * i + e] = t[e];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kEPT; ++i) {
        const int j = i * kST + (int)threadIdx.x;
        v[i] = x[lo + (j < n ? j : 0)];
      }
    }
  }
  // element k of this thread lies in the slice (n = hi - lo; a float4 is whole or absent)
  __device__ __forceinline__ static bool valid(int k, int n) {
    if constexpr (VEC) return 4 * ((k / 4) * kST + (int)threadIdx.x) < n;
    else return k * kST + (int)threadIdx.x < n;
  }
};

__device__ float block_max512(float v, float* sh) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  float t = sh[0];
#pragma unroll
  for (int i = 1; i < kSW; ++i) t = fmaxf(t, sh[i]);
  return t;
}

__device__ uint64_t block_sum512(uint64_t v, uint64_t* sh) {
  v = wave_sum_u64(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int i = 0; i < kSW; ++i) t += sh[i];
  return t;
}

// inclusive block scan in thread order; total receives the block sum
__device__ uint64_t block_scan512(uint64_t v, uint64_t* sh, uint64_t& total) {
  const uint64_t incl = wave_incl_scan_u64(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 63) sh[w] = incl;
  __syncthreads();
  uint64_t before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kSW; ++i) {
    if (i < w) before += sh[i];
    tot += sh[i];
  }
  total = tot;
  return before + incl;
}

// ---- pass 1: slice maxima of y; slice 0 clears the row's merged accumulators
template <bool VEC, bool TONE>
__global__ __launch_bounds__(kST) void samp_max_kernel(SampArgs a) {
  __shared__ float sh[kSW];
  const int r = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const float* x = samp_row(a, r);
  const int mul = samp_mul(a, r);
  const float T = a.T, inv_t = 1.0f / T;
  const int64_t lo = min(a.V, (int64_t)s * a.slen), hi = min(a.V, lo + a.slen);
  SliceRegs<VEC> xr;
  xr.load(x, lo, hi);
  float m = -__builtin_inff();
  const int n = (int)(hi - lo);
#pragma unroll
  for (int k = 0; k < kEPT; ++k)
    if (xr.valid(k, n)) m = fmaxf(m, yv<TONE>(xr.v[k], mul, T, inv_t));
  m = block_max512(m, sh);
  if (threadIdx.x == 0) a.gmax[r * kMaxSlices + s] = m;
  if (s == 0) {
    if (threadIdx.x == 0) a.zsum[r] = 0;
    if (a.do_k || a.do_p) {
      for (int b = threadIdx.x; b < kL1; b += kST) {
        a.hcnt[r * kL1 + b] = 0;
        a.hwgt[r * kL1 + b] = 0;
      }
      if (threadIdx.x < 2) a.ccnt[r * 2 + threadIdx.x] = 0;
    }
  }
}

// ---- pass 2: Z and the first-level histogram, merged per row by integer atomics. Lanes
// spread their LDS atomics over kHistCopies copies (copy = lane % kHistCopies) so lanes of one
// wave that hit the same bucket mostly hit different addresses.
template <bool VEC, bool TONE>
__global__ __launch_bounds__(kST) void samp_stats_kernel(SampArgs a) {
  __shared__ uint32_t hc[kHistCopies][kL1 + 1];  // +1: copies start in different LDS banks
  __shared__ unsigned long long hw[kHistCopies][kL1 + 1];
  __shared__ uint64_t sh[kSW];
  const int r = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const bool trunc = a.do_k || a.do_p;
  const float* x = samp_row(a, r);
  const int mul = samp_mul(a, r);
  const float T = a.T, inv_t = 1.0f / T;
  const int64_t lo = min(a.V, (int64_t)s * a.slen), hi = min(a.V, lo + a.slen);
  SliceRegs<VEC> xr;
  xr.load(x, lo, hi);  // in flight while the row max is read and the histogram cleared
  const float m = row_max(a, r);
  uint32_t* hcp = hc[threadIdx.x % kHistCopies];
  unsigned long long* hwp = hw[threadIdx.x % kHistCopies];
  if (trunc) {
    for (int b = threadIdx.x; b < kHistCopies * (kL1 + 1); b += kST) {
      hc[b / (kL1 + 1)][b % (kL1 + 1)] = 0;
      hw[b / (kL1 + 1)][b % (kL1 + 1)] = 0;
    }
    __syncthreads();
  }
  uint64_t z = 0;
  const int n = (int)(hi - lo);
  // element by element (uniform branches on the histogram flags keep few registers live: three
  // workgroups per CU, which the histogram copies' LDS allows)
#pragma unroll
  for (int k = 0; k < kEPT; ++k) {
    if (!xr.valid(k, n)) continue;
    const float e = dsk_expf_le0(yv<TONE>(xr.v[k], mul, T, inv_t) - m);
    const uint64_t w = fx(e);
    z += w;
    if (trunc) {
      const uint32_t b = min(f32_bits(e) >> kL1Shift, (uint32_t)kL1 - 1);  // NaN stays in bounds
      if (a.do_k) atomicAdd(hcp + b, 1u);
      if (w) atomicAdd(hwp + b, (unsigned long long)w);  // zero masses pile up in the low buckets
    }
  }
  z = block_sum512(z, sh);
  if (threadIdx.x == 0) atomicAdd((unsigned long long*)&a.zsum[r], (unsigned long long)z);
  if (trunc) {
    __syncthreads();
    for (int b = threadIdx.x; b < kL1; b += kST) {
      uint32_t c = 0;
      unsigned long long w = 0;
#pragma unroll
      for (int k = 0; k < kHistCopies; ++k) {
        c += hc[k][b];
        w += hw[k][b];
      }
      if (c) atomicAdd(&a.hcnt[r * kL1 + b], c);
      if (w) atomicAdd((unsigned long long*)&a.hwgt[r * kL1 + b], w);
    }
  }
}

// A window of x = y - m that holds every element whose e lands in first-level bucket b (empty
// for kNone): exp here is within 2 ulp of the true exp (a CPU test of the oracle's copy checks
// this), so a 1e-3 margin on the logarithms of the bucket's bounds is far wider than needed.
// The lowest buckets (e below 2^-122, where the flush to 0 lives) keep no upper bound.
__device__ inline void bucket_window(uint32_t b, float& lo, float& hi) {
  if (b == kNone) {
    lo = __builtin_inff();
    hi = -__builtin_inff();
    return;
  }
  lo = b == 0 ? -__builtin_inff() : logf(bits_f32(b << kL1Shift)) - 1e-3f;
  hi = b <= 8 ? __builtin_inff() : logf(bits_f32((b + 1) << kL1Shift)) + 1e-3f;
}

// ---- pass 3a (truncation), one workgroup per row: the threshold buckets from the merged
// histogram (buckets scanned in descending order, thread t holding bucket kL1 - 1 - t), the
// mass and count above them, and the window of x = y - m the gather stages.
__global__ __launch_bounds__(kST) void samp_select_kernel(SampArgs a) {
  __shared__ uint64_t sh[kSW];
  __shared__ uint32_t sel[4];
  __shared__ uint64_t selw[2];
  const int r = blockIdx.x;
  const uint64_t Z = a.zsum[r];
  const uint64_t TP = a.do_p ? top_p_target(a.top_p, Z) : 0;
  const int bb = kL1 - 1 - (int)threadIdx.x;
  const uint64_t c = a.hcnt[r * kL1 + bb];
  const uint64_t w = a.hwgt[r * kL1 + bb];
  if (threadIdx.x == 0) {
    sel[0] = kNone;
    sel[1] = kNone;
  }
  uint64_t tot;
  const uint64_t ic = block_scan512(c, sh, tot);
  const uint64_t iw = block_scan512(w, sh, tot);
  if (a.do_k && ic - c < (uint64_t)a.top_k && ic >= (uint64_t)a.top_k) {
    sel[0] = (uint32_t)bb;
    sel[2] = (uint32_t)(ic - c);
    selw[0] = iw - w;
  }
  if (a.do_p && TP > 0 && iw - w < TP && iw >= TP) {
    sel[1] = (uint32_t)bb;
    selw[1] = iw - w;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  RowInfo inf;
  inf.bk = sel[0];
  inf.bp = sel[1];
  inf.above_k = inf.bk == kNone ? 0 : sel[2];
  inf.pad = 0;
  inf.wabove_k = inf.bk == kNone ? 0 : selw[0];
  inf.wabove_p = inf.bp == kNone ? 0 : selw[1];
  inf.tp = TP;
  const uint32_t bq = (inf.bp == inf.bk) ? kNone : inf.bp;
  float klo, khi, qlo, qhi;
  bucket_window(inf.bk, klo, khi);
  bucket_window(bq, qlo, qhi);
  inf.wlo = fminf(klo, qlo);
  inf.whi = fmaxf(khi, qhi);
  // with T == 1 the window moves to the raw values (y = v): v - m in [wlo, whi] holds for every
  // v in [m + wlo, m + whi] widened by one part in 2^20 of the bounds' magnitudes
  const float m = row_max(a, r);
  inf.vlo = (m + inf.wlo) - fabsf(m + inf.wlo) * 0x1p-20f - 0x1p-100f;
  inf.vhi = (m + inf.whi) + fabsf(m + inf.whi) * 0x1p-20f + 0x1p-100f;
  a.info[r] = inf;
}

// ---- pass 3b (truncation): the candidates of the threshold buckets. A cheap window test
// stages each wave's window elements in LDS by ballot; the exact keys of the staged elements are
// then computed densely, so exp never runs divergently.
template <bool VEC, bool TONE>
__global__ __launch_bounds__(kST) void samp_gather_kernel(SampArgs a) {
  __shared__ uint64_t sh[kSW];
  __shared__ uint32_t base[2];
  __shared__ uint32_t xs[kSW][64 * kEPT];  // per wave: staged x bits, then their keys
  const int r = blockIdx.x / a.S, s = blockIdx.x % a.S;
  const float* x = samp_row(a, r);
  const int mul = samp_mul(a, r);
  const float T = a.T, inv_t = 1.0f / T;
  const int64_t lo = min(a.V, (int64_t)s * a.slen), hi = min(a.V, lo + a.slen);
  const int n = (int)(hi - lo);
  SliceRegs<VEC> xr;
  xr.load(x, lo, hi);
  const RowInfo inf = a.info[r];
  const float m = row_max(a, r);
  const uint32_t bk = inf.bk, bq = (inf.bp == inf.bk) ? kNone : inf.bp;
  if (bk == kNone && bq == kNone) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t* xw = xs[wv];
  uint32_t cnt = 0;  // elements this wave staged (wave-uniform)
#pragma unroll
  for (int k = 0; k < kEPT; ++k) {  // every lane of the wave takes part in each ballot
    const float v = xr.v[k];
    bool inw;
    if constexpr (TONE) inw = v >= inf.vlo && v <= inf.vhi;
    else {
      const float xx = yv<TONE>(v, mul, T, inv_t) - m;
      inw = xx >= inf.wlo && xx <= inf.whi;
    }
    inw = inw && xr.valid(k, n);
    const uint64_t bal = __ballot(inw);
    if (bal) {
      if (inw) xw[cnt + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u))] =
          f32_bits(yv<TONE>(v, mul, T, inv_t) - m);
      cnt += (uint32_t)__popcll(bal);
    }
  }
  // exact keys of the staged elements (a wave reads only its own staging area)
  __syncthreads();
  uint32_t nk = 0, np = 0;
  for (uint32_t k = lane; k < cnt; k += 64) {
    const uint32_t key = f32_bits(dsk_expf_le0(bits_f32(xw[k])));
    const uint32_t b = key >> kL1Shift;
    const uint32_t kept = (b == bk || b == bq) ? key : kNone;
    xw[k] = kept;
    nk += (kept != kNone && b == bk);
    np += (kept != kNone && b == bq);
  }
  uint64_t totk, totp;
  const uint64_t offk = block_scan512(nk, sh, totk) - nk;
  const uint64_t offp = block_scan512(np, sh, totp) - np;
  if (threadIdx.x == 0) {
    base[0] = totk ? atomicAdd(&a.ccnt[r * 2], (uint32_t)totk) : 0;
    base[1] = totp ? atomicAdd(&a.ccnt[r * 2 + 1], (uint32_t)totp) : 0;
  }
  __syncthreads();
  uint32_t* ck = a.cand + (int64_t)r * a.V;
  uint32_t pk = base[0] + (uint32_t)offk, pp = base[1] + (uint32_t)offp;
  for (uint32_t k = lane; k < cnt; k += 64) {
    const uint32_t key = xw[k];
    if (key == kNone) continue;
    if ((key >> kL1Shift) == bk) ck[pk++] = key;
    else ck[a.V - 1 - (pp++)] = key;
  }
}

// ---- pass 4: per row, the exact thresholds from the candidates and the kept mass
struct FinSmem {
  unsigned long long hist[2048];
  uint32_t keys[kFinCap];
  uint64_t sh[kSW];
  uint32_t bc32;
  uint64_t bc64;
};

// Key K among the n candidate keys (all in first-level bucket `bucket`) with
// weight(> K) < target <= weight(>= K), weight 1 per key (count) or fx(value) (mass); two
// radix levels over the key's low 21 bits (11 then 10 bits).
__device__ uint32_t select_key(const uint32_t* cand, uint32_t n, bool mass, uint64_t target, uint32_t bucket,
                               FinSmem& sm) {
  uint32_t prefix = bucket << kL1Shift;
  uint64_t above = 0;
  const int shifts[2] = {10, 0};
  const int widths[2] = {11, 10};
  for (int lv = 0; lv < 2; ++lv) {
    const int sh = shifts[lv], nb = 1 << widths[lv];
    __syncthreads();
    for (int i = threadIdx.x; i < nb; i += kST) sm.hist[i] = 0;
    if (threadIdx.x == 0) sm.bc32 = kNone;
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < n; c += kST) {
      const uint32_t key = cand[c];
      if (lv == 1 && (key >> 10) != (prefix >> 10)) continue;
      const uint64_t w = mass ? fx(bits_f32(key)) : 1;
      if (w) atomicAdd(&sm.hist[(key >> sh) & (nb - 1)], (unsigned long long)w);
    }
    __syncthreads();
    // descending scan: thread t owns buckets nb-1-4t .. nb-4-4t
    const int nthr = nb / 4;
    uint64_t loc[4] = {0, 0, 0, 0}, tsum = 0;
    if ((int)threadIdx.x < nthr) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        loc[q] = sm.hist[nb - 1 - (int)threadIdx.x * 4 - q];
        tsum += loc[q];
      }
    }
    uint64_t tot;
    uint64_t run = above + block_scan512(tsum, sm.sh, tot) - tsum;
    if ((int)threadIdx.x < nthr) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t nrun = run + loc[q];
        if (run < target && nrun >= target) {
          sm.bc32 = (uint32_t)(nb - 1 - (int)threadIdx.x * 4 - q);
          sm.bc64 = run;
        }
        run = nrun;
      }
    }
    __syncthreads();
    if (sm.bc32 == kNone) return prefix;  // unreachable: the bucket holds the target
    above = sm.bc64;
    prefix |= sm.bc32 << sh;
  }
  return prefix;
}

__device__ uint64_t mass_at_or_above(const uint32_t* cand, uint32_t n, uint32_t K, FinSmem& sm) {
  uint64_t t = 0;
  for (uint32_t c = threadIdx.x; c < n; c += kST) {
    const uint32_t key = cand[c];
    if (key >= K) t += fx(bits_f32(key));
  }
  return block_sum512(t, sm.sh);
}

__global__ __launch_bounds__(kST) void samp_finish_kernel(SampArgs a) {
  __shared__ FinSmem sm;
  const int r = blockIdx.x;
  RowParam rp;
  rp.m = row_max(a, r);
  rp.pad = 0;
  const uint64_t Z = a.zsum[r];
  if (!a.do_k && !a.do_p) {
    rp.thr = 0;
    rp.sf = fx_to_float(Z);
  } else if (a.do_p && a.info[r].tp == 0) {  // empty nucleus
    rp.thr = kNone;
    rp.sf = 0.0f;
  } else {
    const RowInfo inf = a.info[r];
    const uint32_t* gk = a.cand + (int64_t)r * a.V;
    const uint32_t nk = a.ccnt[r * 2];
    const bool shared = inf.bp == inf.bk;
    const uint32_t np = shared ? nk : a.ccnt[r * 2 + 1];
    const uint32_t* gp = shared ? gk : gk + (a.V - np);
    // stage both lists in LDS when they fit (one read of the candidates), else read them in place
    const uint32_t* ck = gk;
    const uint32_t* cq = gp;
    if ((uint64_t)nk + (shared ? 0 : np) <= (uint64_t)kFinCap) {
      for (uint32_t c = threadIdx.x; c < nk; c += kST) sm.keys[c] = gk[c];
      if (!shared)
        for (uint32_t c = threadIdx.x; c < np; c += kST) sm.keys[nk + c] = gp[c];
      __syncthreads();
      ck = sm.keys;
      cq = shared ? sm.keys : sm.keys + nk;
    }
    uint32_t kth = 0, cut = 0;
    if (a.do_k && inf.bk != kNone) kth = select_key(ck, nk, false, (uint64_t)a.top_k - inf.above_k, inf.bk, sm);
    if (a.do_p && inf.bp != kNone) cut = select_key(cq, np, true, inf.tp - inf.wabove_p, inf.bp, sm);
    uint64_t S;
    if (a.do_p && inf.bp != kNone && cut >= kth) {
      rp.thr = cut;
      S = inf.wabove_p + mass_at_or_above(cq, np, cut, sm);
    } else if (a.do_k && inf.bk != kNone) {
      rp.thr = kth;
      S = inf.wabove_k + mass_at_or_above(ck, nk, kth, sm);
    } else {  // unreachable: an active threshold always finds its bucket
      rp.thr = 0;
      S = Z;
    }
    rp.sf = fx_to_float(S);
  }
  if (threadIdx.x == 0) a.prm[r] = rp;
}

// accept test of the drafted token at position i of batch row b (a draft id outside [0, V) is
// rejected): u < min(1, p'(d) / max(q'(d), 1e-9)), q' = 1 for one-hot drafts
__device__ int accept_test(const SampArgs& a, int b, int i, uint32_t off) {
  const float T = a.T, inv_t = 1.0f / T;
  const int32_t d = a.draft[(int64_t)b * a.L + i];
  const bool dvalid = d >= 0 && (int64_t)d < a.V;
  const int prow = b * (a.L + 1) + i;
  const float pd = dvalid ? final_prob(a.prm[prow], samp_row(a, prow)[d], a.p_mul, T, inv_t) : 0.0f;
  float qd = 1.0f;
  if (dvalid && a.Rq) {
    const int qrow = a.Rp + b * a.L + i;
    qd = final_prob(a.prm[qrow], samp_row(a, qrow)[d], a.q_mul, T, inv_t);
  }
  const float u = u24_to_float(philox_word(a.seed, (uint32_t)i, (uint32_t)b, 0u, off));
  float ratio = pd / (qd > 1e-9f ? qd : 1e-9f);
  if (ratio > 1.0f) ratio = 1.0f;
  return u < ratio;
}

// ---- the distribution one draw uses
struct DrawSpec {
  int prow, qrow;       // p row, q row of a residual draw (qrow -1: bonus / row draw)
  int32_t d;            // drafted token of a residual draw with one-hot q (qrow -2)
  RowParam pp, qp;
  const float* px;
  const float* qx;
  int pmul, qmul;
  int b, pos, n;        // acceptance: batch row, drawn position, accepted count
  uint32_t word;
};

__device__ __forceinline__ uint64_t draw_weight(const DrawSpec& ds, int64_t j, float T, float inv_t) {
  const float pj = final_prob(ds.pp, ds.px[j], ds.pmul, T, inv_t);
  if (ds.qrow == -1) return fx(pj);
  const float qj = ds.qrow == -2 ? (j == ds.d ? 1.0f : 0.0f) : final_prob(ds.qp, ds.qx[j], ds.qmul, T, inv_t);
  const float t = pj - qj;
  return fx(t > 0.0f ? t : 0.0f);
}

// The draw of `unit` (acceptance: batch row b, or (b, position) when every position draws; row
// sampling: row r); n is batch row b's accepted count (acceptance).
__device__ DrawSpec draw_spec(const SampArgs& a, int unit, int n) {
  DrawSpec ds;
  ds.qrow = -1;
  ds.d = -1;
  ds.n = n;
  ds.b = 0;
  ds.pos = 0;
  const uint32_t off = samp_offset(a);
  if (a.mode == 0) {
    ds.b = a.all_pos ? unit / (a.L + 1) : unit;
    ds.pos = a.all_pos ? unit % (a.L + 1) : n;
    ds.prow = ds.b * (a.L + 1) + ds.pos;
    if (ds.pos < a.L) {
      ds.d = a.draft[(int64_t)ds.b * a.L + ds.pos];
      ds.qrow = a.Rq ? a.Rp + ds.b * a.L + ds.pos : -2;
    }
    ds.word = philox_word(a.seed, (uint32_t)ds.pos, (uint32_t)ds.b, 1u, off);
  } else {
    ds.prow = unit;
    ds.word = philox_word(a.seed, (uint32_t)(a.row0 + unit), 0u, 2u, off);
  }
  ds.pp = a.prm[ds.prow];
  ds.px = samp_row(a, ds.prow);
  ds.pmul = samp_mul(a, ds.prow);
  if (ds.qrow >= 0) {
    ds.qp = a.prm[ds.qrow];
    ds.qx = samp_row(a, ds.qrow);
    ds.qmul = samp_mul(a, ds.qrow);
  } else {
    ds.qp = ds.pp;
    ds.qx = ds.px;
    ds.qmul = ds.pmul;
  }
  return ds;
}

// ---- pass 5: the accept tests (every workgroup of a batch row repeats them; slice 0 stores
// them), then the per-slice mass of each draw's distribution (row sampling also stores p')
__global__ __launch_bounds__(kST) void samp_wsum_kernel(SampArgs a) {
  __shared__ uint64_t sh[kSW];
  __shared__ int sacc[256];
  __shared__ int sn;
  const int unit = blockIdx.x / a.Sd, s = blockIdx.x % a.Sd;
  int n = 0;
  if (a.mode == 0) {
    const int b = a.all_pos ? unit / (a.L + 1) : unit;
    const uint32_t off = samp_offset(a);
    if ((int)threadIdx.x < a.L) sacc[threadIdx.x] = accept_test(a, b, threadIdx.x, off);
    __syncthreads();
    if (threadIdx.x == 0) {
      int k = 0;
      while (k < a.L && sacc[k]) ++k;
      sn = k;
    }
    if (s == 0 && (!a.all_pos || unit % (a.L + 1) == 0) && (int)threadIdx.x < a.L)
      a.acc[(int64_t)b * a.L + threadIdx.x] = sacc[threadIdx.x];
    __syncthreads();
    n = sn;
  }
  const DrawSpec ds = draw_spec(a, unit, n);
  const float T = a.T, inv_t = 1.0f / T;
  const int64_t lo = min(a.V, (int64_t)s * a.slen_d), hi = min(a.V, lo + a.slen_d);
  // this thread's elements j = lo + tid + k * kST, loads first
  // (without branches, as in SliceRegs::load: a j past the slice reads element lo; such j are
  // skipped below)
  float pv[kDrawEPT], qv[kDrawEPT] = {};
  const int64_t jc = hi > lo ? lo : 0;
#pragma unroll
  for (int k = 0; k < kDrawEPT; ++k) {
    const int64_t j = lo + threadIdx.x + (int64_t)k * kST;
    pv[k] = ds.px[j < hi ? j : jc];
  }
  if (ds.qrow >= 0) {
#pragma unroll
    for (int k = 0; k < kDrawEPT; ++k) {
      const int64_t j = lo + threadIdx.x + (int64_t)k * kST;
      qv[k] = ds.qx[j < hi ? j : jc];
    }
  }
  uint64_t t = 0;
  float* po = (a.mode == 1 && a.probs_out) ? a.probs_out + (int64_t)unit * a.V : nullptr;
#pragma unroll
  for (int k = 0; k < kDrawEPT; ++k) {
    const int64_t j = lo + threadIdx.x + (int64_t)k * kST;
    if (j >= hi) continue;
    const float pj = final_prob(ds.pp, pv[k], ds.pmul, T, inv_t);
    if (ds.qrow == -1) {
      if (po) po[j] = pj;
      t += fx(pj);
    } else {
      const float qj = ds.qrow == -2 ? (j == ds.d ? 1.0f : 0.0f) : final_prob(ds.qp, qv[k], ds.qmul, T, inv_t);
      const float r = pj - qj;
      t += fx(r > 0.0f ? r : 0.0f);
    }
  }
  t = block_sum512(t, sh);
  if (threadIdx.x == 0) a.wsum[(int64_t)unit * kMaxDrawSlices + s] = t;
}

// ---- pass 6: the inverse-CDF draw (the slice holding the uniform's mass, then the element:
// each thread takes a contiguous run of the slice, one block scan finds the run), the outputs
__global__ __launch_bounds__(kST) void samp_draw_kernel(SampArgs a) {
  __shared__ uint64_t sh[kSW];
  __shared__ int64_t found;
  __shared__ uint64_t sbase;
  __shared__ int sslice;
  __shared__ int sn;
  const int unit = blockIdx.x;
  if (threadIdx.x == 0) {
    sn = a.L;
    found = -1;
    sslice = -1;
  }
  __syncthreads();
  if (a.mode == 0 && (int)threadIdx.x < a.L) {  // n = the first rejected position (flags read in parallel)
    const int b = a.all_pos ? unit / (a.L + 1) : unit;
    if (!a.acc[(int64_t)b * a.L + threadIdx.x]) atomicMin(&sn, (int)threadIdx.x);
  }
  __syncthreads();
  const int n = a.mode == 0 ? sn : 0;
  const DrawSpec ds = draw_spec(a, unit, n);
  const float T = a.T, inv_t = 1.0f / T;
  const uint64_t* ws = a.wsum + (int64_t)unit * kMaxDrawSlices;
  const uint64_t u = ds.word >> 8;
  {  // the slice holding the target: slice sums scanned in thread order (Sd <= kST)
    const uint64_t mine = (int)threadIdx.x < a.Sd ? ws[threadIdx.x] : 0;
    uint64_t W;
    const uint64_t incl = block_scan512(mine, sh, W);
    if (W == 0) {
      if (threadIdx.x == 0) found = (int64_t)((u * (uint64_t)a.V) >> 24);
    } else {
      const uint64_t t = (W >> 24) * u + (((W & 0xFFFFFFull) * u) >> 24);
      if (incl - mine <= t && t < incl) {
        sslice = (int)threadIdx.x;
        sbase = t - (incl - mine);  // the target inside the slice
      }
    }
  }
  __syncthreads();
  if (found < 0 && sslice >= 0) {
    const uint64_t tt = sbase;
    const int64_t lo = min(a.V, (int64_t)sslice * a.slen_d), hi = min(a.V, lo + a.slen_d);
    const int64_t per = ceil_div(hi - lo, kST);  // <= kDrawEPT
    const int64_t j0 = lo + (int64_t)threadIdx.x * per;
    uint64_t w[kDrawEPT], tsum = 0;
#pragma unroll
    for (int e = 0; e < kDrawEPT; ++e) {
      const int64_t j = j0 + e;
      w[e] = (e < per && j < hi) ? draw_weight(ds, j, T, inv_t) : 0;
      tsum += w[e];
    }
    uint64_t tot;
    const uint64_t incl = block_scan512(tsum, sh, tot);
    uint64_t r0 = incl - tsum;
    if (r0 <= tt && tt < incl) {  // exactly one thread holds the crossing
#pragma unroll
      for (int e = 0; e < kDrawEPT; ++e) {
        if (tt < r0 + w[e]) {
          found = j0 + e;
          break;
        }
        r0 += w[e];
      }
    }
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  const int32_t tok = (int32_t)(found >= 0 ? found : 0);
  if (a.mode == 1) {
    a.tok_rows[unit] = tok;
    return;
  }
  if (a.sample_out) a.sample_out[(int64_t)ds.b * (a.L + 1) + ds.pos] = tok;
  if (ds.pos != ds.n) return;
  a.n_out[ds.b] = ds.n;
  a.token_out[ds.b] = tok;
  if (a.seq_lens) a.seq_lens[ds.b] += ds.n + 1;
  if (a.accept_out)
    for (int k = 0; k < a.L; ++k) a.accept_out[(int64_t)ds.b * a.L + k] = (uint8_t)a.acc[(int64_t)ds.b * a.L + k];
}

// ---- workspace layout of the sampled paths
struct SampLayout {
  size_t gmax, zsum, hcnt, hwgt, ccnt, info, prm, acc, wsum, cand, total;
};

__host__ inline SampLayout samp_layout(size_t rows, size_t draws, size_t accs, int64_t V) {
  SampLayout L;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  L.gmax = take(rows * kMaxSlices * 4);
  L.zsum = take(rows * 8);
  L.hcnt = take(rows * kL1 * 4);
  L.hwgt = take(rows * kL1 * 8);
  L.ccnt = take(rows * 2 * 4);
  L.info = take(rows * sizeof(RowInfo));
  L.prm = take(rows * sizeof(RowParam));
  L.acc = take(accs * 4);
  L.wsum = take(draws * kMaxDrawSlices * 8);
  L.cand = take(rows * (size_t)V * 4);
  L.total = off;
  return L;
}

__host__ inline void samp_bind(SampArgs& a, void* base, const SampLayout& L) {
  uint8_t* p = reinterpret_cast<uint8_t*>(base);
  a.gmax = reinterpret_cast<float*>(p + L.gmax);
  a.zsum = reinterpret_cast<uint64_t*>(p + L.zsum);
  a.hcnt = reinterpret_cast<uint32_t*>(p + L.hcnt);
  a.hwgt = reinterpret_cast<uint64_t*>(p + L.hwgt);
  a.ccnt = reinterpret_cast<uint32_t*>(p + L.ccnt);
  a.info = reinterpret_cast<RowInfo*>(p + L.info);
  a.prm = reinterpret_cast<RowParam*>(p + L.prm);
  a.acc = reinterpret_cast<int32_t*>(p + L.acc);
  a.wsum = reinterpret_cast<uint64_t*>(p + L.wsum);
  a.cand = reinterpret_cast<uint32_t*>(p + L.cand);
}

// slices per row: at least enough for the gather pass's registers, about 1024 workgroups in
// all, at most kMaxSlices, never slices shorter than 512 elements
__host__ inline int samp_slices(int rows, int64_t V) {
  int64_t S = ceil_div(1024, rows);
  S = std::min<int64_t>(S, std::max<int64_t>(1, V / 512));
  S = std::max<int64_t>(S, ceil_div(V, kMaxSlice));
  return (int)std::min<int64_t>(S, kMaxSlices);
}

__host__ inline int64_t samp_slice_len(int64_t V, int S) { return (ceil_div(V, S) + 3) & ~(int64_t)3; }

// draw slices: about 1024 workgroups over the draws, slices of at most kST * kDrawEPT elements
__host__ inline int samp_draw_slices(int draws, int64_t V) {
  int64_t S = std::max<int64_t>(ceil_div(1024, draws), ceil_div(V, (int64_t)kST * kDrawEPT));
  S = std::min<int64_t>(S, std::max<int64_t>(ceil_div(V, (int64_t)kST * kDrawEPT), ceil_div(V, 256)));
  return (int)std::max<int64_t>(1, std::min<int64_t>(S, kMaxDrawSlices));
}

}  // namespace dsk

using namespace dsk;

// Pass 1 over `rows` rows of logits into ws.gval / ws.gidx; 16-byte chunk loads when every row
// starts 16-byte aligned.
static void launch_slice_argmax(const void* logits, int dtype, int64_t ldl, int64_t V, int rows, const GreedyWs& ws,
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

// The sampled chain (passes 1-6) for the rows and draws a describes.
static int launch_sampled(SampArgs& a, int draws, hipStream_t st, const char* who) {
  const int rows = a.Rp + a.Rq;
  const dim3 blk(kST);
  const dim3 grow((unsigned)(rows * a.S));
  const bool one = a.T == 1.0f;
#define DSK_ROW_PASSES(VEC_, ONE_)                                                 \
  hipLaunchKernelGGL((samp_max_kernel<VEC_, ONE_>), grow, blk, 0, st, a);          \
  hipLaunchKernelGGL((samp_stats_kernel<VEC_, ONE_>), grow, blk, 0, st, a);        \
  if (a.do_k || a.do_p) {                                                          \
    hipLaunchKernelGGL(samp_select_kernel, dim3((unsigned)rows), blk, 0, st, a);   \
    hipLaunchKernelGGL((samp_gather_kernel<VEC_, ONE_>), grow, blk, 0, st, a);     \
  }
  if (a.vec && one) {
    DSK_ROW_PASSES(true, true)
  } else if (a.vec) {
    DSK_ROW_PASSES(true, false)
  } else if (one) {
    DSK_ROW_PASSES(false, true)
  } else {
    DSK_ROW_PASSES(false, false)
  }
#undef DSK_ROW_PASSES
  hipLaunchKernelGGL(samp_finish_kernel, dim3((unsigned)rows), blk, 0, st, a);
  hipLaunchKernelGGL(samp_wsum_kernel, dim3((unsigned)(draws * a.Sd)), blk, 0, st, a);
  hipLaunchKernelGGL(samp_draw_kernel, dim3((unsigned)draws), blk, 0, st, a);
  DSK_LAUNCH_CHECK(who);
  return DSK_OK;
}

static void samp_common(SampArgs& a, int64_t V, int rows, float T, float top_p, int top_k) {
  a.V = V;
  a.T = T;
  a.top_p = top_p;
  a.top_k = top_k;
  a.do_k = (top_k > 0 && (int64_t)top_k < V);
  a.do_p = (top_p < 1.0f);
  a.S = samp_slices(rows, V);
  a.slen = samp_slice_len(V, a.S);
}

static void samp_draws(SampArgs& a, int draws) {
  a.Sd = samp_draw_slices(draws, a.V);
  a.slen_d = samp_slice_len(a.V, a.Sd);
}

static size_t accept_sample_ws(int B, int L, int64_t V) {
  const size_t rows = (size_t)B * (2 * L + 1);
  return samp_layout(rows, (size_t)B * (L + 1), (size_t)B * std::max(L, 1), V).total;
}

extern "C" size_t dsk_accept_ws_bytes(int B, int W, int64_t V) {
  if (B <= 0 || W <= 0 || V <= 0) return 0;
  return std::max(greedy_ws_bytes((size_t)B * W), accept_sample_ws(B, W - 1, V));
}

extern "C" int dsk_accept_ws_init(void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  // No kernel of this file keeps state in the workspace between calls: nothing to initialise.
  (void)stream;
  DSK_REQUIRE(workspace && ws_bytes > 0, "dsk_accept_ws_init: empty workspace");
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
  DSK_REQUIRE(ws_bytes >= greedy_ws_bytes((size_t)B * W), "dsk_accept_greedy: workspace %zu < %zu", ws_bytes,
              greedy_ws_bytes((size_t)B * W));
  GreedyWs ws = greedy_ws(workspace, (size_t)B * W);
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
  GreedyWs ws;
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
  return greedy_ws_bytes((size_t)R);
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
  GreedyWs ws = greedy_ws(workspace, (size_t)R);
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
  DSK_REQUIRE(B > 0 && B <= 1024 && L >= 0 && L < 255 && V > 0 && V <= (1ll << 19),
              "dsk_accept_sample: bad shape B=%d L=%d V=%lld (V <= 2^19)", B, L, (long long)V);
  DSK_REQUIRE(temperature > 0.0f, "dsk_accept_sample: temperature must be > 0");
  const size_t need = accept_sample_ws(B, L, V);
  DSK_REQUIRE(ws_bytes >= need, "dsk_accept_sample: workspace %zu < %zu", ws_bytes, need);
  SampArgs a{};
  a.p = p_logits;
  a.q = q_logits;
  a.Rp = B * (L + 1);
  a.Rq = q_logits ? B * L : 0;
  samp_common(a, V, a.Rp + a.Rq, temperature, top_p, top_k);
  a.p_mul = 0;
  a.q_mul = q_mul_inv_t;
  a.mode = 0;
  a.B = B;
  a.L = L;
  a.all_pos = sample_out != nullptr;
  a.draft = draft;
  a.seed = seed;
  a.offset = offset;
  a.offset_dev = offset_dev;
  a.n_out = n_out;
  a.token_out = token_out;
  a.seq_lens = seq_lens;
  a.accept_out = accept_out;
  a.sample_out = sample_out;
  samp_bind(a, workspace, samp_layout((size_t)B * (2 * L + 1), (size_t)B * (L + 1), (size_t)B * std::max(L, 1), V));
  a.vec = V % 4 == 0 && ((uintptr_t)p_logits & 15) == 0 && ((uintptr_t)q_logits & 15) == 0;
  const int draws = a.all_pos ? B * (L + 1) : B;
  samp_draws(a, draws);
  return launch_sampled(a, draws, as_stream(stream), "dsk_accept_sample");
}

extern "C" size_t dsk_sample_ws_bytes(int R, int64_t V) {
  if (R <= 0 || V <= 0) return 0;
  return std::max(R <= 1024 ? greedy_ws_bytes((size_t)R) : 0, samp_layout((size_t)R, (size_t)R, 1, V).total);
}

extern "C" int dsk_sample_rows(const float* logits, int64_t V, int R, float temperature, float top_p, int top_k,
                               int mul_inv_t, uint64_t seed, uint32_t offset, int row0, int32_t* token_out,
                               float* probs_out, const uint32_t* offset_dev, void* workspace, size_t ws_bytes,
                               dsk_stream_t stream) {
  DSK_REQUIRE(logits && token_out && workspace, "dsk_sample_rows: null pointer");
  DSK_REQUIRE(R > 0 && V > 0 && V <= (1ll << 19), "dsk_sample_rows: bad shape R=%d V=%lld (V <= 2^19)", R,
              (long long)V);
  DSK_REQUIRE(ws_bytes >= dsk_sample_ws_bytes(R, V), "dsk_sample_rows: workspace %zu < %zu", ws_bytes,
              dsk_sample_ws_bytes(R, V));
  const hipStream_t st = as_stream(stream);
  if (temperature <= 0.0f) {
    DSK_REQUIRE(R <= 1024, "dsk_sample_rows: greedy picks take at most 1024 rows");
    GreedyWs ws = greedy_ws(workspace, (size_t)R);
    launch_slice_argmax(logits, DSK_F32, V, V, R, ws, st);
    hipLaunchKernelGGL(argmax_merge_kernel, dim3((unsigned)R), dim3(64), 0, st, V, ws.gval, ws.gidx, token_out);
    DSK_LAUNCH_CHECK("dsk_sample_rows");
    return DSK_OK;
  }
  SampArgs a{};
  a.p = logits;
  a.q = nullptr;
  a.Rp = R;
  a.Rq = 0;
  samp_common(a, V, R, temperature, top_p, top_k);
  a.p_mul = mul_inv_t;
  a.q_mul = 0;
  a.mode = 1;
  a.seed = seed;
  a.offset = offset;
  a.offset_dev = offset_dev;
  a.row0 = row0;
  a.tok_rows = token_out;
  a.probs_out = probs_out;
  samp_bind(a, workspace, samp_layout((size_t)R, (size_t)R, 1, V));
  a.vec = V % 4 == 0 && ((uintptr_t)logits & 15) == 0;
  samp_draws(a, R);
  return launch_sampled(a, R, st, "dsk_sample_rows");
}
