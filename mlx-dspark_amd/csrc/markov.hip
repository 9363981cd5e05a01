// DSpark block sampling with the rank-R Markov head on gfx950.
//
// Position i of a drafted block takes token argmax_v (base[i][v] + bias_v(prev)), where
// bias_v(p) = w2[v] . w1[p] (a rank-R embedding row of the previous token, projected back to
// the vocabulary) and prev is position i-1's token (the pending token for i = 0). The
// dependency makes the block sequential; each step streams all of w2.
//
// One launch per step. A step's workgroups (1) recover prev from the previous step's
// per-workgroup argmax partials (every workgroup reduces them the same way), (2) gather and
// dequantise w1[prev] into LDS as an MFMA A operand (batch rows = M), (3) stream their share
// of w2's 16-row tiles through v_mfma_f32_16x16x32_bf16 (the W8 GEMM arithmetic: q exact in
// bf16, group sums X from a ones operand), form bf16(bf16(base) + bf16(bias)) and keep the
// running argmax (lowest index on ties), (4) publish one (value, index) partial per batch
// row. A final launch reduces the last step. Rounding points follow a bf16 graph: the
// logits, the bias and their sum are bf16.
#include "common.h"

namespace dsk {

constexpr int kMarkovR = 256;          // rank supported (the DSpark checkpoints use 256)
constexpr int kMarkovTilesPerBlock = 20;  // 5 per wave: one round of 2 waves per SIMD holds every tile of V = 151936
constexpr int kMarkovMaxB = 16;

struct MarkovArgs {
  const float* base;     // [B][cap][V] f32 (row (b, i) at (b * cap + i) * ldb)
  int64_t ldb;
  int B, cap, step;
  int64_t V;
  const int32_t* first_prev;  // [B]
  const uint8_t* w1q;          // [V][R] u8 (MLX layout), scales / biases [V][R/64] bf16
  const uint16_t* w1s;
  const uint16_t* w1b;
  const u32x4* w2t;            // tiled [V/16][R/64][64][16 B]
  const uint32_t* w2sb;        // [V/16][R/64][16]
  int32_t* tok;                // [B][cap]
  float* logits_out;           // sampled mode: [B][cap][V] rows for this step, else null
  float* pval;                 // [2][B][nblk] partials (ping-pong by step parity)
  int32_t* pidx;
  int nblk;
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// wave-wide argmax over (v, i) pairs, lowest index on ties
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, 64);
    const int oi = __shfl_xor(i, o, 64);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// argmax over n (value, index) partials by one wave: 8 loads per lane in flight per round
__device__ __forceinline__ void reduce_partials(const float* pv, const int32_t* pi, int n, int lane, float& bv,
                                                int& bi) {
  for (int k0 = 0; k0 < n; k0 += 512) {
    float v[8];
    int id[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // without branches: every load in flight at once
      const int k = k0 + u * 64 + lane;
      v[u] = pv[min(k, n - 1)];
      id[u] = pi[min(k, n - 1)];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + u * 64 + lane >= n) {
        v[u] = -__builtin_inff();
        id[u] = 0x7fffffff;
      }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (better(v[u], id[u], bv, bi)) {
        bv = v[u];
        bi = id[u];
      }
  }
  wave_argmax(bv, bi);
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void markov_step_kernel(MarkovArgs a) {
  constexpr int R = kMarkovR, G = R / 64;
  __shared__ int prev_s[kMarkovMaxB];
  __shared__ __attribute__((aligned(16))) uint16_t e_lds[16 * R];  // [row][R]
  __shared__ float red_v[4][kMarkovMaxB];
  __shared__ int red_i[4][kMarkovMaxB];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const bool greedy = a.logits_out == nullptr;

  // ---- 0. the wave's w2 tiles, their scales and the base logits, issued first: they do not
  // depend on the previous token, so they stream in while it and its w1 row are found (a tile
  // index past the block's tiles re-reads its last tile, a row past B row B - 1: not used)
  constexpr int TPW = kMarkovTilesPerBlock / 4;  // tiles per wave
  const int64_t ntiles = a.V / 16;
  const int64_t t_lo = (int64_t)blockIdx.x * kMarkovTilesPerBlock;
  const int64_t t_hi = min(ntiles, t_lo + kMarkovTilesPerBlock);
  u32x4 wq[TPW][G];
  uint32_t sv[TPW][G];
  float bs[TPW][4];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int64_t t = min(t_lo + wv + 4 * i, t_hi - 1);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      wq[i][g] = __builtin_nontemporal_load(&a.w2t[(t * G + g) * 64 + lane]);
      sv[i][g] = a.w2sb[(t * G + g) * 16 + (lane & 15)];
    }
    const int64_t v = t * 16 + (lane & 15);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int b = min((lane >> 4) * 4 + r, a.B - 1);
      bs[i][r] = a.base[((int64_t)b * a.cap + a.step) * a.ldb + v];
    }
  }

  // ---- 1. previous token of every batch row
  if (a.step == 0) {
    if (threadIdx.x < a.B) prev_s[threadIdx.x] = a.first_prev[threadIdx.x];
  } else if (!greedy) {
    if (threadIdx.x < a.B) prev_s[threadIdx.x] = a.tok[threadIdx.x * a.cap + a.step - 1];
  } else {
    const int par = (a.step - 1) & 1;
    for (int b = wv; b < a.B; b += 4) {
      float bv = -__builtin_inff();
      int bi = 0x7fffffff;
      const float* pv = a.pval + ((size_t)par * a.B + b) * a.nblk;
      const int32_t* pi = a.pidx + ((size_t)par * a.B + b) * a.nblk;
      reduce_partials(pv, pi, a.nblk, lane, bv, bi);
      if (lane == 0) {
        const int t = (bi >= 0 && (int64_t)bi < a.V) ? bi : 0;
        prev_s[b] = t;
        if (blockIdx.x == 0) a.tok[b * a.cap + a.step - 1] = t;
      }
    }
  }
  __syncthreads();

  // ---- 2. e = bf16(deq(w1)[prev]) for every batch row (rows >= B are zero)
  for (int idx = threadIdx.x; idx < 16 * R; idx += 256) {
    const int b = idx / R, r = idx % R;
    float e = 0.0f;
    if (b < a.B) {
      int64_t p = prev_s[b];
      if (p < 0 || p >= a.V) p = 0;
      const int g = r / 64;
      e = round_bf16(fmaf(bf16_to_f32(a.w1s[p * G + g]), (float)a.w1q[p * R + r], bf16_to_f32(a.w1b[p * G + g])));
    }
    e_lds[idx] = f32_to_bf16(e);
  }
  __syncthreads();

  // A operand fragments: lane l holds row l%16, columns 64g + 16(l/16) + [0, 16)
  bf16x8 ea[G][2];
  f32x4 X[G];
  const u32x4 ones_u = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const bf16x8 ones = __builtin_bit_cast(bf16x8, ones_u);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const uint16_t* p = e_lds + (lane & 15) * R + 64 * g + 16 * (lane >> 4);
    ea[g][0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
    ea[g][1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p + 8));
    X[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ea[g][0], ones, f32x4{0, 0, 0, 0}, 0, 0, 0);
    X[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ea[g][1], ones, X[g], 0, 0, 0);
  }

  // ---- 3. this block's tiles, round-robin over the waves (loaded in step 0)
  float bestv[4];
  int besti[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    bestv[r] = -__builtin_inff();
    besti[r] = 0x7fffffff;
  }
#pragma unroll
  for (int it = 0; it < TPW; ++it) {
    const int64_t t = t_lo + wv + 4 * it;
    if (t >= t_hi) break;
    const int64_t v = t * 16 + (lane & 15);
    f32x4 acc = {0, 0, 0, 0};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      bf16x8 b0, b1;
      {
        uint32_t rr[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t q = wq[it][g][i];
          rr[2 * i] = __builtin_amdgcn_perm(f32_bits((float)((q >> 8) & 0xffu)), f32_bits((float)(q & 0xffu)),
                                            0x07060302u);
          rr[2 * i + 1] = __builtin_amdgcn_perm(f32_bits((float)(q >> 24)), f32_bits((float)((q >> 16) & 0xffu)),
                                                0x07060302u);
        }
        b0 = __builtin_bit_cast(bf16x8, (u32x4{rr[0], rr[1], rr[2], rr[3]}));
        b1 = __builtin_bit_cast(bf16x8, (u32x4{rr[4], rr[5], rr[6], rr[7]}));
      }
      f32x4 tq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ea[g][0], b0, f32x4{0, 0, 0, 0}, 0, 0, 0);
      tq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ea[g][1], b1, tq, 0, 0, 0);
      const float s = bf16_to_f32((uint16_t)(sv[it][g] & 0xffffu)), bb = bf16_to_f32((uint16_t)(sv[it][g] >> 16));
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = fmaf(s, tq[r], fmaf(bb, X[g][r], acc[r]));
    }
    // lane holds bias[b = 4 * (lane / 16) + r][v]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int b = (lane >> 4) * 4 + r;
      if (b >= a.B) continue;
      const float lg = round_bf16(round_bf16(bs[it][r]) + round_bf16(acc[r]));
      if (a.logits_out) a.logits_out[((int64_t)b * a.cap + a.step) * a.V + v] = lg;
      if (better(lg, (int)v, bestv[r], besti[r])) {
        bestv[r] = lg;
        besti[r] = (int)v;
      }
    }
  }
  if (!greedy) return;

  // ---- 4. per-row argmax of the block: 16 lanes share a row within a wave, then the waves
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = bestv[r];
    int i = besti[r];
    for (int o = 8; o > 0; o >>= 1) {
      const float ov = __shfl_xor(v, o, 16);
      const int oi = __shfl_xor(i, o, 16);
      if (better(ov, oi, v, i)) {
        v = ov;
        i = oi;
      }
    }
    const int b = (lane >> 4) * 4 + r;
    if ((lane & 15) == 0 && b < a.B) {
      red_v[wv][b] = v;
      red_i[wv][b] = i;
    }
  }
  __syncthreads();
  if (threadIdx.x < a.B) {
    const int b = threadIdx.x;
    float v = red_v[0][b];
    int i = red_i[0][b];
    for (int w = 1; w < 4; ++w)
      if (better(red_v[w][b], red_i[w][b], v, i)) {
        v = red_v[w][b];
        i = red_i[w][b];
      }
    const int par = a.step & 1;
    a.pval[((size_t)par * a.B + b) * a.nblk + blockIdx.x] = v;
    a.pidx[((size_t)par * a.B + b) * a.nblk + blockIdx.x] = i;
  }
}

// the last step's partials -> its tokens
__global__ __launch_bounds__(64) void markov_final_kernel(MarkovArgs a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int par = (a.cap - 1) & 1;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  const float* pv = a.pval + ((size_t)par * a.B + b) * a.nblk;
  const int32_t* pi = a.pidx + ((size_t)par * a.B + b) * a.nblk;
  reduce_partials(pv, pi, a.nblk, lane, bv, bi);
  if (lane == 0) a.tok[b * a.cap + a.cap - 1] = (bi >= 0 && (int64_t)bi < a.V) ? bi : 0;
}

static int markov_nblk(int64_t V) { return (int)ceil_div(V / 16, kMarkovTilesPerBlock); }

}  // namespace dsk

using namespace dsk;

extern "C" size_t dsk_markov_ws_bytes(int B, int64_t V, int sampled) {
  if (B <= 0 || V <= 0) return 0;
  const size_t part = (size_t)2 * B * markov_nblk(V) * (sizeof(float) + sizeof(int32_t));
  return ((part + 255) & ~(size_t)255) + (sampled ? dsk_sample_ws_bytes(1, V) : 0);
}

extern "C" int dsk_markov_block(const float* base, int64_t ldb, int B, int cap, int64_t V, int R,
                                const int32_t* first_prev, const uint8_t* w1q, const uint16_t* w1s,
                                const uint16_t* w1b, const uint8_t* w2t, const uint32_t* w2sb, float temperature,
                                float top_p, int top_k, uint64_t seed, uint32_t offset, int row0, int32_t* tok_out,
                                float* q_logits_out, void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(base && first_prev && w1q && w1s && w1b && w2t && w2sb && tok_out && workspace,
              "dsk_markov_block: null pointer");
  DSK_REQUIRE(R == kMarkovR, "dsk_markov_block: markov rank %d not supported (%d)", R, kMarkovR);
  DSK_REQUIRE(B > 0 && B <= kMarkovMaxB && cap > 0 && cap <= 64, "dsk_markov_block: B=%d cap=%d", B, cap);
  DSK_REQUIRE(row0 >= 0, "dsk_markov_block: row0=%d", row0);
  DSK_REQUIRE(V > 0 && V % 16 == 0 && V < (1ll << 31) && ldb >= V, "dsk_markov_block: bad V=%lld / ldb",
              (long long)V);
  const bool sampled = temperature > 0.0f;
  DSK_REQUIRE(!sampled || q_logits_out, "dsk_markov_block: sampling needs q_logits_out [B, cap, V]");
  DSK_REQUIRE(ws_bytes >= dsk_markov_ws_bytes(B, V, sampled), "dsk_markov_block: workspace %zu < %zu", ws_bytes,
              dsk_markov_ws_bytes(B, V, sampled));
  MarkovArgs a;
  a.base = base;
  a.ldb = ldb;
  a.B = B;
  a.cap = cap;
  a.V = V;
  a.first_prev = first_prev;
  a.w1q = w1q;
  a.w1s = w1s;
  a.w1b = w1b;
  a.w2t = reinterpret_cast<const u32x4*>(w2t);
  a.w2sb = w2sb;
  a.tok = tok_out;
  a.logits_out = sampled ? q_logits_out : nullptr;
  a.nblk = markov_nblk(V);
  const size_t part = (size_t)2 * B * a.nblk;
  a.pval = reinterpret_cast<float*>(workspace);
  a.pidx = reinterpret_cast<int32_t*>(a.pval + part);
  void* sample_ws = reinterpret_cast<uint8_t*>(workspace) + (((part * 8) + 255) & ~(size_t)255);
  const size_t sample_ws_bytes = sampled ? dsk_sample_ws_bytes(1, V) : 0;
  hipStream_t st = as_stream(stream);
  for (int s = 0; s < cap; ++s) {
    a.step = s;
    hipLaunchKernelGGL(markov_step_kernel, dim3((unsigned)a.nblk), dim3(256), 0, st, a);
    DSK_LAUNCH_CHECK("dsk_markov_block (step)");
    if (sampled) {
      // q_i = truncate(softmax(logits_i * (1/T))), sampled; Philox rows (row0 + b) * cap + s
      for (int b = 0; b < B; ++b) {
        const int rc = dsk_sample_rows(q_logits_out + ((int64_t)b * cap + s) * V, V, 1, temperature, top_p, top_k, 1,
                                       seed, offset, (row0 + b) * cap + s, tok_out + b * cap + s, nullptr, nullptr,
                                       sample_ws,
                                       sample_ws_bytes, stream);
        if (rc != DSK_OK) return rc;
      }
    }
  }
  if (!sampled) {
    hipLaunchKernelGGL(markov_final_kernel, dim3((unsigned)B), dim3(64), 0, st, a);
    DSK_LAUNCH_CHECK("dsk_markov_block (final)");
  }
  return DSK_OK;
}
