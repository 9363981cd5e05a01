// W8 affine group-64 weights on gfx950: quantizer, MLX-layout -> tiled-layout repack,
// activation packing (with the residual add and RMSNorm that precede every projection),
// and the skinny GEMM used by every target and drafter projection of the verify step.
//
// Packed activation layout (the GEMM's A operand, see common.h apack_index):
//   P[m/16][k/64][lane][16 bf16], lane = m%16 + 16 * ((k%64)/16): one 2 KiB block per
//   (16-row tile, 64-column group), and each lane's 32 bytes are the two 8-element
//   fragments it feeds to v_mfma_f32_16x16x32_bf16, so every activation load of the GEMM
//   is a contiguous 1 KiB wave-wide read.
//
// Tiled HBM layout (what dsk_w8_gemm streams):
//   wt[t][g][lane][16 B]: tile t = 16 output rows (n = 16t + lane%16), group g = 64 input
//   columns, lane/16 selects the 16-column chunk inside the group. One wave-wide dwordx4
//   load reads one 1 KiB tile-group, contiguous, and lands every byte in the lane that
//   feeds it to v_mfma_f32_16x16x32_bf16 as the B operand (bytes 0-7: first MFMA, 8-15:
//   second).
//   sb[t][g][16]: u32 = bf16 scale | bf16 bias << 16 for n = 16t + 0..15.
//   Paired repack (gated MLPs): the source rows [0, N/2) are the gate projection and
//   [N/2, N) the up projection; destination tile 2p holds gate rows 16p..16p+15 and tile
//   2p+1 the up rows 16p..16p+15, so one workgroup owning both tiles can apply the
//   activation in its epilogue.
//
// W4 (dsk_w4_gemm): the same tiles with two codes per byte (8 bytes per lane per tile-group),
// converted to 1 + q/16 in bf16 by byte permutes, the scale taken 16 times and the sum x term
// folded into the bias.
//
// GEMM arithmetic. With w = s*q + b per group, sum_k x_k w_k = s * sum x_k q_k + b * sum x_k.
// q (0..255) is exact in bf16, the bf16 activations go to the MFMA unchanged, so the MFMA
// yields t = sum x q exactly up to fp32 accumulation; X = sum x over the group comes from
// one more MFMA against a B operand of ones; the group adds s * t + b * X to the fp32
// accumulator.
#include <stdlib.h>

#include "common.h"

namespace dsk {

// =====================================================================================
// quantize: one thread per (row, group)
// =====================================================================================
__global__ void w8_quantize_kernel(const void* __restrict__ w, int w_bf16, int64_t N, int64_t K,
                                   uint8_t* __restrict__ q, uint16_t* __restrict__ scales,
                                   uint16_t* __restrict__ biases, float levels) {
  int64_t G = K / 64;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * G) return;
  int64_t n = idx / G, g = idx % G;
  float v[64];
  const int64_t base = n * K + g * 64;
  if (w_bf16) {
    const uint16_t* p = (const uint16_t*)w + base;
#pragma unroll
    for (int i = 0; i < 64; ++i) v[i] = bf16_to_f32(p[i]);
  } else {
    const float* p = (const float*)w + base;
#pragma unroll
    for (int i = 0; i < 64; ++i) v[i] = p[i];
  }
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int i = 1; i < 64; ++i) {
    lo = fminf(lo, v[i]);
    hi = fmaxf(hi, v[i]);
  }
  float s = (hi - lo) / levels;
  uint16_t sb16 = f32_to_bf16(s);
  float sf = bf16_to_f32(sb16);
  if (!(sf > 0.0f)) {
    sb16 = 0x3f80;  // 1.0
    sf = 1.0f;
  }
  uint16_t bb16 = f32_to_bf16(lo);
  float bf = bf16_to_f32(bb16);
  scales[idx] = sb16;
  biases[idx] = bb16;
  uint8_t* qo = q + base;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    float t = rintf((v[i] - bf) / sf);
    t = fminf(fmaxf(t, 0.0f), levels);
    qo[i] = (uint8_t)(int)t;
  }
}

// =====================================================================================
// repack: MLX layout -> tiled layout
// =====================================================================================
__device__ __forceinline__ int64_t repack_src_row(int64_t n, int64_t N, int paired) {
  if (!paired) return n;
  const int64_t t = n >> 4, r = n & 15;
  return (t & 1) * (N / 2) + (t >> 1) * 16 + r;
}

__global__ void w8_repack_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                 const uint16_t* __restrict__ b, int64_t N, int64_t K, int paired,
                                 u32x4* __restrict__ wt, uint32_t* __restrict__ sb) {
  const int64_t G = K / 64;
  const int64_t chunks = N * K / 16;  // 16-byte chunks
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < chunks) {
    // destination order: t, g, lane
    int64_t lane = idx & 63;
    int64_t tg = idx >> 6;
    int64_t g = tg % G, t = tg / G;
    int64_t n = repack_src_row(t * 16 + (lane & 15), N, paired);
    int64_t k = g * 64 + (lane >> 4) * 16;
    wt[idx] = *reinterpret_cast<const u32x4*>(q + n * K + k);
  }
  if (idx < N * G) {
    // destination order: t, g, n%16
    int64_t r = idx & 15;
    int64_t tg = idx >> 4;
    int64_t g = tg % G, t = tg / G;
    int64_t n = repack_src_row(t * 16 + r, N, paired);
    uint32_t sv = s[n * G + g], bv = b[n * G + g];
    sb[idx] = sv | (bv << 16);
  }
}

// W4 tiled layout: wt4[t][g][lane][8 B], the same (row, 16-column chunk) per lane as the W8
// layout with two codes per byte: byte j holds columns 2j (low nibble) and 2j + 1 (high nibble)
// of the lane's 16. One thread per lane-chunk; sb as for W8 (written by the W8 repack's loop).
__global__ void w4_repack_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                 const uint16_t* __restrict__ b, int64_t N, int64_t K, int paired,
                                 uint2* __restrict__ wt, uint32_t* __restrict__ sb) {
  const int64_t G = K / 64;
  const int64_t chunks = N * K / 16;
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < chunks) {
    int64_t lane = idx & 63;
    int64_t tg = idx >> 6;
    int64_t g = tg % G, t = tg / G;
    int64_t n = repack_src_row(t * 16 + (lane & 15), N, paired);
    int64_t k = g * 64 + (lane >> 4) * 16;
    const u32x4 v = *reinterpret_cast<const u32x4*>(q + n * K + k);
    uint32_t o[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t lo = v[2 * h], hi = v[2 * h + 1];  // codes 8h .. 8h + 7, one per byte
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t src = j < 2 ? lo : hi;
        const int sh = (j & 1) * 16;
        const uint32_t c0 = (src >> sh) & 0xfu, c1 = (src >> (sh + 8)) & 0xfu;
        w |= (c0 | (c1 << 4)) << (8 * j);
      }
      o[h] = w;
    }
    wt[idx] = uint2{o[0], o[1]};
  }
  if (idx < N * G) {
    int64_t r = idx & 15;
    int64_t tg = idx >> 4;
    int64_t g = tg % G, t = tg / G;
    int64_t n = repack_src_row(t * 16 + r, N, paired);
    uint32_t sv = s[n * G + g], bv = b[n * G + g];
    sb[idx] = sv | (bv << 16);
  }
}

// =====================================================================================
// activation pack: one workgroup per row, every 16-byte chunk of the row loaded up front.
//   v = sum of the fp32 partial slices (in slice order), plus the bf16 residual h (written
//   back rounded to bf16), or h alone; optional copy of v (hidden-state tap); optional
//   RMSNorm bf16((v * rsqrt(mean(v^2) + eps)) * w); output in the packed layout.
// =====================================================================================
constexpr int kPackThreads = 512;
constexpr int kPackMaxSplits = 16;

struct PackArgs {
  const float* part;   // [nsplit][M][K] (slice stride M * K), or null
  int nsplit;
  uint16_t* h;         // bf16 row-major, row stride ldh, or null
  int64_t ldh;
  uint16_t* copy;      // bf16 row-major, row stride ldc, or null
  int64_t ldc;
  int M;
  int64_t K;
  const uint16_t* norm_w;
  float eps;
  uint16_t* out;       // packed, or null
  const uint16_t* res_norm_w;  // RMSNorm of the partial sum before the residual add, or null
  float out_scale;             // the residual-stream result is multiplied by this (rounded again)
  float* ssq_out;              // normed later: out = bf16(v * norm_w), ssq_out[m][k / 16] = sum of
                               // the 16 columns' v^2 (the consuming GEMM applies the row scale)
};

template <int NV, int MAXS>
__global__ __launch_bounds__(kPackThreads) void act_pack_kernel(PackArgs a) {
  __shared__ float red[kPackThreads / 64];
  const int m = blockIdx.x, tid = threadIdx.x;
  const int64_t nchunk = a.K / 8;
  const int64_t G = a.K / 64;
  const int S = a.part ? a.nsplit : 0;
  // ---- every load up front, all in flight at once: norm weights, residual, each split's 8
  // values per chunk (slices past S re-read slice S - 1 and are not added), the sandwich norm's
  // weights
  u32x4 v[NV], wv[NV], hv[NV], w1v[NV];
  f32x4 pl[NV][MAXS > 0 ? MAXS : 1], ph[NV][MAXS > 0 ? MAXS : 1];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = min(tid + (int64_t)i * kPackThreads, nchunk - 1);
    if (a.norm_w) wv[i] = *reinterpret_cast<const u32x4*>(a.norm_w + c * 8);
    if (a.h) hv[i] = *reinterpret_cast<const u32x4*>(a.h + (int64_t)m * a.ldh + c * 8);
    if (a.res_norm_w) w1v[i] = *reinterpret_cast<const u32x4*>(a.res_norm_w + c * 8);
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
      const float* p = a.part + ((int64_t)min(s, S - 1) * a.M + m) * a.K + c * 8;
      pl[i][s] = *reinterpret_cast<const f32x4*>(p);
      ph[i][s] = *reinterpret_cast<const f32x4*>(p + 4);
    }
  }
  // block-wide sum (red is reused: barriers on both sides)
  auto block_sum = [&](float x) {
    x = wave_sum(x);
    __syncthreads();
    if ((tid & 63) == 0) red[tid >> 6] = x;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < kPackThreads / 64; ++i) t += red[i];
    return t;
  };
  // ---- partial sum in split order
  float fv[NV][8];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) fv[i][e] = 0.0f;
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {  // selects, not a branch: the loads stay ahead of any wait
      const bool in = s < S;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        fv[i][e] = in ? fv[i][e] + pl[i][s][e] : fv[i][e];
        fv[i][4 + e] = in ? fv[i][4 + e] + ph[i][s][e] : fv[i][4 + e];
      }
    }
  }
  // ---- sandwich norm: the projection output (rounded to bf16) normed before the residual add
  if (a.res_norm_w && S) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = tid + (int64_t)i * kPackThreads;
      if (c >= nchunk) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        fv[i][e] = round_bf16(fv[i][e]);
        ss = fmaf(fv[i][e], fv[i][e], ss);
      }
    }
    const float r1 = rsqrtf(block_sum(ss) / (float)a.K + a.eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint16_t* g = reinterpret_cast<const uint16_t*>(&w1v[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) fv[i][e] = round_bf16((fv[i][e] * r1) * bf16_to_f32(g[e]));
    }
  }
  // ---- residual add, rounded once
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    uint16_t o[8];
    const uint16_t* hh = reinterpret_cast<const uint16_t*>(&hv[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = a.h ? (S ? f32_to_bf16(bf16_to_f32(hh[e]) + fv[i][e]) : hh[e]) : f32_to_bf16(fv[i][e]);
      if (a.out_scale != 1.0f) o[e] = f32_to_bf16(bf16_to_f32(o[e]) * a.out_scale);
    }
    v[i] = *reinterpret_cast<const u32x4*>(o);
  }
  float r = 1.0f;
  if (a.ssq_out) {
    // per 16-column tile: this thread's 8 columns as ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + ...),
    // plus the neighbouring thread's 8 (the GEMM epilogue's 16-lane tree, in the same order)
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = tid + (int64_t)i * kPackThreads;
      const uint16_t* hv2 = reinterpret_cast<const uint16_t*>(&v[i]);
      float q[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = c < nchunk ? bf16_to_f32(hv2[e]) : 0.0f;
        q[e] = f * f;
      }
      float t8 = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
      t8 += __shfl_xor(t8, 1, 64);
      if (c < nchunk && (c & 1) == 0) a.ssq_out[(int64_t)m * (a.K / 16) + (c >> 1)] = t8;
    }
  } else if (a.norm_w) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t c = tid + (int64_t)i * kPackThreads;
      if (c >= nchunk) continue;
      const uint16_t* hv2 = reinterpret_cast<const uint16_t*>(&v[i]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float f = bf16_to_f32(hv2[e]);
        ss = fmaf(f, f, ss);
      }
    }
    r = rsqrtf(block_sum(ss) / (float)a.K + a.eps);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = tid + (int64_t)i * kPackThreads;
    if (c >= nchunk) continue;
    if (a.h && S) *reinterpret_cast<u32x4*>(a.h + (int64_t)m * a.ldh + c * 8) = v[i];
    if (a.copy) *reinterpret_cast<u32x4*>(a.copy + (int64_t)m * a.ldc + c * 8) = v[i];
    if (!a.out) continue;
    u32x4 ov = v[i];
    if (a.norm_w) {
      const uint16_t* hv2 = reinterpret_cast<const uint16_t*>(&v[i]);
      const uint16_t* g = reinterpret_cast<const uint16_t*>(&wv[i]);
      uint16_t o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = f32_to_bf16((bf16_to_f32(hv2[e]) * r) * bf16_to_f32(g[e]));
      ov = *reinterpret_cast<const u32x4*>(o);
    }
    *reinterpret_cast<u32x4*>(a.out + apack_index(m, c * 8, G)) = ov;
  }
}

// =====================================================================================
// skinny GEMM
// =====================================================================================
// u8 x 16 -> two bf16 x 8 (exact: q <= 255 needs 8 significant bits, the fp32 from
// v_cvt_f32_ubyteN is truncated to its top half).
__device__ __forceinline__ void u8x16_to_bf16(const u32x4 w, bf16x8& lo, bf16x8& hi) {
  uint32_t r[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = w[i];
    const float f0 = (float)(v & 0xffu), f1 = (float)((v >> 8) & 0xffu);
    const float f2 = (float)((v >> 16) & 0xffu), f3 = (float)(v >> 24);
    r[2 * i] = __builtin_amdgcn_perm(f32_bits(f1), f32_bits(f0), 0x07060302u);
    r[2 * i + 1] = __builtin_amdgcn_perm(f32_bits(f3), f32_bits(f2), 0x07060302u);
  }
  lo = __builtin_bit_cast(bf16x8, (u32x4{r[0], r[1], r[2], r[3]}));
  hi = __builtin_bit_cast(bf16x8, (u32x4{r[4], r[5], r[6], r[7]}));
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float gelu_tanh_f(float x) {
  const float c = 0.7978845608028654f;  // sqrt(2/pi)
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

struct GemmArgs {
  const u32x4* xp;  // packed activation
  const u32x4* wt;
  const uint32_t* sb;
  int M;
  int64_t N, K, G;
  int SK;           // K splits (DSK_EPI_PARTIAL)
  int64_t gpb;      // groups per split, a multiple of the batch size
  int n_slabs;      // N / (16 * NT)
  int epi;          // DSK_EPI_*
  void* y;
  int y_f32;
  int64_t ldy;
  const uint16_t* res;
  int64_t ldr;
  float softcap;
  int bits;         // weight code width: 8 (dsk_w8_gemm) or 4 (dsk_w4_gemm)
  // RMSNorm of x applied after the product (x = bf16(h * w) packed): every output of row m is
  // multiplied by r_m = rsqrt(sum_{t < rs_tiles} rs_ssq[m * rs_tiles + t] / K + rs_eps) first
  const float* rs_ssq;
  int rs_tiles;
  float rs_eps;
  // DSK_EPI_RESIDUAL: h[m][n] = bf16(h[m][n] + y) in place (row stride ldh), copy[m][n] = h
  // (tap, row stride ldc), y = packed bf16(h * g[n]) (or h when g is null; y may be null) and
  // ssq_out[m][tile] = sum over the tile's 16 columns of h^2 (row stride N / 16)
  uint16_t* h;
  int64_t ldh;
  uint16_t* copy;
  int64_t ldc;
  const uint16_t* g;
  float* ssq_out;
};

// Sum of 16 values held by 16 consecutive lanes (the same balanced tree in every lane):
// ((v0 + v1) + (v2 + v3)) + ... ; dsk_act_pack's normed-later path sums 8 + 8 the same way.
__device__ __forceinline__ float sum16_lanes(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  v += __shfl_xor(v, 8, 64);
  return v;
}

__device__ __forceinline__ void gemm_store(const GemmArgs& a, int m, int64_t n, float v) {
  if (a.res) v += bf16_to_f32(a.res[(int64_t)m * a.ldr + n]);
  if (a.softcap > 0.0f) v = tanhf(v / a.softcap) * a.softcap;
  if (a.y_f32)
    reinterpret_cast<float*>(a.y)[(int64_t)m * a.ldy + n] = v;
  else
    reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.ldy + n] = f32_to_bf16(v);
}

// gated epilogue: g, u are the two projections of one column (rounded to bf16 as the
// projection outputs are), act = bf16(bf16(act_fn(g)) * u), stored packed (K' = N / 2)
__device__ __forceinline__ void gemm_store_gated(const GemmArgs& a, int m, int64_t col, float g, float u) {
  const float gb = round_bf16(g), ub = round_bf16(u);
  const float act = round_bf16(a.epi == DSK_EPI_SWIGLU ? silu_f(gb) : gelu_tanh_f(gb));
  reinterpret_cast<uint16_t*>(a.y)[apack_index(m, col, a.N / 128)] = f32_to_bf16(act * ub);
}

// One batch of U groups: the weight, scale/bias and activation registers of U consecutive
// groups for NT tiles. Padding rows of the packed activation hold arbitrary values; their
// outputs are never stored.
// 16 4-bit codes (8 bytes, byte j = codes 2j | 2j+1 << 4) -> two bf16 x 8 holding 1 + code / 16
// (exact: 0x3f80 | c << 3 is the bf16 of 1 + c / 16, c in the top four mantissa bits); the group
// then adds 16 s (x . (1 + q/16)) + (b - 16 s) X. A form 128 + c (0x4300 | c) would need no shift,
// but its products are ~135 x against ~7.5 x for the codes themselves, so the float32 rounding of
// the accumulated products, left over when the 128 X is subtracted again, would be ~18 times that
// of the exact codes; with 1 + c/16 the offset is ~3 times the codes' part.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void u4x16_to_bf16(const u32x2 w, bf16x8& lo, bf16x8& hi) {
  uint32_t r[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t v = w[h];
    // even / odd codes times 8, one per byte (8 c < 128: no carry into the next byte)
    const uint32_t t = (v << 3) & 0x78787878u, u = (v >> 1) & 0x78787878u;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r[4 * h + i] = __builtin_amdgcn_perm(u, t, 0x0c040c00u + 0x00010001u * i) | 0x3f803f80u;
  }
  lo = __builtin_bit_cast(bf16x8, (u32x4{r[0], r[1], r[2], r[3]}));
  hi = __builtin_bit_cast(bf16x8, (u32x4{r[4], r[5], r[6], r[7]}));
}

template <int BITS> struct WeightChunk;
template <> struct WeightChunk<8> { using type = u32x4; };
template <> struct WeightChunk<4> { using type = u32x2; };

template <int MT, int NT, int U, int BITS>
struct Batch {
  typename WeightChunk<BITS>::type wv[U][NT];
  uint32_t sv[U][NT];
  u32x4 xv[U][MT][2];
};

template <int MT, int NT, int U, int BITS>
__device__ __forceinline__ void batch_load(const GemmArgs& a, int64_t t0, int64_t g0, int lane,
                                           Batch<MT, NT, U, BITS>& r) {
  using WT = typename WeightChunk<BITS>::type;
  const WT* wt = reinterpret_cast<const WT*>(a.wt);
#pragma unroll
  for (int c = 0; c < U; ++c)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t tg = (t0 + j) * a.G + g0 + c;
      r.wv[c][j] = __builtin_nontemporal_load(&wt[tg * 64 + lane]);
    }
#pragma unroll
  for (int c = 0; c < U; ++c)
#pragma unroll
    for (int j = 0; j < NT; ++j) r.sv[c][j] = a.sb[((t0 + j) * a.G + g0 + c) * 16 + (lane & 15)];
#pragma unroll
  for (int c = 0; c < U; ++c)
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const u32x4* px = a.xp + (((int64_t)i * a.G + g0 + c) * 64 + lane) * 2;
      r.xv[c][i][0] = px[0];
      r.xv[c][i][1] = px[1];
    }
}

template <int MT, int NT, int U, int BITS>
__device__ __forceinline__ void batch_compute(const Batch<MT, NT, U, BITS>& r, f32x4 (&acc)[MT][NT]) {
  const u32x4 ones_u = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  const bf16x8 ones = __builtin_bit_cast(bf16x8, ones_u);
#pragma unroll
  for (int c = 0; c < U; ++c) {
    f32x4 X[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      X[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.xv[c][i][0]), ones,
                                                     f32x4{0, 0, 0, 0}, 0, 0, 0);
      X[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.xv[c][i][1]), ones, X[i], 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      bf16x8 b0, b1;
      float s = bf16_to_f32((uint16_t)(r.sv[c][j] & 0xffffu));
      float bb = bf16_to_f32((uint16_t)(r.sv[c][j] >> 16));
      if constexpr (BITS == 8) {
        u8x16_to_bf16(r.wv[c][j], b0, b1);
      } else {
        u4x16_to_bf16(r.wv[c][j], b0, b1);
        bb = fmaf(-16.0f, s, bb);  // s q + b = 16 s (1 + q/16) + (b - 16 s)
        s *= 16.0f;
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.xv[c][i][0]), b0,
                                                          f32x4{0, 0, 0, 0}, 0, 0, 0);
        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, r.xv[c][i][1]), b1, t, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[i][j][q] = fmaf(s, t[q], fmaf(bb, X[i][q], acc[i][j][q]));
      }
    }
  }
}

// Workgroup = NT consecutive 16-row weight tiles x one K split; its WAVES waves take the
// split's batches round-robin, each accumulating all NT tiles (every activation fragment a
// wave loads feeds NT tiles), then reduce through LDS in wave order.
// EK: the epilogue family (0 store, 1 gated, 2 split-K partial) as a template parameter, so each
// family is its own (smaller) kernel. PF: software-pipelined batch loads (two register sets).
// EKR = EK + 4 * RS: RS, the row scale of a normed-later x, is compiled into its own kernels
// (its registers would otherwise weigh on every plan).
template <int MT, int NT, int U, int WAVES, int EKR, bool PF, int BITS>
__global__ __launch_bounds__(WAVES * 64) void w8_gemm_kernel(GemmArgs a) {
  constexpr int EK = EKR & 3;
  constexpr bool RS = EKR >= 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slab = blockIdx.x / a.SK, ks = blockIdx.x % a.SK;
  const int64_t g_lo = min(a.G, (int64_t)ks * a.gpb);  // a trailing split may be empty: it stores zeros
  const int64_t g_hi = min(a.G, g_lo + a.gpb);
  const int nbatch = (int)((g_hi - g_lo) / U);
  const int64_t t0 = (int64_t)slab * NT;

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

  // Row scales of x: wave w owns rows w, w + WAVES, ...; lane l sums the tile partials
  // l, l + 64, l + 128, ... in that order, then the wave sums its lanes (the same order for
  // every plan). The first 256 partials of each row go straight from memory into LDS before the
  // main loop (global_load_lds: no registers held across it); the barrier before the epilogue
  // waits for them.
  constexpr int RPW = (MT * 16 + WAVES - 1) / WAVES;
  constexpr int PRE = MT == 1 ? 4 : 0;  // 64-partial blocks per row staged in LDS (one row tile)
  __shared__ float ssq_lds[RS && PRE ? MT * 16 * 64 * PRE : 1];
  if constexpr (RS && PRE > 0) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int m = wave + WAVES * i;
      if (m >= MT * 16) break;
#pragma unroll
      for (int j = 0; j < PRE; ++j) {
        const int t = lane + 64 * j;
        // lanes past the row count or the tile count load a valid word that is never summed
        const float* src = (m < a.M && t < a.rs_tiles) ? a.rs_ssq + (int64_t)m * a.rs_tiles + t : a.rs_ssq;
        __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(ssq_lds + (m * PRE + j) * 64),
                                         4, 0, 0);
      }
    }
  }

  // residual epilogue: the residual h and the next norm's gain of each output this thread
  // stores, loaded before the main loop (after it they would cost two more memory round trips)
  constexpr int NOUT = MT * NT * 256;
  constexpr int PL = EK == 3 ? (NOUT + WAVES * 64 - 1) / (WAVES * 64) : 1;
  uint16_t hpre[PL], gpre[PL];
  if constexpr (EK == 3) {
#pragma unroll
    for (int u = 0; u < PL; ++u) {
      const int o = threadIdx.x + u * WAVES * 64;
      const int i = (o >> 8) / NT, j = (o >> 8) % NT;
      const int m = i * 16 + ((o & 63) >> 4) * 4 + ((o >> 6) & 3);
      const int64_t n = (t0 + j) * 16 + (o & 15);
      if constexpr (WAVES <= 8) {
        // without branches, so both loads stay in flight through the main loop (guarded, each
        // took its own round trip first): a dead output (o past NOUT or m past M: n is still a
        // column of the slab) reads row M - 1 of its column, and gpre is used only when a.g is
        // set. Measured slower with 16 waves (most of them then hold dead outputs only), which
        // keep the guarded loads.
        hpre[u] = a.h[(int64_t)min(m, a.M - 1) * a.ldh + n];
        gpre[u] = (a.g ? a.g : a.h)[n];
      } else {
        const bool live = o < NOUT && m < a.M;
        hpre[u] = live ? a.h[(int64_t)m * a.ldh + n] : 0;
        gpre[u] = (live && a.g) ? a.g[n] : 0;
      }
    }
  }

  if constexpr (PF) {
    // software pipeline over the wave's batches (bt = wave, wave + WAVES, ...): the next
    // batch's loads are issued before the current one is computed, alternating two register sets
    if (wave < nbatch) {
      Batch<MT, NT, U, BITS> ra, rb;
      batch_load<MT, NT, U, BITS>(a, t0, g_lo + (int64_t)wave * U, lane, ra);
      // vmcnt(0) retires the staged row-scale partials with ra: the compiler cannot count
      // LDS-direct loads and would otherwise wait for every load in flight at each batch
      if constexpr (RS && PRE > 0) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __builtin_amdgcn_sched_barrier(0);
      }
      for (int bt = wave;;) {
        if (bt + WAVES < nbatch) batch_load<MT, NT, U, BITS>(a, t0, g_lo + (int64_t)(bt + WAVES) * U, lane, rb);
        batch_compute<MT, NT, U, BITS>(ra, acc);
        bt += WAVES;
        if (bt >= nbatch) break;
        if (bt + WAVES < nbatch) batch_load<MT, NT, U, BITS>(a, t0, g_lo + (int64_t)(bt + WAVES) * U, lane, ra);
        batch_compute<MT, NT, U, BITS>(rb, acc);
        bt += WAVES;
        if (bt >= nbatch) break;
      }
    }
  } else {
    // registers per thread: 512 / (waves per SIMD); the batch, the accumulators and ~48 more
    constexpr bool kWholeBatch =
        sizeof(Batch<MT, NT, U, BITS>) / 4 + MT * NT * 4 + 48 <= 2048 / WAVES;
    for (int bt = wave; bt < nbatch; bt += WAVES) {
      Batch<MT, NT, U, BITS> r;
      batch_load<MT, NT, U, BITS>(a, t0, g_lo + (int64_t)bt * U, lane, r);
      // every load of the batch is issued before one wait for all of them (the batch is waited
      // for in full anyway): left to itself the scheduler interleaves the loads with partial
      // waits and MFMAs, so a batch took several memory round trips. Held to where the whole
      // batch fits the plan's registers (1024-thread plans with wide batches would spill). The
      // vmcnt(0) also retires staged row-scale partials, so the compiler keeps exact load counts
      // (it cannot count LDS-direct loads).
      if constexpr (kWholeBatch || (RS && PRE > 0)) {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0x0f70);
        __builtin_amdgcn_sched_barrier(0);
      }
      batch_compute<MT, NT, U, BITS>(r, acc);
    }
  }

  __shared__ float red[WAVES][NOUT];
  __shared__ float rsc[RS ? MT * 16 : 1];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][((i * NT + j) * 4 + r) * 64 + lane] = acc[i][j][r];
  constexpr bool rowscale = RS;
  if constexpr (RS) {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int m = wave + WAVES * i;
      if (m >= MT * 16) break;
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < PRE; ++j)
        if (lane + 64 * j < a.rs_tiles) s += ssq_lds[(m * PRE + j) * 64 + lane];
      for (int t = lane + 64 * PRE; t < a.rs_tiles; t += 64)
        if (m < a.M) s += a.rs_ssq[(int64_t)m * a.rs_tiles + t];
      s = wave_sum(s);
      if (lane == 0) rsc[m] = m < a.M ? rsqrtf(s / (float)a.K + a.rs_eps) : 1.0f;
    }
  }
  __syncthreads();

  // output element o: lane ln = o % 64, r = (o / 64) % 4, tile (i, j) = o / 256
  constexpr bool gated = EK == 1;
  if constexpr (EK == 3) {
    // every lane of a wave runs the same iterations (NOUT and the stride are multiples of 64),
    // so the 16-lane column sums below see whole row segments
#pragma unroll
    for (int u = 0; u < PL; ++u) {
      const int o = threadIdx.x + u * WAVES * 64;
      if (o >= NOUT) break;
      const int i = (o >> 8) / NT, j = (o >> 8) % NT;
      const int m = i * 16 + ((o & 63) >> 4) * 4 + ((o >> 6) & 3);
      const bool live = m < a.M;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) v += red[w][o];
      const int64_t n = (t0 + j) * 16 + (o & 15);
      float hn = 0.0f;
      if (live) {
        const uint16_t hb = f32_to_bf16(bf16_to_f32(hpre[u]) + v);
        a.h[(int64_t)m * a.ldh + n] = hb;
        hn = bf16_to_f32(hb);
        if (a.copy) a.copy[(int64_t)m * a.ldc + n] = hb;
        if (a.y)
          reinterpret_cast<uint16_t*>(a.y)[apack_index(m, n, a.N / 64)] =
              a.g ? f32_to_bf16(hn * bf16_to_f32(gpre[u])) : hb;
      }
      const float sq = sum16_lanes(hn * hn);
      if (live && a.ssq_out && (o & 15) == 0) a.ssq_out[(int64_t)m * (a.N / 16) + t0 + j] = sq;
    }
    return;
  }
  for (int o = threadIdx.x; o < NOUT; o += WAVES * 64) {
    const int i = (o >> 8) / NT, j = (o >> 8) % NT;
    const int m = i * 16 + ((o & 63) >> 4) * 4 + ((o >> 6) & 3);
    if (m >= a.M || (gated && (j & 1))) continue;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) v += red[w][o];
    if constexpr (rowscale) v *= rsc[m];
    const int64_t n = (t0 + j) * 16 + (o & 15);
    if constexpr (EK == 2) {
      reinterpret_cast<float*>(a.y)[((int64_t)ks * a.M + m) * a.N + n] = v;
    } else if constexpr (!gated) {
      gemm_store(a, m, n, v);
    } else {
      float u = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) u += red[w][o + 256];
      if constexpr (rowscale) u *= rsc[m];
      gemm_store_gated(a, m, ((t0 + j) >> 1) * 16 + (o & 15), v, u);
    }
  }
}

// =====================================================================================
// embedding gather
// =====================================================================================
__global__ void w8_embed_kernel(const int32_t* __restrict__ ids, const uint8_t* __restrict__ q,
                                const uint16_t* __restrict__ s, const uint16_t* __restrict__ b,
                                int64_t V, int64_t H, float scale, uint16_t* __restrict__ out,
                                int64_t ldo) {
  const int i = blockIdx.y;
  int64_t row = ids[i];
  if (row < 0 || row >= V) row = 0;  // out-of-range ids read row 0 (never out of bounds)
  const int64_t G = H / 64;
  for (int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; k < H; k += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = k / 64;
    float w = bf16_to_f32(s[row * G + g]) * (float)q[row * H + k] + bf16_to_f32(b[row * G + g]);
    w = round_bf16(w);
    out[(int64_t)i * ldo + k] = f32_to_bf16(w * scale);
  }
}

// =====================================================================================
// host side: tile selection
// =====================================================================================
struct GemmPlan {
  int nt, u, waves, sk;
  int64_t gpb;
  bool pf;
};

// NT tiles per workgroup amortise the activation reads (L2 -> CU traffic is the limit once
// the weights stream at full rate); K splits (partial outputs only) bring small-N projections
// to >= 512 workgroups; 4 waves per workgroup with several 2-group batches each, or up to 16
// waves of one batch when a split is short (wide short-K partials, like the fused qkv: pairs of
// tiles, 4 K splits, 8 waves). Rules fitted to a sweep on MI355X at M = 16 over
// the Qwen3-8B verify shapes (qkv 6144x4096, o 4096x4096, gate_up 24576x4096, down
// 4096x12288, head 151936x4096): each lands within 5% of the best configuration measured.
// Plans measured best for the verify-step shapes of the five benchmark configurations where the
// rules below land more than ~3% behind (bench.py --gemm-sweep M --target T: every plan of each
// shape timed in a graph of one launch per layer). Key: row tiles, N, K, epilogue family
// (0 store, 1 gated, 2 split-K partial, 3 residual), 8-bit codes.
struct TunedPlan {
  int mt;
  int64_t n, k;
  int fam;
  int nt, u, waves, sk;
  bool pf;
  int bits;
};
static const TunedPlan kTunedPlans[] = {
    // Qwen3-8B, 16-row verify: qkv 7.35 us (rules 8.38), down 14.37 (14.97), o 6.94 (7.15);
    // gate_up 21.59 (21.70), in the verify step 2850 -> 2842 us
    {1, 6144, 4096, 2, 3, 2, 16, 2, false, 8},
    {1, 4096, 12288, 3, 1, 2, 8, 1, false, 8},
    {1, 4096, 4096, 3, 1, 2, 16, 1, true, 8},
    {1, 24576, 4096, 1, 2, 2, 8, 1, false, 8},
    // Qwen3-0.6B, 9-row verify: qkv 3.32 (3.60), gate_up 4.88 (6.37), head 38.8 (40.7)
    {1, 4096, 1024, 2, 1, 4, 4, 1, true, 8},
    {1, 6144, 1024, 1, 2, 2, 16, 1, true, 8},
    {1, 151936, 1024, 0, 4, 2, 4, 1, false, 8},
    // Gemma-style 12B (sandwich norms), 9-row verify: o 5.41 (5.81), gate_up 24.2 (25.7),
    // down 13.0 (14.3), head 176.4 (179.6)
    {1, 3840, 4096, 2, 2, 2, 8, 2, false, 8},
    {1, 30720, 3840, 1, 4, 2, 8, 1, false, 8},
    {1, 3840, 15360, 2, 2, 2, 8, 2, false, 8},
    {1, 262144, 3840, 0, 4, 2, 8, 1, false, 8},
    // Qwen3-8B, 17-row verify (16 drafts and the bonus row): qkv 9.52 (10.13), gate_up 30.4 (33.3)
    {2, 6144, 4096, 2, 2, 2, 8, 4, false, 8},
    {2, 24576, 4096, 1, 2, 2, 8, 1, false, 8},
    // Qwen3-8B, 36-row batch: qkv 11.85 (12.46)
    {3, 6144, 4096, 2, 2, 2, 4, 4, false, 8},
    // 4-bit DFlash drafter of the Qwen3-8B shape: 16 block rows o 7.22 (7.76), gate_up 16.82
    // (19.09), down 10.67 (12.61); 17 context rows fc 20.76 (22.14), k|v 7.33 (8.10)
    {1, 4096, 4096, 2, 4, 2, 4, 8, true, 4},
    {1, 24576, 4096, 1, 6, 2, 8, 1, false, 4},
    {1, 4096, 12288, 2, 4, 4, 8, 4, false, 4},
    {2, 4096, 20480, 2, 4, 2, 8, 4, false, 4},
    {2, 2048, 4096, 2, 2, 2, 8, 8, false, 4},
};

static GemmPlan plan_gemm(int M, int64_t N, int64_t K, int epi, int bits = 8) {
  const int64_t G = K / 64;
  const int64_t tiles = N / 16;
  const int MT = (M + 15) / 16;
  const bool partial = epi == DSK_EPI_PARTIAL, gated = epi == DSK_EPI_SWIGLU || epi == DSK_EPI_GEGLU;
  GemmPlan p;
  const int fam = partial ? 2 : (gated ? 1 : (epi == DSK_EPI_RESIDUAL ? 3 : 0));
  for (const TunedPlan& t : kTunedPlans)
    if (t.bits == bits && t.mt == MT && t.n == N && t.k == K && t.fam == fam) {
      p.nt = t.nt;
      p.u = t.u;
      p.waves = t.waves;
      p.sk = t.sk;
      p.gpb = ((G / t.u + t.sk - 1) / t.sk) * t.u;
      p.pf = t.pf;
      return p;
    }
  if (epi == DSK_EPI_RESIDUAL) {
    // the residual-add epilogue needs whole rows of the product in one workgroup: no K split;
    // one tile per workgroup and up to 16 waves splitting K (reduced through LDS)
    p.nt = 1;
    p.sk = 1;
    p.u = ((MT == 1 || MT == 3) && G / 4 >= 16 && G % 4 == 0) ? 4 : 2;
    p.gpb = G;
    const int64_t nb = G / p.u;
    p.waves = nb >= 16 ? 16 : (nb >= 8 ? 8 : 4);
    // more than one row tile (a sweep at M = 24, 36, 64 over o 4096x4096 and down 4096x12288):
    // 8 waves of 2-group batches at two and four tiles, 16 waves of 4-group batches at three
    if ((MT == 2 || MT == 4) && p.waves > 8) p.waves = 8;
    while ((size_t)p.waves * MT * 1024 > 65536) p.waves /= 2;
    p.pf = false;  // pipelined loads measured slower here (down 4096x12288: 18.5 -> 23.2 us)
    return p;
  }
  p.u = 2;
  if (partial) p.nt = G >= 128 ? 4 : 2;
  else p.nt = 4;
  if (MT > 2 && p.nt > 2) p.nt = 2;
  while (p.nt > 1 && tiles % p.nt) p.nt /= 2;
  if (gated && p.nt < 2) p.nt = 2;
  const int64_t slabs = tiles / p.nt;
  const int64_t batches = G / p.u;  // per tile
  p.sk = 1;
  if (partial)
    // at most 8 splits: the consumer sums every slice of each row in one workgroup (16 slices of
    // the Gemma-style 12B down projection, 3840 x 15360, cost that sum 20.7 us per layer against
    // 6.6 us for 8, more than the GEMM loses: 6436 -> 5647 us per 9-row verify step)
    while (slabs * p.sk < 512 && batches / (p.sk * 2) >= 4 && p.sk < 8) p.sk *= 2;
  // batches per split, rounded up: the last split takes what is left (K = 9728 in 8 splits:
  // 7 x 20 groups + 12)
  const int64_t bps = (batches + p.sk - 1) / p.sk;
  p.gpb = bps * p.u;
  p.waves = (bps >= 8 && bps < 12) ? 8 : 4;
  if (!partial && slabs < 128) p.waves = bps >= 32 ? 16 : (bps >= 8 ? 8 : 4);
  p.pf = false;
  // wide gated projections (>= 1024 tiles): pairs of tiles, 8 waves, pipelined loads (4-group
  // batches won a standalone sweep at M = 16 but not the verify forward, and slowed the Gemma-style
  // GeGLU projection)
  if (gated && MT == 1 && tiles >= 1024 && tiles % 2 == 0) {
    p.nt = 2;
    p.sk = 1;
    p.gpb = G;
    p.waves = 8;
    p.pf = true;
  }
  // one row tile, a sweep at M = 16 over the Qwen3-8B verify shapes: wide partial sums with a long K (qkv 6144x4096) run whole K
  // ranges in pairs of tiles, 16 waves, pipelined loads (8.7 us against 10.5 for 4 K splits of
  // 8 waves); wide plain stores (the logits, 151936x4096) 8 waves (110.4 against 117.9 us)
  if (MT == 1 && bits == 8 && partial && G >= 64 && tiles >= 384 && tiles % 2 == 0) {
    p.nt = 2;
    p.sk = 1;
    p.u = 2;
    p.gpb = G;
    p.waves = 16;
    p.pf = true;
  }
  if (MT == 1 && bits == 8 && epi == DSK_EPI_STORE && tiles >= 4096 && G >= 64 && p.nt == 4) p.waves = 8;
  // more than one row tile, from a sweep at M = 24, 36 and 64 over the Qwen3-8B verify shapes
  // (the 16-row rules above stay as fitted): the activation rows read per weight byte grow with
  // M, and the plans that won keep whole K ranges and wide slabs. Partial sums: pairs of tiles,
  // no K split, 16 waves at two tiles, 8 above (qkv 6144x4096 at M = 36: 27.2 -> 17.6 us); gated:
  // 8 waves at four tiles (gate_up 24576x4096 at M = 64: 72.1 -> 63.6 us); plain stores (the
  // logits): slabs of 4 tiles at two and three (head 151936x4096 at M = 36: 223.5 -> 192.4 us).
  if (MT >= 2 && bits == 8) {
    if (partial) {
      p.nt = tiles % 2 == 0 ? 2 : 1;
      p.sk = 1;
      p.u = 2;
      p.gpb = G;
      p.waves = MT == 2 ? 16 : 8;
    } else if (gated) {
      p.waves = MT >= 4 ? 8 : p.waves;
    } else if (MT <= 3 && tiles % 4 == 0) {
      p.nt = 4;
      p.u = 2;
      p.gpb = G;
      p.waves = 4;
    }
  }
  while ((size_t)p.waves * MT * p.nt * 1024 > 65536) p.waves /= 2;  // LDS of the reduction
  // 4-bit codes: a wave's load of one tile-group is 512 B, half the 8-bit one. Where the waves
  // of the plan above each run several unpipelined batches (4 waves: down, the head), batches
  // of 4 groups halve the iterations at the same bytes in flight (W4 down 4096x12288 at M = 16:
  // 13.6 -> 10.6 us, head 151936x4096: 120 -> 71 us); with 8 waves of one batch each (qkv, o)
  // or the pipelined gated plan, 2-group batches measured faster.
  if (bits == 4 && MT == 1 && !p.pf && p.waves == 4 && (p.nt == 1 || p.nt == 2 || p.nt == 4)) {
    p.u = 4;
    p.gpb = ((G / 4 + p.sk - 1) / p.sk) * 4;
  }
  return p;
}

template <int MT, int NT, int U, int WAVES, bool PF, int BITS>
static bool launch_gemm_t(const GemmArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)(a.n_slabs * a.SK)), blk(WAVES * 64);
  const bool rs = a.rs_ssq != nullptr;
  if (a.epi == DSK_EPI_PARTIAL) {
    if (rs) hipLaunchKernelGGL((w8_gemm_kernel<MT, NT, U, WAVES, 6, PF, BITS>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((w8_gemm_kernel<MT, NT, U, WAVES, 2, PF, BITS>), grid, blk, 0, st, a);
  } else if (a.epi == DSK_EPI_RESIDUAL) {
    if constexpr (NT > 2) return false;
    else if (rs) return false;  // the residual products' x (attention output, gated MLP) is never normed later
    else hipLaunchKernelGGL((w8_gemm_kernel<MT, NT, U, WAVES, 3, PF, BITS>), grid, blk, 0, st, a);
  } else if (a.epi == DSK_EPI_STORE) {
    if (rs) hipLaunchKernelGGL((w8_gemm_kernel<MT, NT, U, WAVES, 4, PF, BITS>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((w8_gemm_kernel<MT, NT, U, WAVES, 0, PF, BITS>), grid, blk, 0, st, a);
  } else {
    if constexpr (NT % 2 != 0) return false;  // gated tiles come in gate|up pairs
    else if (rs) hipLaunchKernelGGL((w8_gemm_kernel<MT, NT, U, WAVES, 5, PF, BITS>), grid, blk, 0, st, a);
    else hipLaunchKernelGGL((w8_gemm_kernel<MT, NT, U, WAVES, 1, PF, BITS>), grid, blk, 0, st, a);
  }
  return true;
}

template <int MT, int NT, int U, bool PF, int BITS>
static bool launch_gemm_w(const GemmArgs& a, int waves, hipStream_t st) {
  constexpr int max_waves = 65536 / (MT * NT * 1024);  // LDS of the cross-wave reduction
  switch (waves) {
    case 4: if constexpr (max_waves >= 4) return launch_gemm_t<MT, NT, U, 4, PF, BITS>(a, st); return false;
    case 8: if constexpr (max_waves >= 8) return launch_gemm_t<MT, NT, U, 8, PF, BITS>(a, st); return false;
    case 16: if constexpr (max_waves >= 16) return launch_gemm_t<MT, NT, U, 16, PF, BITS>(a, st); return false;
  }
  return false;
}

template <int BITS>
static bool launch_gemm_bits(const GemmArgs& a, int MT, const GemmPlan& p, hipStream_t st) {
  if (p.pf) {  // the pipelined variant is built for the shapes the planner gives it
    if (MT == 1 && p.nt == 2 && p.u == 2) return launch_gemm_w<1, 2, 2, true, BITS>(a, p.waves, st);
    if (MT == 1 && p.nt == 2 && p.u == 4) return launch_gemm_w<1, 2, 4, true, BITS>(a, p.waves, st);
    if (MT == 1 && p.nt == 4 && p.u == 2) return launch_gemm_w<1, 4, 2, true, BITS>(a, p.waves, st);
    if (MT == 1 && p.nt == 1 && p.u == 4) return launch_gemm_w<1, 1, 4, true, BITS>(a, p.waves, st);
    if (MT == 1 && p.nt == 1 && p.u == 2) return launch_gemm_w<1, 1, 2, true, BITS>(a, p.waves, st);
    return false;
  }
#define DSK_GEMM_CASE(MT_, NT_, U_) \
  if (MT == MT_ && p.nt == NT_ && p.u == U_) return launch_gemm_w<MT_, NT_, U_, false, BITS>(a, p.waves, st);
  DSK_GEMM_CASE(1, 1, 2) DSK_GEMM_CASE(1, 2, 2) DSK_GEMM_CASE(1, 4, 2) DSK_GEMM_CASE(1, 8, 2)
  DSK_GEMM_CASE(1, 3, 2) DSK_GEMM_CASE(1, 6, 2)
  DSK_GEMM_CASE(1, 1, 4) DSK_GEMM_CASE(1, 2, 4) DSK_GEMM_CASE(1, 4, 4)
  DSK_GEMM_CASE(2, 1, 2) DSK_GEMM_CASE(2, 2, 2) DSK_GEMM_CASE(2, 4, 2)
  DSK_GEMM_CASE(3, 1, 2) DSK_GEMM_CASE(3, 2, 2) DSK_GEMM_CASE(3, 4, 2) DSK_GEMM_CASE(3, 1, 4)
  DSK_GEMM_CASE(4, 1, 2) DSK_GEMM_CASE(4, 2, 2)
#undef DSK_GEMM_CASE
  return false;
}

static bool launch_gemm(const GemmArgs& a, int MT, const GemmPlan& p, hipStream_t st) {
  return a.bits == 4 ? launch_gemm_bits<4>(a, MT, p, st) : launch_gemm_bits<8>(a, MT, p, st);
}

// Fills GemmArgs for a plan; shared by the entry point and the tuning harness.
static void gemm_prepare(GemmArgs& a, const GemmPlan& p, const void* xp, const uint8_t* wt, const uint32_t* sb,
                         int M, int64_t N, int64_t K, int epi, void* y, int y_dtype, int64_t ldy,
                         const uint16_t* residual, int64_t ldr, float softcap) {
  a.xp = reinterpret_cast<const u32x4*>(xp);
  a.wt = reinterpret_cast<const u32x4*>(wt);
  a.sb = sb;
  a.M = M;
  a.N = N;
  a.K = K;
  a.G = K / 64;
  a.SK = p.sk;
  a.gpb = p.gpb;
  a.n_slabs = (int)(N / 16 / p.nt);
  a.epi = epi;
  a.y = y;
  a.y_f32 = (y_dtype == DSK_F32);
  a.ldy = ldy;
  a.res = residual;
  a.ldr = ldr;
  a.softcap = softcap;
  a.bits = 8;
  a.rs_ssq = nullptr;
  a.rs_tiles = 0;
  a.rs_eps = 0.0f;
  a.h = nullptr;
  a.ldh = 0;
  a.copy = nullptr;
  a.ldc = 0;
  a.g = nullptr;
  a.ssq_out = nullptr;
}

// chunks per thread (NV) x split slices kept in registers (MAXS): NV * MAXS <= 16
static bool pack_launch(const PackArgs& a, hipStream_t st) {
  const int64_t per = ceil_div(a.K / 8, kPackThreads);
  const int S = a.part ? a.nsplit : 0;
  const int ms = S == 0 ? 0 : (S <= 4 ? 4 : (S <= 8 ? 8 : 16));
  const dim3 grid((unsigned)a.M), blk(kPackThreads);
#define DSK_PACK_CASE(NV_, MS_) \
  if (per <= NV_ && ms == MS_) { hipLaunchKernelGGL((act_pack_kernel<NV_, MS_>), grid, blk, 0, st, a); return true; }
  DSK_PACK_CASE(1, 0) DSK_PACK_CASE(1, 4) DSK_PACK_CASE(1, 8) DSK_PACK_CASE(1, 16)
  DSK_PACK_CASE(2, 0) DSK_PACK_CASE(2, 4) DSK_PACK_CASE(2, 8)
  DSK_PACK_CASE(3, 0) DSK_PACK_CASE(3, 4)
  DSK_PACK_CASE(6, 0)
#undef DSK_PACK_CASE
  return false;
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_w8_quantize(const void* w, int w_dtype, int64_t N, int64_t K, uint8_t* q,
                               uint16_t* scales, uint16_t* biases, dsk_stream_t stream) {
  DSK_REQUIRE(w && q && scales && biases, "dsk_w8_quantize: null pointer");
  DSK_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "dsk_w8_quantize: need K %% 64 == 0 (N=%lld K=%lld)",
              (long long)N, (long long)K);
  DSK_REQUIRE(w_dtype == DSK_F32 || w_dtype == DSK_BF16, "dsk_w8_quantize: dtype must be f32 or bf16");
  int64_t total = N * (K / 64);
  int threads = 256;
  hipLaunchKernelGGL(w8_quantize_kernel, dim3((unsigned)ceil_div(total, threads)), dim3(threads), 0,
                     as_stream(stream), w, w_dtype == DSK_BF16 ? 1 : 0, N, K, q, scales, biases, 255.0f);
  DSK_LAUNCH_CHECK("dsk_w8_quantize");
  return DSK_OK;
}

extern "C" int dsk_w4_quantize(const void* w, int w_dtype, int64_t N, int64_t K, uint8_t* q,
                               uint16_t* scales, uint16_t* biases, dsk_stream_t stream) {
  DSK_REQUIRE(w && q && scales && biases, "dsk_w4_quantize: null pointer");
  DSK_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "dsk_w4_quantize: need K %% 64 == 0 (N=%lld K=%lld)",
              (long long)N, (long long)K);
  DSK_REQUIRE(w_dtype == DSK_F32 || w_dtype == DSK_BF16, "dsk_w4_quantize: dtype must be f32 or bf16");
  int64_t total = N * (K / 64);
  int threads = 256;
  hipLaunchKernelGGL(w8_quantize_kernel, dim3((unsigned)ceil_div(total, threads)), dim3(threads), 0,
                     as_stream(stream), w, w_dtype == DSK_BF16 ? 1 : 0, N, K, q, scales, biases, 15.0f);
  DSK_LAUNCH_CHECK("dsk_w4_quantize");
  return DSK_OK;
}

extern "C" int dsk_w8_repack(const uint8_t* q, const uint16_t* scales, const uint16_t* biases, int64_t N,
                             int64_t K, int paired, uint8_t* wt, uint32_t* sb, dsk_stream_t stream) {
  DSK_REQUIRE(q && scales && biases && wt && sb, "dsk_w8_repack: null pointer");
  DSK_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0,
              "dsk_w8_repack: need N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  DSK_REQUIRE(!paired || N % 32 == 0, "dsk_w8_repack: paired layout needs N %% 32 == 0 (N=%lld)", (long long)N);
  int64_t total = N * K / 16;
  int threads = 256;
  hipLaunchKernelGGL(w8_repack_kernel, dim3((unsigned)ceil_div(total, threads)), dim3(threads), 0,
                     as_stream(stream), q, scales, biases, N, K, paired ? 1 : 0, reinterpret_cast<u32x4*>(wt), sb);
  DSK_LAUNCH_CHECK("dsk_w8_repack");
  return DSK_OK;
}

extern "C" int dsk_w4_repack(const uint8_t* q, const uint16_t* scales, const uint16_t* biases, int64_t N,
                             int64_t K, int paired, uint8_t* wt, uint32_t* sb, dsk_stream_t stream) {
  DSK_REQUIRE(q && scales && biases && wt && sb, "dsk_w4_repack: null pointer");
  DSK_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0,
              "dsk_w4_repack: need N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  DSK_REQUIRE(!paired || N % 32 == 0, "dsk_w4_repack: paired layout needs N %% 32 == 0 (N=%lld)", (long long)N);
  DSK_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)wt & 7) == 0, "dsk_w4_repack: q 16-byte, wt 8-byte aligned");
  int64_t total = N * K / 16;
  int threads = 256;
  hipLaunchKernelGGL(w4_repack_kernel, dim3((unsigned)ceil_div(total, threads)), dim3(threads), 0,
                     as_stream(stream), q, scales, biases, N, K, paired ? 1 : 0, reinterpret_cast<uint2*>(wt), sb);
  DSK_LAUNCH_CHECK("dsk_w4_repack");
  return DSK_OK;
}

extern "C" size_t dsk_act_pack_bytes(int M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 64) return 0;
  return (size_t)((M + 15) / 16) * (size_t)K * 32;
}

extern "C" int dsk_act_pack_scaled(const float* part, int nsplit, const uint16_t* part_norm_w, uint16_t* h,
                                   int64_t ldh, uint16_t* copy, int64_t ldc, int M, int64_t K, const uint16_t* norm_w,
                                   float eps, float out_scale, uint16_t* out, dsk_stream_t stream) {
  DSK_REQUIRE(part || h, "dsk_act_pack: needs partial sums or an input h");
  DSK_REQUIRE(out || copy || (h && part), "dsk_act_pack: no output");
  DSK_REQUIRE(!part || (nsplit > 0 && nsplit <= kPackMaxSplits), "dsk_act_pack: nsplit=%d outside [1, %d]", nsplit,
              kPackMaxSplits);
  DSK_REQUIRE(!part || (int64_t)(nsplit <= 4 ? 4 : (nsplit <= 8 ? 8 : 16)) * ceil_div(K / 8, kPackThreads) <= 16,
              "dsk_act_pack: %d partial slices of K=%lld exceed the kernel's registers", nsplit, (long long)K);
  DSK_REQUIRE(M > 0 && M <= 64, "dsk_act_pack: M=%d outside [1, 64]", M);
  DSK_REQUIRE(K > 0 && K % 64 == 0 && K <= 6 * 8 * kPackThreads,
              "dsk_act_pack: K=%lld must be a multiple of 64 <= %d", (long long)K, 6 * 8 * kPackThreads);
  DSK_REQUIRE(!h || (ldh >= K && ldh % 8 == 0), "dsk_act_pack: bad ldh");
  DSK_REQUIRE(!copy || (ldc >= K && ldc % 8 == 0), "dsk_act_pack: bad ldc");
  DSK_REQUIRE((((uintptr_t)part | (uintptr_t)h | (uintptr_t)copy | (uintptr_t)norm_w | (uintptr_t)out |
                (uintptr_t)part_norm_w) & 15) == 0,
              "dsk_act_pack: pointers must be 16-byte aligned");
  DSK_REQUIRE(!part_norm_w || part, "dsk_act_pack: part_norm_w needs partial sums");
  PackArgs a{part, nsplit, h, ldh, copy, ldc, M, K, norm_w, eps, out, part_norm_w, out_scale, nullptr};
  DSK_REQUIRE(pack_launch(a, as_stream(stream)), "dsk_act_pack: no kernel for K=%lld with %d slices", (long long)K,
              nsplit);
  DSK_LAUNCH_CHECK("dsk_act_pack");
  return DSK_OK;
}

extern "C" int dsk_act_pack_rn(const float* part, int nsplit, uint16_t* h, int64_t ldh, uint16_t* copy, int64_t ldc,
                               int M, int64_t K, const uint16_t* norm_w, uint16_t* out, float* ssq_out,
                               dsk_stream_t stream) {
  DSK_REQUIRE(h && out && ssq_out, "dsk_act_pack_rn: needs h, out and ssq_out");
  DSK_REQUIRE(!part || (nsplit > 0 && nsplit <= kPackMaxSplits), "dsk_act_pack_rn: nsplit=%d outside [1, %d]", nsplit,
              kPackMaxSplits);
  DSK_REQUIRE(!part || (int64_t)(nsplit <= 4 ? 4 : (nsplit <= 8 ? 8 : 16)) * ceil_div(K / 8, kPackThreads) <= 16,
              "dsk_act_pack_rn: %d partial slices of K=%lld exceed the kernel's registers", nsplit, (long long)K);
  DSK_REQUIRE(M > 0 && M <= 64, "dsk_act_pack_rn: M=%d outside [1, 64]", M);
  DSK_REQUIRE(K > 0 && K % 64 == 0 && K <= 6 * 8 * kPackThreads,
              "dsk_act_pack_rn: K=%lld must be a multiple of 64 <= %d", (long long)K, 6 * 8 * kPackThreads);
  DSK_REQUIRE(ldh >= K && ldh % 8 == 0 && (!copy || (ldc >= K && ldc % 8 == 0)), "dsk_act_pack_rn: bad row stride");
  DSK_REQUIRE((((uintptr_t)part | (uintptr_t)h | (uintptr_t)copy | (uintptr_t)norm_w | (uintptr_t)out) & 15) == 0,
              "dsk_act_pack_rn: pointers must be 16-byte aligned");
  PackArgs a{part, nsplit, h, ldh, copy, ldc, M, K, norm_w, 0.0f, out, nullptr, 1.0f, ssq_out};
  DSK_REQUIRE(pack_launch(a, as_stream(stream)), "dsk_act_pack_rn: no kernel for K=%lld with %d slices", (long long)K,
              nsplit);
  DSK_LAUNCH_CHECK("dsk_act_pack_rn");
  return DSK_OK;
}

extern "C" int dsk_act_pack(const float* part, int nsplit, const uint16_t* part_norm_w, uint16_t* h, int64_t ldh,
                            uint16_t* copy, int64_t ldc, int M, int64_t K, const uint16_t* norm_w, float eps,
                            uint16_t* out, dsk_stream_t stream) {
  return dsk_act_pack_scaled(part, nsplit, part_norm_w, h, ldh, copy, ldc, M, K, norm_w, eps, 1.0f, out, stream);
}

extern "C" int dsk_w8_gemm_splits(int M, int64_t N, int64_t K) {
  if (M <= 0 || M > 64 || N <= 0 || N % 16 || K <= 0 || K % 256) return 0;
  return plan_gemm(M, N, K, DSK_EPI_PARTIAL).sk;
}

extern "C" int dsk_w4_gemm_splits(int M, int64_t N, int64_t K) {
  if (M <= 0 || M > 64 || N <= 0 || N % 16 || K <= 0 || K % 256) return 0;
  return plan_gemm(M, N, K, DSK_EPI_PARTIAL, 4).sk;
}

struct NormIO {
  const float* x_ssq;  // row scale of x (normed later), or null
  int x_tiles;
  float eps;
  uint16_t* h;         // DSK_EPI_RESIDUAL
  int64_t ldh;
  uint16_t* copy;
  int64_t ldc;
  const uint16_t* next_w;
  float* ssq_out;
};

static int gemm_entry(const char* who, int bits, const uint16_t* xp, const uint8_t* wt, const uint32_t* sb, int M,
                      int64_t N, int64_t K, int epi, void* y, int y_dtype, int64_t ldy, const uint16_t* residual,
                      int64_t ldr, float softcap, hipStream_t st, const NormIO* nio = nullptr,
                      const GemmPlan* forced = nullptr);

extern "C" int dsk_w8_gemm(const uint16_t* xp, const uint8_t* wt, const uint32_t* sb, int M, int64_t N, int64_t K,
                           int epi, void* y, int y_dtype, int64_t ldy, const uint16_t* residual, int64_t ldr,
                           float softcap, dsk_stream_t stream) {
  return gemm_entry("dsk_w8_gemm", 8, xp, wt, sb, M, N, K, epi, y, y_dtype, ldy, residual, ldr, softcap,
                    as_stream(stream));
}

extern "C" int dsk_w4_gemm(const uint16_t* xp, const uint8_t* wt, const uint32_t* sb, int M, int64_t N, int64_t K,
                           int epi, void* y, int y_dtype, int64_t ldy, const uint16_t* residual, int64_t ldr,
                           float softcap, dsk_stream_t stream) {
  return gemm_entry("dsk_w4_gemm", 4, xp, wt, sb, M, N, K, epi, y, y_dtype, ldy, residual, ldr, softcap,
                    as_stream(stream));
}

extern "C" int dsk_w8_gemm_rn(const uint16_t* xp, const uint8_t* wt, const uint32_t* sb, int bits, int M, int64_t N,
                              int64_t K, int epi, void* y, int y_dtype, int64_t ldy, float softcap, const float* x_ssq,
                              int x_tiles, float eps, uint16_t* h, int64_t ldh, uint16_t* copy, int64_t ldc,
                              const uint16_t* next_norm_w, float* ssq_out, dsk_stream_t stream) {
  DSK_REQUIRE(bits == 8 || bits == 4, "dsk_w8_gemm_rn: bits=%d (8 or 4)", bits);
  DSK_REQUIRE(!x_ssq || (x_tiles == K / 16 && eps >= 0.0f),
              "dsk_w8_gemm_rn: the row scale of x needs K / 16 = %lld tile partials (got %d)", (long long)(K / 16),
              x_tiles);
  NormIO nio{x_ssq, x_ssq ? x_tiles : 0, eps, h, ldh, copy, ldc, next_norm_w, ssq_out};
  return gemm_entry("dsk_w8_gemm_rn", bits, xp, wt, sb, M, N, K, epi, y, y_dtype, ldy, nullptr, 0, softcap,
                    as_stream(stream), &nio);
}

extern "C" int dsk_w8_gemm_rn_planned(const uint16_t* xp, const uint8_t* wt, const uint32_t* sb, int bits, int M,
                                      int64_t N, int64_t K, int epi, void* y, int y_dtype, int64_t ldy, float softcap,
                                      const float* x_ssq, int x_tiles, float eps, uint16_t* h, int64_t ldh,
                                      uint16_t* copy, int64_t ldc, const uint16_t* next_norm_w, float* ssq_out,
                                      int slab_tiles, int batch_groups, int waves, int k_splits, int pipelined,
                                      dsk_stream_t stream) {
  const char* who = "dsk_w8_gemm_rn_planned";
  DSK_REQUIRE(bits == 8 || bits == 4, "%s: bits=%d (8 or 4)", who, bits);
  DSK_REQUIRE(!x_ssq || (x_tiles == K / 16 && eps >= 0.0f), "%s: the row scale of x needs K / 16 tile partials",
              who);
  const int64_t G = K / 64, tiles = N / 16;
  const int MT = (M + 15) / 16;
  DSK_REQUIRE(slab_tiles >= 1 && slab_tiles <= 8 && N % 16 == 0 && tiles % slab_tiles == 0,
              "%s: %d tiles per slab do not divide N / 16 = %lld", who, slab_tiles, (long long)tiles);
  DSK_REQUIRE((batch_groups == 2 || batch_groups == 4) && K % 64 == 0 && G % batch_groups == 0,
              "%s: batches of %d groups", who, batch_groups);
  DSK_REQUIRE(waves == 4 || waves == 8 || waves == 16, "%s: %d waves", who, waves);
  DSK_REQUIRE(k_splits >= 1 && (k_splits == 1 || epi == DSK_EPI_PARTIAL) && k_splits <= G / batch_groups,
              "%s: %d K splits (partial sums only, at most one batch each)", who, k_splits);
  DSK_REQUIRE((size_t)waves * MT * slab_tiles * 1024 <= 65536, "%s: the cross-wave reduction exceeds 64 KB of LDS",
              who);
  GemmPlan p;
  p.nt = slab_tiles;
  p.u = batch_groups;
  p.waves = waves;
  p.sk = k_splits;
  p.gpb = ((G / batch_groups + k_splits - 1) / k_splits) * batch_groups;
  p.pf = pipelined != 0;
  NormIO nio{x_ssq, x_ssq ? x_tiles : 0, eps, h, ldh, copy, ldc, next_norm_w, ssq_out};
  return gemm_entry(who, bits, xp, wt, sb, M, N, K, epi, y, y_dtype, ldy, nullptr, 0, softcap, as_stream(stream),
                    &nio, &p);
}

extern "C" int dsk_w8_gemm_plan(int M, int64_t N, int64_t K, int epi, int bits, int* plan) {
  DSK_REQUIRE(plan, "dsk_w8_gemm_plan: null output");
  DSK_REQUIRE(bits == 8 || bits == 4, "dsk_w8_gemm_plan: bits=%d (8 or 4)", bits);
  DSK_REQUIRE(M > 0 && M <= 64 && N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0,
              "dsk_w8_gemm_plan: shape M=%d N=%lld K=%lld outside the GEMM's limits", M, (long long)N, (long long)K);
  const GemmPlan p = plan_gemm(M, N, K, epi, bits);
  plan[0] = p.nt;
  plan[1] = p.u;
  plan[2] = p.waves;
  plan[3] = p.sk;
  plan[4] = p.pf ? 1 : 0;
  return DSK_OK;
}

static int gemm_entry(const char* who, int bits, const uint16_t* xp, const uint8_t* wt, const uint32_t* sb, int M,
                      int64_t N, int64_t K, int epi, void* y, int y_dtype, int64_t ldy, const uint16_t* residual,
                      int64_t ldr, float softcap, hipStream_t st, const NormIO* nio, const GemmPlan* forced) {
  DSK_REQUIRE(xp && wt && sb && (y || epi == DSK_EPI_RESIDUAL), "dsk_w8_gemm: null pointer");
  DSK_REQUIRE(M > 0 && M <= 64, "dsk_w8_gemm: M=%d outside [1, 64]", M);
  DSK_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0,
              "dsk_w8_gemm: need N %% 16 == 0, K %% 256 == 0 (N=%lld K=%lld)", (long long)N, (long long)K);
  DSK_REQUIRE(((uintptr_t)xp & 15) == 0 && ((uintptr_t)wt & 15) == 0, "dsk_w8_gemm: x and W must be 16-byte aligned");
  DSK_REQUIRE(epi >= DSK_EPI_STORE && epi <= (nio ? DSK_EPI_RESIDUAL : DSK_EPI_PARTIAL), "%s: bad epilogue %d", who,
              epi);
  const bool gated = epi == DSK_EPI_SWIGLU || epi == DSK_EPI_GEGLU;
  if (epi == DSK_EPI_RESIDUAL) {
    DSK_REQUIRE(nio->h && nio->ldh >= N && (!nio->copy || nio->ldc >= N), "%s: the residual epilogue needs h [M, N]"
                " (and copy) with row strides >= N", who);
    DSK_REQUIRE(N % 64 == 0, "%s: the residual epilogue needs N %% 64 == 0 (N=%lld)", who, (long long)N);
    DSK_REQUIRE(!y || y_dtype == DSK_BF16, "%s: the residual epilogue's packed output is bf16", who);
    DSK_REQUIRE(!nio->next_w || nio->ssq_out, "%s: a later-normed output needs ssq_out", who);
    DSK_REQUIRE(softcap == 0.0f, "%s: no soft-cap in the residual epilogue", who);
  } else if (epi == DSK_EPI_STORE) {
    DSK_REQUIRE(y_dtype == DSK_F32 || y_dtype == DSK_BF16, "dsk_w8_gemm: y dtype must be f32 or bf16");
    DSK_REQUIRE(ldy >= N, "dsk_w8_gemm: ldy=%lld < N", (long long)ldy);
    DSK_REQUIRE(!residual || ldr >= N, "dsk_w8_gemm: ldr=%lld < N", (long long)ldr);
    DSK_REQUIRE(!(residual && y_dtype != DSK_BF16 && (const void*)residual == y),
                "dsk_w8_gemm: in-place residual needs bf16 output");
  } else {
    DSK_REQUIRE(!residual && softcap == 0.0f, "dsk_w8_gemm: residual / soft-cap need DSK_EPI_STORE");
    DSK_REQUIRE(!gated || (N % 256 == 0 && y_dtype == DSK_BF16),
                "dsk_w8_gemm: gated epilogue needs N %% 256 == 0 and a bf16 (packed) output");
    DSK_REQUIRE(gated || y_dtype == DSK_F32, "dsk_w8_gemm: partial sums are f32");
  }
  const GemmPlan p = forced ? *forced : plan_gemm(M, N, K, epi, bits);
  DSK_REQUIRE(!(gated && p.nt % 2), "%s: gated tiles come in gate|up pairs (slab of %d tiles)", who, p.nt);
  GemmArgs a;
  gemm_prepare(a, p, xp, wt, sb, M, N, K, epi, y, y_dtype, ldy, residual, ldr, softcap);
  a.bits = bits;
  if (nio) {
    a.rs_ssq = nio->x_ssq;
    a.rs_tiles = nio->x_tiles;
    a.rs_eps = nio->eps;
    if (epi == DSK_EPI_RESIDUAL) {
      a.h = nio->h;
      a.ldh = nio->ldh;
      a.copy = nio->copy;
      a.ldc = nio->ldc;
      a.g = nio->next_w;
      a.ssq_out = nio->ssq_out;
    }
  }
  if (!launch_gemm(a, (M + 15) / 16, p, st)) {
    set_error("%s: no kernel for M=%d NT=%d U=%d waves=%d", who, M, p.nt, p.u, p.waves);
    return DSK_EINVAL;
  }
  DSK_LAUNCH_CHECK(who);
  return DSK_OK;
}

extern "C" int dsk_w8_embed(const int32_t* ids, int n, const uint8_t* q, const uint16_t* scales,
                            const uint16_t* biases, int64_t V, int64_t H, float scale, uint16_t* out,
                            int64_t ldo, dsk_stream_t stream) {
  DSK_REQUIRE(ids && q && scales && biases && out, "dsk_w8_embed: null pointer");
  DSK_REQUIRE(n > 0 && V > 0 && H > 0 && H % 64 == 0 && ldo >= H, "dsk_w8_embed: bad shape");
  dim3 grid((unsigned)ceil_div(H, 256), (unsigned)n);
  hipLaunchKernelGGL(w8_embed_kernel, grid, dim3(256), 0, as_stream(stream), ids, q, scales, biases, V, H,
                     scale, out, ldo);
  DSK_LAUNCH_CHECK("dsk_w8_embed");
  return DSK_OK;
}
