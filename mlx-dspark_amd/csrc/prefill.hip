// Dense prefill pieces on gfx950: W8/W4 weights expanded to bf16 rows (once per layer, for the
// library GEMM of a long prompt), and the row-wise RMSNorm and gated activations that sit between
// those GEMMs. Every kernel works on plain row-major bf16 [M, K] activations of any row count.
#include "common.h"

namespace dsk {

// source row of tile row 16 t + r (paired gate|up repacks interleave the halves' tiles)
__device__ __forceinline__ int64_t tiled_src_row(int64_t t, int r, int64_t N, int paired) {
  if (!paired) return t * 16 + r;
  return (t & 1) * (N / 2) + (t >> 1) * 16 + r;
}

// One thread per (tile, group, lane) chunk of 16 codes: out[n][k] = bf16(s * q + b) for the chunk's
// 16 columns of source row n (the tile order undone, so a paired weight comes out gate rows
// first, then up rows).
template <int BITS>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ wt,
                                                           const uint32_t* __restrict__ sb, int64_t N, int64_t K,
                                                           int paired, uint16_t* __restrict__ out) {
  const int64_t G = K / 64;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= N * K / 16) return;
  const int lane = (int)(idx & 63);
  const int64_t tg = idx >> 6, g = tg % G, t = tg / G;
  const int r = lane & 15, c = lane >> 4;
  const uint32_t sbv = sb[(t * G + g) * 16 + r];
  const float s = bf16_to_f32((uint16_t)(sbv & 0xffffu)), b = bf16_to_f32((uint16_t)(sbv >> 16));
  uint32_t codes[4];
  if constexpr (BITS == 8) {
    const u32x4 w = reinterpret_cast<const u32x4*>(wt)[idx];
#pragma unroll
    for (int i = 0; i < 4; ++i) codes[i] = w[i];
  } else {
    // byte j holds columns 2j (low nibble) and 2j + 1 (high nibble): spread to one code per byte
    const uint2 w = reinterpret_cast<const uint2*>(wt)[idx];
    const uint32_t ww[2] = {w.x, w.y};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t v = ww[h];
      uint32_t o0 = 0, o1 = 0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t by0 = (v >> (8 * j)) & 0xffu, by1 = (v >> (8 * (j + 2))) & 0xffu;
        o0 |= ((by0 & 0xfu) | ((by0 >> 4) << 8)) << (16 * j);
        o1 |= ((by1 & 0xfu) | ((by1 >> 4) << 8)) << (16 * j);
      }
      codes[2 * h] = o0;
      codes[2 * h + 1] = o1;
    }
  }
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t q = codes[i / 2] >> (16 * (i & 1));
    const float w0 = fmaf(s, (float)(q & 0xffu), b), w1 = fmaf(s, (float)((q >> 8) & 0xffu), b);
    o[i] = (uint32_t)f32_to_bf16(w0) | ((uint32_t)f32_to_bf16(w1) << 16);
  }
  const int64_t n = tiled_src_row(t, r, N, paired);
  u32x4* dst = reinterpret_cast<u32x4*>(out + n * K + g * 64 + c * 16);
  dst[0] = u32x4{o[0], o[1], o[2], o[3]};
  dst[1] = u32x4{o[4], o[5], o[6], o[7]};
}

// One workgroup per row: y = bf16((x * rsqrt(mean(x^2) + eps)) * w), the normalise-first
// RMSNorm (the same formula as the activation pack's norm).
constexpr int kRowThreads = 256;
__global__ __launch_bounds__(kRowThreads) void rows_rmsnorm_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                   const uint16_t* __restrict__ w, float eps,
                                                                   int64_t K, uint16_t* __restrict__ y,
                                                                   int64_t ldy) {
  const int64_t m = blockIdx.x;
  const uint16_t* xr = x + m * ldx;
  float ss = 0.0f;
  for (int64_t k = threadIdx.x * 8; k < K; k += kRowThreads * 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + k);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float f = bf16_to_f32(h[e]);
      ss = fmaf(f, f, ss);
    }
  }
  __shared__ float red[kRowThreads / 64];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < kRowThreads / 64; ++i) t += red[i];
  const float r = rsqrtf(t / (float)K + eps);
  for (int64_t k = threadIdx.x * 8; k < K; k += kRowThreads * 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + k);
    const u32x4 gv = *reinterpret_cast<const u32x4*>(w + k);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
    const uint16_t* g = reinterpret_cast<const uint16_t*>(&gv);
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = f32_to_bf16((bf16_to_f32(h[e]) * r) * bf16_to_f32(g[e]));
    *reinterpret_cast<u32x4*>(y + m * ldy + k) = *reinterpret_cast<const u32x4*>(o);
  }
}

__device__ __forceinline__ float silu_r(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float gelu_tanh_r(float x) {
  const float c = 0.7978845608028654f;  // sqrt(2/pi)
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

// out[m][i] = bf16(bf16(act(gate[m][i])) * up[m][i]) with gate = gu[m][i], up = gu[m][I + i]
// (bf16 projections; act = SiLU or tanh-GeLU), as the GEMM's gated epilogue computes it.
template <bool GELU>
__global__ __launch_bounds__(256) void rows_gated_kernel(const uint16_t* __restrict__ gu, int64_t ldg, int64_t I,
                                                         int64_t M, uint16_t* __restrict__ out, int64_t ldo) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 8 columns each
  const int64_t per_row = I / 8;
  if (idx >= M * per_row) return;
  const int64_t m = idx / per_row, i = (idx % per_row) * 8;
  const u32x4 gv = *reinterpret_cast<const u32x4*>(gu + m * ldg + i);
  const u32x4 uv = *reinterpret_cast<const u32x4*>(gu + m * ldg + I + i);
  const uint16_t* g = reinterpret_cast<const uint16_t*>(&gv);
  const uint16_t* u = reinterpret_cast<const uint16_t*>(&uv);
  uint16_t o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gb = bf16_to_f32(g[e]);
    const float act = round_bf16(GELU ? gelu_tanh_r(gb) : silu_r(gb));
    o[e] = f32_to_bf16(act * bf16_to_f32(u[e]));
  }
  *reinterpret_cast<u32x4*>(out + m * ldo + i) = *reinterpret_cast<const u32x4*>(o);
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_w8_dequant_rows(const uint8_t* wt, const uint32_t* sb, int bits, int64_t N, int64_t K,
                                   int paired, uint16_t* out, dsk_stream_t stream) {
  DSK_REQUIRE(wt && sb && out, "dsk_w8_dequant_rows: null pointer");
  DSK_REQUIRE(bits == 8 || bits == 4, "dsk_w8_dequant_rows: bits=%d (8 or 4)", bits);
  DSK_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 64 == 0 && (!paired || N % 32 == 0),
              "dsk_w8_dequant_rows: bad shape N=%lld K=%lld", (long long)N, (long long)K);
  DSK_REQUIRE((((uintptr_t)wt | (uintptr_t)out) & 15) == 0, "dsk_w8_dequant_rows: 16-byte aligned pointers");
  const int64_t chunks = N * K / 16;
  const dim3 grid((unsigned)ceil_div(chunks, 256));
  if (bits == 8)
    hipLaunchKernelGGL(dequant_rows_kernel<8>, grid, dim3(256), 0, as_stream(stream), wt, sb, N, K, paired, out);
  else
    hipLaunchKernelGGL(dequant_rows_kernel<4>, grid, dim3(256), 0, as_stream(stream), wt, sb, N, K, paired, out);
  DSK_LAUNCH_CHECK("dsk_w8_dequant_rows");
  return DSK_OK;
}

extern "C" int dsk_rows_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* w, float eps, int64_t M, int64_t K,
                                uint16_t* y, int64_t ldy, dsk_stream_t stream) {
  DSK_REQUIRE(x && w && y, "dsk_rows_rmsnorm: null pointer");
  DSK_REQUIRE(M > 0 && M < (1ll << 31) && K > 0 && K % 8 == 0 && ldx >= K && ldy >= K && ldx % 8 == 0 &&
                  ldy % 8 == 0,
              "dsk_rows_rmsnorm: bad shape");
  DSK_REQUIRE((((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) & 15) == 0, "dsk_rows_rmsnorm: 16-byte aligned pointers");
  hipLaunchKernelGGL(rows_rmsnorm_kernel, dim3((unsigned)M), dim3(kRowThreads), 0, as_stream(stream), x, ldx, w, eps,
                     K, y, ldy);
  DSK_LAUNCH_CHECK("dsk_rows_rmsnorm");
  return DSK_OK;
}

extern "C" int dsk_rows_gated(const uint16_t* gu, int64_t ldg, int64_t M, int64_t I, int act, uint16_t* out,
                              int64_t ldo, dsk_stream_t stream) {
  DSK_REQUIRE(gu && out, "dsk_rows_gated: null pointer");
  DSK_REQUIRE(act == DSK_EPI_SWIGLU || act == DSK_EPI_GEGLU, "dsk_rows_gated: act must be SWIGLU or GEGLU");
  DSK_REQUIRE(M > 0 && I > 0 && I % 8 == 0 && ldg >= 2 * I && ldo >= I && ldg % 8 == 0 && ldo % 8 == 0,
              "dsk_rows_gated: bad shape");
  DSK_REQUIRE((((uintptr_t)gu | (uintptr_t)out) & 15) == 0, "dsk_rows_gated: 16-byte aligned pointers");
  const dim3 grid((unsigned)ceil_div(M * (I / 8), 256));
  if (act == DSK_EPI_GEGLU)
    hipLaunchKernelGGL(rows_gated_kernel<true>, grid, dim3(256), 0, as_stream(stream), gu, ldg, I, M, out, ldo);
  else
    hipLaunchKernelGGL(rows_gated_kernel<false>, grid, dim3(256), 0, as_stream(stream), gu, ldg, I, M, out, ldo);
  DSK_LAUNCH_CHECK("dsk_rows_gated");
  return DSK_OK;
}
