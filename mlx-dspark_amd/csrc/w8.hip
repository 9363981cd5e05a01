// W8 affine group-64 weights on gfx950: quantizer, MLX-layout -> tiled-layout repack,
// activation pack (RMSNorm / SiLU / GeLU prologue) and the skinny GEMM used by every
// target and drafter projection of the verify step.
//
// Tiled HBM layout (what dsk_w8_gemm streams):
//   wt[t][g][lane][16 B]: tile t = 16 output rows (n = 16t + lane%16), group g = 64 input
//   columns, lane/16 selects the 16-column chunk inside the group. One wave-wide dwordx4
//   load reads one 1 KiB tile-group, contiguous, and lands every byte in the lane that
//   feeds it to v_mfma_f32_16x16x32_f16 as the B operand.
//   sb[t][n%16][g]: u32 = bf16 scale | bf16 bias << 16.
//
// GEMM arithmetic. With w = s*q + b per group, sum_k x_k w_k = s * sum x_k q_k + b * sum x_k.
// q (0..255) becomes the fp16 1024 + q with a single v_perm_b32 per two weights (0x64 in
// the high byte of each half), so the MFMA yields acc = sum x (1024 + q) and the group's
// contribution is s * acc + (b - 1024 s) * X with X = sum x over the group (precomputed by
// the activation pack). Activations are exact in fp16 after a per-row power-of-two scale
// (bf16 has 8 significant bits, fp16 11), undone in the epilogue.
#include "common.h"

namespace dsk {

// =====================================================================================
// quantize: one thread per (row, group)
// =====================================================================================
__global__ void w8_quantize_kernel(const void* __restrict__ w, int w_bf16, int64_t N, int64_t K,
                                   uint8_t* __restrict__ q, uint16_t* __restrict__ scales,
                                   uint16_t* __restrict__ biases) {
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
  float s = (hi - lo) / 255.0f;
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
    t = fminf(fmaxf(t, 0.0f), 255.0f);
    qo[i] = (uint8_t)(int)t;
  }
}

// =====================================================================================
// repack: MLX layout -> tiled layout
// =====================================================================================
__global__ void w8_repack_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                 const uint16_t* __restrict__ b, int64_t N, int64_t K,
                                 u32x4* __restrict__ wt, uint32_t* __restrict__ sb) {
  const int64_t G = K / 64;
  const int64_t chunks = N * K / 16;  // 16-byte chunks
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < chunks) {
    // destination order: t, g, lane
    int64_t lane = idx & 63;
    int64_t tg = idx >> 6;
    int64_t g = tg % G, t = tg / G;
    int64_t n = t * 16 + (lane & 15);
    int64_t k = g * 64 + (lane >> 4) * 16;
    const u32x4* src = reinterpret_cast<const u32x4*>(q + n * K + k);
    wt[idx] = *src;
  }
  if (idx < N * G) {
    // destination order: t, n%16, g
    int64_t g = idx % G;
    int64_t tn = idx / G;  // = t*16 + n%16 = n
    int64_t n = tn;
    uint32_t sv = s[n * G + g], bv = b[n * G + g];
    sb[idx] = sv | (bv << 16);
  }
}

// =====================================================================================
// activation pack
// =====================================================================================
struct PackLayout {
  int MT;
  int64_t G;
  size_t xp_off, xs_off, xe_off, total;
};

__host__ __device__ inline PackLayout pack_layout(int M, int64_t K) {
  PackLayout L;
  L.MT = (M + 15) / 16;
  L.G = K / 64;
  L.xp_off = 0;
  L.xs_off = (size_t)L.MT * L.G * 2048;
  L.xe_off = L.xs_off + (size_t)L.MT * L.G * 64;
  L.total = L.xe_off + (size_t)L.MT * 64;
  return L;
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float gelu_tanh_f(float x) {
  const float c = 0.7978845608028654f;  // sqrt(2/pi)
  return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}

constexpr int kPackThreads = 256;
constexpr int kPackMaxK = 24576;

// One workgroup per (padded) row. Row values are formed in fp32, rounded to bf16 (the
// activation dtype between kernels), kept in LDS, then scaled by 2^s and stored as fp16.
__global__ __launch_bounds__(kPackThreads) void act_pack_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int M, int64_t K, int mode,
    const uint16_t* __restrict__ norm_w, float eps, uint8_t* __restrict__ out) {
  __shared__ uint16_t row[kPackMaxK];
  __shared__ float red[kPackThreads / 64];
  const PackLayout L = pack_layout(M, K);
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t nchunk = K / 16;
  _Float16* xp = reinterpret_cast<_Float16*>(out + L.xp_off);
  float* xs = reinterpret_cast<float*>(out + L.xs_off);
  float* xe = reinterpret_cast<float*>(out + L.xe_off);
  const int mt = m >> 4, mr = m & 15;

  if (m >= M) {  // padding rows: zeros
    for (int64_t c = tid; c < nchunk; c += kPackThreads) {
      int64_t g = c >> 2, j = c & 3;
      u32x4* dst = reinterpret_cast<u32x4*>(xp + (((int64_t)mt * L.G + g) * 64 + mr + 16 * j) * 16);
      dst[0] = u32x4{0, 0, 0, 0};
      dst[1] = u32x4{0, 0, 0, 0};
      if (j == 0) xs[((int64_t)mt * L.G + g) * 16 + mr] = 0.0f;
    }
    if (tid == 0) xe[m] = 1.0f;
    return;
  }

  const uint16_t* xr = x + (int64_t)m * ldx;
  float rscale = 1.0f;
  if (mode == DSK_PACK_RMSNORM) {
    float ss = 0.0f;
    for (int64_t k = tid; k < K; k += kPackThreads) {
      float v = bf16_to_f32(xr[k]);
      ss += v * v;
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < kPackThreads / 64; ++i) tot += red[i];
    rscale = rsqrtf(tot / (float)K + eps);
    __syncthreads();
  }

  // pass 1: values -> LDS (bf16), running max |v|
  float amax = 0.0f;
  for (int64_t k = tid; k < K; k += kPackThreads) {
    float v;
    if (mode == DSK_PACK_PLAIN) {
      v = bf16_to_f32(xr[k]);
    } else if (mode == DSK_PACK_RMSNORM) {
      v = (bf16_to_f32(xr[k]) * rscale) * bf16_to_f32(norm_w[k]);
    } else {
      float g = bf16_to_f32(xr[k]);
      float u = bf16_to_f32(xr[K + k]);
      // activation rounds to bf16 before the product, as the bf16 graph does
      float a = round_bf16(mode == DSK_PACK_SILU ? silu_f(g) : gelu_tanh_f(g));
      v = a * u;
    }
    uint16_t h = f32_to_bf16(v);
    row[k] = h;
    amax = fmaxf(amax, fabsf(bf16_to_f32(h)));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  float mx = 0.0f;
  for (int i = 0; i < kPackThreads / 64; ++i) mx = fmaxf(mx, red[i]);
  // power-of-two scale bringing max |v| into [2^14, 2^15)
  int e = 0;
  if (mx > 0.0f) {
    int ex;
    frexpf(mx, &ex);  // mx = f * 2^ex, f in [0.5, 1)
    e = 15 - ex;      // mx * 2^e in [2^14, 2^15)
  }
  const float up = ldexpf(1.0f, e);
  if (tid == 0) xe[m] = ldexpf(1.0f, -e);

  // pass 2: fp16 operand + group sums. Chunk c = 16 columns; the four chunks of a group
  // are handled by four consecutive threads, combined with lane shuffles.
  const int64_t nchunk_pad = ((nchunk + kPackThreads - 1) / kPackThreads) * kPackThreads;
  for (int64_t c = tid; c < nchunk_pad; c += kPackThreads) {
    float part = 0.0f;
    if (c < nchunk) {
      int64_t g = c >> 2, j = c & 3;
      _Float16 hv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float v = bf16_to_f32(row[c * 16 + i]) * up;
        _Float16 h = (_Float16)v;
        hv[i] = h;
        part += (float)h;
      }
      u32x4* dst = reinterpret_cast<u32x4*>(xp + (((int64_t)mt * L.G + g) * 64 + mr + 16 * j) * 16);
      const u32x4* srcv = reinterpret_cast<const u32x4*>(hv);
      dst[0] = srcv[0];
      dst[1] = srcv[1];
    }
    part += __shfl_xor(part, 1, 64);
    part += __shfl_xor(part, 2, 64);
    if (c < nchunk && (c & 3) == 0) xs[((int64_t)mt * L.G + (c >> 2)) * 16 + mr] = part;
  }
}

// =====================================================================================
// skinny GEMM
// =====================================================================================
__device__ __forceinline__ half8 w8_to_h8_lo(uint32_t a, uint32_t b) {
  // bytes q0..q3 of a, q4..q7 of b -> fp16 (1024 + q) x 8
  uint32_t h0 = __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u);
  uint32_t h1 = __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u);
  uint32_t h2 = __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u);
  uint32_t h3 = __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u);
  u32x4 u = {h0, h1, h2, h3};
  return __builtin_bit_cast(half8, u);
}

struct GemmArgs {
  const uint8_t* xpack;
  const u32x4* wt;
  const uint32_t* sb;
  int M;
  int64_t N, K, G;
  int SK;           // K splits
  int64_t gps;      // groups per split
  int n_slabs;      // N / (16 * NTW)
  void* y;
  int y_f32;
  int64_t ldy;
  const uint16_t* res;
  int64_t ldr;
  float softcap;
  float* part;      // [SK][M][N] f32 partials (SK > 1)
  int* cnt;         // [n_slabs] arrival counters (SK > 1)
};

template <int MT, int NTW>
__device__ __forceinline__ void gemm_store(const GemmArgs& a, int m, int64_t n, float v) {
  if (a.res) v += bf16_to_f32(a.res[(int64_t)m * a.ldr + n]);
  if (a.softcap > 0.0f) v = tanhf(v / a.softcap) * a.softcap;
  if (a.y_f32)
    reinterpret_cast<float*>(a.y)[(int64_t)m * a.ldy + n] = v;
  else
    reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.ldy + n] = f32_to_bf16(v);
}

template <int MT, int NTW, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void w8_gemm_kernel(GemmArgs a) {
  constexpr int CH = 4;  // groups per load batch
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;

  // XCD-aware block mapping: the SK blocks of one slab share blockIdx % 8 (one XCD, one L2)
  int slab, ks;
  const int total = a.n_slabs * a.SK;
  if ((a.n_slabs & 7) == 0) {
    int id = blockIdx.x;
    int xcd = id & 7, j = id >> 3;
    slab = (j / a.SK) * 8 + xcd;
    ks = j % a.SK;
  } else {
    slab = blockIdx.x / a.SK;
    ks = blockIdx.x % a.SK;
  }
  (void)total;

  const int64_t g_lo = (int64_t)ks * a.gps;
  const int64_t g_hi = min(a.G, g_lo + a.gps);
  const int64_t span = g_hi - g_lo;
  const int64_t gpw = (span + WAVES - 1) / WAVES;
  const int64_t wg0 = g_lo + wave * gpw;
  const int64_t wg1 = min(g_hi, wg0 + gpw);

  const PackLayout L = pack_layout(a.M, a.K);
  const u32x4* xp = reinterpret_cast<const u32x4*>(a.xpack + L.xp_off);
  const f32x4* xs = reinterpret_cast<const f32x4*>(a.xpack + L.xs_off);
  const float* xe = reinterpret_cast<const float*>(a.xpack + L.xe_off);

  const int64_t t0 = (int64_t)slab * NTW;
  f32x4 acc[MT][NTW];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

  for (int64_t g = wg0; g < wg1; g += CH) {
    const int nb = (int)min((int64_t)CH, wg1 - g);
    u32x4 wv[CH][NTW];
    uint32_t sbv[CH][NTW];
    u32x4 xv[CH][MT][2];
    f32x4 xsv[CH][MT];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (c < nb) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          wv[c][j] = __builtin_nontemporal_load(&a.wt[((t0 + j) * a.G + g + c) * 64 + lane]);
          sbv[c][j] = a.sb[((t0 + j) * 16 + (lane & 15)) * a.G + g + c];
        }
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const u32x4* px = xp + (((int64_t)i * a.G + g + c) * 64 + lane) * 2;
          xv[c][i][0] = px[0];
          xv[c][i][1] = px[1];
          xsv[c][i] = xs[((int64_t)i * a.G + g + c) * 4 + (lane >> 4)];
        }
      }
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (c < nb) {
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const half8 b0 = w8_to_h8_lo(wv[c][j].x, wv[c][j].y);
          const half8 b1 = w8_to_h8_lo(wv[c][j].z, wv[c][j].w);
          const float s = bf16_to_f32((uint16_t)(sbv[c][j] & 0xffffu));
          const float bb = bf16_to_f32((uint16_t)(sbv[c][j] >> 16));
          const float bprime = fmaf(-1024.0f, s, bb);
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            const half8 a0 = __builtin_bit_cast(half8, xv[c][i][0]);
            const half8 a1 = __builtin_bit_cast(half8, xv[c][i][1]);
            f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, f32x4{0, 0, 0, 0}, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, t, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] = fmaf(s, t[r], fmaf(bprime, xsv[c][i][r], acc[i][j][r]));
          }
        }
      }
    }
  }

  // cross-wave reduction
  __shared__ float red[WAVES][MT * NTW * 256];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][((i * NTW + j) * 4 + r) * 64 + lane] = acc[i][j][r];
  __syncthreads();

  constexpr int NOUT = MT * NTW * 256;
  if (a.SK == 1) {
    for (int o = threadIdx.x; o < NOUT; o += WAVES * 64) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) v += red[w][o];
      const int ln = o & 63, r = (o >> 6) & 3, ij = o >> 8;
      const int i = ij / NTW, j = ij % NTW;
      const int m = i * 16 + (ln >> 4) * 4 + r;
      const int64_t n = (t0 + j) * 16 + (ln & 15);
      if (m < a.M) gemm_store<MT, NTW>(a, m, n, v * xe[m]);
    }
    return;
  }

  // split-K: publish partial, last arriving block of the slab reduces in fixed order
  for (int o = threadIdx.x; o < NOUT; o += WAVES * 64) {
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) v += red[w][o];
    const int ln = o & 63, r = (o >> 6) & 3, ij = o >> 8;
    const int i = ij / NTW, j = ij % NTW;
    const int m = i * 16 + (ln >> 4) * 4 + r;
    const int64_t n = (t0 + j) * 16 + (ln & 15);
    if (m < a.M) a.part[((int64_t)ks * a.M + m) * a.N + n] = v * xe[m];
  }
  __threadfence();
  __syncthreads();
  __shared__ int last;
  if (threadIdx.x == 0) {
    int prev = atomicAdd(&a.cnt[slab], 1);
    last = (prev == a.SK - 1);
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (int o = threadIdx.x; o < NOUT; o += WAVES * 64) {
    const int ln = o & 63, r = (o >> 6) & 3, ij = o >> 8;
    const int i = ij / NTW, j = ij % NTW;
    const int m = i * 16 + (ln >> 4) * 4 + r;
    const int64_t n = (t0 + j) * 16 + (ln & 15);
    if (m >= a.M) continue;
    float v = 0.0f;
    for (int s = 0; s < a.SK; ++s) v += __builtin_nontemporal_load(&a.part[((int64_t)s * a.M + m) * a.N + n]);
    gemm_store<MT, NTW>(a, m, n, v);
  }
  if (threadIdx.x == 0) a.cnt[slab] = 0;  // leave the counter zeroed for the next call
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
  int ntw, sk, waves;
  int64_t gps;
};

static GemmPlan plan_gemm(int M, int64_t N, int64_t K) {
  (void)M;
  const int64_t G = K / 64;
  const int64_t tiles = N / 16;
  GemmPlan p;
  p.waves = 4;
  // widest slab that still gives >= 256 blocks without split-K
  p.ntw = 1;
  if (tiles % 4 == 0 && tiles / 4 >= 512) p.ntw = 4;
  else if (tiles % 2 == 0 && tiles / 2 >= 384) p.ntw = 2;
  const int64_t slabs = tiles / p.ntw;
  p.sk = 1;
  while (slabs * p.sk < 256 && G / (p.sk * 2) >= 16) p.sk *= 2;
  p.gps = (G + p.sk - 1) / p.sk;
  return p;
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
                     as_stream(stream), w, w_dtype == DSK_BF16 ? 1 : 0, N, K, q, scales, biases);
  DSK_LAUNCH_CHECK("dsk_w8_quantize");
  return DSK_OK;
}

extern "C" int dsk_w8_repack(const uint8_t* q, const uint16_t* scales, const uint16_t* biases,
                             int64_t N, int64_t K, uint8_t* wt, uint32_t* sb, dsk_stream_t stream) {
  DSK_REQUIRE(q && scales && biases && wt && sb, "dsk_w8_repack: null pointer");
  DSK_REQUIRE(N > 0 && K > 0 && N % 16 == 0 && K % 64 == 0,
              "dsk_w8_repack: need N %% 16 == 0 and K %% 64 == 0 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  int64_t total = N * K / 16;
  int threads = 256;
  hipLaunchKernelGGL(w8_repack_kernel, dim3((unsigned)ceil_div(total, threads)), dim3(threads), 0,
                     as_stream(stream), q, scales, biases, N, K, reinterpret_cast<u32x4*>(wt), sb);
  DSK_LAUNCH_CHECK("dsk_w8_repack");
  return DSK_OK;
}

extern "C" size_t dsk_act_pack_bytes(int M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 64) return 0;
  return pack_layout(M, K).total;
}

extern "C" int dsk_act_pack(const uint16_t* x, int64_t ldx, int M, int64_t K, int mode,
                            const uint16_t* norm_w, float eps, void* out, dsk_stream_t stream) {
  DSK_REQUIRE(x && out, "dsk_act_pack: null pointer");
  DSK_REQUIRE(M > 0 && M <= 64, "dsk_act_pack: M=%d outside [1, 64]", M);
  DSK_REQUIRE(K > 0 && K % 64 == 0 && K <= kPackMaxK, "dsk_act_pack: K=%lld must be a multiple of 64 <= %d",
              (long long)K, kPackMaxK);
  DSK_REQUIRE(mode >= DSK_PACK_PLAIN && mode <= DSK_PACK_GELU, "dsk_act_pack: bad mode %d", mode);
  DSK_REQUIRE(mode != DSK_PACK_RMSNORM || norm_w, "dsk_act_pack: RMSNORM needs norm_w");
  int64_t need = (mode == DSK_PACK_SILU || mode == DSK_PACK_GELU) ? 2 * K : K;
  DSK_REQUIRE(ldx >= need, "dsk_act_pack: ldx=%lld < %lld", (long long)ldx, (long long)need);
  const int MT = (M + 15) / 16;
  hipLaunchKernelGGL(act_pack_kernel, dim3(MT * 16), dim3(kPackThreads), 0, as_stream(stream), x, ldx, M, K,
                     mode, norm_w, eps, reinterpret_cast<uint8_t*>(out));
  DSK_LAUNCH_CHECK("dsk_act_pack");
  return DSK_OK;
}

static constexpr size_t kCounterBytes = 65536;  // 16384 slab counters at the workspace head

extern "C" size_t dsk_w8_gemm_ws_bytes(int M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  GemmPlan p = plan_gemm(M, N, K);
  size_t part = p.sk > 1 ? (size_t)p.sk * M * N * sizeof(float) : 0;
  return kCounterBytes + part;
}

extern "C" int dsk_w8_gemm_ws_init(void* workspace, size_t ws_bytes, dsk_stream_t stream) {
  DSK_REQUIRE(workspace && ws_bytes >= kCounterBytes, "dsk_w8_gemm_ws_init: workspace too small");
  hipError_t e = hipMemsetAsync(workspace, 0, kCounterBytes, as_stream(stream));
  if (e != hipSuccess) {
    set_error("dsk_w8_gemm_ws_init: %s", hipGetErrorString(e));
    return DSK_ELAUNCH;
  }
  return DSK_OK;
}

template <int MT, int NTW>
static void launch_gemm(const GemmArgs& a, int waves, hipStream_t st) {
  dim3 grid((unsigned)(a.n_slabs * a.SK));
  (void)waves;
  hipLaunchKernelGGL((w8_gemm_kernel<MT, NTW, 4>), grid, dim3(256), 0, st, a);
}

extern "C" int dsk_w8_gemm(const void* a_, const uint8_t* wt, const uint32_t* sb, int M, int64_t N,
                           int64_t K, void* y, int y_dtype, int64_t ldy, const uint16_t* residual,
                           int64_t ldr, float softcap, void* workspace, size_t ws_bytes,
                           dsk_stream_t stream) {
  DSK_REQUIRE(a_ && wt && sb && y, "dsk_w8_gemm: null pointer");
  DSK_REQUIRE(M > 0 && M <= 64, "dsk_w8_gemm: M=%d outside [1, 64]", M);
  DSK_REQUIRE(N > 0 && N % 16 == 0 && K > 0 && K % 64 == 0,
              "dsk_w8_gemm: need N %% 16 == 0, K %% 64 == 0 (N=%lld K=%lld)", (long long)N, (long long)K);
  DSK_REQUIRE(y_dtype == DSK_F32 || y_dtype == DSK_BF16, "dsk_w8_gemm: y dtype must be f32 or bf16");
  DSK_REQUIRE(ldy >= N, "dsk_w8_gemm: ldy=%lld < N", (long long)ldy);
  DSK_REQUIRE(!residual || ldr >= N, "dsk_w8_gemm: ldr=%lld < N", (long long)ldr);
  DSK_REQUIRE(!(residual && y_dtype != DSK_BF16 && (const void*)residual == y),
              "dsk_w8_gemm: in-place residual needs bf16 output");
  GemmPlan p = plan_gemm(M, N, K);
  const size_t need = dsk_w8_gemm_ws_bytes(M, N, K);
  DSK_REQUIRE(workspace && ws_bytes >= need, "dsk_w8_gemm: workspace %zu < %zu bytes", ws_bytes, need);
  GemmArgs a;
  a.xpack = reinterpret_cast<const uint8_t*>(a_);
  a.wt = reinterpret_cast<const u32x4*>(wt);
  a.sb = sb;
  a.M = M;
  a.N = N;
  a.K = K;
  a.G = K / 64;
  a.SK = p.sk;
  a.gps = p.gps;
  a.n_slabs = (int)(N / 16 / p.ntw);
  DSK_REQUIRE((int64_t)a.n_slabs <= (int64_t)(kCounterBytes / sizeof(int)) || p.sk == 1,
              "dsk_w8_gemm: too many slabs for split-K counters");
  a.y = y;
  a.y_f32 = (y_dtype == DSK_F32);
  a.ldy = ldy;
  a.res = residual;
  a.ldr = ldr;
  a.softcap = softcap;
  a.cnt = reinterpret_cast<int*>(workspace);
  a.part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + kCounterBytes);
  hipStream_t st = as_stream(stream);
  const int MT = (M + 15) / 16;
#define DSK_GEMM_CASE(MT_, NTW_) \
  if (MT == MT_ && p.ntw == NTW_) { launch_gemm<MT_, NTW_>(a, p.waves, st); DSK_LAUNCH_CHECK("dsk_w8_gemm"); return DSK_OK; }
  DSK_GEMM_CASE(1, 1) DSK_GEMM_CASE(1, 2) DSK_GEMM_CASE(1, 4)
  DSK_GEMM_CASE(2, 1) DSK_GEMM_CASE(2, 2) DSK_GEMM_CASE(2, 4)
  DSK_GEMM_CASE(3, 1) DSK_GEMM_CASE(3, 2) DSK_GEMM_CASE(3, 4)
  DSK_GEMM_CASE(4, 1) DSK_GEMM_CASE(4, 2) DSK_GEMM_CASE(4, 4)
#undef DSK_GEMM_CASE
  set_error("dsk_w8_gemm: no kernel for MT=%d NTW=%d", MT, p.ntw);
  return DSK_EINVAL;
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
