// Small device-side bookkeeping kernels.
#include "common.h"

namespace dsk {

__global__ void lens_add_kernel(int32_t* __restrict__ lens, const int32_t* __restrict__ n, int B, int add) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) lens[b] += (n ? n[b] : 0) + add;
}

// one workgroup per logits row; the row's CSR entries are applied in order by one lane each
// (ids within a row are distinct, so there are no write conflicts)
__global__ void penalize_kernel(float* __restrict__ logits, int64_t ldl, const int32_t* __restrict__ row_ptr,
                                const int32_t* __restrict__ ids, const float* __restrict__ vals) {
  const int r = blockIdx.x;
  for (int j = row_ptr[r] + threadIdx.x; j < row_ptr[r + 1]; j += blockDim.x) logits[(int64_t)r * ldl + ids[j]] -= vals[j];
}

// One workgroup per row: a max / sum-of-exp pass for the log-normaliser, then top_k
// selection passes, each taking the largest entry that ranks below the previous pick in the
// order (value descending, index ascending), so ties resolve to the lowest index.
constexpr int kLpThreads = 1024;

__device__ __forceinline__ bool lp_before(float va, int64_t ia, float vb, int64_t ib) {
  return va > vb || (va == vb && ia < ib);
}

__global__ __launch_bounds__(kLpThreads) void row_logprobs_kernel(const float* __restrict__ logits, int64_t ldl,
                                                                  int64_t V, const int32_t* __restrict__ tokens,
                                                                  int top_k, float* __restrict__ chosen,
                                                                  int32_t* __restrict__ top_ids,
                                                                  float* __restrict__ top_vals) {
  __shared__ float sv[kLpThreads / 64];
  __shared__ int64_t si[kLpThreads / 64];
  const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float* x = logits + (int64_t)r * ldl;
  float m = -__builtin_inff();
  for (int64_t j = tid; j < V; j += kLpThreads) m = fmaxf(m, x[j]);
  m = wave_max(m);
  if (lane == 0) sv[wv] = m;
  __syncthreads();
  m = -__builtin_inff();
  for (int i = 0; i < kLpThreads / 64; ++i) m = fmaxf(m, sv[i]);
  __syncthreads();
  float se = 0.0f;
  for (int64_t j = tid; j < V; j += kLpThreads) se += expf(x[j] - m);
  se = wave_sum(se);
  if (lane == 0) sv[wv] = se;
  __syncthreads();
  se = 0.0f;
  for (int i = 0; i < kLpThreads / 64; ++i) se += sv[i];
  const float lse = m + logf(se);
  if (tid == 0) {
    int64_t t = tokens[r];
    t = t < 0 ? 0 : (t >= V ? V - 1 : t);
    chosen[r] = x[t] - lse;
  }
  float pv = __builtin_inff();
  int64_t pi = -1;
  for (int k = 0; k < top_k; ++k) {
    float bv = -__builtin_inff();
    int64_t bi = V;
    for (int64_t j = tid; j < V; j += kLpThreads) {
      const float v = x[j];
      if (lp_before(pv, pi, v, j) && lp_before(v, j, bv, bi)) {
        bv = v;
        bi = j;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int64_t oi = __shfl_xor(bi, o, 64);
      if (lp_before(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    __syncthreads();
    if (lane == 0) {
      sv[wv] = bv;
      si[wv] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
    for (int i = 1; i < kLpThreads / 64; ++i)
      if (lp_before(sv[i], si[i], bv, bi)) {
        bv = sv[i];
        bi = si[i];
      }
    if (tid == 0) {
      top_ids[(int64_t)r * top_k + k] = (int32_t)(bi < V ? bi : 0);
      top_vals[(int64_t)r * top_k + k] = bi < V ? bv - lse : -__builtin_inff();
    }
    pv = bv;
    pi = bi;
  }
}

// Reads [p, p + n16 * 16) and keeps nothing: the bytes pass through the memory-side cache on
// their way, so a kernel that reads them soon after finds them there. Each thread issues
// kPrefetchLoads 16-byte loads before it uses any (a lane past the end re-reads the last chunk),
// so a workgroup keeps 32 KB in flight. The xor of everything read is stored only if it equals a
// value no real weight image produces in practice, and then into the caller's 16-byte sink, so
// the loads cannot be dropped.
constexpr int kPrefetchLoads = 8;

__global__ __launch_bounds__(256) void prefetch_kernel(const uint4* __restrict__ p, int64_t n16,
                                                       uint4* __restrict__ sink) {
  uint4 acc = {0, 0, 0, 0};
  const int64_t step = (int64_t)gridDim.x * 256 * kPrefetchLoads;
  for (int64_t base = (int64_t)blockIdx.x * 256 * kPrefetchLoads + threadIdx.x; base < n16; base += step) {
    uint4 v[kPrefetchLoads];
#pragma unroll
    for (int u = 0; u < kPrefetchLoads; ++u) v[u] = p[min(base + u * 256, n16 - 1)];
#pragma unroll
    for (int u = 0; u < kPrefetchLoads; ++u) {
      acc.x ^= v[u].x;
      acc.y ^= v[u].y;
      acc.z ^= v[u].z;
      acc.w ^= v[u].w;
    }
  }
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == 0xf39cc060u && acc.w == 0x5ced1a3bu) *sink = acc;
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_row_logprobs(const float* logits, int64_t ldl, int R, int64_t V, const int32_t* tokens,
                                int top_k, float* chosen, int32_t* top_ids, float* top_vals, dsk_stream_t stream) {
  DSK_REQUIRE(logits && tokens && chosen && R > 0 && V > 0 && ldl >= V, "dsk_row_logprobs: bad arguments");
  DSK_REQUIRE(top_k >= 0 && top_k <= 64 && (top_k == 0 || (top_ids && top_vals)),
              "dsk_row_logprobs: top_k=%d outside [0, 64] or no output", top_k);
  hipLaunchKernelGGL(row_logprobs_kernel, dim3((unsigned)R), dim3(kLpThreads), 0, as_stream(stream), logits, ldl, V,
                     tokens, top_k, chosen, top_ids, top_vals);
  DSK_LAUNCH_CHECK("dsk_row_logprobs");
  return DSK_OK;
}

extern "C" int dsk_logits_penalize(float* logits, int64_t ldl, int R, const int32_t* row_ptr, const int32_t* ids,
                                   const float* vals, dsk_stream_t stream) {
  DSK_REQUIRE(logits && row_ptr && ids && vals && R > 0, "dsk_logits_penalize: bad arguments");
  hipLaunchKernelGGL(penalize_kernel, dim3((unsigned)R), dim3(64), 0, as_stream(stream), logits, ldl, row_ptr, ids,
                     vals);
  DSK_LAUNCH_CHECK("dsk_logits_penalize");
  return DSK_OK;
}

extern "C" int dsk_prefetch(const void* p, size_t bytes, int workgroups, void* sink, dsk_stream_t stream) {
  DSK_REQUIRE(p && sink && workgroups > 0, "dsk_prefetch: bad arguments");
  DSK_REQUIRE(((uintptr_t)p & 15) == 0 && bytes % 16 == 0 && ((uintptr_t)sink & 15) == 0,
              "dsk_prefetch: 16-byte aligned pointers and a multiple of 16 bytes");
  if (bytes == 0) return DSK_OK;
  hipLaunchKernelGGL(prefetch_kernel, dim3((unsigned)workgroups), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint4*>(p), (int64_t)(bytes / 16), reinterpret_cast<uint4*>(sink));
  DSK_LAUNCH_CHECK("dsk_prefetch");
  return DSK_OK;
}

extern "C" int dsk_lens_add(int32_t* lens, const int32_t* n, int B, int add, dsk_stream_t stream) {
  DSK_REQUIRE(lens && B > 0, "dsk_lens_add: bad arguments");
  hipLaunchKernelGGL(lens_add_kernel, dim3((unsigned)ceil_div(B, 256)), dim3(256), 0, as_stream(stream), lens, n,
                     B, add);
  DSK_LAUNCH_CHECK("dsk_lens_add");
  return DSK_OK;
}
