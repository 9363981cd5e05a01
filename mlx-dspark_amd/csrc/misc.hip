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

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_logits_penalize(float* logits, int64_t ldl, int R, const int32_t* row_ptr, const int32_t* ids,
                                   const float* vals, dsk_stream_t stream) {
  DSK_REQUIRE(logits && row_ptr && ids && vals && R > 0, "dsk_logits_penalize: bad arguments");
  hipLaunchKernelGGL(penalize_kernel, dim3((unsigned)R), dim3(64), 0, as_stream(stream), logits, ldl, row_ptr, ids,
                     vals);
  DSK_LAUNCH_CHECK("dsk_logits_penalize");
  return DSK_OK;
}

extern "C" int dsk_lens_add(int32_t* lens, const int32_t* n, int B, int add, dsk_stream_t stream) {
  DSK_REQUIRE(lens && B > 0, "dsk_lens_add: bad arguments");
  hipLaunchKernelGGL(lens_add_kernel, dim3((unsigned)ceil_div(B, 256)), dim3(256), 0, as_stream(stream), lens, n,
                     B, add);
  DSK_LAUNCH_CHECK("dsk_lens_add");
  return DSK_OK;
}
