// Small device-side bookkeeping kernels.
#include "common.h"

namespace dsk {

__global__ void lens_add_kernel(int32_t* __restrict__ lens, const int32_t* __restrict__ n, int B, int add) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) lens[b] += (n ? n[b] : 0) + add;
}

}  // namespace dsk

using namespace dsk;

extern "C" int dsk_lens_add(int32_t* lens, const int32_t* n, int B, int add, dsk_stream_t stream) {
  DSK_REQUIRE(lens && B > 0, "dsk_lens_add: bad arguments");
  hipLaunchKernelGGL(lens_add_kernel, dim3((unsigned)ceil_div(B, 256)), dim3(256), 0, as_stream(stream), lens, n,
                     B, add);
  DSK_LAUNCH_CHECK("dsk_lens_add");
  return DSK_OK;
}
