// Zero fill as a kernel rather than hipMemsetAsync, so that a caller may capture it into a HIP graph (memset nodes in
// captured graphs have given wrong results on replay on this platform).
#include "omt_internal.h"

namespace omt {

__global__ void __launch_bounds__(256) zero_fill_kernel(unsigned char* __restrict__ dst, int64_t bytes) {
  const int64_t n16 = bytes >> 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if ((((uintptr_t)dst) & 15) == 0) {
    for (int64_t i = t; i < n16; i += stride) reinterpret_cast<uint4*>(dst)[i] = make_uint4(0, 0, 0, 0);
    for (int64_t i = (n16 << 4) + t; i < bytes; i += stride) dst[i] = 0;
  } else {
    for (int64_t i = t; i < bytes; i += stride) dst[i] = 0;
  }
}

}  // namespace omt

using namespace omt;

OMT_EXPORT int omt_memset_zero(void* dst, size_t bytes, void* stream) {
  if (bytes == 0) return OMT_OK;
  if (!dst) return fail(OMT_INVALID, "omt_memset_zero: null pointer");
  hipLaunchKernelGGL(zero_fill_kernel, dim3(grid1d(cdiv((int64_t)bytes, 16), 256, 8192)), dim3(256), 0,
                     stream_of(stream), (unsigned char*)dst, (int64_t)bytes);
  return launch_check("zero_fill_kernel");
}
