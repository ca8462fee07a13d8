// Zero fill of device words (counter buffers).  A kernel rather than
// hipMemsetAsync, so that a HIP graph capturing the call records a kernel
// node: memset nodes have given wrong results on replays after the first.
#include "pa_device.hpp"
#include "pa_internal.hpp"

namespace pa {

constexpr int kFillThreads = 256;

__global__ void __launch_bounds__(kFillThreads)
fill_zero_kernel(uint32_t* __restrict__ p, size_t words) {
  const size_t stride = (size_t)gridDim.x * kFillThreads;
  for (size_t i = (size_t)blockIdx.x * kFillThreads + threadIdx.x; i < words; i += stride) p[i] = 0u;
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
  const size_t words = bytes / 4;
  if (words == 0) return hipSuccess;
  const size_t want = (words + kFillThreads - 1) / kFillThreads;
  const int grid = (int)(want < 1024 ? want : 1024);
  fill_zero_kernel<<<grid, kFillThreads, 0, stream>>>(static_cast<uint32_t*>(p), words);
  return hipGetLastError();
}

}  // namespace pa
