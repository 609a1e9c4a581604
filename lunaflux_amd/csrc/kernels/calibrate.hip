// calibrate.hip - measurement support: a plain streaming copy of a known
// number of bytes. Profiling runs read the hardware byte counters for this
// kernel next to the projection kernels, to convert counter units into bytes.
#include "device_common.h"

extern "C" __global__ __launch_bounds__(256) void lf_calibrate_copy(const int64_t *count16,
                                                                    const uint4 *src,
                                                                    uint4 *dst) {
  const int64_t n = *count16;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    dst[i] = src[i];
  }
}
