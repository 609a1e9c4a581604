// scratch.hip - lunaflux_hip_function_launch_scratch: a launch that
// allocates nothing. The kernel's workspace (the trailing argument) is this
// library's own device array `scratch`, one copy per GPU, instead of a
// caller region. For callers that cannot call hipMalloc (code under HIP graph
// capture, tight serving loops, harnesses that forbid allocation).
//
// `scratch` is a file-scope device array, so in host code its name is only a
// stand-in for the symbol: its device address on a GPU comes from
// hipGetSymbolAddress with that GPU current, once per device (the first
// scratch launch on it), and only that address is ever handed to a kernel or
// to the clearing kernel below.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "runtime_internal.h"

namespace {

constexpr int64_t kScratchBytes = LF_SCRATCH_MAX_BYTES;
static_assert(kScratchBytes % 16 == 0, "cleared in 16-byte stores");

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Zero-fills the first `chunks` 16-byte chunks of the scratch array (a kernel,
// not hipMemsetAsync, so the launch may also be captured into a graph).
__global__ void lf_scratch_clear(uint4 *base, uint64_t chunks) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < chunks;
       i += stride) {
    base[i] = make_uint4(0u, 0u, 0u, 0u);
  }
}

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void *g_address[kMaxDevices];  // the array's address on each device, once known

// The array's device address on `ordinal` (which must be the current
// device): looked up the first time, then kept.
int32_t scratch_address(int32_t ordinal, void **out) {
  if (ordinal < 0 || ordinal >= kMaxDevices) return LF_UNSUPPORTED;
  std::lock_guard<std::mutex> guard(g_lock);
  if (g_address[ordinal] == nullptr) {
    void *address = nullptr;
    if (hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)) != hipSuccess || address == nullptr) {
      return LF_DRIVER_FAILURE;
    }
    g_address[ordinal] = address;
  }
  *out = g_address[ordinal];
  return LF_OK;
}

struct Request {
  int64_t bytes;
  bool clear;
};

int32_t prepare(void *context, int32_t ordinal, hipStream_t stream, uintptr_t *value) {
  const Request *request = static_cast<const Request *>(context);
  void *address = nullptr;
  int32_t status = scratch_address(ordinal, &address);
  if (status != LF_OK) return status;
  if (request->clear) {
    uint4 *base = static_cast<uint4 *>(address);
    uint64_t chunks = static_cast<uint64_t>(request->bytes + 15) / 16;
    uint64_t blocks = (chunks + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    void *args[] = {&base, &chunks};
    if (hipLaunchKernel(reinterpret_cast<const void *>(&lf_scratch_clear),
                        dim3(static_cast<unsigned>(blocks)), dim3(256), args, 0,
                        stream) != hipSuccess) {
      return LF_DRIVER_FAILURE;
    }
  }
  *value = reinterpret_cast<uintptr_t>(address);
  return LF_OK;
}

}  // namespace

extern "C" int32_t lunaflux_hip_function_launch_scratch(
    lf_function *function, lf_stream *stream, int32_t grid_x, int32_t grid_y, int32_t grid_z,
    int32_t block_x, int32_t block_y, int32_t block_z, int32_t shared_memory_bytes,
    int32_t argument_count, lf_allocation *const *allocations, const int64_t *offsets,
    const int64_t *byte_counts, const int64_t *alignments, int64_t scratch_bytes,
    int32_t clear) {
  if (scratch_bytes <= 0 || scratch_bytes > kScratchBytes) return LF_INVALID_ARGUMENT;
  Request request{scratch_bytes, clear != 0};
  const lunaflux::LaunchExtra extra{prepare, &request};
  return lunaflux::checked_launch(function, stream, grid_x, grid_y, grid_z, block_x, block_y,
                                  block_z, shared_memory_bytes, argument_count, allocations,
                                  offsets, byte_counts, alignments, true, &extra);
}
