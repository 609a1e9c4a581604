// runtime_internal.h - what the library's other translation units (and its
// CPU test build) use from runtime.cpp; not part of the C ABI.
#pragma once

#include "lunaflux_hip.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace lunaflux {

// Every HIP runtime call runtime.cpp makes goes through this table, the
// counterpart of the reference's driver dispatch table (lf_cuda_api,
// internal/cuda/cuda_abi.h:56-141). The library fills it with the HIP
// runtime's own entry points; the CPU test build (LUNAFLUX_HIP_FAKE) starts
// it empty and installs fakes, as the reference's fake-driver probes do
// (internal/cuda/launch_probe.c, region_probe.c, lifecycle_probe.c).
struct HipApi {
  hipError_t (*DriverGetVersion)(int *);
  hipError_t (*GetDeviceCount)(int *);
  hipError_t (*GetDeviceProperties)(hipDeviceProp_t *, int);
  hipError_t (*DeviceTotalMem)(size_t *, hipDevice_t);
  hipError_t (*SetDevice)(int);
  hipError_t (*DeviceSynchronize)();
  hipError_t (*Malloc)(void **, size_t);
  hipError_t (*Free)(void *);
  hipError_t (*Memcpy)(void *, const void *, size_t, hipMemcpyKind);
  hipError_t (*StreamCreateWithFlags)(hipStream_t *, unsigned int);
  hipError_t (*StreamDestroy)(hipStream_t);
  hipError_t (*StreamSynchronize)(hipStream_t);
  hipError_t (*EventCreate)(hipEvent_t *);
  hipError_t (*EventDestroy)(hipEvent_t);
  hipError_t (*EventRecord)(hipEvent_t, hipStream_t);
  hipError_t (*EventSynchronize)(hipEvent_t);
  hipError_t (*EventElapsedTime)(float *, hipEvent_t, hipEvent_t);
  hipError_t (*ModuleLoadData)(hipModule_t *, const void *);
  hipError_t (*ModuleUnload)(hipModule_t);
  hipError_t (*ModuleGetFunction)(hipFunction_t *, hipModule_t, const char *);
  hipError_t (*ModuleLaunchKernel)(hipFunction_t, unsigned int, unsigned int, unsigned int,
                                   unsigned int, unsigned int, unsigned int, unsigned int,
                                   hipStream_t, void **, void **);
};

const HipApi &hip();

// `prepare` runs once every check of the launch has passed, with the
// context's device current and the function, module, stream and every
// allocation held open: it may enqueue work on `stream` ahead of the kernel
// and must store the trailing argument's value in *value. A status other
// than LF_OK abandons the launch and is returned.
struct LaunchExtra {
  int32_t (*prepare)(void *context, int32_t ordinal, hipStream_t stream, uintptr_t *value);
  void *context;
};

// lunaflux_hip_function_launch(_async) with, when extra is not null, one
// more kernel argument after the argc regions (argc + 1 <= 32).
int32_t checked_launch(lf_function *function, lf_stream *stream, int32_t grid_x,
                       int32_t grid_y, int32_t grid_z, int32_t block_x, int32_t block_y,
                       int32_t block_z, int32_t shared_memory_bytes, int32_t argc,
                       lf_allocation *const *allocations, const int64_t *offsets,
                       const int64_t *byte_counts, const int64_t *alignments,
                       bool synchronous, const LaunchExtra *extra);

#ifdef LUNAFLUX_HIP_FAKE
// CPU test build only: install the fake runtime (before any other call), and
// read a handle's lifecycle counters {state, active operations, children,
// references}; state 0 LIVE, 1 CLOSING, 2 CLOSED. Returns false for a
// pointer that is not a handle of this library.
void install_hip_api(const HipApi &api);
bool inspect(const void *handle, int32_t out[4]);
#endif

}  // namespace lunaflux
