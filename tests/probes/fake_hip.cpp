// fake_hip.cpp - the fake HIP runtime behind tests/probes/fake_hip.h.
#include "fake_hip.h"

#include <cstdlib>
#include <cstring>

#include "runtime_internal.h"

namespace {

lf_fake_hip_state g_state;

bool take(int32_t &flag) {
  if (flag == 0) return false;
  flag = 0;
  return true;
}

hipError_t fake_driver_version(int *v) {
  *v = 70200000;
  return hipSuccess;
}

hipError_t fake_device_count(int *n) {
  *n = g_state.device_count;
  return g_state.device_count > 0 ? hipSuccess : hipErrorNoDevice;
}

hipError_t fake_properties(hipDeviceProp_t *p, int ordinal) {
  if (ordinal < 0 || ordinal >= g_state.device_count) return hipErrorInvalidDevice;
  std::memset(p, 0, sizeof(*p));
  p->major = 9;
  p->minor = 5;
  std::strncpy(p->name, "AMD Instinct MI355X", sizeof(p->name) - 1);
  std::strncpy(p->gcnArchName, "gfx950:sramecc+:xnack-", sizeof(p->gcnArchName) - 1);
  return hipSuccess;
}

hipError_t fake_total_mem(size_t *bytes, hipDevice_t ordinal) {
  if (ordinal < 0 || ordinal >= g_state.device_count) return hipErrorInvalidDevice;
  *bytes = static_cast<size_t>(288) << 30;
  return hipSuccess;
}

hipError_t fake_set_device(int ordinal) {
  g_state.set_device_calls += 1;
  return ordinal >= 0 && ordinal < g_state.device_count ? hipSuccess : hipErrorInvalidDevice;
}

hipError_t fake_device_sync() {
  g_state.device_syncs += 1;
  g_state.free_calls_at_last_device_sync = g_state.free_calls;
  return hipSuccess;
}

hipError_t fake_malloc(void **p, size_t n) {
  g_state.malloc_calls += 1;
  if (take(g_state.fail_malloc_once)) return hipErrorOutOfMemory;
  void *q = nullptr;
  if (posix_memalign(&q, 4096, n) != 0) return hipErrorOutOfMemory;
  std::memset(q, 0xA5, n);
  *p = q;
  g_state.live_allocations += 1;
  return hipSuccess;
}

hipError_t fake_free(void *p) {
  if (p == nullptr) return hipSuccess;  // context initialisation
  g_state.free_calls += 1;
  if (take(g_state.fail_free_once)) return hipErrorInvalidValue;
  std::free(p);
  g_state.live_allocations -= 1;
  return hipSuccess;
}

hipError_t fake_memcpy(void *dst, const void *src, size_t n, hipMemcpyKind) {
  g_state.memcpy_calls += 1;
  std::memcpy(dst, src, n);
  return hipSuccess;
}

uintptr_t g_next_handle = 0x1000;

hipError_t fake_stream_create(hipStream_t *s, unsigned int flags) {
  if (flags != hipStreamNonBlocking) return hipErrorInvalidValue;
  g_state.stream_creates += 1;
  *s = reinterpret_cast<hipStream_t>(g_next_handle += 16);
  return hipSuccess;
}

hipError_t fake_stream_destroy(hipStream_t) {
  if (take(g_state.fail_stream_destroy_once)) return hipErrorInvalidHandle;
  g_state.stream_destroys += 1;
  return hipSuccess;
}

hipError_t fake_stream_sync(hipStream_t) {
  g_state.stream_syncs += 1;
  return take(g_state.fail_stream_sync_once) ? hipErrorLaunchFailure : hipSuccess;
}

hipError_t fake_event_create(hipEvent_t *e) {
  g_state.event_creates += 1;
  *e = reinterpret_cast<hipEvent_t>(g_next_handle += 16);
  return hipSuccess;
}

hipError_t fake_event_destroy(hipEvent_t) {
  g_state.event_destroys += 1;
  return hipSuccess;
}

hipError_t fake_event_record(hipEvent_t, hipStream_t) {
  g_state.event_records += 1;
  return hipSuccess;
}

hipError_t fake_event_sync(hipEvent_t) { return hipSuccess; }

hipError_t fake_elapsed(float *ms, hipEvent_t, hipEvent_t) {
  *ms = 1.5f;
  return hipSuccess;
}

hipError_t fake_module_load(hipModule_t *m, const void *image) {
  if (std::memcmp(image, lf_fake_module_image, sizeof(lf_fake_module_image)) != 0) {
    return hipErrorInvalidImage;
  }
  g_state.module_loads += 1;
  *m = reinterpret_cast<hipModule_t>(g_next_handle += 16);
  return hipSuccess;
}

hipError_t fake_module_unload(hipModule_t) {
  if (take(g_state.fail_module_unload_once)) return hipErrorInvalidHandle;
  g_state.module_unloads += 1;
  return hipSuccess;
}

hipError_t fake_get_function(hipFunction_t *f, hipModule_t, const char *name) {
  if (std::strcmp(name, "kernel_a") != 0 && std::strcmp(name, "kernel_b") != 0) {
    return hipErrorNotFound;
  }
  g_state.function_loads += 1;
  *f = reinterpret_cast<hipFunction_t>(g_next_handle += 16);
  return hipSuccess;
}

hipError_t fake_launch(hipFunction_t f, unsigned int gx, unsigned int gy, unsigned int gz,
                       unsigned int bx, unsigned int by, unsigned int bz, unsigned int lds,
                       hipStream_t stream, void **params, void **extra) {
  g_state.launches += 1;
  if (extra != nullptr || params == nullptr) return hipErrorInvalidValue;
  g_state.grid[0] = gx;
  g_state.grid[1] = gy;
  g_state.grid[2] = gz;
  g_state.block[0] = bx;
  g_state.block[1] = by;
  g_state.block[2] = bz;
  g_state.shared_memory_bytes = lds;
  g_state.stream = stream;
  g_state.function = f;
  for (int32_t i = 0; i < g_state.expected_params && i < LF_FAKE_MAX_PARAMS; ++i) {
    std::memcpy(&g_state.params[i], params[i], sizeof(uintptr_t));
  }
  if (g_state.on_launch != nullptr) g_state.on_launch(g_state.on_launch_user);
  return take(g_state.fail_launch_once) ? hipErrorLaunchFailure : hipSuccess;
}

}  // namespace

extern "C" {

const uint8_t lf_fake_module_image[16] = {'F', 'A', 'K', 'E', 'M', 'O', 'D', 0,
                                          1, 2, 3, 4, 5, 6, 7, 8};

lf_fake_hip_state *lf_fake_hip(void) { return &g_state; }

void lf_fake_hip_install(void) {
  std::memset(&g_state, 0, sizeof(g_state));
  g_state.device_count = 1;
  lunaflux::HipApi api{};
  api.DriverGetVersion = fake_driver_version;
  api.GetDeviceCount = fake_device_count;
  api.GetDeviceProperties = fake_properties;
  api.DeviceTotalMem = fake_total_mem;
  api.SetDevice = fake_set_device;
  api.DeviceSynchronize = fake_device_sync;
  api.Malloc = fake_malloc;
  api.Free = fake_free;
  api.Memcpy = fake_memcpy;
  api.StreamCreateWithFlags = fake_stream_create;
  api.StreamDestroy = fake_stream_destroy;
  api.StreamSynchronize = fake_stream_sync;
  api.EventCreate = fake_event_create;
  api.EventDestroy = fake_event_destroy;
  api.EventRecord = fake_event_record;
  api.EventSynchronize = fake_event_sync;
  api.EventElapsedTime = fake_elapsed;
  api.ModuleLoadData = fake_module_load;
  api.ModuleUnload = fake_module_unload;
  api.ModuleGetFunction = fake_get_function;
  api.ModuleLaunchKernel = fake_launch;
  lunaflux::install_hip_api(api);
}

int32_t lf_fake_inspect(const void *handle, int32_t out[4]) {
  return lunaflux::inspect(handle, out) ? 1 : 0;
}

}  // extern "C"
