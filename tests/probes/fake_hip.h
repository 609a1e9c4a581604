/*
 * fake_hip.h - a fake HIP runtime for CPU tests of the C ABI, in the spirit
 * of the reference's fake-driver probes (internal/cuda/launch_probe.c:40-131,
 * region_probe.c, lifecycle_probe.c): the library's dispatch table
 * (lunaflux::HipApi) is pointed at these functions, which record every call
 * and can be told to fail once. Device memory is host memory, so transfers
 * round-trip for real. Only the library's CPU test build (LUNAFLUX_HIP_FAKE)
 * links this.
 */
#ifndef LUNAFLUX_TEST_FAKE_HIP_H
#define LUNAFLUX_TEST_FAKE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LF_FAKE_MAX_PARAMS 40

typedef struct lf_fake_hip_state {
  int32_t device_count;
  /* call counts */
  int32_t set_device_calls, malloc_calls, free_calls, memcpy_calls;
  int32_t stream_creates, stream_destroys, stream_syncs, device_syncs;
  int32_t event_creates, event_destroys, event_records;
  int32_t module_loads, module_unloads, function_loads, launches;
  int32_t live_allocations; /* successful mallocs minus successful frees */
  /* failure injection: the next such call fails (then the flag clears) */
  int32_t fail_launch_once, fail_stream_sync_once, fail_stream_destroy_once;
  int32_t fail_free_once, fail_module_unload_once, fail_malloc_once;
  /* the last launch */
  uint32_t grid[3], block[3], shared_memory_bytes;
  void *stream, *function;
  int32_t expected_params; /* how many kernel parameters to record */
  uintptr_t params[LF_FAKE_MAX_PARAMS];
  /* the order of the last device synchronization relative to frees */
  int32_t free_calls_at_last_device_sync;
  /* called inside the fake launch, while the library holds every operand */
  void (*on_launch)(void *user);
  void *on_launch_user;
} lf_fake_hip_state;

/* Installs the fake runtime into the library's dispatch table (call first). */
void lf_fake_hip_install(void);
lf_fake_hip_state *lf_fake_hip(void);
/* The fake code object image lunaflux_hip_module_load accepts. */
extern const uint8_t lf_fake_module_image[16];
/* Library handle counters: {state, active operations, children, references};
 * returns 0 for a pointer that is not a library handle. */
int32_t lf_fake_inspect(const void *handle, int32_t out[4]);

#ifdef __cplusplus
}
#endif

#endif
