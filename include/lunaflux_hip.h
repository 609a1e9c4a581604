/*
 * lunaflux_hip.h - HIP (gfx950) device ABI that replaces LunaFlux's private
 * CUDA ABI (/root/reference/internal/cuda). The MoonBit `device` package is
 * the only caller (its externs live in internal/cuda/ffi.mbt:29-240); each
 * entry point below names the export it replaces.
 *
 * Conventions kept from the reference:
 *  - status codes and their values (internal/cuda/cuda_abi.h:44-54);
 *  - availability codes (internal/cuda/cuda_abi.h:34-42);
 *  - every create returns a handle even on failure, with the outcome in
 *    *status, and the handle is then CLOSED (resources.c:367-396);
 *  - resources are LIVE -> CLOSING -> CLOSED with an active-operation
 *    counter; closing a resource that is in use or has open children returns
 *    LF_BUSY (resources.c:280-312);
 *  - device pointers, driver codes and strings never cross the boundary:
 *    kernels receive `allocation base + offset` resolved inside the library
 *    after bounds and alignment checks (regions.c:5-32);
 *  - a launch is synchronous: it returns after the stream has drained
 *    (launch.c:146-163).
 *
 * Differences forced by a plain C ABI (no MoonBit runtime on this side):
 *  - arrays arrive as pointer + explicit count instead of MoonBit arrays,
 *    and byte buffers as pointer + length;
 *  - handles are reference counted by the library instead of being MoonBit
 *    external objects: a child holds a reference on its parent (the
 *    reference's moonbit_incref), and `lunaflux_hip_release` drops the
 *    caller's reference (what the MoonBit finalizer does); the device
 *    resource is destroyed at `_close` or when the last reference goes.
 *  - `lunaflux_hip_copy_to_host` fills a caller buffer instead of returning
 *    a fresh MoonBit Bytes.
 *  - `lunaflux_hip_function_launch_async` is an addition for callers that
 *    pipeline launches on one stream (benchmarks, graph-free batching); it
 *    performs every check of the synchronous launch but does not wait.
 */
#ifndef LUNAFLUX_HIP_H
#define LUNAFLUX_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* internal/cuda/cuda_abi.h:34-42 */
enum lf_availability {
  LF_AVAILABLE = 0,
  LF_UNSUPPORTED_PLATFORM = 1,
  LF_DRIVER_LIBRARY_MISSING = 2,
  LF_DRIVER_ABI_INCOMPLETE = 3,
  LF_DRIVER_INITIALIZATION_FAILED = 4,
  LF_NO_DEVICES = 5,
  LF_INVENTORY_FAILED = 6
};

/* internal/cuda/cuda_abi.h:44-54 */
enum lf_status {
  LF_OK = 0,
  LF_UNAVAILABLE = -1,
  LF_INVALID_ARGUMENT = -2,
  LF_CLOSED = -3,
  LF_BUSY = -4,
  LF_DRIVER_FAILURE = -5,
  LF_HOST_ALLOCATION_FAILED = -6,
  LF_SIZE_OVERFLOW = -7,
  LF_UNSUPPORTED = -8
};

/* Launch limits the reference enforces (internal/cuda/launch.c:6-10,
 * device/kernel_launch_types.mbt:14, internal/cuda/modules.c:135). */
#define LF_MAX_KERNEL_ARGUMENTS 32
#define LF_MAX_GRID_YZ 65535
#define LF_MAX_BLOCK_DIMENSION 1024
#define LF_MAX_THREADS_PER_BLOCK 1024
#define LF_MAX_SHARED_MEMORY_BYTES 98304
#define LF_MAX_REGION_ALIGNMENT 4096
#define LF_MAX_SYMBOL_BYTES 128
#define LF_DEVICE_NAME_BYTES 96

typedef struct lf_context lf_context;
typedef struct lf_stream lf_stream;
typedef struct lf_event lf_event;
typedef struct lf_allocation lf_allocation;
typedef struct lf_allocation_lease lf_allocation_lease;
typedef struct lf_module lf_module;
typedef struct lf_function lf_function;
typedef struct lf_blas lf_blas;
typedef struct lf_gemm_plan lf_gemm_plan;

/* Replaces lunaflux_cuda_probe (internal/cuda/loader.c:205-212;
 * ffi.mbt:29-30). output = {driver version, device count, vendor GEMM
 * available (always 0 here)}; returns an lf_availability code. */
int32_t lunaflux_hip_probe(int64_t output[3]);

/* Replaces lunaflux_cuda_device_info (loader.c:214-252; ffi.mbt:33-38).
 * numeric = {total bytes, major, minor, supports_bf16, supports_vendor_gemm}
 * with (major, minor) = (9, 5) for gfx950; name is NUL-terminated. */
int32_t lunaflux_hip_device_info(int32_t ordinal, int64_t numeric[5],
                                 uint8_t name[LF_DEVICE_NAME_BYTES]);

/* Generic reference drop for every handle type below (the MoonBit
 * finalizer's role, resources.c:363-365). Closes the device resource when
 * this was the last reference. NULL is ignored. */
void lunaflux_hip_release(void *handle);

/* Replaces lunaflux_cuda_context_create/_close (resources.c:367-401;
 * ffi.mbt:41-46). */
lf_context *lunaflux_hip_context_create(int32_t ordinal, int32_t *status);
int32_t lunaflux_hip_context_close(lf_context *context);

/* Replaces lunaflux_cuda_stream_create/_close/_synchronize (ffi.mbt:49-58).
 * Streams are non-blocking and keep the default priority. */
lf_stream *lunaflux_hip_stream_create(lf_context *context, int32_t *status);
int32_t lunaflux_hip_stream_close(lf_stream *stream);
int32_t lunaflux_hip_stream_synchronize(lf_stream *stream);

/* Replaces lunaflux_cuda_event_* (resources.c:250-365; ffi.mbt:61-82).
 * elapsed returns milliseconds between two recorded events. */
lf_event *lunaflux_hip_event_create(lf_context *context, int32_t *status);
int32_t lunaflux_hip_event_close(lf_event *event);
int32_t lunaflux_hip_event_record(lf_event *event, lf_stream *stream);
int32_t lunaflux_hip_event_synchronize(lf_event *event);
double lunaflux_hip_event_elapsed(lf_event *start, lf_event *finish,
                                  int32_t *status);

/* Replaces lunaflux_cuda_allocation_create/_close (resources.c:369-452;
 * ffi.mbt:85-94). Device memory, at least 256-byte aligned. */
lf_allocation *lunaflux_hip_allocation_create(lf_context *context,
                                              int64_t byte_count,
                                              int32_t *status);
int32_t lunaflux_hip_allocation_close(lf_allocation *allocation);

/* Replaces lunaflux_cuda_allocation_lease_create/_close
 * (allocation_lease.c; ffi.mbt:97-106): keeps the allocation open (its
 * close returns LF_BUSY) until the lease is closed. */
lf_allocation_lease *lunaflux_hip_allocation_lease_create(
  lf_context *context, lf_allocation *allocation, int32_t *status);
int32_t lunaflux_hip_allocation_lease_close(lf_allocation_lease *lease);

/* Replaces lunaflux_cuda_context_validate_allocation_region
 * (regions.c:34-79; ffi.mbt:109-116). */
int32_t lunaflux_hip_context_validate_allocation_region(
  lf_context *context, lf_allocation *allocation, int64_t offset,
  int64_t byte_count, int64_t alignment);

/* Replaces lunaflux_cuda_copy_to_device (transfers.c:48-75;
 * ffi.mbt:119-126): copies source[source_offset, +byte_count) to the
 * allocation at destination_offset, synchronously. */
int32_t lunaflux_hip_copy_to_device(lf_allocation *allocation,
                                    const uint8_t *source,
                                    int64_t source_length,
                                    int64_t source_offset,
                                    int64_t destination_offset,
                                    int64_t byte_count);
/* Replaces lunaflux_cuda_context_copy_fixed_to_device / _device_to_fixed
 * (transfers.c:77-250; ffi.mbt:129-148). */
int32_t lunaflux_hip_context_copy_fixed_to_device(
  lf_context *context, lf_allocation *allocation, const uint8_t *source,
  int64_t source_length, int64_t source_offset, int64_t destination_offset,
  int64_t byte_count);
int32_t lunaflux_hip_context_copy_device_to_fixed(
  lf_context *context, lf_allocation *allocation, uint8_t *destination,
  int64_t destination_length, int64_t source_offset,
  int64_t destination_offset, int64_t byte_count);
/* Replaces lunaflux_cuda_copy_to_host (ffi.mbt:151-157): copies
 * [source_offset, +byte_count) of the allocation into destination. */
int32_t lunaflux_hip_copy_to_host(lf_allocation *allocation,
                                  int64_t source_offset, int64_t byte_count,
                                  uint8_t *destination,
                                  int64_t destination_length);

/* Replaces lunaflux_cuda_module_load/_close (modules.c:39-111;
 * ffi.mbt:160-169). image is a gfx950 HSA code object (hipcc --genco). */
lf_module *lunaflux_hip_module_load(lf_context *context, const uint8_t *image,
                                    int64_t image_length, int32_t *status);
int32_t lunaflux_hip_module_close(lf_module *module);

/* Replaces lunaflux_cuda_function_load/_close (modules.c:118-172;
 * ffi.mbt:172-181). name: 1..128 bytes, no NUL, an identifier
 * [A-Za-z_][A-Za-z0-9_]* (kernels/artifact/admit.mbt:56-92). */
lf_function *lunaflux_hip_function_load(lf_module *module,
                                        const uint8_t *name,
                                        int64_t name_length, int32_t *status);
int32_t lunaflux_hip_function_close(lf_function *function);

/* Replaces lunaflux_cuda_function_launch (launch.c:41-173; ffi.mbt:184-199).
 * Every kernel parameter is one device region: allocations[i] base +
 * offsets[i], checked against byte_counts[i] and alignments[i] (a power of
 * two <= 4096). Grid, block and dynamic LDS are validated as in
 * launch.c:12-38. Returns after the stream has drained. */
int32_t lunaflux_hip_function_launch(
  lf_function *function, lf_stream *stream, int32_t grid_x, int32_t grid_y,
  int32_t grid_z, int32_t block_x, int32_t block_y, int32_t block_z,
  int32_t shared_memory_bytes, int32_t argument_count,
  lf_allocation *const *allocations, const int64_t *offsets,
  const int64_t *byte_counts, const int64_t *alignments);
/* Same checks, but returns once the launch is enqueued (addition; see the
 * file comment). */
int32_t lunaflux_hip_function_launch_async(
  lf_function *function, lf_stream *stream, int32_t grid_x, int32_t grid_y,
  int32_t grid_z, int32_t block_x, int32_t block_y, int32_t block_z,
  int32_t shared_memory_bytes, int32_t argument_count,
  lf_allocation *const *allocations, const int64_t *offsets,
  const int64_t *byte_counts, const int64_t *alignments);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): a synchronous launch with every check of
 * lunaflux_hip_function_launch, whose kernel receives argument_count region
 * arguments followed by one more: the device address of this library's
 * scratch array on the stream's device. The array is LF_SCRATCH_MAX_BYTES
 * (16 MiB), held by each GPU the library launches on until the process ends;
 * the kernel may use its first scratch_bytes (1 .. LF_SCRATCH_MAX_BYTES,
 * else LF_INVALID_ARGUMENT, with nothing launched). With clear != 0 those
 * bytes are zeroed first, by a fill kernel on the same stream. Nothing is
 * allocated (no hipMalloc, hipFree or allocating library call). Every call on
 * one GPU shares that GPU's array, which keeps the last call's contents
 * (clear what must start at zero); calls that overlap on one GPU (several
 * threads or streams) race. argument_count + 1 <= 32. */
#define LF_SCRATCH_MAX_BYTES (16 << 20)
int32_t lunaflux_hip_function_launch_scratch(
  lf_function *function, lf_stream *stream, int32_t grid_x, int32_t grid_y,
  int32_t grid_z, int32_t block_x, int32_t block_y, int32_t block_z,
  int32_t shared_memory_bytes, int32_t argument_count,
  lf_allocation *const *allocations, const int64_t *offsets,
  const int64_t *byte_counts, const int64_t *alignments,
  int64_t scratch_bytes, int32_t clear);

/* Replace lunaflux_cuda_cublas_create/_close and the BF16 vendor GEMM plan
 * (gemm.c:108-397; ffi.mbt:202-240). This ABI ships no vendor GEMM: create
 * returns a CLOSED handle with LF_UNSUPPORTED, matching device_info's
 * supports_vendor_gemm = 0, so the catalog never selects it. */
lf_blas *lunaflux_hip_blas_create(lf_context *context, int32_t *status);
int32_t lunaflux_hip_blas_close(lf_blas *blas);
lf_gemm_plan *lunaflux_hip_bf16_gemm_plan_create(lf_blas *blas, int64_t rows,
                                                 int64_t inner,
                                                 int64_t columns,
                                                 int64_t workspace_byte_count,
                                                 int32_t *status);
int32_t lunaflux_hip_bf16_gemm_plan_close(lf_gemm_plan *plan);
int32_t lunaflux_hip_bf16_gemm_plan_run(
  lf_gemm_plan *plan, lf_allocation *left, int64_t left_offset,
  lf_allocation *right, int64_t right_offset, lf_allocation *output,
  int64_t output_offset, lf_allocation *workspace, int64_t workspace_offset,
  lf_stream *stream);

#ifdef __cplusplus
}
#endif

#endif
