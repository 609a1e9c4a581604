/*
 * lunaflux_hip_moonbit.c - the MoonBit-facing stub layer over the HIP C ABI
 * (include/lunaflux_hip.h). One function per extern of the reference's
 * private FFI (internal/cuda/ffi.mbt:29-240), taking and returning the values
 * MoonBit's C backend passes for those extern signatures:
 *
 *   FixedArray[Int64] / FixedArray[Byte]   int64_t * / uint8_t * (length in
 *                                          the object header,
 *                                          Moonbit_array_length)
 *   Bytes                                  moonbit_bytes_t
 *   Ref[Int]                               int32_t * (the cell's value)
 *   abstract handle types (Context, ...)   an external object from
 *                                          moonbit_make_external_object
 *   FixedArray[Allocation]                 an array of such objects
 *
 * These shapes are the reference's, so ffi.mbt keeps its signatures and
 * #borrow annotations; only each extern's symbol string changes, from
 * "lunaflux_cuda_<name>" to "lunaflux_hip_mbt_<name>". The reference's
 * ownership rules hold (internal/cuda/resources.c:104-133, modules.c:39-90):
 *  - every create returns an external object, also on failure (its handle is
 *    then a CLOSED library handle, or none), with the outcome in *status;
 *  - arguments are borrowed: nothing here consumes a reference the caller
 *    passes in;
 *  - the finalizer drops the object's library reference; a child handle
 *    holds a library reference on its parent (what the reference does with
 *    moonbit_incref on the parent object), so the device resource of a
 *    parent outlives every open child, and is destroyed at its explicit
 *    close or once its last reference is gone.
 * copy_to_host returns fresh Bytes (empty on failure), as
 * internal/cuda/transfers.c:207-250 does.
 *
 * Built with the MoonBit package's other native stubs (moonbit.h comes with
 * the MoonBit toolchain); links against liblunaflux_hip.so.
 */
#include <stdint.h>
#include <stdlib.h>

#include "lunaflux_hip.h"
#include "moonbit.h"

typedef struct lf_mbt_object {
  void *handle; /* the library handle, or NULL when creation failed early */
} lf_mbt_object;

static void lf_mbt_finalize(void *self) {
  lf_mbt_object *object = (lf_mbt_object *)self;
  lunaflux_hip_release(object->handle);
  object->handle = NULL;
}

static lf_mbt_object *lf_mbt_wrap(void *handle) {
  lf_mbt_object *object = (lf_mbt_object *)moonbit_make_external_object(
    lf_mbt_finalize, (uint32_t)sizeof(lf_mbt_object));
  object->handle = handle;
  return object;
}

static void *lf_mbt_handle(lf_mbt_object *object) {
  return object == NULL ? NULL : object->handle;
}

static int64_t lf_mbt_bytes_length(moonbit_bytes_t bytes) {
  return bytes == NULL ? 0 : (int64_t)Moonbit_array_length(bytes);
}

/* ffi.mbt:29-30 */
MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_probe(int64_t *output) {
  if (output == NULL || Moonbit_array_length(output) < 3) return LF_INVALID_ARGUMENT;
  return lunaflux_hip_probe(output);
}

/* ffi.mbt:33-38 */
MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_device_info(int32_t ordinal, int64_t *numeric,
                                                        uint8_t *name) {
  if (numeric == NULL || name == NULL || Moonbit_array_length(numeric) < 5 ||
      Moonbit_array_length(name) < LF_DEVICE_NAME_BYTES) {
    return LF_INVALID_ARGUMENT;
  }
  return lunaflux_hip_device_info(ordinal, numeric, name);
}

/* ffi.mbt:41-46 */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_context_create(int32_t ordinal,
                                                                  int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_context_create(ordinal, status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_context_close(lf_mbt_object *context) {
  void *h = lf_mbt_handle(context);
  return h == NULL ? LF_CLOSED : lunaflux_hip_context_close((lf_context *)h);
}

/* ffi.mbt:49-58 */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_stream_create(lf_mbt_object *context,
                                                                 int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_stream_create((lf_context *)lf_mbt_handle(context), status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_stream_close(lf_mbt_object *stream) {
  void *h = lf_mbt_handle(stream);
  return h == NULL ? LF_CLOSED : lunaflux_hip_stream_close((lf_stream *)h);
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_stream_synchronize(lf_mbt_object *stream) {
  return lunaflux_hip_stream_synchronize((lf_stream *)lf_mbt_handle(stream));
}

/* ffi.mbt:61-82 */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_event_create(lf_mbt_object *context,
                                                                int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_event_create((lf_context *)lf_mbt_handle(context), status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_event_close(lf_mbt_object *event) {
  void *h = lf_mbt_handle(event);
  return h == NULL ? LF_CLOSED : lunaflux_hip_event_close((lf_event *)h);
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_event_record(lf_mbt_object *event,
                                                         lf_mbt_object *stream) {
  return lunaflux_hip_event_record((lf_event *)lf_mbt_handle(event),
                                   (lf_stream *)lf_mbt_handle(stream));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_event_synchronize(lf_mbt_object *event) {
  return lunaflux_hip_event_synchronize((lf_event *)lf_mbt_handle(event));
}

MOONBIT_FFI_EXPORT double lunaflux_hip_mbt_event_elapsed(lf_mbt_object *start,
                                                         lf_mbt_object *finish,
                                                         int32_t *status) {
  return lunaflux_hip_event_elapsed((lf_event *)lf_mbt_handle(start),
                                    (lf_event *)lf_mbt_handle(finish), status);
}

/* ffi.mbt:85-94 */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_allocation_create(lf_mbt_object *context,
                                                                     int64_t byte_count,
                                                                     int32_t *status) {
  return lf_mbt_wrap(
    lunaflux_hip_allocation_create((lf_context *)lf_mbt_handle(context), byte_count, status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_allocation_close(lf_mbt_object *allocation) {
  void *h = lf_mbt_handle(allocation);
  return h == NULL ? LF_CLOSED : lunaflux_hip_allocation_close((lf_allocation *)h);
}

/* ffi.mbt:97-106 */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_allocation_lease_create(
  lf_mbt_object *context, lf_mbt_object *allocation, int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_allocation_lease_create(
    (lf_context *)lf_mbt_handle(context), (lf_allocation *)lf_mbt_handle(allocation), status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_allocation_lease_close(lf_mbt_object *lease) {
  void *h = lf_mbt_handle(lease);
  return h == NULL ? LF_CLOSED : lunaflux_hip_allocation_lease_close((lf_allocation_lease *)h);
}

/* ffi.mbt:109-116 */
MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_context_validate_allocation_region(
  lf_mbt_object *context, lf_mbt_object *allocation, int64_t offset, int64_t byte_count,
  int64_t alignment) {
  return lunaflux_hip_context_validate_allocation_region(
    (lf_context *)lf_mbt_handle(context), (lf_allocation *)lf_mbt_handle(allocation), offset,
    byte_count, alignment);
}

/* ffi.mbt:119-126 */
MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_copy_to_device(lf_mbt_object *allocation,
                                                           moonbit_bytes_t source,
                                                           int64_t source_offset,
                                                           int64_t destination_offset,
                                                           int64_t byte_count) {
  return lunaflux_hip_copy_to_device((lf_allocation *)lf_mbt_handle(allocation), source,
                                     lf_mbt_bytes_length(source), source_offset,
                                     destination_offset, byte_count);
}

/* ffi.mbt:129-138 */
MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_context_copy_fixed_to_device(
  lf_mbt_object *context, lf_mbt_object *allocation, uint8_t *source, int64_t source_offset,
  int64_t destination_offset, int64_t byte_count) {
  return lunaflux_hip_context_copy_fixed_to_device(
    (lf_context *)lf_mbt_handle(context), (lf_allocation *)lf_mbt_handle(allocation), source,
    lf_mbt_bytes_length(source), source_offset, destination_offset, byte_count);
}

/* ffi.mbt:141-148 */
MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_context_copy_device_to_fixed(
  lf_mbt_object *context, lf_mbt_object *allocation, uint8_t *destination,
  int64_t source_offset, int64_t destination_offset, int64_t byte_count) {
  return lunaflux_hip_context_copy_device_to_fixed(
    (lf_context *)lf_mbt_handle(context), (lf_allocation *)lf_mbt_handle(allocation),
    destination, lf_mbt_bytes_length(destination), source_offset, destination_offset,
    byte_count);
}

/* ffi.mbt:151-157; internal/cuda/transfers.c:207-250 */
MOONBIT_FFI_EXPORT moonbit_bytes_t lunaflux_hip_mbt_copy_to_host(lf_mbt_object *allocation,
                                                                 int64_t source_offset,
                                                                 int64_t byte_count,
                                                                 int32_t *status) {
  if (lf_mbt_handle(allocation) == NULL) {
    *status = LF_CLOSED;
    return moonbit_make_bytes(0, 0);
  }
  if (source_offset < 0 || byte_count < 0 || byte_count > INT32_MAX) {
    *status = LF_SIZE_OVERFLOW;
    return moonbit_make_bytes(0, 0);
  }
  moonbit_bytes_t output = moonbit_make_bytes((int32_t)byte_count, 0);
  *status = lunaflux_hip_copy_to_host((lf_allocation *)lf_mbt_handle(allocation), source_offset,
                                      byte_count, output, byte_count);
  if (*status != LF_OK) {
    moonbit_decref(output);
    return moonbit_make_bytes(0, 0);
  }
  return output;
}

/* ffi.mbt:160-169 */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_module_load(lf_mbt_object *context,
                                                               moonbit_bytes_t image,
                                                               int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_module_load((lf_context *)lf_mbt_handle(context), image,
                                              lf_mbt_bytes_length(image), status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_module_close(lf_mbt_object *module) {
  void *h = lf_mbt_handle(module);
  return h == NULL ? LF_CLOSED : lunaflux_hip_module_close((lf_module *)h);
}

/* ffi.mbt:172-181 */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_function_load(lf_mbt_object *module,
                                                                 moonbit_bytes_t name,
                                                                 int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_function_load((lf_module *)lf_mbt_handle(module), name,
                                                lf_mbt_bytes_length(name), status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_function_close(lf_mbt_object *function) {
  void *h = lf_mbt_handle(function);
  return h == NULL ? LF_CLOSED : lunaflux_hip_function_close((lf_function *)h);
}

/* ffi.mbt:184-199. The four arrays must have one entry per kernel argument
 * (1 .. 32), as internal/cuda/launch.c:66-72 requires. */
MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_function_launch(
  lf_mbt_object *function, lf_mbt_object *stream, int32_t grid_x, int32_t grid_y,
  int32_t grid_z, int32_t block_x, int32_t block_y, int32_t block_z,
  int32_t shared_memory_bytes, lf_mbt_object **allocations, int64_t *offsets,
  int64_t *byte_counts, int64_t *alignments) {
  if (allocations == NULL || offsets == NULL || byte_counts == NULL || alignments == NULL) {
    return LF_INVALID_ARGUMENT;
  }
  int32_t count = (int32_t)Moonbit_array_length(allocations);
  if (count <= 0 || count > LF_MAX_KERNEL_ARGUMENTS ||
      (int32_t)Moonbit_array_length(offsets) != count ||
      (int32_t)Moonbit_array_length(byte_counts) != count ||
      (int32_t)Moonbit_array_length(alignments) != count) {
    return LF_INVALID_ARGUMENT;
  }
  lf_allocation *handles[LF_MAX_KERNEL_ARGUMENTS];
  for (int32_t i = 0; i < count; i += 1) {
    handles[i] = (lf_allocation *)lf_mbt_handle(allocations[i]);
  }
  return lunaflux_hip_function_launch(
    (lf_function *)lf_mbt_handle(function), (lf_stream *)lf_mbt_handle(stream), grid_x, grid_y,
    grid_z, block_x, block_y, block_z, shared_memory_bytes, count, handles, offsets, byte_counts,
    alignments);
}

/* ffi.mbt:202-240: the vendor BF16 GEMM. This ABI ships none
 * (device_info reports supports_vendor_gemm = 0, so the catalog never
 * selects it); every call reports LF_UNSUPPORTED. */
MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_cublas_create(lf_mbt_object *context,
                                                                 int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_blas_create((lf_context *)lf_mbt_handle(context), status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_cublas_close(lf_mbt_object *handle) {
  void *h = lf_mbt_handle(handle);
  return h == NULL ? LF_CLOSED : lunaflux_hip_blas_close((lf_blas *)h);
}

MOONBIT_FFI_EXPORT lf_mbt_object *lunaflux_hip_mbt_bf16_gemm_plan_create(
  lf_mbt_object *handle, int64_t rows, int64_t inner, int64_t columns,
  int64_t workspace_byte_count, int32_t *status) {
  return lf_mbt_wrap(lunaflux_hip_bf16_gemm_plan_create(
    (lf_blas *)lf_mbt_handle(handle), rows, inner, columns, workspace_byte_count, status));
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_bf16_gemm_plan_close(lf_mbt_object *plan) {
  void *h = lf_mbt_handle(plan);
  return h == NULL ? LF_CLOSED : lunaflux_hip_bf16_gemm_plan_close((lf_gemm_plan *)h);
}

MOONBIT_FFI_EXPORT int32_t lunaflux_hip_mbt_bf16_gemm_plan_run(
  lf_mbt_object *plan, lf_mbt_object *left, int64_t left_offset, lf_mbt_object *right,
  int64_t right_offset, lf_mbt_object *output, int64_t output_offset, lf_mbt_object *workspace,
  int64_t workspace_offset, lf_mbt_object *stream) {
  return lunaflux_hip_bf16_gemm_plan_run(
    (lf_gemm_plan *)lf_mbt_handle(plan), (lf_allocation *)lf_mbt_handle(left), left_offset,
    (lf_allocation *)lf_mbt_handle(right), right_offset, (lf_allocation *)lf_mbt_handle(output),
    output_offset, (lf_allocation *)lf_mbt_handle(workspace), workspace_offset,
    (lf_stream *)lf_mbt_handle(stream));
}
