/*
 * moonbit_probe.c - CPU probe of the MoonBit stub layer
 * (lunaflux_amd/csrc/moonbit/lunaflux_hip_moonbit.c): every function the
 * `device` package's externs bind (internal/cuda/ffi.mbt:29-240, symbol
 * strings renamed to lunaflux_hip_mbt_*), called with the values MoonBit
 * passes (FixedArray, Bytes, Ref[Int] cells, external objects), over the
 * fake HIP runtime. Checks the reference's conventions at this layer:
 * creates return an object also on failure, with the outcome in the status
 * cell; array lengths come from the object headers (all four launch arrays
 * must agree, 1..32 entries, internal/cuda/launch.c:66-72); copy_to_host
 * returns fresh Bytes, empty on failure (internal/cuda/transfers.c:207-250);
 * finalizers release every device resource, a parent's only after its
 * children's, and leave no object behind.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fake_hip.h"
#include "lunaflux_hip.h"
#include "moonbit.h"

#define CHECK(cond)                                                             \
  do {                                                                          \
    if (!(cond)) {                                                              \
      fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      return 1;                                                                 \
    }                                                                           \
  } while (0)

typedef void *obj;

/* the stub layer's exports (what ffi.mbt's externs bind) */
int32_t lunaflux_hip_mbt_probe(int64_t *output);
int32_t lunaflux_hip_mbt_device_info(int32_t ordinal, int64_t *numeric, uint8_t *name);
obj lunaflux_hip_mbt_context_create(int32_t ordinal, int32_t *status);
int32_t lunaflux_hip_mbt_context_close(obj context);
obj lunaflux_hip_mbt_stream_create(obj context, int32_t *status);
int32_t lunaflux_hip_mbt_stream_close(obj stream);
int32_t lunaflux_hip_mbt_stream_synchronize(obj stream);
obj lunaflux_hip_mbt_event_create(obj context, int32_t *status);
int32_t lunaflux_hip_mbt_event_close(obj event);
int32_t lunaflux_hip_mbt_event_record(obj event, obj stream);
int32_t lunaflux_hip_mbt_event_synchronize(obj event);
double lunaflux_hip_mbt_event_elapsed(obj start, obj finish, int32_t *status);
obj lunaflux_hip_mbt_allocation_create(obj context, int64_t byte_count, int32_t *status);
int32_t lunaflux_hip_mbt_allocation_close(obj allocation);
obj lunaflux_hip_mbt_allocation_lease_create(obj context, obj allocation, int32_t *status);
int32_t lunaflux_hip_mbt_allocation_lease_close(obj lease);
int32_t lunaflux_hip_mbt_context_validate_allocation_region(obj context, obj allocation,
                                                            int64_t offset, int64_t byte_count,
                                                            int64_t alignment);
int32_t lunaflux_hip_mbt_copy_to_device(obj allocation, moonbit_bytes_t source,
                                        int64_t source_offset, int64_t destination_offset,
                                        int64_t byte_count);
int32_t lunaflux_hip_mbt_context_copy_fixed_to_device(obj context, obj allocation,
                                                      uint8_t *source, int64_t source_offset,
                                                      int64_t destination_offset,
                                                      int64_t byte_count);
int32_t lunaflux_hip_mbt_context_copy_device_to_fixed(obj context, obj allocation,
                                                      uint8_t *destination,
                                                      int64_t source_offset,
                                                      int64_t destination_offset,
                                                      int64_t byte_count);
moonbit_bytes_t lunaflux_hip_mbt_copy_to_host(obj allocation, int64_t source_offset,
                                              int64_t byte_count, int32_t *status);
obj lunaflux_hip_mbt_module_load(obj context, moonbit_bytes_t image, int32_t *status);
int32_t lunaflux_hip_mbt_module_close(obj module);
obj lunaflux_hip_mbt_function_load(obj module, moonbit_bytes_t name, int32_t *status);
int32_t lunaflux_hip_mbt_function_close(obj function);
int32_t lunaflux_hip_mbt_function_launch(obj function, obj stream, int32_t grid_x,
                                         int32_t grid_y, int32_t grid_z, int32_t block_x,
                                         int32_t block_y, int32_t block_z,
                                         int32_t shared_memory_bytes, obj *allocations,
                                         int64_t *offsets, int64_t *byte_counts,
                                         int64_t *alignments);
obj lunaflux_hip_mbt_cublas_create(obj context, int32_t *status);
int32_t lunaflux_hip_mbt_cublas_close(obj handle);
obj lunaflux_hip_mbt_bf16_gemm_plan_create(obj handle, int64_t rows, int64_t inner,
                                           int64_t columns, int64_t workspace_byte_count,
                                           int32_t *status);
int32_t lunaflux_hip_mbt_bf16_gemm_plan_close(obj plan);
int32_t lunaflux_hip_mbt_bf16_gemm_plan_run(obj plan, obj left, int64_t left_offset, obj right,
                                            int64_t right_offset, obj output,
                                            int64_t output_offset, obj workspace,
                                            int64_t workspace_offset, obj stream);

static moonbit_bytes_t bytes_of(const void *data, int32_t n) {
  moonbit_bytes_t b = moonbit_make_bytes(n, 0);
  memcpy(b, data, (size_t)n);
  return b;
}

static int64_t *int64s(int32_t n, const int64_t *values) {
  int64_t *a = moonbit_shim_int64_array(n);
  for (int32_t i = 0; i < n; ++i) a[i] = values[i];
  return a;
}

static int probe_device_queries(void) {
  int64_t *out = moonbit_shim_int64_array(3);
  CHECK(lunaflux_hip_mbt_probe(out) == LF_AVAILABLE && out[1] == 1 && out[2] == 0);
  moonbit_decref(out);
  int64_t *short_out = moonbit_shim_int64_array(2);
  CHECK(lunaflux_hip_mbt_probe(short_out) == LF_INVALID_ARGUMENT);
  moonbit_decref(short_out);
  int64_t *numeric = moonbit_shim_int64_array(5);
  uint8_t *name = moonbit_shim_byte_array(LF_DEVICE_NAME_BYTES);
  CHECK(lunaflux_hip_mbt_device_info(0, numeric, name) == LF_OK);
  CHECK(numeric[1] == 9 && numeric[2] == 5 && numeric[3] == 1 && numeric[4] == 0);
  CHECK(strcmp((const char *)name, "AMD Instinct MI355X") == 0);
  uint8_t *short_name = moonbit_shim_byte_array(95);
  CHECK(lunaflux_hip_mbt_device_info(0, numeric, short_name) == LF_INVALID_ARGUMENT);
  moonbit_decref(numeric);
  moonbit_decref(name);
  moonbit_decref(short_name);
  return 0;
}

static int probe_resources_and_transfers(void) {
  lf_fake_hip_state *f = lf_fake_hip();
  int32_t st = -99;
  obj bad = lunaflux_hip_mbt_context_create(7, &st);
  CHECK(bad != NULL && st == LF_INVALID_ARGUMENT);  /* an object, also on failure */
  obj bad_stream = lunaflux_hip_mbt_stream_create(bad, &st);
  CHECK(bad_stream != NULL && st == LF_CLOSED);
  CHECK(lunaflux_hip_mbt_stream_synchronize(bad_stream) == LF_CLOSED);
  moonbit_decref(bad_stream);
  moonbit_decref(bad);

  obj ctx = lunaflux_hip_mbt_context_create(0, &st);
  CHECK(st == LF_OK);
  obj s = lunaflux_hip_mbt_stream_create(ctx, &st);
  CHECK(st == LF_OK && lunaflux_hip_mbt_stream_synchronize(s) == LF_OK);
  obj e0 = lunaflux_hip_mbt_event_create(ctx, &st);
  obj e1 = lunaflux_hip_mbt_event_create(ctx, &st);
  CHECK(lunaflux_hip_mbt_event_record(e0, s) == LF_OK && lunaflux_hip_mbt_event_record(e1, s) == LF_OK);
  CHECK(lunaflux_hip_mbt_event_synchronize(e1) == LF_OK);
  CHECK(lunaflux_hip_mbt_event_elapsed(e0, e1, &st) == 1.5 && st == LF_OK);
  CHECK(lunaflux_hip_mbt_context_close(ctx) == LF_BUSY);
  CHECK(lunaflux_hip_mbt_event_close(e0) == LF_OK && lunaflux_hip_mbt_event_close(e1) == LF_OK);

  obj a = lunaflux_hip_mbt_allocation_create(ctx, 128, &st);
  CHECK(st == LF_OK);
  obj none = lunaflux_hip_mbt_allocation_create(ctx, 0, &st);
  CHECK(none != NULL && st == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_mbt_context_validate_allocation_region(ctx, a, 64, 64, 64) == LF_OK);
  CHECK(lunaflux_hip_mbt_context_validate_allocation_region(ctx, a, 64, 65, 1) ==
        LF_INVALID_ARGUMENT);
  obj lease = lunaflux_hip_mbt_allocation_lease_create(ctx, a, &st);
  CHECK(st == LF_OK && lunaflux_hip_mbt_allocation_close(a) == LF_BUSY);
  CHECK(lunaflux_hip_mbt_allocation_lease_close(lease) == LF_OK);

  uint8_t pattern[48];
  for (int i = 0; i < 48; ++i) pattern[i] = (uint8_t)(3 * i + 5);
  moonbit_bytes_t src = bytes_of(pattern, 48);
  CHECK(lunaflux_hip_mbt_copy_to_device(a, src, 8, 0, 40) == LF_OK);
  CHECK(lunaflux_hip_mbt_copy_to_device(a, src, 9, 0, 40) == LF_INVALID_ARGUMENT);  /* past src */
  CHECK(lunaflux_hip_mbt_copy_to_device(a, src, -1, 0, 4) == LF_SIZE_OVERFLOW);
  moonbit_bytes_t back = lunaflux_hip_mbt_copy_to_host(a, 0, 40, &st);
  CHECK(st == LF_OK && Moonbit_array_length(back) == 40 && memcmp(back, pattern + 8, 40) == 0);
  moonbit_decref(back);
  uint8_t *fixed = moonbit_shim_byte_array(16);
  memcpy(fixed, pattern, 16);
  CHECK(lunaflux_hip_mbt_context_copy_fixed_to_device(ctx, a, fixed, 0, 100, 16) == LF_OK);
  CHECK(lunaflux_hip_mbt_context_copy_fixed_to_device(ctx, a, fixed, 4, 100, 16) ==
        LF_INVALID_ARGUMENT);
  uint8_t *dst = moonbit_shim_byte_array(16);
  CHECK(lunaflux_hip_mbt_context_copy_device_to_fixed(ctx, a, dst, 100, 0, 16) == LF_OK);
  CHECK(memcmp(dst, pattern, 16) == 0);
  CHECK(lunaflux_hip_mbt_context_copy_device_to_fixed(ctx, a, dst, 120, 0, 16) ==
        LF_INVALID_ARGUMENT);
  /* failures return empty Bytes, with the status */
  moonbit_bytes_t empty = lunaflux_hip_mbt_copy_to_host(a, 100, 29, &st);
  CHECK(st == LF_INVALID_ARGUMENT && Moonbit_array_length(empty) == 0);
  moonbit_decref(empty);
  empty = lunaflux_hip_mbt_copy_to_host(a, 0, -1, &st);
  CHECK(st == LF_SIZE_OVERFLOW && Moonbit_array_length(empty) == 0);
  moonbit_decref(empty);
  empty = lunaflux_hip_mbt_copy_to_host(a, 0, 0, &st);
  CHECK(st == LF_OK && Moonbit_array_length(empty) == 0);
  moonbit_decref(empty);
  CHECK(lunaflux_hip_mbt_allocation_close(a) == LF_OK);
  empty = lunaflux_hip_mbt_copy_to_host(a, 0, 8, &st);
  CHECK(st == LF_CLOSED && Moonbit_array_length(empty) == 0);
  moonbit_decref(empty);

  moonbit_decref(src);
  moonbit_decref(fixed);
  moonbit_decref(dst);
  moonbit_decref(lease);
  moonbit_decref(a);
  moonbit_decref(none);
  moonbit_decref(e0);
  moonbit_decref(e1);
  /* finalizing the context's object first: the stream's hold keeps the
   * context open, so the stream still works; finalizing the stream then
   * releases both */
  int32_t destroys = f->stream_destroys;
  moonbit_decref(ctx);
  CHECK(lunaflux_hip_mbt_stream_synchronize(s) == LF_OK);
  moonbit_decref(s);
  CHECK(f->stream_destroys == destroys + 1);
  return 0;
}

static int probe_modules_and_launch(void) {
  lf_fake_hip_state *f = lf_fake_hip();
  int32_t st = -99;
  obj ctx = lunaflux_hip_mbt_context_create(0, &st);
  obj s = lunaflux_hip_mbt_stream_create(ctx, &st);
  moonbit_bytes_t image = bytes_of(lf_fake_module_image, 16);
  obj m = lunaflux_hip_mbt_module_load(ctx, image, &st);
  CHECK(st == LF_OK);
  moonbit_bytes_t junk = moonbit_make_bytes(16, 0);
  obj bad_module = lunaflux_hip_mbt_module_load(ctx, junk, &st);
  CHECK(bad_module != NULL && st == LF_DRIVER_FAILURE);
  moonbit_bytes_t nothing = moonbit_make_bytes(0, 0);
  obj empty_module = lunaflux_hip_mbt_module_load(ctx, nothing, &st);
  CHECK(empty_module != NULL && st == LF_INVALID_ARGUMENT);
  moonbit_bytes_t name = bytes_of("kernel_a", 8);
  obj fn = lunaflux_hip_mbt_function_load(m, name, &st);
  CHECK(st == LF_OK);
  moonbit_bytes_t bad_name = bytes_of("kernel-a", 8);
  obj bad_fn = lunaflux_hip_mbt_function_load(m, bad_name, &st);
  CHECK(bad_fn != NULL && st == LF_INVALID_ARGUMENT);

  obj first = lunaflux_hip_mbt_allocation_create(ctx, 256, &st);
  obj second = lunaflux_hip_mbt_allocation_create(ctx, 256, &st);
  /* device addresses of the two allocations, through offset-0 launches */
  obj *one = (obj *)moonbit_shim_object_array(2);
  one[0] = first;
  one[1] = second;
  const int64_t z2[2] = {0, 0}, o2[2] = {1, 1};
  int64_t *off2 = int64s(2, z2), *bytes2 = int64s(2, o2), *al2 = int64s(2, o2);
  f->expected_params = 2;
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, one, off2, bytes2, al2) ==
        LF_OK);
  uintptr_t base1 = f->params[0], base2 = f->params[1];

  obj *args = (obj *)moonbit_shim_object_array(3);
  args[0] = first;
  args[1] = second;
  args[2] = first;
  const int64_t offs[3] = {16, 32, 64}, sizes[3] = {16, 32, 64};
  int64_t *offsets = int64s(3, offs), *bytes = int64s(3, sizes), *aligns = int64s(3, sizes);
  f->expected_params = 3;
  int32_t launches = f->launches;
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 3, 2, 1, 8, 4, 2, 64, args, offsets, bytes,
                                         aligns) == LF_OK);
  CHECK(f->launches == launches + 1);
  CHECK(f->params[0] == base1 + 16 && f->params[1] == base2 + 32 && f->params[2] == base1 + 64);
  CHECK(f->grid[0] == 3 && f->block[2] == 2 && f->shared_memory_bytes == 64);
  /* the four arrays must agree in length, 1..32 */
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, args, off2, bytes,
                                         aligns) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, args, offsets, bytes2,
                                         aligns) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, args, offsets, bytes,
                                         al2) == LF_INVALID_ARGUMENT);
  obj *none = (obj *)moonbit_shim_object_array(0);
  int64_t *z0 = moonbit_shim_int64_array(0);
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, none, z0, z0, z0) ==
        LF_INVALID_ARGUMENT);
  obj *many = (obj *)moonbit_shim_object_array(33);
  int64_t *z33 = moonbit_shim_int64_array(33);
  for (int i = 0; i < 33; ++i) {
    many[i] = first;
    z33[i] = 1;
  }
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, many, z33, z33, z33) ==
        LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1025, 1, 1, 0, args, offsets, bytes,
                                         aligns) == LF_INVALID_ARGUMENT);
  CHECK(f->launches == launches + 1);
  /* a closed function or operand */
  CHECK(lunaflux_hip_mbt_allocation_close(second) == LF_OK);
  CHECK(lunaflux_hip_mbt_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, args, offsets, bytes,
                                         aligns) == LF_CLOSED);
  CHECK(lunaflux_hip_mbt_module_close(m) == LF_BUSY);
  CHECK(lunaflux_hip_mbt_function_close(fn) == LF_OK && lunaflux_hip_mbt_module_close(m) == LF_OK);

  /* the vendor GEMM: objects returned, every call UNSUPPORTED */
  obj blas = lunaflux_hip_mbt_cublas_create(ctx, &st);
  CHECK(blas != NULL && st == LF_UNSUPPORTED);
  obj plan = lunaflux_hip_mbt_bf16_gemm_plan_create(blas, 4, 4, 4, 0, &st);
  CHECK(plan != NULL && st == LF_UNSUPPORTED);
  CHECK(lunaflux_hip_mbt_bf16_gemm_plan_run(plan, first, 0, first, 0, first, 0, first, 0, s) ==
        LF_UNSUPPORTED);
  CHECK(lunaflux_hip_mbt_bf16_gemm_plan_close(plan) == LF_OK);
  CHECK(lunaflux_hip_mbt_cublas_close(blas) == LF_OK);

  obj objects[] = {plan, blas, fn, bad_fn, m, bad_module, empty_module, first, second, s, ctx};
  for (size_t i = 0; i < sizeof(objects) / sizeof(objects[0]); ++i) moonbit_decref(objects[i]);
  void *arrays[] = {image, junk, nothing, name, bad_name, one, off2, bytes2, al2, args,
                    offsets, bytes, aligns, none, z0, many, z33};
  for (size_t i = 0; i < sizeof(arrays) / sizeof(arrays[0]); ++i) moonbit_decref(arrays[i]);
  return 0;
}

int main(void) {
  lf_fake_hip_install();
  struct {
    const char *name;
    int (*run)(void);
  } probes[] = {{"device_queries", probe_device_queries},
                {"resources_and_transfers", probe_resources_and_transfers},
                {"modules_and_launch", probe_modules_and_launch}};
  for (size_t i = 0; i < sizeof(probes) / sizeof(probes[0]); ++i) {
    if (probes[i].run() != 0) {
      fprintf(stderr, "probe %s failed\n", probes[i].name);
      return 1;
    }
    printf("ok %s\n", probes[i].name);
  }
  lf_fake_hip_state *f = lf_fake_hip();
  if (moonbit_shim_live_objects() != 0 || f->live_allocations != 0 ||
      f->module_loads != f->module_unloads || f->stream_creates != f->stream_destroys ||
      f->event_creates != f->event_destroys) {
    fprintf(stderr, "leak: %d objects, %d allocations, modules %d/%d, streams %d/%d\n",
            moonbit_shim_live_objects(), f->live_allocations, f->module_loads,
            f->module_unloads, f->stream_creates, f->stream_destroys);
    return 1;
  }
  printf("ok all\n");
  return 0;
}
