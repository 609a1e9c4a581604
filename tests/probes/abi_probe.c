/*
 * abi_probe.c - CPU probes of the HIP C ABI (include/lunaflux_hip.h) over the
 * fake HIP runtime, covering what the reference's fake-driver probes cover
 * for internal/cuda: lifecycle interlocks and retryable closes
 * (lifecycle_probe.c), region checks and leases (region_probe.c,
 * allocation_lease_probe.c), transfers (transfer_probe.c), and the launch
 * path (launch_probe.c:40-131: every operand held during the launch, close
 * -> LF_BUSY, kernel parameter = allocation base + offset, dimension and
 * argument limits, injected launch and synchronization failures). Also the
 * symbol grammar (kernels/artifact/admit.mbt:56-92) and this ABI's own
 * addition, the asynchronous launch: a module or allocation it used is only
 * released after its device has drained.
 *
 * Prints one "ok <probe>" line per probe; exits non-zero at the first
 * failed check, naming it.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fake_hip.h"
#include "lunaflux_hip.h"

#define CHECK(cond)                                                  \
  do {                                                               \
    if (!(cond)) {                                                   \
      fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      return 1;                                                      \
    }                                                                \
  } while (0)

enum { kLive = 0, kClosing = 1, kClosed = 2 };

static int32_t state_of(const void *h) {
  int32_t c[4];
  return lf_fake_inspect(h, c) ? c[0] : -1;
}
static int32_t active_of(const void *h) {
  int32_t c[4];
  return lf_fake_inspect(h, c) ? c[1] : -1;
}
static int32_t children_of(const void *h) {
  int32_t c[4];
  return lf_fake_inspect(h, c) ? c[2] : -1;
}

/* releases a handle a check only needs the creation status of */
static int released(void *handle) {
  lunaflux_hip_release(handle);
  return handle != NULL;
}

static lf_context *new_context(void) {
  int32_t st = -99;
  lf_context *c = lunaflux_hip_context_create(0, &st);
  return st == LF_OK ? c : NULL;
}

static int probe_availability(void) {
  int64_t out[3] = {0, 0, 7};
  CHECK(lunaflux_hip_probe(out) == LF_AVAILABLE);
  CHECK(out[0] == 70200000 && out[1] == 1 && out[2] == 0);
  int64_t numeric[5];
  uint8_t name[LF_DEVICE_NAME_BYTES];
  CHECK(lunaflux_hip_device_info(0, numeric, name) == LF_OK);
  CHECK(numeric[0] == (int64_t)288 << 30 && numeric[1] == 9 && numeric[2] == 5);
  CHECK(numeric[3] == 1 && numeric[4] == 0);
  CHECK(strcmp((const char *)name, "AMD Instinct MI355X") == 0);
  CHECK(lunaflux_hip_device_info(1, numeric, name) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_device_info(-1, numeric, name) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_device_info(0, NULL, name) == LF_INVALID_ARGUMENT);
  return 0;
}

static int probe_lifecycle(void) {
  lf_fake_hip_state *f = lf_fake_hip();
  int32_t st = -99;
  /* a failed create still returns a handle, CLOSED, with the outcome */
  lf_context *bad = lunaflux_hip_context_create(3, &st);
  CHECK(bad != NULL && st == LF_INVALID_ARGUMENT && state_of(bad) == kClosed);
  CHECK(released(lunaflux_hip_stream_create(bad, &st)) && st == LF_CLOSED);
  CHECK(lunaflux_hip_context_close(bad) == LF_OK);
  lunaflux_hip_release(bad);

  lf_context *ctx = new_context();
  CHECK(ctx != NULL && state_of(ctx) == kLive);
  lf_stream *s = lunaflux_hip_stream_create(ctx, &st);
  CHECK(st == LF_OK && children_of(ctx) == 1);
  lf_event *e = lunaflux_hip_event_create(ctx, &st);
  CHECK(st == LF_OK && children_of(ctx) == 2);
  /* closing a parent with open children is refused and changes nothing */
  CHECK(lunaflux_hip_context_close(ctx) == LF_BUSY && state_of(ctx) == kLive);
  /* a close whose driver call fails leaves the object LIVE; a retry works */
  f->fail_stream_destroy_once = 1;
  CHECK(lunaflux_hip_stream_close(s) == LF_DRIVER_FAILURE && state_of(s) == kLive);
  CHECK(children_of(ctx) == 2);
  CHECK(lunaflux_hip_stream_synchronize(s) == LF_OK);
  CHECK(lunaflux_hip_stream_close(s) == LF_OK && state_of(s) == kClosed);
  CHECK(lunaflux_hip_stream_close(s) == LF_OK);  /* idempotent */
  CHECK(children_of(ctx) == 1);
  CHECK(lunaflux_hip_stream_synchronize(s) == LF_CLOSED);
  /* events: elapsed needs both recorded */
  lf_stream *s2 = lunaflux_hip_stream_create(ctx, &st);
  lf_event *e2 = lunaflux_hip_event_create(ctx, &st);
  CHECK(lunaflux_hip_event_elapsed(e, e2, &st) == 0.0 && st == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_event_record(e, s2) == LF_OK && lunaflux_hip_event_record(e2, s2) == LF_OK);
  CHECK(lunaflux_hip_event_elapsed(e, e2, &st) == 1.5 && st == LF_OK);
  CHECK(lunaflux_hip_event_synchronize(e2) == LF_OK);
  /* dropping the last reference closes a live child and frees its slot */
  lunaflux_hip_release(e2);
  lunaflux_hip_release(e);
  CHECK(children_of(ctx) == 1);
  CHECK(lunaflux_hip_stream_close(s2) == LF_OK);
  lunaflux_hip_release(s2);
  lunaflux_hip_release(s);
  CHECK(children_of(ctx) == 0);
  CHECK(lunaflux_hip_context_close(ctx) == LF_OK && state_of(ctx) == kClosed);
  /* a handle of the wrong kind is refused */
  CHECK(lunaflux_hip_stream_close((lf_stream *)ctx) == LF_INVALID_ARGUMENT);
  lunaflux_hip_release(ctx);
  return 0;
}

static int probe_regions(void) {
  int32_t st = -99;
  lf_context *ctx = new_context();
  lf_context *other = new_context();
  lf_allocation *a = lunaflux_hip_allocation_create(ctx, 4096, &st);
  CHECK(st == LF_OK);
  lf_allocation *b = lunaflux_hip_allocation_create(other, 64, &st);
  CHECK(st == LF_OK);
  CHECK(released(lunaflux_hip_allocation_create(ctx, 0, &st)) && st == LF_INVALID_ARGUMENT);
  CHECK(released(lunaflux_hip_allocation_create(ctx, -5, &st)) && st == LF_INVALID_ARGUMENT);
  lf_fake_hip()->fail_malloc_once = 1;
  lf_allocation *failed = lunaflux_hip_allocation_create(ctx, 64, &st);
  CHECK(failed != NULL && st == LF_DRIVER_FAILURE && state_of(failed) == kClosed);
  lunaflux_hip_release(failed);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 0, 4096, 256) == LF_OK);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 16, 16, 16) == LF_OK);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 4095, 1, 1) == LF_OK);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 4095, 2, 1) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 4096, 1, 1) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, -1, 1, 1) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 0, 0, 1) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 8, 16, 16) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 0, 16, 3) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 0, 16, 0) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 0, 16, 4096) == LF_OK);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 0, 16, 8192) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, b, 0, 16, 16) == LF_INVALID_ARGUMENT);
  CHECK(active_of(a) == 0 && active_of(ctx) == 0);  /* guards released */
  /* a lease keeps the allocation open */
  lf_allocation_lease *lease = lunaflux_hip_allocation_lease_create(ctx, a, &st);
  CHECK(st == LF_OK && active_of(a) == 1);
  CHECK(released(lunaflux_hip_allocation_lease_create(other, a, &st)) && st == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_allocation_close(a) == LF_BUSY && state_of(a) == kLive);
  CHECK(lunaflux_hip_context_close(ctx) == LF_BUSY);
  CHECK(lunaflux_hip_allocation_lease_close(lease) == LF_OK && active_of(a) == 0);
  lunaflux_hip_release(lease);
  int32_t frees = lf_fake_hip()->free_calls;
  CHECK(lunaflux_hip_allocation_close(a) == LF_OK && state_of(a) == kClosed);
  CHECK(lf_fake_hip()->free_calls == frees + 1);
  CHECK(lunaflux_hip_context_validate_allocation_region(ctx, a, 0, 16, 16) == LF_CLOSED);
  /* a failed free leaves the allocation LIVE and retryable */
  lf_fake_hip()->fail_free_once = 1;
  CHECK(lunaflux_hip_allocation_close(b) == LF_DRIVER_FAILURE && state_of(b) == kLive);
  CHECK(lunaflux_hip_allocation_close(b) == LF_OK);
  lunaflux_hip_release(a);
  lunaflux_hip_release(b);
  CHECK(lunaflux_hip_context_close(ctx) == LF_OK && lunaflux_hip_context_close(other) == LF_OK);
  lunaflux_hip_release(ctx);
  lunaflux_hip_release(other);
  return 0;
}

static int probe_transfers(void) {
  int32_t st = -99;
  lf_context *ctx = new_context();
  lf_context *other = new_context();
  lf_allocation *a = lunaflux_hip_allocation_create(ctx, 64, &st);
  uint8_t src[32], dst[32];
  for (int i = 0; i < 32; ++i) src[i] = (uint8_t)(i * 7 + 1);
  memset(dst, 0, sizeof(dst));
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, 4, 8, 20) == LF_OK);
  CHECK(lunaflux_hip_copy_to_host(a, 8, 20, dst, 20) == LF_OK);
  CHECK(memcmp(dst, src + 4, 20) == 0);
  CHECK(lunaflux_hip_context_copy_fixed_to_device(ctx, a, src, 32, 0, 32, 32) == LF_OK);
  memset(dst, 0, sizeof(dst));
  CHECK(lunaflux_hip_context_copy_device_to_fixed(ctx, a, dst, 32, 32, 0, 32) == LF_OK);
  CHECK(memcmp(dst, src, 32) == 0);
  /* empty copies are valid; negative spans overflow; spans outside either
   * buffer are invalid (internal/cuda/transfers.c:6-45) */
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, 0, 64, 0) == LF_OK);
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, -1, 0, 4) == LF_SIZE_OVERFLOW);
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, 0, -1, 4) == LF_SIZE_OVERFLOW);
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, 0, 0, -4) == LF_SIZE_OVERFLOW);
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, 30, 0, 4) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, 0, 62, 4) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_copy_to_device(a, NULL, 0, 0, 0, 0) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_copy_to_host(a, 60, 8, dst, 32) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_copy_to_host(a, 0, 33, dst, 32) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_copy_fixed_to_device(other, a, src, 32, 0, 0, 4) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_context_copy_device_to_fixed(NULL, a, dst, 32, 0, 0, 4) == LF_CLOSED);
  CHECK(active_of(a) == 0);
  CHECK(lunaflux_hip_allocation_close(a) == LF_OK);
  CHECK(lunaflux_hip_copy_to_device(a, src, 32, 0, 0, 4) == LF_CLOSED);
  CHECK(lunaflux_hip_copy_to_host(a, 0, 4, dst, 32) == LF_CLOSED);
  lunaflux_hip_release(a);
  CHECK(lunaflux_hip_context_close(ctx) == LF_OK && lunaflux_hip_context_close(other) == LF_OK);
  lunaflux_hip_release(ctx);
  lunaflux_hip_release(other);
  return 0;
}

typedef struct launch_scene {
  lf_function *fn;
  lf_module *module;
  lf_stream *stream;
  lf_allocation *first, *second;
  int checks_passed;
} launch_scene;

/* Inside the fake launch: every operand is held (the first allocation twice,
 * as two arguments name it) and no close gets through (launch_probe.c). */
static void interlocks(void *user) {
  launch_scene *s = (launch_scene *)user;
  s->checks_passed = active_of(s->fn) == 1 && active_of(s->module) == 1 &&
                     active_of(s->stream) == 1 && active_of(s->first) == 2 &&
                     active_of(s->second) == 1 &&
                     lunaflux_hip_function_close(s->fn) == LF_BUSY &&
                     lunaflux_hip_module_close(s->module) == LF_BUSY &&
                     lunaflux_hip_stream_close(s->stream) == LF_BUSY &&
                     lunaflux_hip_allocation_close(s->first) == LF_BUSY &&
                     lunaflux_hip_allocation_close(s->second) == LF_BUSY;
}

static int probe_launch(void) {
  lf_fake_hip_state *f = lf_fake_hip();
  int32_t st = -99;
  lf_context *ctx = new_context();
  lf_context *other = new_context();
  lf_module *m = lunaflux_hip_module_load(ctx, lf_fake_module_image, 16, &st);
  CHECK(st == LF_OK);
  uint8_t junk[16] = {0};
  lf_module *badm = lunaflux_hip_module_load(ctx, junk, 16, &st);
  CHECK(badm != NULL && st == LF_DRIVER_FAILURE);
  lunaflux_hip_release(badm);
  CHECK(released(lunaflux_hip_module_load(ctx, junk, 0, &st)) && st == LF_INVALID_ARGUMENT);
  /* symbol grammar: [A-Za-z_][A-Za-z0-9_]*, 1..128 bytes, no NUL */
  const char *bad_names[] = {"9kernel", "kernel-a", "kernel a", "", "k\xe9"};
  for (int i = 0; i < 5; ++i) {
    lf_function *g = lunaflux_hip_function_load(m, (const uint8_t *)bad_names[i],
                                                 (int64_t)strlen(bad_names[i]), &st);
    CHECK(g != NULL && st == LF_INVALID_ARGUMENT);
    lunaflux_hip_release(g);
  }
  uint8_t long_name[129];
  memset(long_name, 'a', sizeof(long_name));
  lunaflux_hip_release(lunaflux_hip_function_load(m, long_name, 129, &st));
  CHECK(st == LF_INVALID_ARGUMENT);
  lunaflux_hip_release(lunaflux_hip_function_load(m, (const uint8_t *)"kernel_a\0", 9, &st));
  CHECK(st == LF_INVALID_ARGUMENT);
  lunaflux_hip_release(lunaflux_hip_function_load(m, (const uint8_t *)"missing_kernel", 14, &st));
  CHECK(st == LF_DRIVER_FAILURE);
  lf_function *fn = lunaflux_hip_function_load(m, (const uint8_t *)"kernel_a", 8, &st);
  CHECK(st == LF_OK && children_of(m) == 1);
  lf_stream *s = lunaflux_hip_stream_create(ctx, &st);
  lf_stream *s_other = lunaflux_hip_stream_create(other, &st);
  lf_allocation *first = lunaflux_hip_allocation_create(ctx, 256, &st);
  lf_allocation *second = lunaflux_hip_allocation_create(ctx, 256, &st);
  lf_allocation *foreign = lunaflux_hip_allocation_create(other, 256, &st);
  uintptr_t base1 = 0, base2 = 0;
  {
    /* the allocations' device addresses, read back through a launch */
    lf_allocation *args[2] = {first, second};
    int64_t offs[2] = {0, 0}, bytes[2] = {1, 1}, al[2] = {1, 1};
    f->expected_params = 2;
    CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 2, args, offs, bytes, al) == LF_OK);
    base1 = f->params[0];
    base2 = f->params[1];
    CHECK(base1 % 256 == 0 && base2 % 256 == 0 && base1 != base2);
  }
  launch_scene scene = {fn, m, s, first, second, 0};
  lf_allocation *args[3] = {first, second, first};
  int64_t offsets[3] = {16, 32, 64}, bytes[3] = {16, 32, 64}, aligns[3] = {16, 32, 64};
  f->on_launch = interlocks;
  f->on_launch_user = &scene;
  f->expected_params = 3;
  int32_t launches = f->launches, syncs = f->stream_syncs;
  CHECK(lunaflux_hip_function_launch(fn, s, 3, 2, 1, 8, 4, 2, 64, 3, args, offsets, bytes,
                                     aligns) == LF_OK);
  CHECK(scene.checks_passed);
  CHECK(f->launches == launches + 1 && f->stream_syncs == syncs + 1);  /* synchronous */
  CHECK(f->grid[0] == 3 && f->grid[1] == 2 && f->grid[2] == 1);
  CHECK(f->block[0] == 8 && f->block[1] == 4 && f->block[2] == 2 && f->shared_memory_bytes == 64);
  CHECK(f->params[0] == base1 + 16 && f->params[1] == base2 + 32 && f->params[2] == base1 + 64);
  CHECK(active_of(fn) == 0 && active_of(m) == 0 && active_of(s) == 0 && active_of(first) == 0);
  f->on_launch = NULL;
  /* launch limits (internal/cuda/launch.c:12-38): nothing reaches the driver */
  launches = f->launches;
  const int32_t bad_dims[][7] = {{0, 1, 1, 1, 1, 1, 0},      {1, 65536, 1, 1, 1, 1, 0},
                                 {1, 1, 65536, 1, 1, 1, 0},  {1, 1, 1, 1025, 1, 1, 0},
                                 {1, 1, 1, 32, 32, 2, 0},    {1, 1, 1, 1, 1, 1, 98305},
                                 {1, 1, 1, 1, 1, 1, -1},     {1, 1, 1, 0, 1, 1, 0},
                                 {-1, 1, 1, 1, 1, 1, 0}};
  for (int i = 0; i < 9; ++i) {
    const int32_t *d = bad_dims[i];
    CHECK(lunaflux_hip_function_launch(fn, s, d[0], d[1], d[2], d[3], d[4], d[5], d[6], 3, args,
                                       offsets, bytes, aligns) == LF_INVALID_ARGUMENT);
  }
  CHECK(lunaflux_hip_function_launch(fn, s, 65536, 65535, 65535, 1024, 1, 1, 98304, 3, args,
                                     offsets, bytes, aligns) == LF_OK);
  launches = f->launches;
  /* argument count 1..32 */
  lf_allocation *many[33];
  int64_t zo[33], ob[33], oa[33];
  for (int i = 0; i < 33; ++i) {
    many[i] = first;
    zo[i] = 0;
    ob[i] = 1;
    oa[i] = 1;
  }
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 33, many, zo, ob, oa) ==
        LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 0, many, zo, ob, oa) ==
        LF_INVALID_ARGUMENT);
  CHECK(f->launches == launches);
  f->expected_params = 32;
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 32, many, zo, ob, oa) == LF_OK);
  CHECK(active_of(first) == 0);
  f->expected_params = 3;
  launches = f->launches;
  /* region rejections, guards released */
  int64_t off_range[3] = {16, 32, 250};
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, off_range, bytes,
                                     aligns) == LF_INVALID_ARGUMENT);
  int64_t misaligned[3] = {16, 33, 64};
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, misaligned, bytes,
                                     aligns) == LF_INVALID_ARGUMENT);
  int64_t zero_bytes[3] = {16, 0, 64};
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, offsets, zero_bytes,
                                     aligns) == LF_INVALID_ARGUMENT);
  int64_t odd_align[3] = {16, 32, 3};
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, offsets, bytes,
                                     odd_align) == LF_INVALID_ARGUMENT);
  int64_t huge_align[3] = {0, 0, 8192};
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, huge_align, bytes,
                                     huge_align) == LF_INVALID_ARGUMENT);
  lf_allocation *mixed[3] = {first, foreign, second};
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, mixed, offsets, bytes,
                                     aligns) == LF_INVALID_ARGUMENT);
  CHECK(lunaflux_hip_function_launch(fn, s_other, 1, 1, 1, 1, 1, 1, 0, 3, args, offsets, bytes,
                                     aligns) == LF_INVALID_ARGUMENT);
  CHECK(f->launches == launches);
  CHECK(active_of(first) == 0 && active_of(second) == 0 && active_of(foreign) == 0);
  CHECK(active_of(fn) == 0 && active_of(m) == 0 && active_of(s) == 0);
  /* injected failures: reported, every hold released */
  f->fail_launch_once = 1;
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, offsets, bytes,
                                     aligns) == LF_DRIVER_FAILURE);
  f->fail_stream_sync_once = 1;
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, offsets, bytes,
                                     aligns) == LF_DRIVER_FAILURE);
  CHECK(active_of(first) == 0 && active_of(fn) == 0 && active_of(s) == 0 && active_of(m) == 0);
  /* a closed operand: LF_CLOSED before the driver */
  launches = f->launches;
  CHECK(lunaflux_hip_allocation_close(second) == LF_OK);
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, offsets, bytes,
                                     aligns) == LF_CLOSED);
  CHECK(f->launches == launches && active_of(first) == 0);
  /* the module stays open while a function of it is */
  CHECK(lunaflux_hip_module_close(m) == LF_BUSY);
  CHECK(lunaflux_hip_function_close(fn) == LF_OK && children_of(m) == 0);
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 1, 1, 1, 0, 3, args, offsets, bytes,
                                     aligns) == LF_CLOSED);
  f->fail_module_unload_once = 1;
  CHECK(lunaflux_hip_module_close(m) == LF_DRIVER_FAILURE && state_of(m) == kLive);
  CHECK(lunaflux_hip_module_close(m) == LF_OK);
  lunaflux_hip_release(fn);
  lunaflux_hip_release(m);
  lunaflux_hip_release(first);
  lunaflux_hip_release(second);
  lunaflux_hip_release(foreign);
  lunaflux_hip_release(s);
  lunaflux_hip_release(s_other);
  CHECK(children_of(ctx) == 0 && children_of(other) == 0);
  CHECK(lunaflux_hip_context_close(ctx) == LF_OK && lunaflux_hip_context_close(other) == LF_OK);
  lunaflux_hip_release(ctx);
  lunaflux_hip_release(other);
  return 0;
}

static int probe_async_release(void) {
  lf_fake_hip_state *f = lf_fake_hip();
  int32_t st = -99;
  lf_context *ctx = new_context();
  lf_module *m = lunaflux_hip_module_load(ctx, lf_fake_module_image, 16, &st);
  lf_function *fn = lunaflux_hip_function_load(m, (const uint8_t *)"kernel_b", 8, &st);
  lf_stream *s = lunaflux_hip_stream_create(ctx, &st);
  lf_allocation *a = lunaflux_hip_allocation_create(ctx, 256, &st);
  lf_allocation *b = lunaflux_hip_allocation_create(ctx, 256, &st);
  lf_allocation *args[1] = {a};
  int64_t off[1] = {0}, bytes[1] = {256}, al[1] = {256};
  f->expected_params = 1;
  /* a synchronous launch leaves nothing queued: closing b needs no drain */
  CHECK(lunaflux_hip_function_launch(fn, s, 1, 1, 1, 64, 1, 1, 0, 1, args, off, bytes, al) == LF_OK);
  int32_t drains = f->device_syncs;
  int32_t syncs = f->stream_syncs;
  CHECK(lunaflux_hip_allocation_close(b) == LF_OK && f->device_syncs == drains);
  /* an asynchronous launch returns once enqueued, holding nothing ... */
  CHECK(lunaflux_hip_function_launch_async(fn, s, 1, 1, 1, 64, 1, 1, 0, 1, args, off, bytes,
                                           al) == LF_OK);
  CHECK(f->stream_syncs == syncs && active_of(a) == 0 && active_of(fn) == 0);
  /* ... so closing what it used first waits for the device, then frees */
  int32_t frees = f->free_calls;
  CHECK(lunaflux_hip_allocation_close(a) == LF_OK);
  CHECK(f->device_syncs == drains + 1 && f->free_calls_at_last_device_sync == frees);
  CHECK(f->free_calls == frees + 1);
  CHECK(lunaflux_hip_function_close(fn) == LF_OK);
  int32_t unloads = f->module_unloads;
  CHECK(lunaflux_hip_module_close(m) == LF_OK && f->device_syncs == drains + 2);
  CHECK(f->module_unloads == unloads + 1);
  lunaflux_hip_release(a);
  lunaflux_hip_release(b);
  lunaflux_hip_release(fn);
  lunaflux_hip_release(m);
  lunaflux_hip_release(s);
  CHECK(lunaflux_hip_context_close(ctx) == LF_OK);
  lunaflux_hip_release(ctx);
  return 0;
}

static int probe_vendor_gemm(void) {
  int32_t st = -99;
  lf_context *ctx = new_context();
  lf_blas *blas = lunaflux_hip_blas_create(ctx, &st);
  CHECK(blas != NULL && st == LF_UNSUPPORTED && state_of(blas) == kClosed);
  lf_gemm_plan *plan = lunaflux_hip_bf16_gemm_plan_create(blas, 1, 1, 1, 0, &st);
  CHECK(plan != NULL && st == LF_UNSUPPORTED);
  CHECK(lunaflux_hip_bf16_gemm_plan_run(plan, NULL, 0, NULL, 0, NULL, 0, NULL, 0, NULL) ==
        LF_UNSUPPORTED);
  CHECK(lunaflux_hip_bf16_gemm_plan_close(plan) == LF_OK && lunaflux_hip_blas_close(blas) == LF_OK);
  lunaflux_hip_release(plan);
  lunaflux_hip_release(blas);
  CHECK(lunaflux_hip_context_close(ctx) == LF_OK);
  lunaflux_hip_release(ctx);
  return 0;
}

int main(void) {
  lf_fake_hip_install();
  struct {
    const char *name;
    int (*run)(void);
  } probes[] = {{"availability", probe_availability}, {"lifecycle", probe_lifecycle},
                {"regions", probe_regions},           {"transfers", probe_transfers},
                {"launch", probe_launch},             {"async_release", probe_async_release},
                {"vendor_gemm", probe_vendor_gemm}};
  for (size_t i = 0; i < sizeof(probes) / sizeof(probes[0]); ++i) {
    if (probes[i].run() != 0) {
      fprintf(stderr, "probe %s failed\n", probes[i].name);
      return 1;
    }
    printf("ok %s\n", probes[i].name);
  }
  lf_fake_hip_state *f = lf_fake_hip();
  if (f->live_allocations != 0) {
    fprintf(stderr, "device memory leaked: %d allocations live\n", f->live_allocations);
    return 1;
  }
  printf("ok all\n");
  return 0;
}
