/*
 * moonbit.h - test stand-in for the MoonBit runtime header, so the MoonBit
 * stub layer (lunaflux_amd/csrc/moonbit/lunaflux_hip_moonbit.c) builds and
 * runs without the MoonBit toolchain. It provides the names that layer uses
 * with the semantics the MoonBit C backend gives them: objects carry a
 * header (reference count, length) in front of the payload the pointer
 * designates; Moonbit_array_length reads the length; external objects run
 * their finalizer when the count reaches zero. Test-only helpers (prefixed
 * moonbit_shim_) build the FixedArray and Ref values MoonBit would pass and
 * count live objects.
 */
#ifndef LUNAFLUX_TEST_MOONBIT_H
#define LUNAFLUX_TEST_MOONBIT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOONBIT_FFI_EXPORT
#define MOONBIT_EXPORT

typedef uint8_t *moonbit_bytes_t;

struct moonbit_shim_header {
  int32_t rc;
  int32_t length;
  void (*finalize)(void *self);
  uint64_t pad; /* keeps the payload 16-byte aligned */
};

#define Moonbit_array_length(obj) \
  (((struct moonbit_shim_header *)(void *)(obj)) - 1)->length

void *moonbit_make_external_object(void (*finalize)(void *self), uint32_t payload_size);
moonbit_bytes_t moonbit_make_bytes(int32_t size, int value);
void moonbit_incref(void *object);
void moonbit_decref(void *object);

/* test helpers */
int64_t *moonbit_shim_int64_array(int32_t length);
uint8_t *moonbit_shim_byte_array(int32_t length);
void **moonbit_shim_object_array(int32_t length);
int32_t moonbit_shim_live_objects(void);

#ifdef __cplusplus
}
#endif

#endif
