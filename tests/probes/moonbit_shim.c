/* moonbit_shim.c - the test stand-in runtime behind tests/probes/moonbit.h. */
#include "moonbit.h"

#include <stdlib.h>
#include <string.h>

static int32_t live_objects;

static void *shim_alloc(int64_t payload, int32_t length, void (*finalize)(void *)) {
  struct moonbit_shim_header *h =
    (struct moonbit_shim_header *)calloc(1, sizeof(*h) + (size_t)(payload > 0 ? payload : 1));
  if (h == NULL) abort();
  h->rc = 1;
  h->length = length;
  h->finalize = finalize;
  live_objects += 1;
  return h + 1;
}

void *moonbit_make_external_object(void (*finalize)(void *self), uint32_t payload_size) {
  return shim_alloc(payload_size, 0, finalize);
}

moonbit_bytes_t moonbit_make_bytes(int32_t size, int value) {
  uint8_t *p = (uint8_t *)shim_alloc(size, size, NULL);
  memset(p, value, (size_t)(size > 0 ? size : 0));
  return p;
}

void moonbit_incref(void *object) { (((struct moonbit_shim_header *)object) - 1)->rc += 1; }

void moonbit_decref(void *object) {
  struct moonbit_shim_header *h = ((struct moonbit_shim_header *)object) - 1;
  h->rc -= 1;
  if (h->rc == 0) {
    if (h->finalize != NULL) h->finalize(object);
    live_objects -= 1;
    free(h);
  }
}

int64_t *moonbit_shim_int64_array(int32_t length) {
  return (int64_t *)shim_alloc((int64_t)length * 8, length, NULL);
}

uint8_t *moonbit_shim_byte_array(int32_t length) {
  return (uint8_t *)shim_alloc(length, length, NULL);
}

void **moonbit_shim_object_array(int32_t length) {
  return (void **)shim_alloc((int64_t)length * (int64_t)sizeof(void *), length, NULL);
}

int32_t moonbit_shim_live_objects(void) { return live_objects; }
