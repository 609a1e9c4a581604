// runtime.cpp - implementation of include/lunaflux_hip.h over the HIP
// runtime (libamdhip64). Host code only; the kernels live in a separate
// gfx950 code object loaded through lunaflux_hip_module_load. Every HIP call
// goes through the dispatch table lunaflux::hip() (runtime_internal.h).
//
// Lifecycle model (same observable behaviour as internal/cuda/resources.c):
// each handle carries state (LIVE/CLOSING/CLOSED), an active-operation count
// and a child count. An operation brackets itself with op_begin/op_end; close
// moves LIVE -> CLOSING only when nothing is active and no child is open,
// otherwise it reports LF_BUSY; a close whose driver call fails leaves the
// object LIVE, so the close can be retried (resources.c:17-57). Memory is
// reference counted: the creator holds one reference, every open child holds
// one on its parent, and the object is freed (after closing its device
// resource) when the count drops to zero.
//
// Asynchronous launches (lunaflux_hip_function_launch_async, an addition to
// the reference's synchronous ABI) release their hold on the function,
// module, stream and allocations once the kernel is enqueued. So that a close
// can never free what a queued kernel still reads, the module and every
// allocation of such a launch are marked, and closing a marked module or
// allocation first waits for its device to go idle.
#include "runtime_internal.h"

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

namespace lunaflux {

#ifdef LUNAFLUX_HIP_FAKE
namespace {
HipApi g_api{};
}
void install_hip_api(const HipApi &api) { g_api = api; }
const HipApi &hip() { return g_api; }
#else
const HipApi &hip() {
  static const HipApi api = {
      &hipDriverGetVersion,  &hipGetDeviceCount,       &hipGetDeviceProperties,
      &hipDeviceTotalMem,    &hipSetDevice,            &hipDeviceSynchronize,
      &hipMalloc,            &hipFree,                 &hipMemcpy,
      &hipStreamCreateWithFlags, &hipStreamDestroy,    &hipStreamSynchronize,
      &hipEventCreate,       &hipEventDestroy,         &hipEventRecord,
      &hipEventSynchronize,  &hipEventElapsedTime,     &hipModuleLoadData,
      &hipModuleUnload,      &hipModuleGetFunction,    &hipModuleLaunchKernel,
  };
  return api;
}
#endif

}  // namespace lunaflux

using lunaflux::hip;

namespace {

constexpr uint32_t kMagic = 0x4C464855u;  // "UHFL"

enum Kind : int32_t {
  kContext = 1,
  kStream,
  kEvent,
  kAllocation,
  kLease,
  kModule,
  kFunction,
  kBlas,
  kGemmPlan
};

enum State : int32_t { kLive = 0, kClosing = 1, kClosed = 2 };

struct Object {
  uint32_t magic = kMagic;
  int32_t kind = 0;
  std::atomic<int32_t> refs{1};
  std::atomic<int32_t> state{kClosed};
  std::atomic<int32_t> active{0};
  std::atomic<int32_t> children{0};
  // set when an asynchronous launch used this object (module, allocation)
  std::atomic<bool> queued{false};
  Object *parent = nullptr;
  virtual ~Object() { magic = 0; }
  // Releases the device resource; called with the object CLOSING.
  virtual int32_t destroy_device() { return LF_OK; }
};

int32_t map_hip(hipError_t e) { return e == hipSuccess ? LF_OK : LF_DRIVER_FAILURE; }

int32_t op_begin(Object *o) {
  if (o == nullptr) return LF_CLOSED;
  if (o->state.load() != kLive) return LF_CLOSED;
  o->active.fetch_add(1);
  if (o->state.load() != kLive) {
    o->active.fetch_sub(1);
    return LF_BUSY;
  }
  return LF_OK;
}

void op_end(Object *o) { o->active.fetch_sub(1); }

void unref(Object *o);

int32_t close_object(Object *o) {
  if (o == nullptr) return LF_INVALID_ARGUMENT;
  if (o->state.load() == kClosed) return LF_OK;
  if (o->children.load() != 0) return LF_BUSY;
  int32_t expected = kLive;
  if (!o->state.compare_exchange_strong(expected, kClosing)) {
    return expected == kClosed ? LF_OK : LF_BUSY;
  }
  if (o->active.load() != 0 || o->children.load() != 0) {
    o->state.store(kLive);
    return LF_BUSY;
  }
  int32_t result = o->destroy_device();
  if (result != LF_OK) {
    o->state.store(kLive);
    return result;
  }
  o->state.store(kClosed);
  Object *parent = o->parent;
  o->parent = nullptr;
  if (parent != nullptr) {
    parent->children.fetch_sub(1);
    unref(parent);
  }
  return LF_OK;
}

void unref(Object *o) {
  if (o == nullptr) return;
  if (o->refs.fetch_sub(1) == 1) {
    if (o->state.load() == kLive) {
      // The last reference is gone, so nothing can be using the object.
      close_object(o);
    }
    delete o;
  }
}

// Child `c` of `p` becomes LIVE: it holds a reference on p and counts as a
// child (the reference's moonbit_incref + children += 1).
void attach(Object *c, Object *p) {
  p->refs.fetch_add(1);
  p->children.fetch_add(1);
  c->parent = p;
  c->state.store(kLive);
}

template <typename T>
T *checked(void *handle, int32_t kind) {
  Object *o = static_cast<Object *>(handle);
  if (o == nullptr || o->magic != kMagic || o->kind != kind) return nullptr;
  return static_cast<T *>(o);
}

struct ApiState {
  int32_t availability = LF_DRIVER_INITIALIZATION_FAILED;
  int32_t driver_version = 0;
  int32_t device_count = 0;
};

const ApiState &api() {
  static ApiState state = [] {
    ApiState s;
    int version = 0;
    if (hip().DriverGetVersion == nullptr || hip().DriverGetVersion(&version) != hipSuccess) {
      s.availability = LF_DRIVER_INITIALIZATION_FAILED;
      return s;
    }
    s.driver_version = version;
    int count = 0;
    hipError_t e = hip().GetDeviceCount(&count);
    if (e == hipErrorNoDevice || (e == hipSuccess && count == 0)) {
      s.availability = LF_NO_DEVICES;
    } else if (e != hipSuccess) {
      s.availability = LF_INVENTORY_FAILED;
    } else {
      s.availability = LF_AVAILABLE;
      s.device_count = count;
    }
    return s;
  }();
  return state;
}

}  // namespace

struct lf_context : Object {
  int32_t ordinal = -1;
};

namespace {
int32_t set_device_of(Object *child) {
  lf_context *ctx = static_cast<lf_context *>(child->parent);
  return map_hip(hip().SetDevice(ctx->ordinal));
}

// A module or allocation that an asynchronous launch used may still be read
// by a queued kernel: wait for its device before releasing it.
int32_t drain_if_queued(Object *o) {
  if (!o->queued.load()) return LF_OK;
  int32_t r = map_hip(hip().DeviceSynchronize());
  if (r == LF_OK) o->queued.store(false);
  return r;
}
}  // namespace

struct lf_stream : Object {
  hipStream_t handle = nullptr;
  int32_t destroy_device() override {
    int32_t r = set_device_of(this);
    if (r == LF_OK && handle != nullptr) r = map_hip(hip().StreamDestroy(handle));
    if (r == LF_OK) handle = nullptr;
    return r;
  }
};

struct lf_event : Object {
  hipEvent_t handle = nullptr;
  bool recorded = false;
  int32_t destroy_device() override {
    int32_t r = set_device_of(this);
    if (r == LF_OK && handle != nullptr) r = map_hip(hip().EventDestroy(handle));
    if (r == LF_OK) handle = nullptr;
    return r;
  }
};

struct lf_allocation : Object {
  void *base = nullptr;
  size_t size = 0;
  int32_t destroy_device() override {
    int32_t r = set_device_of(this);
    if (r == LF_OK) r = drain_if_queued(this);
    if (r == LF_OK && base != nullptr) r = map_hip(hip().Free(base));
    if (r == LF_OK) {
      base = nullptr;
      size = 0;
    }
    return r;
  }
};

struct lf_allocation_lease : Object {
  lf_allocation *allocation = nullptr;
  // Ends the operation the lease holds open on its allocation and drops the
  // lease's reference to it.
  int32_t destroy_device() override {
    lf_allocation *a = allocation;
    allocation = nullptr;
    if (a != nullptr) {
      op_end(a);
      unref(a);
    }
    return LF_OK;
  }
};

struct lf_module : Object {
  hipModule_t handle = nullptr;
  std::vector<uint8_t> image;
  int32_t destroy_device() override {
    int32_t r = set_device_of(this);
    if (r == LF_OK) r = drain_if_queued(this);
    if (r == LF_OK && handle != nullptr) r = map_hip(hip().ModuleUnload(handle));
    if (r == LF_OK) {
      handle = nullptr;
      image.clear();
    }
    return r;
  }
};

struct lf_function : Object {
  hipFunction_t handle = nullptr;
};

struct lf_blas : Object {};
struct lf_gemm_plan : Object {};

namespace {

lf_context *context_of(Object *o) {
  while (o != nullptr && o->kind != kContext) o = o->parent;
  return static_cast<lf_context *>(o);
}

int32_t make_current(lf_context *ctx) {
  if (ctx == nullptr || ctx->state.load() != kLive) return LF_CLOSED;
  return map_hip(hip().SetDevice(ctx->ordinal));
}

// internal/cuda/regions.c:5-32
int32_t region_address(lf_allocation *a, int64_t offset, int64_t byte_count,
                       int64_t alignment, bool allow_empty, uintptr_t *out) {
  if (a == nullptr || a->state.load() != kLive) return LF_CLOSED;
  if (offset < 0 || byte_count < 0 || (byte_count == 0 && !allow_empty) ||
      alignment <= 0 || alignment > LF_MAX_REGION_ALIGNMENT ||
      (alignment & (alignment - 1)) != 0) {
    return LF_INVALID_ARGUMENT;
  }
  uint64_t start = static_cast<uint64_t>(offset);
  uint64_t count = static_cast<uint64_t>(byte_count);
  if (start > a->size || count > a->size - start) return LF_INVALID_ARGUMENT;
  uintptr_t base = reinterpret_cast<uintptr_t>(a->base);
  if (start > UINTPTR_MAX - base) return LF_SIZE_OVERFLOW;
  uintptr_t resolved = base + static_cast<uintptr_t>(start);
  if (resolved % static_cast<uint64_t>(alignment) != 0) {
    return LF_INVALID_ARGUMENT;
  }
  *out = resolved;
  return LF_OK;
}

// internal/cuda/launch.c:12-38
int32_t validate_dims(int32_t gx, int32_t gy, int32_t gz, int32_t bx,
                      int32_t by, int32_t bz, int32_t lds) {
  if (gx <= 0 || gy <= 0 || gz <= 0 || gy > LF_MAX_GRID_YZ ||
      gz > LF_MAX_GRID_YZ) {
    return LF_INVALID_ARGUMENT;
  }
  if (bx <= 0 || by <= 0 || bz <= 0 || bx > LF_MAX_BLOCK_DIMENSION ||
      by > LF_MAX_BLOCK_DIMENSION || bz > LF_MAX_BLOCK_DIMENSION) {
    return LF_INVALID_ARGUMENT;
  }
  uint64_t threads = static_cast<uint64_t>(bx) * by * bz;
  if (threads > LF_MAX_THREADS_PER_BLOCK || lds < 0 ||
      lds > LF_MAX_SHARED_MEMORY_BYTES) {
    return LF_INVALID_ARGUMENT;
  }
  return LF_OK;
}

template <typename T>
T *new_closed(int32_t kind) {
  T *o = new (std::nothrow) T();
  if (o != nullptr) o->kind = kind;
  return o;
}

}  // namespace

namespace lunaflux {

#ifdef LUNAFLUX_HIP_FAKE
bool inspect(const void *handle, int32_t out[4]) {
  const Object *o = static_cast<const Object *>(handle);
  if (o == nullptr || o->magic != kMagic) return false;
  out[0] = o->state.load();
  out[1] = o->active.load();
  out[2] = o->children.load();
  out[3] = o->refs.load();
  return true;
}
#endif

int32_t checked_launch(lf_function *fn, lf_stream *stream, int32_t gx, int32_t gy,
                       int32_t gz, int32_t bx, int32_t by, int32_t bz, int32_t lds,
                       int32_t argc, lf_allocation *const *allocs,
                       const int64_t *offsets, const int64_t *bytes,
                       const int64_t *aligns, bool synchronous,
                       const LaunchExtra *extra) {
  int32_t status = validate_dims(gx, gy, gz, bx, by, bz, lds);
  if (status != LF_OK) return status;
  // A trailing argument supplied by the library counts against the cap.
  const int32_t max_regions = LF_MAX_KERNEL_ARGUMENTS - (extra != nullptr ? 1 : 0);
  if (argc <= 0 || argc > max_regions || allocs == nullptr ||
      offsets == nullptr || bytes == nullptr || aligns == nullptr) {
    return LF_INVALID_ARGUMENT;
  }
  fn = checked<lf_function>(fn, kFunction);
  stream = checked<lf_stream>(stream, kStream);
  if (fn == nullptr || stream == nullptr) return LF_CLOSED;
  // Acquire function -> module -> stream -> each allocation, as
  // internal/cuda/launch.c:75-104 does; release in reverse.
  status = op_begin(fn);
  if (status != LF_OK) return status;
  lf_module *module = static_cast<lf_module *>(fn->parent);
  bool module_acquired = false;
  bool stream_acquired = false;
  int32_t acquired = 0;
  if (module == nullptr) status = LF_CLOSED;
  if (status == LF_OK) {
    status = op_begin(module);
    module_acquired = status == LF_OK;
  }
  if (status == LF_OK) {
    status = op_begin(stream);
    stream_acquired = status == LF_OK;
  }
  for (int32_t i = 0; status == LF_OK && i < argc; i += 1) {
    lf_allocation *a = checked<lf_allocation>(allocs[i], kAllocation);
    if (a == nullptr) {
      status = LF_CLOSED;
      break;
    }
    status = op_begin(a);
    if (status == LF_OK) acquired += 1;
  }
  uintptr_t values[LF_MAX_KERNEL_ARGUMENTS];
  void *params[LF_MAX_KERNEL_ARGUMENTS];
  lf_context *ctx = nullptr;
  if (status == LF_OK) {
    ctx = context_of(module);
    if (ctx == nullptr || context_of(stream) != ctx) status = LF_INVALID_ARGUMENT;
  }
  for (int32_t i = 0; status == LF_OK && i < argc; i += 1) {
    lf_allocation *a = allocs[i];
    if (context_of(a) != ctx) {
      status = LF_INVALID_ARGUMENT;
      break;
    }
    if (bytes[i] <= 0 || aligns[i] <= 0) {
      status = LF_INVALID_ARGUMENT;
      break;
    }
    status = region_address(a, offsets[i], bytes[i], aligns[i], false, &values[i]);
    params[i] = &values[i];
  }
  if (status == LF_OK) status = make_current(ctx);
  if (status == LF_OK && extra != nullptr) {
    // argc < LF_MAX_KERNEL_ARGUMENTS here (checked above), so the slot exists.
    status = extra->prepare(extra->context, ctx->ordinal, stream->handle, &values[argc]);
    params[argc] = &values[argc];
  }
  if (status == LF_OK) {
    status = map_hip(hip().ModuleLaunchKernel(
        fn->handle, static_cast<unsigned>(gx), static_cast<unsigned>(gy),
        static_cast<unsigned>(gz), static_cast<unsigned>(bx),
        static_cast<unsigned>(by), static_cast<unsigned>(bz),
        static_cast<unsigned>(lds), stream->handle, params, nullptr));
  }
  if (status == LF_OK && synchronous) {
    status = map_hip(hip().StreamSynchronize(stream->handle));
  }
  if (status == LF_OK && !synchronous) {
    module->queued.store(true);
    for (int32_t i = 0; i < argc; i += 1) allocs[i]->queued.store(true);
  }
  for (int32_t i = acquired; i > 0; i -= 1) op_end(allocs[i - 1]);
  if (stream_acquired) op_end(stream);
  if (module_acquired) op_end(module);
  op_end(fn);
  return status;
}

}  // namespace lunaflux

namespace {

bool valid_symbol(const uint8_t *name, int64_t length) {
  if (name == nullptr || length <= 0 || length > LF_MAX_SYMBOL_BYTES) return false;
  for (int64_t i = 0; i < length; i += 1) {
    uint8_t c = name[i];
    bool alpha = (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || c == '_';
    bool digit = c >= '0' && c <= '9';
    if (!(alpha || (i > 0 && digit))) return false;
  }
  return true;
}

// Host <-> device copy of byte_count bytes between host[host_offset..] (a
// buffer of host_length bytes) and the allocation at device_offset, checked
// as internal/cuda/transfers.c:6-45 checks: negative offsets or counts are
// LF_SIZE_OVERFLOW, spans outside either buffer LF_INVALID_ARGUMENT, and an
// empty copy is valid.
int32_t copy_host_device(lf_context *context, lf_allocation *allocation,
                         const uint8_t *source, uint8_t *destination,
                         int64_t host_length, int64_t host_offset,
                         int64_t device_offset, int64_t byte_count) {
  allocation = checked<lf_allocation>(allocation, kAllocation);
  if (allocation == nullptr) return LF_CLOSED;
  if (context != nullptr) {
    context = checked<lf_context>(context, kContext);
    if (context == nullptr) return LF_CLOSED;
  }
  int32_t st = op_begin(allocation);
  if (st != LF_OK) return st;
  uintptr_t address = 0;
  if (source == nullptr && destination == nullptr) {
    st = LF_INVALID_ARGUMENT;
  } else if (host_offset < 0 || device_offset < 0 || byte_count < 0 || host_length < 0) {
    st = LF_SIZE_OVERFLOW;
  } else if (host_offset > host_length || byte_count > host_length - host_offset) {
    st = LF_INVALID_ARGUMENT;
  } else if (context != nullptr && context_of(allocation) != context) {
    st = LF_INVALID_ARGUMENT;
  } else {
    st = region_address(allocation, device_offset, byte_count, 1, true, &address);
  }
  if (st == LF_OK) st = make_current(context_of(allocation));
  if (st == LF_OK && byte_count > 0) {
    void *device = reinterpret_cast<void *>(address);
    if (source != nullptr) {
      st = map_hip(hip().Memcpy(device, source + host_offset,
                                static_cast<size_t>(byte_count), hipMemcpyHostToDevice));
    } else {
      st = map_hip(hip().Memcpy(destination + host_offset, device,
                                static_cast<size_t>(byte_count), hipMemcpyDeviceToHost));
    }
  }
  op_end(allocation);
  return st;
}

}  // namespace

extern "C" {

int32_t lunaflux_hip_probe(int64_t output[3]) {
  const ApiState &s = api();
  if (output != nullptr) {
    output[0] = s.driver_version;
    output[1] = s.device_count;
    output[2] = 0;
  }
  return s.availability;
}

int32_t lunaflux_hip_device_info(int32_t ordinal, int64_t numeric[5],
                                 uint8_t name[LF_DEVICE_NAME_BYTES]) {
  const ApiState &s = api();
  if (s.availability != LF_AVAILABLE) return LF_UNAVAILABLE;
  if (numeric == nullptr || name == nullptr) return LF_INVALID_ARGUMENT;
  if (ordinal < 0 || ordinal >= s.device_count) return LF_INVALID_ARGUMENT;
  hipDeviceProp_t prop;
  std::memset(&prop, 0, sizeof(prop));
  size_t total = 0;
  if (hip().GetDeviceProperties(&prop, ordinal) != hipSuccess ||
      hip().DeviceTotalMem(&total, ordinal) != hipSuccess) {
    return LF_DRIVER_FAILURE;
  }
  numeric[0] = static_cast<int64_t>(total);
  numeric[1] = prop.major;
  numeric[2] = prop.minor;
  // bf16 MFMA exists on every CDNA generation from gfx90a on.
  numeric[3] = prop.major >= 9 ? 1 : 0;
  numeric[4] = 0;
  std::memset(name, 0, LF_DEVICE_NAME_BYTES);
  // Some drivers report an empty marketing name; the architecture name
  // (e.g. "gfx950:sramecc+:xnack-") is always set.
  const char *label = prop.name[0] != '\0' ? prop.name : prop.gcnArchName;
  std::strncpy(reinterpret_cast<char *>(name), label, LF_DEVICE_NAME_BYTES - 1);
  return LF_OK;
}

void lunaflux_hip_release(void *handle) {
  Object *o = static_cast<Object *>(handle);
  if (o == nullptr || o->magic != kMagic) return;
  unref(o);
}

lf_context *lunaflux_hip_context_create(int32_t ordinal, int32_t *status) {
  lf_context *ctx = new_closed<lf_context>(kContext);
  int32_t st = LF_OK;
  if (ctx == nullptr) {
    st = LF_HOST_ALLOCATION_FAILED;
  } else if (api().availability != LF_AVAILABLE) {
    st = LF_UNAVAILABLE;
  } else if (ordinal < 0 || ordinal >= api().device_count) {
    st = LF_INVALID_ARGUMENT;
  } else if (hip().SetDevice(ordinal) != hipSuccess || hip().Free(nullptr) != hipSuccess) {
    st = LF_DRIVER_FAILURE;
  } else {
    ctx->ordinal = ordinal;
    ctx->state.store(kLive);
  }
  if (status != nullptr) *status = st;
  return ctx;
}

int32_t lunaflux_hip_context_close(lf_context *context) {
  context = checked<lf_context>(context, kContext);
  if (context == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(context);
}

lf_stream *lunaflux_hip_stream_create(lf_context *context, int32_t *status) {
  lf_stream *s = new_closed<lf_stream>(kStream);
  context = checked<lf_context>(context, kContext);
  int32_t st = s == nullptr ? LF_HOST_ALLOCATION_FAILED : op_begin(context);
  if (s != nullptr && st == LF_OK) {
    st = make_current(context);
    if (st == LF_OK) {
      st = map_hip(hip().StreamCreateWithFlags(&s->handle, hipStreamNonBlocking));
    }
    if (st == LF_OK) attach(s, context);
    op_end(context);
  }
  if (status != nullptr) *status = st;
  return s;
}

int32_t lunaflux_hip_stream_close(lf_stream *stream) {
  stream = checked<lf_stream>(stream, kStream);
  if (stream == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(stream);
}

int32_t lunaflux_hip_stream_synchronize(lf_stream *stream) {
  stream = checked<lf_stream>(stream, kStream);
  if (stream == nullptr) return LF_CLOSED;
  int32_t st = op_begin(stream);
  if (st != LF_OK) return st;
  st = make_current(context_of(stream));
  if (st == LF_OK) st = map_hip(hip().StreamSynchronize(stream->handle));
  op_end(stream);
  return st;
}

lf_event *lunaflux_hip_event_create(lf_context *context, int32_t *status) {
  lf_event *e = new_closed<lf_event>(kEvent);
  context = checked<lf_context>(context, kContext);
  int32_t st = e == nullptr ? LF_HOST_ALLOCATION_FAILED : op_begin(context);
  if (e != nullptr && st == LF_OK) {
    st = make_current(context);
    if (st == LF_OK) st = map_hip(hip().EventCreate(&e->handle));
    if (st == LF_OK) attach(e, context);
    op_end(context);
  }
  if (status != nullptr) *status = st;
  return e;
}

int32_t lunaflux_hip_event_close(lf_event *event) {
  event = checked<lf_event>(event, kEvent);
  if (event == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(event);
}

int32_t lunaflux_hip_event_record(lf_event *event, lf_stream *stream) {
  event = checked<lf_event>(event, kEvent);
  stream = checked<lf_stream>(stream, kStream);
  if (event == nullptr || stream == nullptr) return LF_CLOSED;
  int32_t st = op_begin(event);
  if (st != LF_OK) return st;
  st = op_begin(stream);
  if (st == LF_OK) {
    if (context_of(event) != context_of(stream)) {
      st = LF_INVALID_ARGUMENT;
    } else {
      st = make_current(context_of(stream));
      if (st == LF_OK) st = map_hip(hip().EventRecord(event->handle, stream->handle));
      if (st == LF_OK) event->recorded = true;
    }
    op_end(stream);
  }
  op_end(event);
  return st;
}

int32_t lunaflux_hip_event_synchronize(lf_event *event) {
  event = checked<lf_event>(event, kEvent);
  if (event == nullptr) return LF_CLOSED;
  int32_t st = op_begin(event);
  if (st != LF_OK) return st;
  st = make_current(context_of(event));
  if (st == LF_OK) st = map_hip(hip().EventSynchronize(event->handle));
  op_end(event);
  return st;
}

double lunaflux_hip_event_elapsed(lf_event *start, lf_event *finish,
                                  int32_t *status) {
  start = checked<lf_event>(start, kEvent);
  finish = checked<lf_event>(finish, kEvent);
  int32_t st = (start == nullptr || finish == nullptr) ? LF_CLOSED : op_begin(start);
  float ms = 0.0f;
  if (st == LF_OK) {
    st = op_begin(finish);
    if (st == LF_OK) {
      if (!start->recorded || !finish->recorded ||
          context_of(start) != context_of(finish)) {
        st = LF_INVALID_ARGUMENT;
      } else {
        st = make_current(context_of(start));
        if (st == LF_OK) {
          st = map_hip(hip().EventElapsedTime(&ms, start->handle, finish->handle));
        }
      }
      op_end(finish);
    }
    op_end(start);
  }
  if (status != nullptr) *status = st;
  return st == LF_OK ? static_cast<double>(ms) : 0.0;
}

lf_allocation *lunaflux_hip_allocation_create(lf_context *context,
                                              int64_t byte_count,
                                              int32_t *status) {
  lf_allocation *a = new_closed<lf_allocation>(kAllocation);
  context = checked<lf_context>(context, kContext);
  int32_t st = LF_OK;
  if (a == nullptr) {
    st = LF_HOST_ALLOCATION_FAILED;
  } else if (byte_count <= 0) {
    st = LF_INVALID_ARGUMENT;
  } else if (static_cast<uint64_t>(byte_count) > SIZE_MAX) {
    st = LF_SIZE_OVERFLOW;
  } else {
    st = op_begin(context);
    if (st == LF_OK) {
      st = make_current(context);
      if (st == LF_OK) st = map_hip(hip().Malloc(&a->base, static_cast<size_t>(byte_count)));
      if (st == LF_OK) {
        a->size = static_cast<size_t>(byte_count);
        attach(a, context);
      } else {
        a->base = nullptr;
      }
      op_end(context);
    }
  }
  if (status != nullptr) *status = st;
  return a;
}

int32_t lunaflux_hip_allocation_close(lf_allocation *allocation) {
  allocation = checked<lf_allocation>(allocation, kAllocation);
  if (allocation == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(allocation);
}

lf_allocation_lease *lunaflux_hip_allocation_lease_create(
    lf_context *context, lf_allocation *allocation, int32_t *status) {
  lf_allocation_lease *lease = new_closed<lf_allocation_lease>(kLease);
  context = checked<lf_context>(context, kContext);
  allocation = checked<lf_allocation>(allocation, kAllocation);
  int32_t st = lease == nullptr ? LF_HOST_ALLOCATION_FAILED : op_begin(context);
  if (lease != nullptr && st == LF_OK) {
    st = allocation == nullptr ? LF_CLOSED : op_begin(allocation);
    if (st == LF_OK) {
      if (context_of(allocation) != context) {
        op_end(allocation);
        st = LF_INVALID_ARGUMENT;
      } else {
        // The lease keeps one operation open on the allocation and one
        // reference on it until the lease closes.
        allocation->refs.fetch_add(1);
        lease->allocation = allocation;
        lease->state.store(kLive);
      }
    }
    op_end(context);
  }
  if (status != nullptr) *status = st;
  return lease;
}

int32_t lunaflux_hip_allocation_lease_close(lf_allocation_lease *lease) {
  lease = checked<lf_allocation_lease>(lease, kLease);
  if (lease == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(lease);
}

int32_t lunaflux_hip_context_validate_allocation_region(
    lf_context *context, lf_allocation *allocation, int64_t offset,
    int64_t byte_count, int64_t alignment) {
  context = checked<lf_context>(context, kContext);
  allocation = checked<lf_allocation>(allocation, kAllocation);
  if (context == nullptr || allocation == nullptr) return LF_CLOSED;
  int32_t st = op_begin(context);
  if (st != LF_OK) return st;
  st = op_begin(allocation);
  if (st == LF_OK) {
    uintptr_t address = 0;
    if (context_of(allocation) != context) {
      st = LF_INVALID_ARGUMENT;
    } else if (byte_count <= 0 || alignment <= 0) {
      st = LF_INVALID_ARGUMENT;
    } else {
      st = region_address(allocation, offset, byte_count, alignment, false, &address);
    }
    op_end(allocation);
  }
  op_end(context);
  return st;
}

int32_t lunaflux_hip_copy_to_device(lf_allocation *allocation,
                                    const uint8_t *source,
                                    int64_t source_length,
                                    int64_t source_offset,
                                    int64_t destination_offset,
                                    int64_t byte_count) {
  if (source == nullptr) {
    return checked<lf_allocation>(allocation, kAllocation) == nullptr ? LF_CLOSED
                                                                      : LF_INVALID_ARGUMENT;
  }
  return copy_host_device(nullptr, allocation, source, nullptr, source_length,
                          source_offset, destination_offset, byte_count);
}

int32_t lunaflux_hip_context_copy_fixed_to_device(
    lf_context *context, lf_allocation *allocation, const uint8_t *source,
    int64_t source_length, int64_t source_offset, int64_t destination_offset,
    int64_t byte_count) {
  if (context == nullptr) return LF_CLOSED;
  if (source == nullptr) return LF_INVALID_ARGUMENT;
  return copy_host_device(context, allocation, source, nullptr, source_length,
                          source_offset, destination_offset, byte_count);
}

int32_t lunaflux_hip_context_copy_device_to_fixed(
    lf_context *context, lf_allocation *allocation, uint8_t *destination,
    int64_t destination_length, int64_t source_offset,
    int64_t destination_offset, int64_t byte_count) {
  if (context == nullptr) return LF_CLOSED;
  if (destination == nullptr) return LF_INVALID_ARGUMENT;
  return copy_host_device(context, allocation, nullptr, destination,
                          destination_length, destination_offset, source_offset,
                          byte_count);
}

int32_t lunaflux_hip_copy_to_host(lf_allocation *allocation,
                                  int64_t source_offset, int64_t byte_count,
                                  uint8_t *destination,
                                  int64_t destination_length) {
  if (destination == nullptr) {
    return checked<lf_allocation>(allocation, kAllocation) == nullptr ? LF_CLOSED
                                                                      : LF_INVALID_ARGUMENT;
  }
  return copy_host_device(nullptr, allocation, nullptr, destination,
                          destination_length, 0, source_offset, byte_count);
}

lf_module *lunaflux_hip_module_load(lf_context *context, const uint8_t *image,
                                    int64_t image_length, int32_t *status) {
  lf_module *m = new_closed<lf_module>(kModule);
  context = checked<lf_context>(context, kContext);
  int32_t st = LF_OK;
  if (m == nullptr) {
    st = LF_HOST_ALLOCATION_FAILED;
  } else if (image == nullptr || image_length <= 0) {
    st = LF_INVALID_ARGUMENT;
  } else {
    st = op_begin(context);
    if (st == LF_OK) {
      try {
        m->image.assign(image, image + image_length);
      } catch (...) {
        st = LF_HOST_ALLOCATION_FAILED;
      }
      if (st == LF_OK) st = make_current(context);
      if (st == LF_OK) st = map_hip(hip().ModuleLoadData(&m->handle, m->image.data()));
      if (st == LF_OK) {
        attach(m, context);
      } else {
        m->handle = nullptr;
        m->image.clear();
      }
      op_end(context);
    }
  }
  if (status != nullptr) *status = st;
  return m;
}

int32_t lunaflux_hip_module_close(lf_module *module) {
  module = checked<lf_module>(module, kModule);
  if (module == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(module);
}

lf_function *lunaflux_hip_function_load(lf_module *module, const uint8_t *name,
                                        int64_t name_length, int32_t *status) {
  lf_function *f = new_closed<lf_function>(kFunction);
  module = checked<lf_module>(module, kModule);
  int32_t st = LF_OK;
  if (f == nullptr) {
    st = LF_HOST_ALLOCATION_FAILED;
  } else if (module == nullptr || module->state.load() != kLive) {
    st = LF_CLOSED;
  } else if (!valid_symbol(name, name_length)) {
    st = LF_INVALID_ARGUMENT;
  } else {
    st = op_begin(module);
    if (st == LF_OK) {
      char symbol[LF_MAX_SYMBOL_BYTES + 1];
      std::memcpy(symbol, name, static_cast<size_t>(name_length));
      symbol[name_length] = '\0';
      st = make_current(context_of(module));
      if (st == LF_OK) {
        st = map_hip(hip().ModuleGetFunction(&f->handle, module->handle, symbol));
      }
      if (st == LF_OK) {
        attach(f, module);
      } else {
        f->handle = nullptr;
      }
      op_end(module);
    }
  }
  if (status != nullptr) *status = st;
  return f;
}

int32_t lunaflux_hip_function_close(lf_function *function) {
  function = checked<lf_function>(function, kFunction);
  if (function == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(function);
}

int32_t lunaflux_hip_function_launch(
    lf_function *function, lf_stream *stream, int32_t grid_x, int32_t grid_y,
    int32_t grid_z, int32_t block_x, int32_t block_y, int32_t block_z,
    int32_t shared_memory_bytes, int32_t argument_count,
    lf_allocation *const *allocations, const int64_t *offsets,
    const int64_t *byte_counts, const int64_t *alignments) {
  return lunaflux::checked_launch(function, stream, grid_x, grid_y, grid_z, block_x, block_y,
                                  block_z, shared_memory_bytes, argument_count, allocations,
                                  offsets, byte_counts, alignments, true, nullptr);
}

int32_t lunaflux_hip_function_launch_async(
    lf_function *function, lf_stream *stream, int32_t grid_x, int32_t grid_y,
    int32_t grid_z, int32_t block_x, int32_t block_y, int32_t block_z,
    int32_t shared_memory_bytes, int32_t argument_count,
    lf_allocation *const *allocations, const int64_t *offsets,
    const int64_t *byte_counts, const int64_t *alignments) {
  return lunaflux::checked_launch(function, stream, grid_x, grid_y, grid_z, block_x, block_y,
                                  block_z, shared_memory_bytes, argument_count, allocations,
                                  offsets, byte_counts, alignments, false, nullptr);
}

lf_blas *lunaflux_hip_blas_create(lf_context *context, int32_t *status) {
  (void)context;
  lf_blas *b = new_closed<lf_blas>(kBlas);
  if (status != nullptr) *status = b == nullptr ? LF_HOST_ALLOCATION_FAILED : LF_UNSUPPORTED;
  return b;
}

int32_t lunaflux_hip_blas_close(lf_blas *blas) {
  blas = checked<lf_blas>(blas, kBlas);
  if (blas == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(blas);
}

lf_gemm_plan *lunaflux_hip_bf16_gemm_plan_create(lf_blas *blas, int64_t rows,
                                                 int64_t inner, int64_t columns,
                                                 int64_t workspace_byte_count,
                                                 int32_t *status) {
  (void)blas;
  (void)rows;
  (void)inner;
  (void)columns;
  (void)workspace_byte_count;
  lf_gemm_plan *p = new_closed<lf_gemm_plan>(kGemmPlan);
  if (status != nullptr) *status = p == nullptr ? LF_HOST_ALLOCATION_FAILED : LF_UNSUPPORTED;
  return p;
}

int32_t lunaflux_hip_bf16_gemm_plan_close(lf_gemm_plan *plan) {
  plan = checked<lf_gemm_plan>(plan, kGemmPlan);
  if (plan == nullptr) return LF_INVALID_ARGUMENT;
  return close_object(plan);
}

int32_t lunaflux_hip_bf16_gemm_plan_run(
    lf_gemm_plan *plan, lf_allocation *left, int64_t left_offset,
    lf_allocation *right, int64_t right_offset, lf_allocation *output,
    int64_t output_offset, lf_allocation *workspace, int64_t workspace_offset,
    lf_stream *stream) {
  (void)plan;
  (void)left;
  (void)left_offset;
  (void)right;
  (void)right_offset;
  (void)output;
  (void)output_offset;
  (void)workspace;
  (void)workspace_offset;
  (void)stream;
  return LF_UNSUPPORTED;
}

}  // extern "C"
