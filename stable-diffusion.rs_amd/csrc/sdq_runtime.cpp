// sdq_runtime.cpp -- handles, errors, streams, evaluation and the caching
// device allocator behind libsdq's C ABI (include/sdq.h).
//
// Mirrors the object model the reference binds through mlx-c
// (crates/sd-tensor/src/mlx.rs:106-121, 338-342, 358-359, 398-416) so that
// the Rust seam can swap one library for the other.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <sstream>
#include <thread>

#include "kernels/launch.hpp"
#include "sdq_internal.hpp"

namespace sdq {

// ---- errors ---------------------------------------------------------------

namespace {

void default_handler(const char *msg, void *) {
  std::fprintf(stderr, "libsdq: %s\n", msg);
}

struct HandlerSlot {
  std::mutex mu;
  sdq_error_handler_func fn = default_handler;
  void *data = nullptr;
  void (*dtor)(void *) = nullptr;
};

HandlerSlot &handler_slot() {
  static HandlerSlot *slot = new HandlerSlot(); // never destroyed: usable at exit
  return *slot;
}

} // namespace

void report(const char *op, const char *msg) {
  std::string text = std::string("[") + op + "] " + msg;
  HandlerSlot &h = handler_slot();
  sdq_error_handler_func fn;
  void *data;
  {
    std::lock_guard<std::mutex> lock(h.mu);
    fn = h.fn;
    data = h.data;
  }
  // Called synchronously, on the calling thread, before the status returns:
  // the reference's thread-local trampoline depends on it (mlx.rs:419-470).
  fn(text.c_str(), data);
}

void fail(const std::string &msg) { throw Error(msg); }

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    (void)hipGetLastError(); // clear the sticky slot for the next call
    fail(std::string(what) + ": " + hipGetErrorString(e));
  }
}

// ---- dtypes -----------------------------------------------------------------

size_t dtype_size(int d) {
  switch (d) {
  case SDQ_BOOL:
  case SDQ_UINT8:
  case SDQ_INT8:
    return 1;
  case SDQ_UINT16:
  case SDQ_INT16:
  case SDQ_FLOAT16:
  case SDQ_BFLOAT16:
    return 2;
  case SDQ_UINT32:
  case SDQ_INT32:
  case SDQ_FLOAT32:
    return 4;
  case SDQ_UINT64:
  case SDQ_INT64:
  case SDQ_FLOAT64:
  case SDQ_COMPLEX64:
    return 8;
  default:
    return 0;
  }
}

const char *dtype_name(int d) {
  static const char *names[] = {"bool",    "uint8",   "uint16",  "uint32",
                                "uint64",  "int8",    "int16",   "int32",
                                "int64",   "float16", "float32", "float64",
                                "bfloat16", "complex64"};
  if (d < 0 || d > SDQ_COMPLEX64) return "unknown";
  return names[d];
}

bool is_float_dtype(int d) {
  return d == SDQ_FLOAT32 || d == SDQ_BFLOAT16 || d == SDQ_FLOAT16;
}

int promote_float(int a, int b) {
  if (a == b) return a;
  // float32 wins; float16 with bfloat16 promotes to float32, as in MLX.
  return SDQ_FLOAT32;
}

// ---- caching allocator --------------------------------------------------------

namespace {

// Makes `device` current for the scope (the allocator is called from any
// thread, with any device current).
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev) != hipSuccess) {
      (void)hipGetLastError();
      prev = -1;
    }
    if (prev != device) (void)hipSetDevice(device);
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

// An event recorded on `stream` when a block was freed: a later user of the
// block on another stream waits for it.
struct Pending {
  hipEvent_t event;
  hipStream_t stream;
};

struct FreeBlock {
  void *ptr;
  size_t capacity;
  std::vector<Pending> pending;
};

struct DevicePool {
  std::multimap<size_t, FreeBlock> free_blocks; // by capacity
  std::vector<hipEvent_t> events;               // recycled, timing disabled
};

struct Pool {
  std::mutex mu;
  std::map<int, DevicePool> devices;
  size_t active = 0;
  size_t peak = 0;
  size_t cached = 0;
  size_t limit = size_t(64) << 30; // cached bytes kept at most
};

Pool &pool() {
  static Pool *p = new Pool(); // never destroyed: buffers may outlive statics
  return *p;
}

hipEvent_t take_event(int device) {
  {
    Pool &p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    auto &ev = p.devices[device].events;
    if (!ev.empty()) {
      hipEvent_t e = ev.back();
      ev.pop_back();
      return e;
    }
  }
  hipEvent_t e = nullptr;
  hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
  return e;
}

void give_events_locked(Pool &p, int device, const std::vector<Pending> &pend) {
  auto &ev = p.devices[device].events;
  for (const Pending &q : pend) ev.push_back(q.event);
}

// Four size classes per octave, 256 B minimum: at most 25% slack, and a
// steady-state call sequence maps onto the same few classes.
size_t round_size(size_t bytes) {
  if (bytes <= 256) return 256;
  size_t p = size_t(1) << (63 - __builtin_clzll(bytes - 1)); // largest pow2 < bytes
  size_t step = std::max<size_t>(p / 4, 256);
  return (bytes + step - 1) / step * step;
}

void trim_locked(Pool &p, size_t target) {
  for (auto &dev : p.devices) {
    auto &fb = dev.second.free_blocks;
    if (p.cached <= target || fb.empty()) continue;
    DeviceGuard guard(dev.first);
    while (p.cached > target && !fb.empty()) {
      auto it = std::prev(fb.end()); // largest first
      // The block's last users must be done before its memory goes back.
      for (const Pending &q : it->second.pending) (void)hipEventSynchronize(q.event);
      give_events_locked(p, dev.first, it->second.pending);
      (void)hipFree(it->second.ptr);
      p.cached -= it->second.capacity;
      fb.erase(it);
    }
  }
}

} // namespace

void Buffer::note_reader(hipStream_t s) {
  if (s == stream) return;
  for (hipStream_t r : readers)
    if (r == s) return;
  readers.push_back(s);
}

Buffer::~Buffer() {
  if (!ptr) return;
  // One event per stream that may still be using the block, recorded now;
  // retired library streams were synchronised when they were destroyed.
  std::vector<Pending> pend;
  {
    DeviceGuard guard(device);
    auto record = [&](hipStream_t s) {
      if (stream_retired(s)) return;
      hipEvent_t e = nullptr;
      try {
        e = take_event(device);
      } catch (const std::exception &) {
        (void)hipStreamSynchronize(s); // no event: wait here instead
        (void)hipGetLastError();
        return;
      }
      if (hipEventRecord(e, s) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipStreamSynchronize(s);
        (void)hipGetLastError();
        (void)hipEventDestroy(e);
        return;
      }
      pend.push_back(Pending{e, s});
    };
    record(stream);
    for (hipStream_t r : readers) record(r);
  }
  Pool &p = pool();
  std::lock_guard<std::mutex> lock(p.mu);
  p.active -= capacity;
  p.devices[device].free_blocks.emplace(capacity, FreeBlock{ptr, capacity, std::move(pend)});
  p.cached += capacity;
  if (p.cached > p.limit) trim_locked(p, p.limit);
}

std::shared_ptr<Buffer> allocate(size_t bytes, int device, hipStream_t stream) {
  auto buf = std::make_shared<Buffer>();
  buf->device = device;
  buf->stream = stream;
  if (bytes == 0) return buf;
  const size_t want = round_size(bytes);
  Pool &p = pool();
  {
    std::unique_lock<std::mutex> lock(p.mu);
    auto &fb = p.devices[device].free_blocks;
    auto it = fb.lower_bound(want);
    if (it != fb.end() && it->first <= want + want / 4) {
      FreeBlock blk = std::move(it->second);
      fb.erase(it);
      p.cached -= blk.capacity;
      p.active += blk.capacity;
      p.peak = std::max(p.peak, p.active);
      lock.unlock();
      // Work already enqueued on `stream` precedes this use by stream order;
      // the block's users on other streams are waited for on the device.
      hipError_t err = hipSuccess;
      for (const Pending &q : blk.pending)
        if (q.stream != stream && err == hipSuccess) err = hipStreamWaitEvent(stream, q.event, 0);
      {
        std::lock_guard<std::mutex> relock(p.mu);
        give_events_locked(p, device, blk.pending);
      }
      buf->ptr = blk.ptr;
      buf->capacity = blk.capacity;
      hip_check(err, "allocator: hipStreamWaitEvent");
      return buf;
    }
  }
  void *ptr = nullptr;
  hipError_t e = hipMalloc(&ptr, want);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    clear_cache();
    hip_check(hipMalloc(&ptr, want), "hipMalloc");
  }
  {
    std::lock_guard<std::mutex> lock(p.mu);
    p.active += want;
    p.peak = std::max(p.peak, p.active);
  }
  buf->ptr = ptr;
  buf->capacity = want;
  return buf;
}

// ---- per-stream workspace ---------------------------------------------------------

namespace {

struct WorkspaceKey {
  int device;
  hipStream_t stream;
  std::thread::id thread; // only for hipStreamPerThread
  bool operator<(const WorkspaceKey &o) const {
    if (device != o.device) return device < o.device;
    if (stream != o.stream) return stream < o.stream;
    return thread < o.thread;
  }
};

struct WorkspaceSlot {
  std::shared_ptr<Buffer> partial;
  size_t partial_floats = 0;
};

std::mutex g_ws_mu;
// Never destroyed, like the pool: a static map's destructor would free its
// buffers (HIP event records) during process teardown, after the HIP runtime
// and any attached profiler have shut down.
std::map<WorkspaceKey, WorkspaceSlot> &g_ws = *new std::map<WorkspaceKey, WorkspaceSlot>();

WorkspaceKey ws_key(int device, hipStream_t stream) {
  WorkspaceKey k{device, stream, std::thread::id()};
  if (stream == hipStreamPerThread) k.thread = std::this_thread::get_id();
  return k;
}

} // namespace

float *stream_workspace(int device, hipStream_t stream, size_t partial_floats) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  WorkspaceSlot &slot = g_ws[ws_key(device, stream)];
  const size_t want = partial_floats + kWorkspaceHeaderFloats;
  if (slot.partial_floats < want) {
    // Grows by at least half again, so a growing sequence reallocates rarely;
    // the old buffer returns to the cache once the stream's work on it is done.
    const size_t n = std::max(want, slot.partial_floats + slot.partial_floats / 2);
    slot.partial = allocate(n * sizeof(float), device, stream);
    slot.partial_floats = n;
    // The header holds the stream-K flags, which each launch leaves zero.
    kern::fill_zero(slot.partial->ptr, kWorkspaceHeaderFloats * sizeof(float), stream);
  }
  return slot.partial ? static_cast<float *>(slot.partial->ptr) : nullptr;
}

void release_stream_workspace(int device, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_ws_mu);
  for (auto it = g_ws.begin(); it != g_ws.end();) {
    if (it->first.device == device && it->first.stream == stream)
      it = g_ws.erase(it);
    else
      ++it;
  }
}

size_t active_memory() {
  std::lock_guard<std::mutex> lock(pool().mu);
  return pool().active;
}
size_t peak_memory() {
  std::lock_guard<std::mutex> lock(pool().mu);
  return pool().peak;
}
size_t cache_memory() {
  std::lock_guard<std::mutex> lock(pool().mu);
  return pool().cached;
}
void reset_peak_memory() {
  std::lock_guard<std::mutex> lock(pool().mu);
  pool().peak = pool().active;
}
size_t set_cache_limit(size_t limit) {
  std::lock_guard<std::mutex> lock(pool().mu);
  size_t old = pool().limit;
  pool().limit = limit;
  if (pool().cached > limit) trim_locked(pool(), limit);
  return old;
}
void clear_cache() {
  {
    // Workspaces go back to the cache first (their users are done after the
    // device synchronisation below).
    std::lock_guard<std::mutex> lock(g_ws_mu);
    g_ws.clear();
  }
  std::lock_guard<std::mutex> lock(pool().mu);
  (void)hipDeviceSynchronize();
  trim_locked(pool(), 0);
}

// ---- streams --------------------------------------------------------------------

namespace {

std::mutex g_stream_mu;
std::map<int, hipStream_t> g_default_streams;
// Owned streams destroyed by sdq_stream_free (each synchronised first).  A
// handle value HIP hands out again for a new stream is taken off the list.
std::set<hipStream_t> g_retired;

hipStream_t default_stream_for(int device) {
  std::lock_guard<std::mutex> lock(g_stream_mu);
  auto it = g_default_streams.find(device);
  if (it != g_default_streams.end()) return it->second;
  hipStream_t s = nullptr;
  // Default priority; non-blocking so the legacy null stream never orders it.
  hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
            "hipStreamCreate");
  g_default_streams[device] = s;
  return s;
}

int current_device() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    fail("no HIP device is visible; libsdq has no CPU backend");
  }
  int d = 0;
  hip_check(hipGetDevice(&d), "hipGetDevice");
  return d;
}

} // namespace

bool stream_retired(hipStream_t s) {
  std::lock_guard<std::mutex> lock(g_stream_mu);
  return g_retired.count(s) != 0;
}

StreamImpl *stream_of(sdq_stream s, const char *op) {
  (void)op;
  auto *impl = static_cast<StreamImpl *>(s.ctx);
  if (!impl) fail("invalid stream handle");
  if (impl->cpu)
    fail("libsdq has no CPU backend; submit this op to a GPU stream "
         "(sdq_default_gpu_stream_new)");
  if (!impl->stream) {
    // Created without a visible device; try again now.
    impl->device = current_device();
    impl->stream = default_stream_for(impl->device);
  }
  return impl;
}

// ---- arrays ---------------------------------------------------------------------

std::string shape_str(const std::vector<int> &shape) {
  std::ostringstream os;
  os << "(";
  for (size_t i = 0; i < shape.size(); ++i) {
    if (i) os << ",";
    os << shape[i];
  }
  os << ")";
  return os.str();
}

ArrayImpl *array_of(sdq_array a, const char *op, const char *name) {
  (void)op;
  auto *impl = static_cast<ArrayImpl *>(a.ctx);
  if (!impl) fail(std::string("`") + name + "` is an empty array handle");
  return impl;
}

std::unique_ptr<ArrayImpl> make_array(const std::vector<int> &shape, int dtype,
                                      const StreamImpl &s) {
  auto a = std::make_unique<ArrayImpl>();
  a->shape = shape;
  a->dtype = dtype;
  size_t n = 1;
  for (int d : shape) {
    if (d < 0) fail("negative dimension in shape " + shape_str(shape));
    n *= size_t(d);
  }
  a->size = n;
  a->device = s.device;
  a->stream = s.stream;
  a->buf = allocate(a->nbytes(), s.device, s.stream);
  return a;
}

ArrayImpl share(const ArrayImpl &a) {
  ArrayImpl c;
  c.shape = a.shape;
  c.dtype = a.dtype;
  c.size = a.size;
  c.buf = a.buf;
  c.device = a.device;
  c.stream = a.stream;
  return c;
}

void set_vector_result(sdq_vector_array *res,
                       std::vector<std::unique_ptr<ArrayImpl>> values) {
  if (!res) fail("result pointer is NULL");
  auto *v = static_cast<VectorImpl *>(res->ctx);
  if (!v) {
    v = new VectorImpl();
    res->ctx = v;
  }
  v->items.clear();
  for (auto &a : values) v->items.push_back(share(*a));
}

void set_result(sdq_array *res, std::unique_ptr<ArrayImpl> value) {
  if (!res) fail("result pointer is NULL");
  if (res->ctx) {
    auto *old = static_cast<ArrayImpl *>(res->ctx);
    *old = std::move(*value);
  } else {
    res->ctx = value.release();
  }
}

} // namespace sdq

using namespace sdq;

// ---- C ABI ------------------------------------------------------------------------

namespace {

template <typename T> const T *host_view(sdq_array arr, int want, const char *op) {
  try {
    ArrayImpl *a = array_of(arr, op, "arr");
    if (a->dtype != want)
      fail(std::string("array is ") + dtype_name(a->dtype) + ", not " +
           dtype_name(want));
    a->host.resize(a->nbytes());
    if (a->nbytes()) {
      hip_check(hipMemcpyAsync(a->host.data(), a->data(), a->nbytes(),
                               hipMemcpyDeviceToHost, a->stream),
                "copy to host");
      hip_check(hipStreamSynchronize(a->stream), "synchronize");
    }
    return reinterpret_cast<const T *>(a->host.data());
  } catch (const std::exception &e) {
    report(op, e.what());
    return nullptr;
  }
}

} // namespace

extern "C" {

void sdq_set_error_handler(sdq_error_handler_func handler, void *data,
                           void (*dtor)(void *)) {
  HandlerSlot &h = handler_slot();
  void (*old_dtor)(void *) = nullptr;
  void *old_data = nullptr;
  {
    std::lock_guard<std::mutex> lock(h.mu);
    old_dtor = h.dtor;
    old_data = h.data;
    h.fn = handler ? handler : default_handler;
    h.data = handler ? data : nullptr;
    h.dtor = handler ? dtor : nullptr;
  }
  if (old_dtor) old_dtor(old_data);
}

sdq_array sdq_array_new(void) { return sdq_array{nullptr}; }

sdq_array sdq_array_new_data(const void *data, const int *shape, int dim,
                             sdq_dtype dtype) {
  try {
    if (dim < 0 || (dim > 0 && !shape)) fail("invalid shape");
    if (dtype_size(dtype) == 0) fail("unsupported dtype");
    std::vector<int> shp(shape, shape + dim);
    StreamImpl s;
    s.device = current_device();
    s.stream = default_stream_for(s.device);
    auto a = make_array(shp, dtype, s);
    if (a->nbytes()) {
      if (!data) fail("data is NULL");
      hip_check(hipMemcpyAsync(a->data(), data, a->nbytes(),
                               hipMemcpyHostToDevice, s.stream),
                "copy to device");
      hip_check(hipStreamSynchronize(s.stream), "synchronize");
    }
    return sdq_array{a.release()};
  } catch (const std::exception &e) {
    report("array_new_data", e.what());
    return sdq_array{nullptr};
  }
}

sdq_array sdq_array_new_float32(float val) {
  return sdq_array_new_data(&val, nullptr, 0, SDQ_FLOAT32);
}

int sdq_array_free(sdq_array arr) {
  delete static_cast<ArrayImpl *>(arr.ctx);
  return 0;
}

size_t sdq_array_size(sdq_array arr) {
  auto *a = static_cast<ArrayImpl *>(arr.ctx);
  return a ? a->size : 0;
}

size_t sdq_array_ndim(sdq_array arr) {
  auto *a = static_cast<ArrayImpl *>(arr.ctx);
  return a ? a->shape.size() : 0;
}

const int *sdq_array_shape(sdq_array arr) {
  auto *a = static_cast<ArrayImpl *>(arr.ctx);
  return (a && !a->shape.empty()) ? a->shape.data() : nullptr;
}

sdq_dtype sdq_array_dtype(sdq_array arr) {
  auto *a = static_cast<ArrayImpl *>(arr.ctx);
  return a ? sdq_dtype(a->dtype) : SDQ_FLOAT32;
}

size_t sdq_array_nbytes(sdq_array arr) {
  auto *a = static_cast<ArrayImpl *>(arr.ctx);
  return a ? a->nbytes() : 0;
}

int sdq_array_eval(sdq_array arr) {
  SDQ_GUARD("eval", {
    ArrayImpl *a = array_of(arr, "eval", "arr");
    if (a->stream) hip_check(hipStreamSynchronize(a->stream), "synchronize");
  });
}

const float *sdq_array_data_float32(sdq_array arr) {
  return host_view<float>(arr, SDQ_FLOAT32, "array_data_float32");
}
const uint32_t *sdq_array_data_uint32(sdq_array arr) {
  return host_view<uint32_t>(arr, SDQ_UINT32, "array_data_uint32");
}
const uint16_t *sdq_array_data_bfloat16(sdq_array arr) {
  return host_view<uint16_t>(arr, SDQ_BFLOAT16, "array_data_bfloat16");
}
const uint16_t *sdq_array_data_float16(sdq_array arr) {
  return host_view<uint16_t>(arr, SDQ_FLOAT16, "array_data_float16");
}

int sdq_array_copy_to_host(void *dst, size_t nbytes, sdq_array arr) {
  SDQ_GUARD("array_copy_to_host", {
    ArrayImpl *a = array_of(arr, "array_copy_to_host", "arr");
    if (nbytes != a->nbytes())
      fail("nbytes " + std::to_string(nbytes) + " does not match the array's " +
           std::to_string(a->nbytes()));
    if (nbytes) {
      if (!dst) fail("dst is NULL");
      hip_check(hipMemcpyAsync(dst, a->data(), nbytes, hipMemcpyDeviceToHost,
                               a->stream),
                "copy to host");
      hip_check(hipStreamSynchronize(a->stream), "synchronize");
    }
  });
}

sdq_vector_array sdq_vector_array_new(void) {
  return sdq_vector_array{new VectorImpl()};
}

sdq_vector_array sdq_vector_array_new_value(sdq_array val) {
  auto *v = new VectorImpl();
  if (auto *a = static_cast<ArrayImpl *>(val.ctx)) v->items.push_back(share(*a));
  return sdq_vector_array{v};
}

int sdq_vector_array_append_value(sdq_vector_array vec, sdq_array val) {
  SDQ_GUARD("vector_array_append_value", {
    auto *v = static_cast<VectorImpl *>(vec.ctx);
    if (!v) fail("invalid vector handle");
    ArrayImpl *a = array_of(val, "vector_array_append_value", "val");
    v->items.push_back(share(*a));
  });
}

size_t sdq_vector_array_size(sdq_vector_array vec) {
  auto *v = static_cast<VectorImpl *>(vec.ctx);
  return v ? v->items.size() : 0;
}

int sdq_vector_array_get(sdq_array *res, sdq_vector_array vec, size_t index) {
  SDQ_GUARD("vector_array_get", {
    auto *v = static_cast<VectorImpl *>(vec.ctx);
    if (!v) fail("invalid vector handle");
    if (index >= v->items.size())
      fail("index " + std::to_string(index) + " out of range for a vector of " +
           std::to_string(v->items.size()));
    set_result(res, std::make_unique<ArrayImpl>(share(v->items[index])));
  });
}

int sdq_vector_array_free(sdq_vector_array vec) {
  delete static_cast<VectorImpl *>(vec.ctx);
  return 0;
}

sdq_stream sdq_default_gpu_stream_new(void) {
  auto *s = new StreamImpl();
  try {
    s->device = current_device();
    s->stream = default_stream_for(s->device);
  } catch (const std::exception &) {
    // No device yet: the handle stays valid and ops on it report the reason.
    s->stream = nullptr;
  }
  return sdq_stream{s};
}

sdq_stream sdq_default_cpu_stream_new(void) {
  auto *s = new StreamImpl();
  s->cpu = true;
  return sdq_stream{s};
}

sdq_stream sdq_gpu_stream_new(void) {
  try {
    auto *s = new StreamImpl();
    s->device = current_device();
    hipStream_t h = nullptr;
    hip_check(hipStreamCreateWithFlags(&h, hipStreamNonBlocking),
              "hipStreamCreate");
    {
      std::lock_guard<std::mutex> lock(g_stream_mu);
      g_retired.erase(h);
    }
    s->stream = h;
    s->owned = true;
    return sdq_stream{s};
  } catch (const std::exception &e) {
    report("gpu_stream_new", e.what());
    return sdq_stream{nullptr};
  }
}

int sdq_stream_free(sdq_stream s) {
  auto *impl = static_cast<StreamImpl *>(s.ctx);
  if (impl && impl->owned && impl->stream) {
    // Everything enqueued on the stream completes before it goes: blocks and
    // arrays still tagged with it then need no wait on it (stream_retired).
    (void)hipStreamSynchronize(impl->stream);
    {
      std::lock_guard<std::mutex> lock(g_stream_mu);
      g_retired.insert(impl->stream);
    }
    release_stream_workspace(impl->device, impl->stream);
    (void)hipStreamDestroy(impl->stream);
  }
  delete impl;
  return 0;
}

int sdq_synchronize(sdq_stream s) {
  SDQ_GUARD("synchronize", {
    StreamImpl *impl = stream_of(s, "synchronize");
    hip_check(hipStreamSynchronize(impl->stream), "hipStreamSynchronize");
  });
}

void *sdq_stream_native(sdq_stream s) {
  auto *impl = static_cast<StreamImpl *>(s.ctx);
  if (!impl || impl->cpu) return nullptr;
  return impl->stream;
}

int sdq_eval(sdq_vector_array outputs) {
  SDQ_GUARD("eval", {
    auto *v = static_cast<VectorImpl *>(outputs.ctx);
    if (!v) fail("invalid vector handle");
    for (const ArrayImpl &a : v->items)
      if (a.stream) hip_check(hipStreamSynchronize(a.stream), "synchronize");
  });
}

int sdq_get_active_memory(size_t *res) {
  SDQ_GUARD("get_active_memory", {
    if (!res) fail("res is NULL");
    *res = active_memory();
  });
}
int sdq_get_peak_memory(size_t *res) {
  SDQ_GUARD("get_peak_memory", {
    if (!res) fail("res is NULL");
    *res = peak_memory();
  });
}
int sdq_get_cache_memory(size_t *res) {
  SDQ_GUARD("get_cache_memory", {
    if (!res) fail("res is NULL");
    *res = cache_memory();
  });
}
int sdq_reset_peak_memory(void) { SDQ_GUARD("reset_peak_memory", reset_peak_memory()); }
int sdq_set_cache_limit(size_t *res, size_t limit) {
  SDQ_GUARD("set_cache_limit", {
    size_t old = set_cache_limit(limit);
    if (res) *res = old;
  });
}
int sdq_clear_cache(void) { SDQ_GUARD("clear_cache", clear_cache()); }

const char *sdq_version(void) { return "sdq 0.1.0 gfx950"; }

int sdq_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

} // extern "C"
