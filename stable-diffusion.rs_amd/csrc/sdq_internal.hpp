// sdq_internal.hpp -- shared declarations of libsdq's host runtime.
//
// The runtime keeps the object model the reference's mlx-c bindings assume
// (crates/sd-tensor/src/mlx.rs:38-98, 558-612): reference-counted arrays
// behind opaque handles, streams as handles, a process-wide error handler,
// and explicit evaluation.  Arrays live in HBM; their buffers come from a
// per-device caching allocator so that steady-state calls never reach
// hipMalloc.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "sdq.h"

namespace sdq {

// Every failure inside the library is thrown as this and turned into a
// status + handler message at the C boundary.
struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const std::string &msg);
void hip_check(hipError_t e, const char *what);

size_t dtype_size(int dtype);
const char *dtype_name(int dtype);
bool is_float_dtype(int dtype);  // float32, bfloat16, float16
int promote_float(int a, int b); // MLX promotion among the three float types

// ---- device memory ------------------------------------------------------

// One device allocation.  `stream` is the stream it was allocated for (its
// producer); `readers` are the other streams that were ordered to use it
// (note_reader, called by the ops that consume it elsewhere).  When the last
// reference goes, one event per such stream is recorded and the block returns
// to the allocator's cache carrying them: whichever stream reuses the block
// first waits on all of them (a device-side wait, no host synchronisation),
// so no stream can overwrite data another stream is still reading.
struct Buffer {
  void *ptr = nullptr;
  size_t capacity = 0;
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<hipStream_t> readers;
  void note_reader(hipStream_t s);
  ~Buffer();
};

std::shared_ptr<Buffer> allocate(size_t bytes, int device, hipStream_t stream);
// True for a stream of sdq_gpu_stream_new that sdq_stream_free has destroyed.
// Such a stream is synchronised before it is destroyed, so its work is known
// to be complete and nothing waits on it afterwards.
bool stream_retired(hipStream_t s);
size_t active_memory();
size_t peak_memory();
size_t cache_memory();
void reset_peak_memory();
size_t set_cache_limit(size_t limit); // returns the previous limit
void clear_cache();

// ---- per-stream workspace ---------------------------------------------------

// Scratch memory of the large-M kernel (f32 partial tiles when it splits K
// across blocks), one buffer per (device, stream): calls on one stream are
// ordered by it, so they share the memory with no synchronisation and no
// per-call allocation.  It grows to the largest request and is kept until
// the stream is freed (release_stream_workspace) or the cache is cleared.
// The per-thread handle hipStreamPerThread names a different stream in each
// host thread, so its workspace is kept per thread.
// The buffer starts with a header of kWorkspaceHeaderFloats floats -- the
// stream-K flags, zeroed when the buffer is allocated and left zero by every
// launch -- followed by partial_floats floats of partial tiles.
constexpr size_t kWorkspaceHeaderFloats = 1024;
float *stream_workspace(int device, hipStream_t stream, size_t partial_floats);
void release_stream_workspace(int device, hipStream_t stream);

// Compute units of a device (cached).
int cu_count(int device);

// ---- streams ------------------------------------------------------------

struct StreamImpl {
  int device = 0;
  hipStream_t stream = nullptr;
  bool cpu = false;
  bool owned = false; // created by sdq_gpu_stream_new, destroyed on free
};

StreamImpl *stream_of(sdq_stream s, const char *op);

// ---- arrays -------------------------------------------------------------

struct ArrayImpl {
  std::vector<int> shape;
  int dtype = SDQ_FLOAT32;
  size_t size = 0; // elements
  std::shared_ptr<Buffer> buf;
  int device = 0;
  hipStream_t stream = nullptr; // the stream whose work produces the data
  std::vector<unsigned char> host; // mirror returned by the data accessors

  size_t nbytes() const { return size * dtype_size(dtype); }
  void *data() const { return buf ? buf->ptr : nullptr; }
};

ArrayImpl *array_of(sdq_array a, const char *op, const char *name);
// A new device array of the given shape, allocated for `s`.
std::unique_ptr<ArrayImpl> make_array(const std::vector<int> &shape, int dtype,
                                      const StreamImpl &s);
// Moves `value` into the result handle (allocating the handle when empty).
void set_result(sdq_array *res, std::unique_ptr<ArrayImpl> value);
// A second reference to the same data (metadata copied, buffer shared).
ArrayImpl share(const ArrayImpl &a);

struct VectorImpl {
  std::vector<ArrayImpl> items;
};
// Replaces the contents of the result vector (allocating it when empty).
void set_vector_result(sdq_vector_array *res,
                       std::vector<std::unique_ptr<ArrayImpl>> values);
std::string shape_str(const std::vector<int> &shape);

// Orders stream `s` after the work producing `a` and records `s` as a user
// of its memory (sdq_ops.cpp).
void order_after(const ArrayImpl *a, const StreamImpl *s);
// Fails unless `a` lives on the stream's device.
void same_device(const ArrayImpl *a, const StreamImpl *s, const char *name);

// Reports `msg` for op `op` through the installed handler.
void report(const char *op, const char *msg);

namespace kern {
struct Epilogue;
}

// y = x @ dequantize(w).T on device pointers with the epilogue `ep` (its
// output layout included), on `stream`; picks the kernel by M
// (sdq_ops.cpp).
void matmul_dispatch(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
                     const uint32_t *w, const void *scales, const void *biases,
                     int s_dtype, int64_t M, int64_t N, int64_t K, int gs, int bits,
                     int device, hipStream_t stream, const kern::Epilogue &ep);

// The Flux attention (sdq_ops_block.cpp): output shape of the qkv inputs,
// and the op writing its merged-heads output at `out` with row stride
// `ld_out` elements.
struct FluxAttnShape {
  int B = 0, N = 0, dtype = SDQ_FLOAT32;
};
FluxAttnShape flux_attention_shape(sdq_array qkv_a, sdq_array qkv_b, int heads, const StreamImpl *st);
void flux_attention_into(void *out, int64_t ld_out, sdq_array qkv_a, sdq_array q_norm_a, sdq_array k_norm_a,
                         sdq_array qkv_b, sdq_array q_norm_b, sdq_array k_norm_b, sdq_array pe_cos,
                         sdq_array pe_sin, int heads, float scale, float eps, const StreamImpl *st);

} // namespace sdq

// Wraps a C entry point body: exceptions become status 1 plus a message.
#define SDQ_GUARD(op, ...)                                                   \
  try {                                                                      \
    __VA_ARGS__;                                                             \
    return 0;                                                                \
  } catch (const std::exception &e) {                                        \
    ::sdq::report(op, e.what());                                             \
    return 1;                                                                \
  } catch (...) {                                                            \
    ::sdq::report(op, "unknown failure");                                    \
    return 1;                                                                \
  }
