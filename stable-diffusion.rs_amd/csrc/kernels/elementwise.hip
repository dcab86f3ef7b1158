// elementwise.hip -- the few elementwise ops around the quantized linear:
// dtype casts (mlx_astype, mlx.rs:149), the bias add after the matmul
// (quantized.rs:314-317), the T5 gate product (t5.rs:211) and tanh-GELU
// (Array::gelu_approx, mlx.rs:1041-1054).  All compute in f32 and round once
// to the output dtype.
#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kThreads = 256;

int grid_for(int64_t items) {
  int64_t blocks = (items + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return int(blocks);
}

template <int A, int O>
__global__ __launch_bounds__(kThreads) void astype_kernel(const typename Elem<A>::T *__restrict__ a,
                                                          typename Elem<O>::T *__restrict__ out,
                                                          int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    out[i] = Elem<O>::store(Elem<A>::load(a[i]));
}

enum class BinOp { kAdd, kMul };

template <BinOp OP, int A, int B, int O>
__global__ __launch_bounds__(kThreads) void binary_kernel(const typename Elem<A>::T *__restrict__ a,
                                                          const typename Elem<B>::T *__restrict__ b,
                                                          typename Elem<O>::T *__restrict__ out,
                                                          int64_t n, int64_t b_n) {
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
    const float x = Elem<A>::load(a[i]);
    const float y = Elem<B>::load(b[b_n == n ? i : i % b_n]);
    out[i] = Elem<O>::store(OP == BinOp::kAdd ? x + y : x * y);
  }
}

// 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3))), the operation order
// of mlx.rs:1048-1053.
// Eight elements per thread with 16-byte accesses where both pointers allow
// (the launch checks), the ragged tail one element per thread.
template <int D>
__global__ __launch_bounds__(kThreads) void gelu_kernel(const typename Elem<D>::T *__restrict__ a,
                                                        typename Elem<D>::T *__restrict__ out,
                                                        int64_t n, bool vec) {
  using T = typename Elem<D>::T;
  constexpr int kWords = int(sizeof(T)) * 8 / 4; // 32-bit words per 8 elements
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  const int64_t tid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t groups = vec ? n / 8 : 0;
  for (int64_t g = tid; g < groups; g += stride) {
    const u32x4 *src = reinterpret_cast<const u32x4 *>(a + g * 8);
    u32x4 *dst = reinterpret_cast<u32x4 *>(out + g * 8);
    u32x4 w[kWords / 4];
#pragma unroll
    for (int q = 0; q < kWords / 4; ++q) w[q] = __builtin_nontemporal_load(src + q);
#pragma unroll
    for (int q = 0; q < kWords / 4; ++q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t word = w[q][j];
        if constexpr (sizeof(T) == 4) {
          w[q][j] = __float_as_uint(gelu_approx_f(__uint_as_float(word)));
        } else {
          const float lo = Elem<D>::load(T(word & 0xffffu));
          const float hi = Elem<D>::load(T(word >> 16));
          w[q][j] = uint32_t(Elem<D>::store(gelu_approx_f(lo))) |
                    (uint32_t(Elem<D>::store(gelu_approx_f(hi))) << 16);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < kWords / 4; ++q) __builtin_nontemporal_store(w[q], dst + q);
  }
  for (int64_t i = groups * 8 + tid; i < n; i += stride)
    out[i] = Elem<D>::store(gelu_approx_f(Elem<D>::load(a[i])));
}


#define SDQ_FLOAT_DISPATCH(dt, NAME, ...)                                    \
  switch (dt) {                                                              \
  case SDQ_FLOAT32: {                                                        \
    constexpr int NAME = SDQ_FLOAT32;                                        \
    __VA_ARGS__;                                                             \
    break;                                                                   \
  }                                                                          \
  case SDQ_BFLOAT16: {                                                       \
    constexpr int NAME = SDQ_BFLOAT16;                                       \
    __VA_ARGS__;                                                             \
    break;                                                                   \
  }                                                                          \
  case SDQ_FLOAT16: {                                                        \
    constexpr int NAME = SDQ_FLOAT16;                                        \
    __VA_ARGS__;                                                             \
    break;                                                                   \
  }                                                                          \
  default:                                                                   \
    fail("unsupported dtype");                                               \
  }

// Zeroes a run of 32-bit words (a kernel rather than hipMemsetAsync, so it
// is also safe inside a captured graph).
__global__ __launch_bounds__(256) void fill_zero_kernel(uint32_t *__restrict__ p, int64_t words) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < words) p[i] = 0u;
}

} // namespace

namespace kern {


void astype(const void *a, int a_dtype, void *out, int out_dtype, int64_t n,
            hipStream_t stream) {
  if (n == 0) return;
  const int grid = grid_for(n);
  SDQ_FLOAT_DISPATCH(a_dtype, AD, SDQ_FLOAT_DISPATCH(out_dtype, OD, {
    astype_kernel<AD, OD><<<grid, kThreads, 0, stream>>>(
        static_cast<const typename Elem<AD>::T *>(a),
        static_cast<typename Elem<OD>::T *>(out), n);
  }));
  hip_check(hipGetLastError(), "astype launch");
}

template <BinOp OP>
static void binary(const void *a, int a_dtype, const void *b, int b_dtype,
                   void *out, int out_dtype, int64_t n, int64_t b_n,
                   hipStream_t stream) {
  if (n == 0) return;
  if (b_n <= 0 || n % b_n != 0) fail("binary op: broadcast shape mismatch");
  const int grid = grid_for(n);
  SDQ_FLOAT_DISPATCH(a_dtype, AD, SDQ_FLOAT_DISPATCH(b_dtype, BD, SDQ_FLOAT_DISPATCH(out_dtype, OD, {
    binary_kernel<OP, AD, BD, OD><<<grid, kThreads, 0, stream>>>(
        static_cast<const typename Elem<AD>::T *>(a),
        static_cast<const typename Elem<BD>::T *>(b),
        static_cast<typename Elem<OD>::T *>(out), n, b_n);
  })));
  hip_check(hipGetLastError(), "binary launch");
}

void add(const void *a, int a_dtype, const void *b, int b_dtype, void *out,
         int out_dtype, int64_t n, int64_t b_n, hipStream_t stream) {
  binary<BinOp::kAdd>(a, a_dtype, b, b_dtype, out, out_dtype, n, b_n, stream);
}

void multiply(const void *a, int a_dtype, const void *b, int b_dtype,
              void *out, int out_dtype, int64_t n, hipStream_t stream) {
  binary<BinOp::kMul>(a, a_dtype, b, b_dtype, out, out_dtype, n, n, stream);
}

void gelu_approx(const void *a, int dtype, void *out, int64_t n,
                 hipStream_t stream) {
  if (n == 0) return;
  const bool vec = reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
  // A few groups of eight per thread keep many loads in flight without a
  // huge grid.
  const int grid = grid_for((vec ? n / 8 : n) / 4 + 1);
  SDQ_FLOAT_DISPATCH(dtype, D, {
    gelu_kernel<D><<<grid, kThreads, 0, stream>>>(
        static_cast<const typename Elem<D>::T *>(a),
        static_cast<typename Elem<D>::T *>(out), n, vec);
  });
  hip_check(hipGetLastError(), "gelu launch");
}


void fill_zero(void *p, size_t bytes, hipStream_t stream) {
  const int64_t words = int64_t(bytes / 4);
  if (words == 0) return;
  const int grid = int((words + 255) / 256);
  fill_zero_kernel<<<grid, 256, 0, stream>>>(static_cast<uint32_t *>(p), words);
  hip_check(hipGetLastError(), "fill_zero launch");
}

} // namespace kern
} // namespace sdq
