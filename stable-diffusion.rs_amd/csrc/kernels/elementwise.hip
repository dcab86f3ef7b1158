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

// Eight consecutive elements of a float32/bfloat16/float16 array as f32,
// and back: 16-byte accesses (two for f32); `p` must be 16-byte aligned.
template <int D>
__device__ __forceinline__ void load8f(const typename Elem<D>::T *p, float (&v)[8]) {
  if constexpr (sizeof(typename Elem<D>::T) == 4) {
    const u32x4 a = reinterpret_cast<const u32x4 *>(p)[0];
    const u32x4 b = reinterpret_cast<const u32x4 *>(p)[1];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = __uint_as_float(a[k]);
      v[4 + k] = __uint_as_float(b[k]);
    }
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = Elem<D>::load(typename Elem<D>::T(a[k] & 0xffffu));
      v[2 * k + 1] = Elem<D>::load(typename Elem<D>::T(a[k] >> 16));
    }
  }
}

template <int D>
__device__ __forceinline__ void store8f(typename Elem<D>::T *p, const float (&v)[8]) {
  if constexpr (sizeof(typename Elem<D>::T) == 4) {
    u32x4 a, b;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a[k] = __float_as_uint(v[k]);
      b[k] = __float_as_uint(v[4 + k]);
    }
    reinterpret_cast<u32x4 *>(p)[0] = a;
    reinterpret_cast<u32x4 *>(p)[1] = b;
  } else {
    u32x4 a;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      a[k] = uint32_t(Elem<D>::store(v[2 * k])) | (uint32_t(Elem<D>::store(v[2 * k + 1])) << 16);
    *reinterpret_cast<u32x4 *>(p) = a;
  }
}

// The epilogue's combine stage over a finished [M, N] output, in place:
// y = r + g * y (COMB 1; G = 0: no gate) or y * r (COMB 2), r [M, N] with row
// stride N.  Used after the large-M kernel, whose tile store does not carry
// the combine stage.  Groups of eight consecutive elements of a row per
// thread, every operand in 16-byte pieces; the host checks that rows are
// whole groups and every pointer is 16-byte aligned.
template <int D, int R, int G, int COMB>
__global__ __launch_bounds__(kThreads) void combine8_kernel(typename Elem<D>::T *__restrict__ y,
                                                            const typename Elem<R>::T *__restrict__ res,
                                                            const void *__restrict__ gate,
                                                            int64_t M, int64_t N) {
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  const int64_t groups = M * N / 8;
  for (int64_t g = int64_t(blockIdx.x) * kThreads + threadIdx.x; g < groups; g += stride) {
    const int64_t e0 = g * 8;
    float v[8], r[8];
    load8f<D>(y + e0, v);
    load8f<R>(res + e0, r);
    if constexpr (COMB == 2) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] *= r[k];
    } else if constexpr (G == 0) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] += r[k];
    } else {
      float gv[8];
      load8f<G>(static_cast<const typename Elem<G>::T *>(gate) + (e0 % N), gv);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = fmaf(gv[k], v[k], r[k]);
    }
    store8f<D>(y + e0, v);
  }
}

// Any shape or alignment: one element per thread.
template <int D>
__global__ __launch_bounds__(kThreads) void combine_kernel(typename Elem<D>::T *__restrict__ y,
                                                           int64_t M, int64_t N,
                                                           kern::Epilogue ep) {
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < M * N; i += stride) {
    const int64_t m = i / N, n = i - m * N;
    y[i] = Elem<D>::store(epi_combine(ep, Elem<D>::load(y[i]), m, n));
  }
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

void combine_inplace(void *y, int y_dtype, int64_t M, int64_t N, const Epilogue &ep,
                     hipStream_t stream) {
  if (M == 0 || N == 0 || ep.combine == 0) return;
  if (!epilogue_ok(ep)) fail("combine: bad epilogue");
  const auto a16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool vec = N % 8 == 0 && ep.ld_res == N && a16(y) && a16(ep.res) && (!ep.gate || a16(ep.gate));
  if (!vec) {
    const int grid = grid_for(M * N / 4 + 1);
    SDQ_FLOAT_DISPATCH(y_dtype, D, {
      combine_kernel<D><<<grid, kThreads, 0, stream>>>(static_cast<typename Elem<D>::T *>(y), M, N, ep);
    });
    hip_check(hipGetLastError(), "combine launch");
    return;
  }
  const int grid = grid_for(M * N / 8 / 4 + 1);
  const int gdt = ep.gate ? ep.gate_dtype : 0;
  SDQ_FLOAT_DISPATCH(y_dtype, D, {
    SDQ_FLOAT_DISPATCH(ep.res_dtype, R, {
      auto *yp = static_cast<typename Elem<D>::T *>(y);
      auto *rp = static_cast<const typename Elem<R>::T *>(ep.res);
      if (ep.combine == 2) {
        combine8_kernel<D, R, 0, 2><<<grid, kThreads, 0, stream>>>(yp, rp, nullptr, M, N);
      } else if (gdt == 0) {
        combine8_kernel<D, R, 0, 1><<<grid, kThreads, 0, stream>>>(yp, rp, nullptr, M, N);
      } else {
        SDQ_FLOAT_DISPATCH(gdt, G, {
          combine8_kernel<D, R, G, 1><<<grid, kThreads, 0, stream>>>(yp, rp, ep.gate, M, N);
        });
      }
    });
  });
  hip_check(hipGetLastError(), "combine launch");
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
