// dense.hip -- y = a @ b.T in f32 accumulation, for the weights that stay
// dense (norm-sized or with an input width that is not a multiple of the
// group size): the `x @ w.T` of the diffusers Linear in
// sd-models/src/mlx/mod.rs:181-189, which quantized::linear falls back to for
// names held dense (quantized.rs:307-312).  Not on the hot path: a plain
// 16 x 16 LDS-tiled kernel with one output per thread, exact f32 products.
#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kTile = 16;

template <int AD, int BD, int OD>
__global__ __launch_bounds__(kTile *kTile) void matmul_nt_kernel(
    const typename Elem<AD>::T *__restrict__ a, const typename Elem<BD>::T *__restrict__ b,
    typename Elem<OD>::T *__restrict__ y, int64_t M, int64_t N, int64_t K) {
  __shared__ float as[kTile][kTile + 1];
  __shared__ float bs[kTile][kTile + 1];
  const int tx = threadIdx.x % kTile; // column within the tile
  const int ty = threadIdx.x / kTile; // row within the tile
  const int64_t row = int64_t(blockIdx.y) * kTile + ty;
  const int64_t col = int64_t(blockIdx.x) * kTile + tx;
  const int64_t brow = int64_t(blockIdx.x) * kTile + ty; // row of b this thread stages
  float acc = 0.0f;
  for (int64_t k0 = 0; k0 < K; k0 += kTile) {
    const int64_t k = k0 + tx;
    as[ty][tx] = (row < M && k < K) ? Elem<AD>::load(a[row * K + k]) : 0.0f;
    bs[ty][tx] = (brow < N && k < K) ? Elem<BD>::load(b[brow * K + k]) : 0.0f;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kTile; ++kk) acc = fmaf(as[ty][kk], bs[tx][kk], acc);
    __syncthreads();
  }
  if (row < M && col < N) y[row * N + col] = Elem<OD>::store(acc);
}

#define SDQ_DENSE_CASE(A, B)                                                          \
  if (a_dtype == A && b_dtype == B) {                                                 \
    constexpr int O = (A == B) ? A : SDQ_FLOAT32;                                     \
    matmul_nt_kernel<A, B, O><<<grid, kTile * kTile, 0, stream>>>(                    \
        static_cast<const typename Elem<A>::T *>(a),                                  \
        static_cast<const typename Elem<B>::T *>(b),                                  \
        static_cast<typename Elem<O>::T *>(y), M, N, K);                              \
    hip_check(hipGetLastError(), "matmul launch");                                    \
    return;                                                                           \
  }

} // namespace

namespace kern {

void matmul_nt(const void *a, int a_dtype, const void *b, int b_dtype, void *y,
               int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (M == 0 || N == 0) return;
  if ((N + kTile - 1) / kTile > 0x7fffffff || (M + kTile - 1) / kTile > 65535)
    fail("matmul: shape too large for the dense kernel");
  const dim3 grid(unsigned((N + kTile - 1) / kTile), unsigned((M + kTile - 1) / kTile));
  SDQ_DENSE_CASE(SDQ_FLOAT32, SDQ_FLOAT32)
  SDQ_DENSE_CASE(SDQ_BFLOAT16, SDQ_BFLOAT16)
  SDQ_DENSE_CASE(SDQ_FLOAT16, SDQ_FLOAT16)
  SDQ_DENSE_CASE(SDQ_BFLOAT16, SDQ_FLOAT32)
  SDQ_DENSE_CASE(SDQ_FLOAT32, SDQ_BFLOAT16)
  SDQ_DENSE_CASE(SDQ_FLOAT16, SDQ_FLOAT32)
  SDQ_DENSE_CASE(SDQ_FLOAT32, SDQ_FLOAT16)
  SDQ_DENSE_CASE(SDQ_BFLOAT16, SDQ_FLOAT16)
  SDQ_DENSE_CASE(SDQ_FLOAT16, SDQ_BFLOAT16)
  fail("matmul: unsupported dtypes");
}

} // namespace kern
} // namespace sdq
