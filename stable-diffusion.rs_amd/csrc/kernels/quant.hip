// quant.hip -- MLX-affine quantize and dequantize for gfx950.
//
// Replaces mlx_quantize / mlx_dequantize (crates/sd-tensor/src/mlx.rs:363-384,
// called from QuantizedArray::quantize / dequantize at mlx.rs:1856-1945).
//
// BUILT WITH -ffp-contract=off: every product and sum below is one IEEE f32
// operation, rounded once, and division is the correctly rounded one, so the
// codes, scales, biases and dequantized values are bit-identical to the CPU
// restatement of the same arithmetic:
//   per group of G values (G = group size along the last axis)
//     scale = max((w_max - w_min) / n_bins, 1e-7), sign chosen so the larger
//     magnitude edge is the bias; q0 = rint(edge / scale); when q0 != 0 the
//     scale is refit to edge / q0 so that edge reconstructs exactly;
//     code = clamp(rint((w - bias) / scale), 0, n_bins), 32/bits codes per
//     word, first element in the least significant bits;
//   dequantize: w = round_T(round_T(q * scale) + bias), T = the scales' dtype.
#include "device_common.hpp"
#include "launch.hpp"
#include "quant_group.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kThreads = 256;

template <int WDT, int N> __device__ __forceinline__ void load_elems(const typename Elem<WDT>::T *p, float (&v)[N]) {
  if constexpr (WDT == SDQ_FLOAT32) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      floatx4 t = *reinterpret_cast<const floatx4 *>(p + i);
      v[i] = t[0];
      v[i + 1] = t[1];
      v[i + 2] = t[2];
      v[i + 3] = t[3];
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 8) {
      u32x4 t = *reinterpret_cast<const u32x4 *>(p + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[i + 2 * j] = Elem<WDT>::load(uint16_t(t[j] & 0xffffu));
        v[i + 2 * j + 1] = Elem<WDT>::load(uint16_t(t[j] >> 16));
      }
    }
  }
}

template <int BITS, int WDT, int GS>
__global__ __launch_bounds__(kThreads) void quantize_kernel(
    const typename Elem<WDT>::T *__restrict__ w, int64_t n_chunks,
    uint32_t *__restrict__ wq, typename Elem<WDT>::T *__restrict__ scales,
    typename Elem<WDT>::T *__restrict__ biases) {
  using Shape = QuantShape<BITS>;
  constexpr int C = Shape::kPerThread;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t c = int64_t(blockIdx.x) * kThreads + threadIdx.x; c < n_chunks;
       c += stride) {
    // n_chunks is a multiple of the lanes per group, which divides the wave,
    // so the lanes of a group are either all in range here or all out of it.
    float v[C];
    load_elems<WDT, C>(w + c * C, v);
    uint32_t words[Shape::kWords];
    float scale, bias;
    quantize_group<BITS, GS>(v, words, scale, bias);
    store_group<BITS, GS, WDT>(c, words, scale, bias, wq, scales, biases);
  }
}

template <int BITS, int SDT, int ODT, int GS>
__global__ __launch_bounds__(kThreads) void dequantize_kernel(
    const uint32_t *__restrict__ wq, const typename Elem<SDT>::T *__restrict__ scales,
    const typename Elem<SDT>::T *__restrict__ biases, int64_t n_words,
    typename Elem<ODT>::T *__restrict__ out) {
  constexpr int kPerWord = 32 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  using OT = typename Elem<ODT>::T;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n_words;
       i += stride) {
    const uint32_t word = wq[i];
    // A word's codes never straddle a group (kPerWord <= 16 <= group size).
    const int64_t g = (i * kPerWord) / GS;
    const float s = Elem<SDT>::load(scales[g]);
    const float b = Elem<SDT>::load(biases[g]);
    OT vals[kPerWord];
#pragma unroll
    for (int e = 0; e < kPerWord; ++e) {
      const float q = float((word >> (e * BITS)) & kMask);
      const float p = Elem<SDT>::round(q * s);
      const float r = Elem<SDT>::round(p + b);
      vals[e] = Elem<ODT>::store(r);
    }
    constexpr int kBytes = kPerWord * int(sizeof(OT));
    OT *dst = out + i * kPerWord;
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int j = 0; j < kBytes / 16; ++j)
        reinterpret_cast<u32x4 *>(dst)[j] = reinterpret_cast<const u32x4 *>(vals)[j];
    } else if constexpr (kBytes == 8) {
      *reinterpret_cast<u32x2 *>(dst) = *reinterpret_cast<const u32x2 *>(vals);
    } else {
#pragma unroll
      for (int e = 0; e < kPerWord; ++e) dst[e] = vals[e];
    }
  }
}

int grid_for(int64_t items) {
  int64_t blocks = (items + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return int(blocks);
}

template <int BITS, int WDT>
void launch_quantize_gs(const void *w, int64_t n, int gs, uint32_t *wq,
                        void *scales, void *biases, hipStream_t st) {
  using T = typename Elem<WDT>::T;
  const int64_t chunks = n / QuantShape<BITS>::kPerThread;
  const int grid = grid_for(chunks);
  auto *wp = static_cast<const T *>(w);
  auto *sp = static_cast<T *>(scales);
  auto *bp = static_cast<T *>(biases);
  switch (gs) {
  case 32:
    quantize_kernel<BITS, WDT, 32><<<grid, kThreads, 0, st>>>(wp, chunks, wq, sp, bp);
    break;
  case 64:
    quantize_kernel<BITS, WDT, 64><<<grid, kThreads, 0, st>>>(wp, chunks, wq, sp, bp);
    break;
  case 128:
    quantize_kernel<BITS, WDT, 128><<<grid, kThreads, 0, st>>>(wp, chunks, wq, sp, bp);
    break;
  default:
    fail("quantize: unsupported group size");
  }
}

template <int BITS>
void launch_quantize_bits(const void *w, int wdt, int64_t n, int gs,
                          uint32_t *wq, void *scales, void *biases,
                          hipStream_t st) {
  switch (wdt) {
  case SDQ_FLOAT32:
    launch_quantize_gs<BITS, SDQ_FLOAT32>(w, n, gs, wq, scales, biases, st);
    break;
  case SDQ_BFLOAT16:
    launch_quantize_gs<BITS, SDQ_BFLOAT16>(w, n, gs, wq, scales, biases, st);
    break;
  case SDQ_FLOAT16:
    launch_quantize_gs<BITS, SDQ_FLOAT16>(w, n, gs, wq, scales, biases, st);
    break;
  default:
    fail("quantize: unsupported dtype");
  }
}

template <int BITS, int SDT, int ODT>
void launch_dequantize_gs(const uint32_t *wq, const void *s, const void *b,
                          int64_t n_words, int gs, void *out, hipStream_t st) {
  using ST = typename Elem<SDT>::T;
  using OT = typename Elem<ODT>::T;
  const int grid = grid_for(n_words);
  auto *sp = static_cast<const ST *>(s);
  auto *bp = static_cast<const ST *>(b);
  auto *op = static_cast<OT *>(out);
  switch (gs) {
  case 32:
    dequantize_kernel<BITS, SDT, ODT, 32><<<grid, kThreads, 0, st>>>(wq, sp, bp, n_words, op);
    break;
  case 64:
    dequantize_kernel<BITS, SDT, ODT, 64><<<grid, kThreads, 0, st>>>(wq, sp, bp, n_words, op);
    break;
  case 128:
    dequantize_kernel<BITS, SDT, ODT, 128><<<grid, kThreads, 0, st>>>(wq, sp, bp, n_words, op);
    break;
  default:
    fail("dequantize: unsupported group size");
  }
}

template <int BITS, int SDT>
void launch_dequantize_out(const uint32_t *wq, const void *s, const void *b,
                           int64_t n_words, int gs, void *out, int odt,
                           hipStream_t st) {
  switch (odt) {
  case SDQ_FLOAT32:
    launch_dequantize_gs<BITS, SDT, SDQ_FLOAT32>(wq, s, b, n_words, gs, out, st);
    break;
  case SDQ_BFLOAT16:
    launch_dequantize_gs<BITS, SDT, SDQ_BFLOAT16>(wq, s, b, n_words, gs, out, st);
    break;
  case SDQ_FLOAT16:
    launch_dequantize_gs<BITS, SDT, SDQ_FLOAT16>(wq, s, b, n_words, gs, out, st);
    break;
  default:
    fail("dequantize: unsupported output dtype");
  }
}

template <int BITS>
void launch_dequantize_bits(const uint32_t *wq, const void *s, const void *b,
                            int sdt, int64_t n_words, int gs, void *out,
                            int odt, hipStream_t st) {
  switch (sdt) {
  case SDQ_FLOAT32:
    launch_dequantize_out<BITS, SDQ_FLOAT32>(wq, s, b, n_words, gs, out, odt, st);
    break;
  case SDQ_BFLOAT16:
    launch_dequantize_out<BITS, SDQ_BFLOAT16>(wq, s, b, n_words, gs, out, odt, st);
    break;
  case SDQ_FLOAT16:
    launch_dequantize_out<BITS, SDQ_FLOAT16>(wq, s, b, n_words, gs, out, odt, st);
    break;
  default:
    fail("dequantize: unsupported scale dtype");
  }
}

} // namespace

namespace kern {

void quantize(const void *w, int w_dtype, int64_t rows, int64_t cols,
              int group_size, int bits, uint32_t *wq, void *scales,
              void *biases, hipStream_t stream) {
  const int64_t n = rows * cols;
  if (n == 0) return;
  if (cols % group_size != 0) fail("quantize: cols % group_size != 0");
  switch (bits) {
  case 2:
    launch_quantize_bits<2>(w, w_dtype, n, group_size, wq, scales, biases, stream);
    break;
  case 4:
    launch_quantize_bits<4>(w, w_dtype, n, group_size, wq, scales, biases, stream);
    break;
  case 8:
    launch_quantize_bits<8>(w, w_dtype, n, group_size, wq, scales, biases, stream);
    break;
  default:
    fail("quantize: unsupported bits");
  }
  hip_check(hipGetLastError(), "quantize launch");
}

void dequantize(const uint32_t *wq, const void *scales, const void *biases,
                int s_dtype, int64_t rows, int64_t cols, int group_size,
                int bits, void *out, int out_dtype, hipStream_t stream) {
  const int64_t n_words = rows * cols * bits / 32;
  if (n_words == 0) return;
  switch (bits) {
  case 2:
    launch_dequantize_bits<2>(wq, scales, biases, s_dtype, n_words, group_size, out, out_dtype, stream);
    break;
  case 4:
    launch_dequantize_bits<4>(wq, scales, biases, s_dtype, n_words, group_size, out, out_dtype, stream);
    break;
  case 8:
    launch_dequantize_bits<8>(wq, scales, biases, s_dtype, n_words, group_size, out, out_dtype, stream);
    break;
  default:
    fail("dequantize: unsupported bits");
  }
  hip_check(hipGetLastError(), "dequantize launch");
}

} // namespace kern
} // namespace sdq
