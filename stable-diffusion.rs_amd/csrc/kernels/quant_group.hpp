// quant_group.hpp -- one MLX-affine group quantized by a run of consecutive
// lanes: the arithmetic shared by quantize (quant.hip) and the fused GGUF
// requantization (gguf.hip), so the two give bit-identical codes, scales and
// biases for the same f32 values.
//
// A translation unit that includes this must be built with -ffp-contract=off:
// every product and sum is then one IEEE f32 operation, rounded once, and the
// divisions are the correctly rounded ones.
//   per group of G values
//     scale = max((w_max - w_min) / n_bins, 1e-7), sign chosen so the larger
//     magnitude edge is the bias; q0 = rint(edge / scale); when q0 != 0 the
//     scale is refit to edge / q0 so that edge reconstructs exactly;
//     code = clamp(rint((w - bias) / scale), 0, n_bins), 32/bits codes per
//     word, first element in the least significant bits.
#pragma once

#include "device_common.hpp"

namespace sdq {
namespace dev {

// Elements handled by one lane: one word at 2 bits, two words at 8 bits,
// one word at 4 bits.  A group's lanes are consecutive lanes of one wave.
template <int BITS> struct QuantShape {
  static constexpr int kPerThread = BITS == 2 ? 16 : 8;
  static constexpr int kPerWord = 32 / BITS;
  static constexpr int kWords = kPerThread / kPerWord;
};

// Quantizes this lane's kPerThread values of a group of GS values spread over
// GS / kPerThread consecutive lanes (a power of two <= 16, aligned to itself
// within the wave).  Every lane of the group must execute this together.
// Returns the lane's packed words and the group's scale and bias.
template <int BITS, int GS>
__device__ __forceinline__ void quantize_group(const float (&v)[QuantShape<BITS>::kPerThread],
                                               uint32_t (&words)[QuantShape<BITS>::kWords],
                                               float &scale_out, float &bias_out) {
  using Shape = QuantShape<BITS>;
  constexpr int C = Shape::kPerThread;
  constexpr int T = GS / C;
  const float n_bins = float((1 << BITS) - 1);
  const float eps = 1e-7f;
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int e = 1; e < C; ++e) {
    lo = fminf(lo, v[e]);
    hi = fmaxf(hi, v[e]);
  }
#pragma unroll
  for (int off = T / 2; off > 0; off >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, off));
    hi = fmaxf(hi, __shfl_xor(hi, off));
  }
  const bool neg_edge = fabsf(lo) > fabsf(hi);
  float scale = (hi - lo) / n_bins;
  scale = scale < eps ? eps : scale;
  scale = neg_edge ? scale : -scale;
  const float edge = neg_edge ? lo : hi;
  const float q0 = rintf(edge / scale);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
#pragma unroll
  for (int i = 0; i < Shape::kWords; ++i) words[i] = 0u;
#pragma unroll
  for (int e = 0; e < C; ++e) {
    float q = rintf((v[e] - bias) / scale);
    q = fminf(fmaxf(q, 0.0f), n_bins);
    words[e / Shape::kPerWord] |= uint32_t(q) << ((e % Shape::kPerWord) * BITS);
  }
  scale_out = scale;
  bias_out = bias;
}

// Stores lane chunk `c`'s words, and the group's scale and bias from the
// group's first lane.
template <int BITS, int GS, int SDT>
__device__ __forceinline__ void store_group(int64_t c, const uint32_t (&words)[QuantShape<BITS>::kWords],
                                            float scale, float bias, uint32_t *__restrict__ wq,
                                            typename Elem<SDT>::T *__restrict__ scales,
                                            typename Elem<SDT>::T *__restrict__ biases) {
  using Shape = QuantShape<BITS>;
  constexpr int T = GS / Shape::kPerThread;
  if constexpr (Shape::kWords == 2) {
    *reinterpret_cast<u32x2 *>(wq + c * 2) = u32x2{words[0], words[1]};
  } else {
    wq[c] = words[0];
  }
  if ((c & (T - 1)) == 0) {
    scales[c / T] = Elem<SDT>::store(scale);
    biases[c / T] = Elem<SDT>::store(bias);
  }
}

} // namespace dev
} // namespace sdq
