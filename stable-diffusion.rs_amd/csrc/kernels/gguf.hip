// gguf.hip -- GGUF tensor blocks decoded on the device, and the fused
// GGUF -> MLX-affine requantization of the quantized loader.
//
// Replaces, in the reference's load path (crates/sd-models/src/mlx/quantized.rs:
// 181-258, from_gguf / from_gguf_renamed), the host-side block decoding of
// Gguf::dequantize (crates/sd-tensor/src/mlx_gguf.rs:235-276, per-type
// decoders 324-438) and the f32 round trip through Array::from_slice_f32 +
// QuantizedArray::quantize that follows it (quantized.rs:190-196).  The raw
// GGML blocks (0.5-1.1 bytes per value) go to HBM as they are; one kernel
// decodes them in registers and, for the loader, quantizes the decoded f32
// values straight to packed codes, so the dense f32 tensor is never written.
//
// BUILT WITH -ffp-contract=off.  Each decoded value is computed with the
// reference decoder's f32 operations in its order (Rust never contracts
// a*b - c), so values are the reference's bit for bit; the requantization is
// quant_group.hpp, the same arithmetic as quantize (quant.hip), so codes,
// scales and biases equal those of decoding then quantizing.
//
// Work layout.  A block of 256 lanes owns 256*C consecutive values (C = 8,
// or 16 for 2-bit codes); their raw bytes, a whole number of GGML blocks and
// a multiple of 16 bytes for every type, are staged in LDS with 16-byte
// loads, then each lane decodes its C values from LDS.  The lanes of one
// MLX group are consecutive lanes of one wave (quant_group.hpp).
#include "device_common.hpp"
#include "launch.hpp"
#include "quant_group.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kThreads = 256;

// GGML type ids as written in the file (mlx_gguf.rs:61-79) and their
// (values, bytes) per block (mlx_gguf.rs:27-40, 81-92).
enum : int { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30 };

template <int T> struct Layout;
template <> struct Layout<T_F32> { static constexpr int kValues = 1, kBytes = 4; };
template <> struct Layout<T_F16> { static constexpr int kValues = 1, kBytes = 2; };
template <> struct Layout<T_BF16> { static constexpr int kValues = 1, kBytes = 2; };
template <> struct Layout<T_Q4_0> { static constexpr int kValues = 32, kBytes = 18; };
template <> struct Layout<T_Q8_0> { static constexpr int kValues = 32, kBytes = 34; };
template <> struct Layout<T_Q4_K> { static constexpr int kValues = 256, kBytes = 144; };
template <> struct Layout<T_Q5_K> { static constexpr int kValues = 256, kBytes = 176; };
template <> struct Layout<T_Q6_K> { static constexpr int kValues = 256, kBytes = 210; };

// f16 -> f32 as mlx_gguf.rs:302-318 defines it: exact for every finite value
// and infinity (built from the fields, so the result does not depend on the
// hardware's f16 denormal mode), and the canonical quiet NaN for every NaN.
__device__ __forceinline__ float half_to_f32(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  if (e == 0) {
    const float v = float(m) * 5.9604644775390625e-8f; // m * 2^-24, exact
    return __uint_as_float(__float_as_uint(v) | sign);
  }
  if (e == 0x1fu) return __uint_as_float(m ? 0x7fc00000u : (sign | 0x7f800000u));
  return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

// A NaN produced by a block's arithmetic as the reference's platform (Apple
// arm64, default-NaN propagation) produces it: the positive quiet NaN.  Its
// only NaN sources are a NaN scale, which decodes to that NaN, and inf * 0 or
// inf - inf, whose default NaN is that NaN too; the hardware here may flip
// the sign in a subtraction.
__device__ __forceinline__ float canon_nan(float v) {
  return v != v ? __uint_as_float(0x7fc00000u) : v;
}

__device__ __forceinline__ uint32_t lds_u16(const uint8_t *p) {
  return *reinterpret_cast<const uint16_t *>(p); // 2-byte aligned in every use
}

// Decodes values [t, t + 8) of the GGML block at `blk` (LDS); t % 8 == 0.
template <int T> struct Decode;

template <> struct Decode<T_F32> {
  static __device__ __forceinline__ void get(const uint8_t *blk, int, float (&v)[8]) {
    const floatx4 a = reinterpret_cast<const floatx4 *>(blk)[0];
    const floatx4 b = reinterpret_cast<const floatx4 *>(blk)[1];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = a[k];
      v[k + 4] = b[k];
    }
  }
};
template <> struct Decode<T_F16> {
  static __device__ __forceinline__ void get(const uint8_t *blk, int, float (&v)[8]) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(blk);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = half_to_f32(a[k] & 0xffffu);
      v[2 * k + 1] = half_to_f32(a[k] >> 16);
    }
  }
};
template <> struct Decode<T_BF16> {
  static __device__ __forceinline__ void get(const uint8_t *blk, int, float (&v)[8]) {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(blk);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __uint_as_float(a[k] << 16);
      v[2 * k + 1] = __uint_as_float(a[k] & 0xffff0000u);
    }
  }
};
// mlx_gguf.rs:324-335: d * (nibble - 8); low nibbles are values 0..15, high
// nibbles 16..31.
template <> struct Decode<T_Q4_0> {
  static __device__ __forceinline__ void get(const uint8_t *blk, int t, float (&v)[8]) {
    const float d = half_to_f32(lds_u16(blk));
    const int shift = t >= 16 ? 4 : 0;
    const uint8_t *q = blk + 2 + (t & 15);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = canon_nan(d * float(int((q[k] >> shift) & 0x0f) - 8));
  }
};
// mlx_gguf.rs:337-344: d * (signed byte).
template <> struct Decode<T_Q8_0> {
  static __device__ __forceinline__ void get(const uint8_t *blk, int t, float (&v)[8]) {
    const float d = half_to_f32(lds_u16(blk));
    const uint8_t *q = blk + 2 + t;
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = canon_nan(d * float(int(int8_t(q[k]))));
  }
};

// mlx_gguf.rs:351-360 (llama.cpp's get_scale_min_k4): the 6-bit scale and
// min of sub-block j from the 12 packed bytes.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, uint32_t &sc, uint32_t &m) {
  if (j < 4) {
    sc = q[j] & 63u;
    m = q[j + 4] & 63u;
  } else {
    sc = (q[j + 4] & 0x0fu) | (uint32_t(q[j - 4] >> 6) << 4);
    m = (uint32_t(q[j + 4]) >> 4) | (uint32_t(q[j] >> 6) << 4);
  }
}

// mlx_gguf.rs:362-409: sub-block j = t / 32 takes the low (even j) or high
// (odd j) nibbles of one 32-byte half; Q5_K adds bit j of qh[i] as the fifth
// bit.  value = (d * sc) * q - dmin * m, each product rounded.
template <bool FIVE> struct DecodeK45 {
  static __device__ __forceinline__ void get(const uint8_t *blk, int t, float (&v)[8]) {
    const float d = half_to_f32(lds_u16(blk));
    const float dmin = half_to_f32(lds_u16(blk + 2));
    const int j = t >> 5, i0 = t & 31;
    uint32_t sc, m;
    scale_min_k4(j, blk + 4, sc, m);
    const float d1 = d * float(sc);
    const float m1 = dmin * float(m);
    const uint8_t *qs = blk + (FIVE ? 48 : 16) + (j >> 1) * 32 + i0;
    const int shift = (j & 1) ? 4 : 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint32_t q = (uint32_t(qs[k]) >> shift) & 0x0fu;
      if constexpr (FIVE) q |= ((uint32_t(blk[16 + i0 + k]) >> j) & 1u) << 4;
      const float prod = d1 * float(q);
      v[k] = canon_nan(prod - m1);
    }
  }
};
template <> struct Decode<T_Q4_K> : DecodeK45<false> {};
template <> struct Decode<T_Q5_K> : DecodeK45<true> {};

// mlx_gguf.rs:411-438: two halves of 128 values; in half n, quarter r of 32
// values takes the low (r < 2) or high nibbles of ql[n*64 + (r&1)*32 + l],
// bits 2r..2r+1 of qh[n*32 + l] as bits 4-5, minus 32, and the signed scale
// sc[n*8 + l/16 + 2r].  value = (d * sc) * q.
template <> struct Decode<T_Q6_K> {
  static __device__ __forceinline__ void get(const uint8_t *blk, int t, float (&v)[8]) {
    const float d = half_to_f32(lds_u16(blk + 208));
    const int n = t >> 7, r = (t >> 5) & 3, l0 = t & 31;
    const uint8_t *ql = blk + n * 64 + (r & 1) * 32 + l0;
    const uint8_t *qh = blk + 128 + n * 32 + l0;
    const float sc = float(int(int8_t(blk[192 + n * 8 + (l0 >> 4) + 2 * r])));
    const float ds = d * sc;
    const int lshift = r >= 2 ? 4 : 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int q = int(((uint32_t(ql[k]) >> lshift) & 0x0fu) | (((uint32_t(qh[k]) >> (2 * r)) & 3u) << 4)) - 32;
      v[k] = canon_nan(ds * float(q));
    }
  }
};

// Stages the raw bytes of values [v0, v0 + 256*C) into LDS: `full` bytes
// (the block's whole share, a multiple of 16) or, for the last block, what
// is left.  raw is 16-byte aligned and v0's byte offset is a multiple of 16.
template <int T, int C>
__device__ __forceinline__ void stage(const uint8_t *__restrict__ raw, int64_t raw_bytes,
                                      uint8_t *lds) {
  using L = Layout<T>;
  constexpr int kValues = kThreads * C;
  constexpr int kRaw = kValues / L::kValues * L::kBytes;
  static_assert(kRaw % 16 == 0, "a block's raw share must be 16-byte pieces");
  const int64_t first = int64_t(blockIdx.x) * kRaw;
  const int64_t left = raw_bytes - first;
  const int here = left < kRaw ? int(left) : kRaw;
  const u32x4 *src = reinterpret_cast<const u32x4 *>(raw + first);
  u32x4 *dst = reinterpret_cast<u32x4 *>(lds);
  for (int i = threadIdx.x; i < here / 16; i += kThreads) dst[i] = src[i];
  for (int b = (here / 16) * 16 + threadIdx.x; b < here; b += kThreads) lds[b] = raw[first + b];
  __syncthreads();
}

template <int T, int C>
__device__ __forceinline__ void decode_lane(const uint8_t *lds, float (&v)[C]) {
  using L = Layout<T>;
#pragma unroll
  for (int h = 0; h < C / 8; ++h) {
    const int local = threadIdx.x * C + h * 8;
    const int blk = local / L::kValues, t = local % L::kValues;
    float part[8];
    Decode<T>::get(lds + blk * L::kBytes, t, part);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[h * 8 + k] = part[k];
  }
}

template <int T>
__global__ __launch_bounds__(kThreads) void gguf_dequantize_kernel(const uint8_t *__restrict__ raw,
                                                                   int64_t raw_bytes, int64_t n,
                                                                   float *__restrict__ out) {
  constexpr int C = 8;
  __shared__ __align__(16) uint8_t lds[kThreads * C / Layout<T>::kValues * Layout<T>::kBytes];
  stage<T, C>(raw, raw_bytes, lds);
  const int64_t e0 = (int64_t(blockIdx.x) * kThreads + threadIdx.x) * C;
  if (e0 >= n) return;
  float v[C];
  decode_lane<T, C>(lds, v);
  if (e0 + C <= n) {
    reinterpret_cast<floatx4 *>(out + e0)[0] = floatx4{v[0], v[1], v[2], v[3]};
    reinterpret_cast<floatx4 *>(out + e0)[1] = floatx4{v[4], v[5], v[6], v[7]};
  } else {
#pragma unroll
    for (int k = 0; k < C; ++k)
      if (e0 + k < n) out[e0 + k] = v[k];
  }
}

template <int T, int BITS, int GS>
__global__ __launch_bounds__(kThreads) void gguf_quantize_kernel(const uint8_t *__restrict__ raw,
                                                                 int64_t raw_bytes, int64_t n_chunks,
                                                                 uint32_t *__restrict__ wq,
                                                                 float *__restrict__ scales,
                                                                 float *__restrict__ biases) {
  constexpr int C = QuantShape<BITS>::kPerThread;
  __shared__ __align__(16) uint8_t lds[kThreads * C / Layout<T>::kValues * Layout<T>::kBytes];
  stage<T, C>(raw, raw_bytes, lds);
  const int64_t c = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  // n_chunks is a multiple of the lanes per group, which divides the wave,
  // so a group's lanes are all in range or all out of it.
  if (c >= n_chunks) return;
  float v[C];
  decode_lane<T, C>(lds, v);
  uint32_t words[QuantShape<BITS>::kWords];
  float scale, bias;
  quantize_group<BITS, GS>(v, words, scale, bias);
  store_group<BITS, GS, SDQ_FLOAT32>(c, words, scale, bias, wq, scales, biases);
}

template <int T> void launch_dequantize(const uint8_t *raw, int64_t raw_bytes, int64_t n, float *out, hipStream_t st) {
  const int64_t per_block = int64_t(kThreads) * 8;
  const int64_t grid = (n + per_block - 1) / per_block;
  if (grid > 0x7fffffff) fail("gguf: tensor too large for one launch");
  gguf_dequantize_kernel<T><<<dim3(unsigned(grid)), kThreads, 0, st>>>(raw, raw_bytes, n, out);
}

template <int T, int BITS, int GS>
void launch_quantize_t(const uint8_t *raw, int64_t raw_bytes, int64_t n, uint32_t *wq, float *sc, float *bi,
                       hipStream_t st) {
  constexpr int C = QuantShape<BITS>::kPerThread;
  const int64_t chunks = n / C;
  const int64_t grid = (chunks + kThreads - 1) / kThreads;
  if (grid > 0x7fffffff) fail("gguf: tensor too large for one launch");
  gguf_quantize_kernel<T, BITS, GS><<<dim3(unsigned(grid)), kThreads, 0, st>>>(raw, raw_bytes, chunks, wq, sc, bi);
}

template <int T, int BITS>
void launch_quantize_gs(const uint8_t *raw, int64_t raw_bytes, int64_t n, int gs, uint32_t *wq, float *sc,
                        float *bi, hipStream_t st) {
  switch (gs) {
  case 32: launch_quantize_t<T, BITS, 32>(raw, raw_bytes, n, wq, sc, bi, st); break;
  case 64: launch_quantize_t<T, BITS, 64>(raw, raw_bytes, n, wq, sc, bi, st); break;
  case 128: launch_quantize_t<T, BITS, 128>(raw, raw_bytes, n, wq, sc, bi, st); break;
  default: fail("gguf quantize: unsupported group size");
  }
}

template <int T>
void launch_quantize_bits(const uint8_t *raw, int64_t raw_bytes, int64_t n, int gs, int bits, uint32_t *wq,
                          float *sc, float *bi, hipStream_t st) {
  switch (bits) {
  case 2: launch_quantize_gs<T, 2>(raw, raw_bytes, n, gs, wq, sc, bi, st); break;
  case 4: launch_quantize_gs<T, 4>(raw, raw_bytes, n, gs, wq, sc, bi, st); break;
  case 8: launch_quantize_gs<T, 8>(raw, raw_bytes, n, gs, wq, sc, bi, st); break;
  default: fail("gguf quantize: unsupported bits");
  }
}

template <template <int> class F, typename... A> void by_type(int type, A... a) {
  switch (type) {
  case T_F32: F<T_F32>::run(a...); break;
  case T_F16: F<T_F16>::run(a...); break;
  case T_BF16: F<T_BF16>::run(a...); break;
  case T_Q4_0: F<T_Q4_0>::run(a...); break;
  case T_Q8_0: F<T_Q8_0>::run(a...); break;
  case T_Q4_K: F<T_Q4_K>::run(a...); break;
  case T_Q5_K: F<T_Q5_K>::run(a...); break;
  case T_Q6_K: F<T_Q6_K>::run(a...); break;
  default: fail("gguf: unsupported GGML type " + std::to_string(type));
  }
}

template <int T> struct RunDequantize {
  static void run(const uint8_t *raw, int64_t raw_bytes, int64_t n, float *out, hipStream_t st) {
    launch_dequantize<T>(raw, raw_bytes, n, out, st);
  }
};
template <int T> struct RunQuantize {
  static void run(const uint8_t *raw, int64_t raw_bytes, int64_t n, int gs, int bits, uint32_t *wq, float *sc,
                  float *bi, hipStream_t st) {
    launch_quantize_bits<T>(raw, raw_bytes, n, gs, bits, wq, sc, bi, st);
  }
};

void check_raw(const uint8_t *raw, int type, int64_t n, int64_t raw_bytes) {
  int64_t per = 0, bytes = 0;
  if (!kern::gguf_block(type, &per, &bytes)) fail("gguf: unsupported GGML type " + std::to_string(type));
  if (n % per != 0) fail("gguf: element count is not a multiple of the block size");
  if (n / per * bytes != raw_bytes) fail("gguf: raw byte count does not match the element count");
  if (reinterpret_cast<uintptr_t>(raw) % 16 != 0) fail("gguf: raw bytes must be 16-byte aligned");
}

} // namespace

namespace kern {

bool gguf_block(int type, int64_t *values, int64_t *bytes) {
  int64_t v = 0, b = 0;
  switch (type) {
  case T_F32: v = Layout<T_F32>::kValues; b = Layout<T_F32>::kBytes; break;
  case T_F16: v = Layout<T_F16>::kValues; b = Layout<T_F16>::kBytes; break;
  case T_BF16: v = Layout<T_BF16>::kValues; b = Layout<T_BF16>::kBytes; break;
  case T_Q4_0: v = Layout<T_Q4_0>::kValues; b = Layout<T_Q4_0>::kBytes; break;
  case T_Q8_0: v = Layout<T_Q8_0>::kValues; b = Layout<T_Q8_0>::kBytes; break;
  case T_Q4_K: v = Layout<T_Q4_K>::kValues; b = Layout<T_Q4_K>::kBytes; break;
  case T_Q5_K: v = Layout<T_Q5_K>::kValues; b = Layout<T_Q5_K>::kBytes; break;
  case T_Q6_K: v = Layout<T_Q6_K>::kValues; b = Layout<T_Q6_K>::kBytes; break;
  default: return false;
  }
  if (values) *values = v;
  if (bytes) *bytes = b;
  return true;
}

void gguf_dequantize(const uint8_t *raw, int type, int64_t n, int64_t raw_bytes, float *out, hipStream_t stream) {
  if (n == 0) return;
  check_raw(raw, type, n, raw_bytes);
  by_type<RunDequantize>(type, raw, raw_bytes, n, out, stream);
  hip_check(hipGetLastError(), "gguf dequantize launch");
}

void gguf_quantize(const uint8_t *raw, int type, int64_t rows, int64_t cols, int64_t raw_bytes, int group_size,
                   int bits, uint32_t *wq, float *scales, float *biases, hipStream_t stream) {
  const int64_t n = rows * cols;
  if (n == 0) return;
  if (cols % group_size != 0) fail("gguf quantize: cols % group_size != 0");
  check_raw(raw, type, n, raw_bytes);
  by_type<RunQuantize>(type, raw, raw_bytes, n, group_size, bits, wq, scales, biases, stream);
  hip_check(hipGetLastError(), "gguf quantize launch");
}

} // namespace kern
} // namespace sdq
