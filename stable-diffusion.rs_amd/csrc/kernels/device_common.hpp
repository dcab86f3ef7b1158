// device_common.hpp -- element types, conversions and vector types shared by
// the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sdq.h"
#include "launch.hpp"

namespace sdq {
namespace dev {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// Round to nearest even (hardware v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, uint16_t(h)));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Two f32 values packed as a bf16 pair (first in the low half), rounded to
// nearest even: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const floatx2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// Hides a value's known bits from the optimizer (no instruction is emitted),
// so that byte-field conversions select v_cvt_f32_ubyte{0..3} directly
// instead of re-extracting fields it believes are narrower.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// Storage type and conversions per dtype code (positions of mlx_dtype).
template <int DT> struct Elem;

template <> struct Elem<SDQ_FLOAT32> {
  using T = float;
  static __device__ __forceinline__ float load(T v) { return v; }
  static __device__ __forceinline__ T store(float f) { return f; }
  static __device__ __forceinline__ float round(float f) { return f; }
};

template <> struct Elem<SDQ_BFLOAT16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(T v) { return bf16_bits_to_f32(v); }
  static __device__ __forceinline__ T store(float f) { return f32_to_bf16_bits(f); }
  static __device__ __forceinline__ float round(float f) {
    return bf16_bits_to_f32(f32_to_bf16_bits(f));
  }
};

template <> struct Elem<SDQ_FLOAT16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(T v) { return f16_bits_to_f32(v); }
  static __device__ __forceinline__ T store(float f) { return f32_to_f16_bits(f); }
  static __device__ __forceinline__ float round(float f) {
    return f16_bits_to_f32(f32_to_f16_bits(f));
  }
};

// Eight consecutive activations as a bf16x8 MFMA operand, from any of the
// three float dtypes.  `p` must be 16-byte aligned for 16-bit types and
// 32-byte aligned for f32.
template <int DT> struct Load8;

template <> struct Load8<SDQ_BFLOAT16> {
  static __device__ __forceinline__ u32x4 get(const uint16_t *p) {
    return *reinterpret_cast<const u32x4 *>(p);
  }
};

template <> struct Load8<SDQ_FLOAT16> {
  static __device__ __forceinline__ u32x4 get(const uint16_t *p) {
    u32x4 v = *reinterpret_cast<const u32x4 *>(p);
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      r[i] = pack_bf16x2(f16_bits_to_f32(v[i] & 0xffffu), f16_bits_to_f32(v[i] >> 16));
    return r;
  }
};

template <> struct Load8<SDQ_FLOAT32> {
  static __device__ __forceinline__ u32x4 get(const float *p) {
    floatx4 a = *reinterpret_cast<const floatx4 *>(p);
    floatx4 b = *reinterpret_cast<const floatx4 *>(p + 4);
    u32x4 r;
    r[0] = pack_bf16x2(a[0], a[1]);
    r[1] = pack_bf16x2(a[2], a[3]);
    r[2] = pack_bf16x2(b[0], b[1]);
    r[3] = pack_bf16x2(b[2], b[3]);
    return r;
  }
};

// Buffer resources: a 32-bit byte window over a global array, addressed as
// (per-lane VGPR offset) + (uniform SGPR offset).  A pipelined loop then
// advances one scalar per step instead of 64-bit addresses per lane.
using Rsrc = __amdgpu_buffer_rsrc_t;

__device__ __forceinline__ Rsrc make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, int(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4 bload16(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

__device__ __forceinline__ uint32_t bload4(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

__device__ __forceinline__ uint32_t bload2(Rsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

// One scale or bias element through a buffer resource, widened to f32.
template <int DT> struct BLoadScalar;
template <> struct BLoadScalar<SDQ_FLOAT32> {
  static __device__ __forceinline__ float get(Rsrc r, uint32_t voff, uint32_t soff) {
    return __uint_as_float(bload4(r, voff, soff));
  }
};
template <> struct BLoadScalar<SDQ_BFLOAT16> {
  static __device__ __forceinline__ float get(Rsrc r, uint32_t voff, uint32_t soff) {
    return bf16_bits_to_f32(bload2(r, voff, soff));
  }
};
template <> struct BLoadScalar<SDQ_FLOAT16> {
  static __device__ __forceinline__ float get(Rsrc r, uint32_t voff, uint32_t soff) {
    return f16_bits_to_f32(bload2(r, voff, soff));
  }
};

// Eight consecutive activations at byte offset voff + soff as a bf16x8 MFMA
// operand (f16 and f32 are converted, rounding to nearest even).
template <int DT> struct BLoad8;
template <> struct BLoad8<SDQ_BFLOAT16> {
  static __device__ __forceinline__ u32x4 get(Rsrc r, uint32_t voff, uint32_t soff) {
    return bload16(r, voff, soff);
  }
};
template <> struct BLoad8<SDQ_FLOAT16> {
  static __device__ __forceinline__ u32x4 get(Rsrc r, uint32_t voff, uint32_t soff) {
    const u32x4 v = bload16(r, voff, soff);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t pair = v[i];
      o[i] = pack_bf16x2(f16_bits_to_f32(pair & 0xffffu), f16_bits_to_f32(pair >> 16));
    }
    return o;
  }
};
template <> struct BLoad8<SDQ_FLOAT32> {
  static __device__ __forceinline__ u32x4 get(Rsrc r, uint32_t voff, uint32_t soff) {
    const u32x4 a = bload16(r, voff, soff);
    const u32x4 b = bload16(r, voff + 16, soff);
    u32x4 o;
    o[0] = pack_bf16x2(__uint_as_float(a[0]), __uint_as_float(a[1]));
    o[1] = pack_bf16x2(__uint_as_float(a[2]), __uint_as_float(a[3]));
    o[2] = pack_bf16x2(__uint_as_float(b[0]), __uint_as_float(b[1]));
    o[3] = pack_bf16x2(__uint_as_float(b[2]), __uint_as_float(b[3]));
    return o;
  }
};

// 0.5 v (1 + tanh(u)), u = sqrt(2/pi) (v + 0.044715 v^3), through the identity
// 1 + tanh(u) = 2 (1 - r) for u >= 0 and 2 r' for u < 0, with
// r = 1 / (1 + exp(2|u|)): each branch keeps full relative precision (no
// cancellation near tanh = -1), exp from the hardware base-2 exponential
// and the reciprocal from the hardware reciprocal (both about 1 ulp).  The
// result stays within 5e-7 of the f32 formula with a correctly rounded tanh
// for |v| <= 8, and saturates cleanly (exp overflows to inf, r to 0).
__device__ __forceinline__ float gelu_approx_f(float v) {
  // sqrt(2 / pi) as the reference evaluates it in f32: sqrtf(2.0f / PI_f32),
  // one ulp below the correctly rounded constant.
  const float c = 0.7978845238685608f;
  const float k = 0.044715f;
  const float kTwoLog2e = 2.8853900817779268f; // 2 / ln 2
  const float u = (v + ((v * v) * v) * k) * c;
  const float e = __builtin_amdgcn_exp2f(fabsf(u) * kTwoLog2e);
  const float r = __builtin_amdgcn_rcpf(e + 1.0f);
  return u >= 0.0f ? v * (1.0f - r) : v * r;
}

// Bytes per element of a float dtype code.
__device__ __forceinline__ int dtype_size_dev(int dt) { return dt == SDQ_FLOAT32 ? 4 : 2; }

// One value of a float32/bfloat16/float16 array as f32.
__device__ __forceinline__ float epi_load(const void *p, int dtype, int64_t i) {
  if (dtype == SDQ_FLOAT32) return static_cast<const float *>(p)[i];
  const uint16_t h = static_cast<const uint16_t *>(p)[i];
  return dtype == SDQ_BFLOAT16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

// The matmul epilogue (kern::Epilogue) on one f32 result: bias of output
// column n, then the activation; the caller rounds once to the output dtype.
__device__ __forceinline__ float epi_bias(const kern::Epilogue &ep, int64_t n) {
  return ep.bias ? epi_load(ep.bias, ep.bias_dtype, n) : 0.0f;
}

__device__ __forceinline__ float epi_apply(const kern::Epilogue &ep, float v, float bias) {
  v += bias;
  return ep.act == 1 ? gelu_approx_f(v) : v;
}

// The output layout of the epilogue: where column n of row m goes, and the
// activation of that column (kern::Epilogue: y with row stride ldy, or y2
// for columns past the split).
template <typename OT>
__device__ __forceinline__ OT *epi_dst(const kern::Epilogue &ep, OT *y, int64_t N, int64_t m, int64_t n) {
  if (ep.split > 0 && n >= ep.split) return static_cast<OT *>(ep.y2) + m * ep.ldy2 + (n - ep.split);
  return y + m * (ep.ldy > 0 ? ep.ldy : N) + n;
}
__device__ __forceinline__ int epi_act(const kern::Epilogue &ep, int64_t n) {
  return ep.split > 0 && n >= ep.split ? ep.act2 : ep.act;
}
__device__ __forceinline__ float epi_apply_col(const kern::Epilogue &ep, float v, float bias, int64_t n) {
  v += bias;
  return epi_act(ep, n) == 1 ? gelu_approx_f(v) : v;
}

// The combine stage of the epilogue for output element (m, n).
__device__ __forceinline__ float epi_combine(const kern::Epilogue &ep, float v, int64_t m, int64_t n) {
  if (ep.combine == 0) return v;
  const float r = epi_load(ep.res, ep.res_dtype, m * ep.ld_res + n);
  if (ep.combine == 2) return v * r;
  const float g = ep.gate ? epi_load(ep.gate, ep.gate_dtype, n) : 1.0f;
  return fmaf(g, v, r);
}

// n consecutive values (n = 4 or 8) of a float32/bfloat16/float16 array at
// element i as f32; one or two 16-byte loads when `vec` (the caller has
// checked the alignment), single elements otherwise.
template <int NV>
__device__ __forceinline__ void epi_loadn(const void *p, int dtype, int64_t i, bool vec, float (&out)[NV]) {
  static_assert(NV == 4 || NV == 8, "4 or 8 values");
  if (!vec) {
#pragma unroll
    for (int k = 0; k < NV; ++k) out[k] = epi_load(p, dtype, i + k);
    return;
  }
  if (dtype == SDQ_FLOAT32) {
    const u32x4 *q = reinterpret_cast<const u32x4 *>(static_cast<const float *>(p) + i);
#pragma unroll
    for (int h = 0; h < NV / 4; ++h) {
      const u32x4 a = q[h];
#pragma unroll
      for (int k = 0; k < 4; ++k) out[4 * h + k] = __uint_as_float(a[k]);
    }
  } else {
    const uint16_t *base = static_cast<const uint16_t *>(p) + i;
    uint32_t w[NV / 2];
    if constexpr (NV == 8) {
      const u32x4 a = *reinterpret_cast<const u32x4 *>(base);
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = a[k];
    } else {
      const u32x2 a = *reinterpret_cast<const u32x2 *>(base);
      w[0] = a[0];
      w[1] = a[1];
    }
#pragma unroll
    for (int k = 0; k < NV / 2; ++k) {
      out[2 * k] = dtype == SDQ_BFLOAT16 ? bf16_bits_to_f32(w[k] & 0xffffu) : f16_bits_to_f32(w[k] & 0xffffu);
      out[2 * k + 1] = dtype == SDQ_BFLOAT16 ? bf16_bits_to_f32(w[k] >> 16) : f16_bits_to_f32(w[k] >> 16);
    }
  }
}

// The combine stage on NV consecutive outputs (m, n .. n + NV - 1), each
// already rounded to the output dtype (as the unfused sequence rounds the
// linear's result): y = r + g * v with one fused multiply-add, or v * r.
// `vec`: residual row and gate 16-byte aligned at n (checked by the caller).
template <int NV>
__device__ __forceinline__ void epi_combine_n(const kern::Epilogue &ep, int64_t m, int64_t n, bool vec,
                                              float (&v)[NV]) {
  float r[NV];
  epi_loadn<NV>(ep.res, ep.res_dtype, m * ep.ld_res + n, vec, r);
  if (ep.combine == 2) {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] *= r[k];
  } else if (!ep.gate) {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] += r[k];
  } else {
    float g[NV];
    epi_loadn<NV>(ep.gate, ep.gate_dtype, n, vec, g);
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = fmaf(g[k], v[k], r[k]);
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

} // namespace dev
} // namespace sdq
