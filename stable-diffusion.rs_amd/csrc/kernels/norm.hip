// norm.hip -- the row normalisations, the rotary embedding and the fused
// q/k/v preparation around the Flux block linears, for gfx950.
//
// Replaces, as single HBM passes:
//   mlx_fast_layer_norm / mlx_fast_rms_norm   crates/sd-tensor/src/mlx.rs:212-227, 1059-1115
//   norm_modulate: layer_norm(x) * (1 + scale) + shift
//                                             sd-models/src/mlx/flux.rs:255-275
//   rotate: interleaved RoPE                  flux.rs:165-205
//   split_qkv -> qk_norm -> rotate (q and k) and the V layout the attention
//   kernel reads                              flux.rs:300-327, 352-380, 446-460
//
// A row (one token's C channels, or one head's 128 dims) is held in one
// wave's registers: C/64 values per lane, so the mean, the variance and the
// output are one read and one write of HBM.  Statistics are f32 sums reduced
// across the wave with butterfly shuffles; each output is rounded once.
// Built with -ffp-contract=off: the rotation's products and sums are
// separately rounded f32 operations, as the reference's composition is.
#include <cmath>

#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

template <int DT> __device__ __forceinline__ void load8(const typename Elem<DT>::T *p, float (&v)[8]) {
  if constexpr (DT == SDQ_FLOAT32) {
    const floatx4 a = reinterpret_cast<const floatx4 *>(p)[0];
    const floatx4 b = reinterpret_cast<const floatx4 *>(p)[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[i + 4] = b[i];
    }
  } else {
    const u32x4 a = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = Elem<DT>::load(uint16_t(a[i] & 0xffffu));
      v[2 * i + 1] = Elem<DT>::load(uint16_t(a[i] >> 16));
    }
  }
}

template <int DT> __device__ __forceinline__ void store8(typename Elem<DT>::T *p, const float (&v)[8]) {
  if constexpr (DT == SDQ_FLOAT32) {
    reinterpret_cast<floatx4 *>(p)[0] = floatx4{v[0], v[1], v[2], v[3]};
    reinterpret_cast<floatx4 *>(p)[1] = floatx4{v[4], v[5], v[6], v[7]};
  } else {
    u32x4 a;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = uint32_t(Elem<DT>::store(v[2 * i])) | (uint32_t(Elem<DT>::store(v[2 * i + 1])) << 16);
    *reinterpret_cast<u32x4 *>(p) = a;
  }
}

enum { NORM_LAYER = 0, NORM_RMS = 1, NORM_MODULATE = 2 };

// One wave per row of C values, VPL values per lane (VPL = 8 * chunks): lane
// `lane` holds elements 8 * (64 j + lane) + 0..7 of chunk j.  vec: rows and
// parameter arrays are 16-byte aligned and C % 8 == 0; otherwise elements are
// moved one by one.
//   LAYER:    y = (x - mean) * rsqrt(var + eps) [* w] [+ b]
//   RMS:      y = x * rsqrt(mean(x^2) + eps) [* w]
//   MODULATE: y = (x - mean) * rsqrt(var + eps) * (1 + scale[g]) + shift[g],
//             g = row / rows_per_group (Flux's [batch, 1, C] modulation rows)
template <int XDT, int ODT, int PDT, int MODE, int VPL>
__global__ __launch_bounds__(kThreads) void norm_kernel(const typename Elem<XDT>::T *__restrict__ x,
                                                        typename Elem<ODT>::T *__restrict__ y, int64_t rows,
                                                        int C, float eps, const typename Elem<PDT>::T *__restrict__ w,
                                                        const typename Elem<PDT>::T *__restrict__ bshift,
                                                        int64_t rows_per_group, bool vec) {
  constexpr int kChunks = VPL / 8;
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const typename Elem<XDT>::T *xr = x + row * C;
  float v[kChunks][8];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c0 = 8 * (64 * j + lane);
    if (vec && c0 + 8 <= C) {
      load8<XDT>(xr + c0, v[j]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = c0 + e < C ? Elem<XDT>::load(xr[c0 + e]) : 0.0f;
    }
  }
  const float inv_c = 1.0f / float(C);
  float mean = 0.0f;
  if constexpr (MODE != NORM_RMS) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kChunks; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[j][e];
    mean = wave_sum(s) * inv_c;
  }
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c0 = 8 * (64 * j + lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = c0 + e < C ? v[j][e] - mean : 0.0f;
      ss += d * d;
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) * inv_c + eps);
  const typename Elem<PDT>::T *sc = nullptr, *sh = nullptr;
  if constexpr (MODE == NORM_MODULATE) {
    const int64_t g = row / rows_per_group;
    sc = w + g * C;
    sh = bshift + g * C;
  }
  typename Elem<ODT>::T *yr = y + row * C;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c0 = 8 * (64 * j + lane);
    if (c0 >= C) break;
    float o[8];
    if (vec && c0 + 8 <= C) {
      // Whole chunk: the parameters come in 16-byte pieces too (vec also
      // covers their alignment).
      float pm[8], pa[8];
      const typename Elem<PDT>::T *mul = MODE == NORM_MODULATE ? sc : w;
      const typename Elem<PDT>::T *add = MODE == NORM_MODULATE ? sh : (MODE == NORM_LAYER ? bshift : nullptr);
      if (mul) load8<PDT>(mul + c0, pm);
      if (add) load8<PDT>(add + c0, pa);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float t = (v[j][e] - mean) * rstd;
        if constexpr (MODE == NORM_MODULATE) {
          t = t * (1.0f + pm[e]) + pa[e];
        } else {
          if (mul) t = t * pm[e];
          if (add) t = t + pa[e];
        }
        o[e] = t;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = c0 + e < C ? c0 + e : C - 1;
        float t = (v[j][e] - mean) * rstd;
        if constexpr (MODE == NORM_MODULATE) {
          t = t * (1.0f + Elem<PDT>::load(sc[c])) + Elem<PDT>::load(sh[c]);
        } else {
          if (w) t = t * Elem<PDT>::load(w[c]);
          if (MODE == NORM_LAYER && bshift) t = t + Elem<PDT>::load(bshift[c]);
        }
        o[e] = t;
      }
    }
    if (vec && c0 + 8 <= C) {
      store8<ODT>(yr + c0, o);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (c0 + e < C) yr[c0 + e] = Elem<ODT>::store(o[e]);
    }
  }
}

// Interleaved rotary embedding (flux.rs:165-205): for pair i of a row of D
// values at position n, (e, o) = (x[2i], x[2i+1]) becomes
//   (e cos[n,i] - o sin[n,i],  e sin[n,i] + o cos[n,i]).
// x: [rows = B*H*N, D], cos/sin: [N, D/2] f32; one thread per pair.
template <int XDT>
__global__ __launch_bounds__(kThreads) void rope_kernel(const typename Elem<XDT>::T *__restrict__ x,
                                                        typename Elem<XDT>::T *__restrict__ y, int64_t pairs,
                                                        int half, int N, const float *__restrict__ cs,
                                                        const float *__restrict__ sn) {
  const int64_t p = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (p >= pairs) return;
  const int i = int(p % half);
  const int n = int((p / half) % N);
  const float e = Elem<XDT>::load(x[2 * p]), o = Elem<XDT>::load(x[2 * p + 1]);
  const float c = cs[int64_t(n) * half + i], s = sn[int64_t(n) * half + i];
  const float ec = e * c, os = o * s, es = e * s, oc = o * c;
  y[2 * p] = Elem<XDT>::store(ec - os);
  y[2 * p + 1] = Elem<XDT>::store(es + oc);
}

// Flux attention input (D = 128): token n of head hd from `qkv` rows laid
// out [3, H, D] along the last axis (split_qkv, flux.rs:300-310).  q and k:
// RMSNorm over the head (mean of squares + 1e-6, times the norm's scale,
// flux.rs:322-327), then the rotary embedding, written bf16 [B, H, N, D];
// v: written transposed, bf16 V^T [B, H, D, ldt].  Two sources a (tokens
// [0, na)) and b (tokens [na, na + nb)) with their own norm scales give the
// double block's text-then-image sequence (flux.rs:375-379).  Block = 32
// tokens of one head; each wave does 8 tokens, two dims per lane.
struct PrepSrc {
  const void *qkv = nullptr;
  int64_t ld = 0;    // elements between tokens
  int64_t sb = 0;    // elements between batch items
  const void *qn = nullptr;
  const void *kn = nullptr;
};

template <int XDT, int WDT>
__global__ __launch_bounds__(kThreads) void flux_prep_kernel(PrepSrc sa, PrepSrc sb, int na, int nb, int H,
                                                             float eps, const float *__restrict__ cs,
                                                             const float *__restrict__ sn, uint16_t *__restrict__ q,
                                                             uint16_t *__restrict__ k, uint16_t *__restrict__ vt,
                                                             int64_t ldt) {
  constexpr int D = 128;
  using XT = typename Elem<XDT>::T;
  using WT = typename Elem<WDT>::T;
  __shared__ uint16_t vtile[D][32 + 2];
  const int N = na + nb;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 32, hd = blockIdx.y, b = blockIdx.z;
  const int64_t qk_head = (int64_t(b) * H + hd) * N;
  for (int t = 0; t < 8; ++t) {
    const int tl = wave * 8 + t;
    const int n = n0 + tl;
    if (n >= N) {
      vtile[2 * lane][tl] = 0;
      vtile[2 * lane + 1][tl] = 0;
      continue;
    }
    const PrepSrc &src = n < na ? sa : sb;
    const int ns = n < na ? n : n - na;
    const XT *row = static_cast<const XT *>(src.qkv) + int64_t(b) * src.sb + int64_t(ns) * src.ld;
    const float c = cs[int64_t(n) * (D / 2) + lane], s = sn[int64_t(n) * (D / 2) + lane];
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const XT *xp = row + int64_t(part) * H * D + int64_t(hd) * D + 2 * lane;
      const float x0 = Elem<XDT>::load(xp[0]), x1 = Elem<XDT>::load(xp[1]);
      const float ms = wave_sum(x0 * x0 + x1 * x1) * (1.0f / D);
      const float rr = 1.0f / sqrtf(ms + eps);
      const WT *wn = static_cast<const WT *>(part == 0 ? src.qn : src.kn);
      const float e = (x0 * rr) * Elem<WDT>::load(wn[2 * lane]);
      const float o = (x1 * rr) * Elem<WDT>::load(wn[2 * lane + 1]);
      const float ec = e * c, os = o * s, es = e * s, oc = o * c;
      const uint32_t pair = uint32_t(f32_to_bf16_bits(ec - os)) | (uint32_t(f32_to_bf16_bits(es + oc)) << 16);
      uint16_t *dst = (part == 0 ? q : k) + (qk_head + n) * D + 2 * lane;
      *reinterpret_cast<uint32_t *>(dst) = pair;
    }
    const XT *vp = row + int64_t(2) * H * D + int64_t(hd) * D + 2 * lane;
    vtile[2 * lane][tl] = f32_to_bf16_bits(Elem<XDT>::load(vp[0]));
    vtile[2 * lane + 1][tl] = f32_to_bf16_bits(Elem<XDT>::load(vp[1]));
  }
  __syncthreads();
  // V^T: 128 rows of 32 tokens, as 16-byte pieces of 8 tokens.
  uint16_t *vdst = vt + (int64_t(b) * H + hd) * D * ldt;
  for (int pc = threadIdx.x; pc < D * 4; pc += kThreads) {
    const int d = pc / 4, c = pc % 4;
    if (n0 + 8 * c >= ldt) continue;
    u32x4 val;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      val[i] = uint32_t(vtile[d][8 * c + 2 * i]) | (uint32_t(vtile[d][8 * c + 2 * i + 1]) << 16);
    *reinterpret_cast<u32x4 *>(vdst + int64_t(d) * ldt + n0 + 8 * c) = val;
  }
}

// ---- host dispatch -----------------------------------------------------------

template <int XDT, int ODT, int PDT, int MODE>
void launch_norm_vpl(const void *x, void *y, int64_t rows, int C, float eps, const void *w, const void *b,
                     int64_t rpg, hipStream_t st) {
  using XT = typename Elem<XDT>::T;
  using OT = typename Elem<ODT>::T;
  using PT = typename Elem<PDT>::T;
  auto a16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool vec = C % 8 == 0 && a16(x) && a16(y) && (!w || a16(w)) && (!b || a16(b));
  const dim3 grid(unsigned((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  auto *xp = static_cast<const XT *>(x);
  auto *yp = static_cast<OT *>(y);
  auto *wp = static_cast<const PT *>(w);
  auto *bp = static_cast<const PT *>(b);
  // 8-value chunks per lane, rounded up to one of the instantiated counts.
  const int need = (C + 511) / 512;
  const int chunks = need <= 2 ? need : need <= 4 ? 4 : need <= 6 ? 6 : need <= 8 ? 8 : need <= 12 ? 12 : need <= 16 ? 16 : 0;
#define SDQ_NORM_CASE(NC)                                                                                   \
  case NC:                                                                                                  \
    norm_kernel<XDT, ODT, PDT, MODE, 8 * NC><<<grid, kThreads, 0, st>>>(xp, yp, rows, C, eps, wp, bp, rpg, vec); \
    break;
  switch (chunks) {
    SDQ_NORM_CASE(1)
    SDQ_NORM_CASE(2)
    SDQ_NORM_CASE(4)
    SDQ_NORM_CASE(6)
    SDQ_NORM_CASE(8)
    SDQ_NORM_CASE(12)
    SDQ_NORM_CASE(16)
  default:
    fail("norm: rows longer than 8192 values are not supported");
  }
#undef SDQ_NORM_CASE
}

template <int XDT, int ODT, int MODE>
void launch_norm_pdt(int pdt, const void *x, void *y, int64_t rows, int C, float eps, const void *w, const void *b,
                     int64_t rpg, hipStream_t st) {
  switch (pdt) {
  case SDQ_FLOAT32: launch_norm_vpl<XDT, ODT, SDQ_FLOAT32, MODE>(x, y, rows, C, eps, w, b, rpg, st); break;
  case SDQ_BFLOAT16: launch_norm_vpl<XDT, ODT, SDQ_BFLOAT16, MODE>(x, y, rows, C, eps, w, b, rpg, st); break;
  case SDQ_FLOAT16: launch_norm_vpl<XDT, ODT, SDQ_FLOAT16, MODE>(x, y, rows, C, eps, w, b, rpg, st); break;
  default: fail("norm: parameters must be float32, bfloat16 or float16");
  }
}

// The output has x's dtype.
template <int MODE>
void launch_norm(int xdt, int odt, int pdt, const void *x, void *y, int64_t rows, int C, float eps, const void *w,
                 const void *b, int64_t rpg, hipStream_t st) {
  if (odt != xdt) fail("norm: the output dtype must be the input's");
  switch (xdt) {
  case SDQ_FLOAT32: launch_norm_pdt<SDQ_FLOAT32, SDQ_FLOAT32, MODE>(pdt, x, y, rows, C, eps, w, b, rpg, st); break;
  case SDQ_BFLOAT16: launch_norm_pdt<SDQ_BFLOAT16, SDQ_BFLOAT16, MODE>(pdt, x, y, rows, C, eps, w, b, rpg, st); break;
  case SDQ_FLOAT16: launch_norm_pdt<SDQ_FLOAT16, SDQ_FLOAT16, MODE>(pdt, x, y, rows, C, eps, w, b, rpg, st); break;
  default: fail("norm: unsupported input dtype");
  }
}

template <int XDT, int WDT>
void launch_prep_w(const PrepSrc &a, const PrepSrc &b, int na, int nb, int B, int H, float eps, const float *cs,
                   const float *sn, uint16_t *q, uint16_t *k, uint16_t *vt, int64_t ldt, hipStream_t st) {
  const dim3 grid(unsigned(ldt / 32), unsigned(H), unsigned(B));
  flux_prep_kernel<XDT, WDT><<<grid, kThreads, 0, st>>>(a, b, na, nb, H, eps, cs, sn, q, k, vt, ldt);
}

template <int XDT>
void launch_prep(int wdt, const PrepSrc &a, const PrepSrc &b, int na, int nb, int B, int H, float eps,
                 const float *cs, const float *sn, uint16_t *q, uint16_t *k, uint16_t *vt, int64_t ldt,
                 hipStream_t st) {
  switch (wdt) {
  case SDQ_FLOAT32: launch_prep_w<XDT, SDQ_FLOAT32>(a, b, na, nb, B, H, eps, cs, sn, q, k, vt, ldt, st); break;
  case SDQ_BFLOAT16: launch_prep_w<XDT, SDQ_BFLOAT16>(a, b, na, nb, B, H, eps, cs, sn, q, k, vt, ldt, st); break;
  case SDQ_FLOAT16: launch_prep_w<XDT, SDQ_FLOAT16>(a, b, na, nb, B, H, eps, cs, sn, q, k, vt, ldt, st); break;
  default: fail("flux attention: norm scales must be float32, bfloat16 or float16");
  }
}

} // namespace

namespace kern {

void layer_norm(const void *x, int x_dtype, void *y, int y_dtype, int64_t rows, int C, float eps, const void *w,
                const void *b, int p_dtype, hipStream_t stream) {
  if (rows == 0 || C == 0) return;
  launch_norm<NORM_LAYER>(x_dtype, y_dtype, p_dtype, x, y, rows, C, eps, w, b, 1, stream);
  hip_check(hipGetLastError(), "layer_norm launch");
}

void rms_norm(const void *x, int x_dtype, void *y, int y_dtype, int64_t rows, int C, float eps, const void *w,
              int p_dtype, hipStream_t stream) {
  if (rows == 0 || C == 0) return;
  launch_norm<NORM_RMS>(x_dtype, y_dtype, p_dtype, x, y, rows, C, eps, w, nullptr, 1, stream);
  hip_check(hipGetLastError(), "rms_norm launch");
}

void norm_modulate(const void *x, int x_dtype, void *y, int y_dtype, int64_t rows, int C, float eps,
                   const void *shift, const void *scale, int p_dtype, int64_t rows_per_group, hipStream_t stream) {
  if (rows == 0 || C == 0) return;
  if (rows_per_group <= 0) fail("norm_modulate: bad group");
  launch_norm<NORM_MODULATE>(x_dtype, y_dtype, p_dtype, x, y, rows, C, eps, scale, shift, rows_per_group, stream);
  hip_check(hipGetLastError(), "norm_modulate launch");
}

void rope(const void *x, int x_dtype, void *y, int64_t rows, int D, int N, const float *cs, const float *sn,
          hipStream_t stream) {
  const int64_t pairs = rows * (D / 2);
  if (pairs == 0) return;
  if (D % 2 != 0) fail("rope: the last dimension must be even");
  const dim3 grid(unsigned((pairs + kThreads - 1) / kThreads));
  switch (x_dtype) {
  case SDQ_FLOAT32:
    rope_kernel<SDQ_FLOAT32><<<grid, kThreads, 0, stream>>>(static_cast<const float *>(x), static_cast<float *>(y),
                                                            pairs, D / 2, N, cs, sn);
    break;
  case SDQ_BFLOAT16:
    rope_kernel<SDQ_BFLOAT16><<<grid, kThreads, 0, stream>>>(static_cast<const uint16_t *>(x),
                                                             static_cast<uint16_t *>(y), pairs, D / 2, N, cs, sn);
    break;
  case SDQ_FLOAT16:
    rope_kernel<SDQ_FLOAT16><<<grid, kThreads, 0, stream>>>(static_cast<const uint16_t *>(x),
                                                            static_cast<uint16_t *>(y), pairs, D / 2, N, cs, sn);
    break;
  default: fail("rope: unsupported dtype");
  }
  hip_check(hipGetLastError(), "rope launch");
}

void flux_attention_prep(const FluxPrepSrc &a, const FluxPrepSrc &b, int x_dtype, int w_dtype, int na, int nb, int B,
                         int H, float eps, const float *cs, const float *sn, uint16_t *q, uint16_t *k, uint16_t *vt,
                         int64_t ldt, hipStream_t stream) {
  if (B == 0 || H == 0 || na + nb == 0) return;
  if (ldt % 32 != 0 || ldt < na + nb) fail("flux attention: bad V^T stride");
  PrepSrc pa{a.qkv, a.ld, a.sb, a.qn, a.kn}, pb{b.qkv, b.ld, b.sb, b.qn, b.kn};
  switch (x_dtype) {
  case SDQ_FLOAT32: launch_prep<SDQ_FLOAT32>(w_dtype, pa, pb, na, nb, B, H, eps, cs, sn, q, k, vt, ldt, stream); break;
  case SDQ_BFLOAT16: launch_prep<SDQ_BFLOAT16>(w_dtype, pa, pb, na, nb, B, H, eps, cs, sn, q, k, vt, ldt, stream); break;
  case SDQ_FLOAT16: launch_prep<SDQ_FLOAT16>(w_dtype, pa, pb, na, nb, B, H, eps, cs, sn, q, k, vt, ldt, stream); break;
  default: fail("flux attention: unsupported qkv dtype");
  }
  hip_check(hipGetLastError(), "flux attention prep launch");
}

} // namespace kern
} // namespace sdq
