/*
 * sdq_oracle.c -- CPU restatement of the MLX-affine quantized linear.
 *
 * TEST INFRASTRUCTURE ONLY (see sdq_oracle.h).  Build with -ffp-contract=off
 * and without -ffast-math: every f32 operation below is meant to be one IEEE
 * operation, rounded once, exactly as written.
 *
 * Specification choices (MLX is not vendored, so these restate MLX's CPU
 * backend as published; they are the contract the HIP kernels are held to
 * bit for bit):
 *   Q1  Per group of `group_size` values along the last axis, in f32:
 *         w_min, w_max (std::min / std::max semantics);
 *         scale = max((w_max - w_min) / n_bins, 1e-7f), n_bins = 2^bits - 1;
 *         if |w_min| > |w_max|: edge = w_min, else edge = w_max, scale = -scale;
 *         q0 = rint(edge / scale);
 *         if q0 != 0: scale = edge / q0, bias = edge; else bias = 0.
 *       The dominant edge of each group is therefore reconstructed exactly.
 *   Q2  code = clamp(rint((w - bias) / scale), 0, n_bins), rint = round half
 *       to even; codes are packed 32/bits per uint32, first element in the
 *       least significant bits.
 *   Q3  Codes are computed from the f32 scale and bias; the stored scale and
 *       bias are those values rounded to the weight's dtype.
 *   D1  dequantize: w = round_T(round_T(q * s) + b), T = the scales' dtype --
 *       a multiply and an add, each rounded, never fused.
 *   M1  quantized_matmul: x and the scales are promoted to one float type;
 *       each output is sum_k x[m,k] * w[n,k], w as in D1, accumulated in that
 *       type in increasing k.
 */
#include "sdq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- SeededRng: crates/sd-tensor/src/lib.rs:115-144 -------------------- */

uint64_t sdo_rng_next_u64(uint64_t *state) {
  /* lib.rs:115-121 */
  *state += 0x9E3779B97F4A7C15ULL;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

double sdo_rng_next_f64(uint64_t *state) {
  /* lib.rs:124-128: 53 bits, shifted off zero, so the result is in (0, 1].
   * The divisor 2^53 + 1 is not representable and rounds to 2^53 in f64, as
   * it does in the Rust source. */
  uint64_t bits = sdo_rng_next_u64(state) >> 11;
  return ((double)bits + 1.0) / (9007199254740992.0 + 1.0);
}

void sdo_rng_normals(uint64_t *state, float *out, size_t n) {
  /* lib.rs:131-144: Box-Muller, the cos draw first, then the sin draw. */
  const double tau = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    double u1 = sdo_rng_next_f64(state);
    double u2 = sdo_rng_next_f64(state);
    double r = sqrt(-2.0 * log(u1));
    double theta = tau * u2;
    out[i++] = (float)(r * cos(theta));
    if (i < n) out[i++] = (float)(r * sin(theta));
  }
}

/* ---- 16-bit storage formats --------------------------------------------- */

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t sdo_bf16_from_f32(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float sdo_f32_from_bf16(uint16_t h) { return bits_f32((uint32_t)h << 16); }

uint16_t sdo_f16_from_f32(float f) {
  uint32_t x = f32_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf or nan */
    uint32_t nan = ax > 0x7f800000u ? (0x0200u | ((ax >> 13) & 0x03ffu)) : 0u;
    return (uint16_t)(sign | 0x7c00u | nan);
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
  if (ax >= 0x38800000u) {                                   /* normal */
    ax += 0xc8000fffu + ((ax >> 13) & 1u);
    return (uint16_t)(sign | (ax >> 13));
  }
  /* subnormal: m * 2^-24, m = rint(|f| * 2^24); m == 1024 is the smallest
   * normal, whose encoding is the same integer. */
  float scaled = fabsf(f) * 16777216.0f;
  return (uint16_t)(sign | (uint32_t)rintf(scaled));
}

float sdo_f32_from_f16(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t m = (uint32_t)h & 0x03ffu;
  if (e == 0x1fu) return bits_f32(sign | 0x7f800000u | (m << 13));
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f); /* exact */
    return sign ? -v : v;
  }
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

float sdo_round_to(float v, int dtype) {
  switch (dtype) {
  case SDO_BFLOAT16:
    return sdo_f32_from_bf16(sdo_bf16_from_f32(v));
  case SDO_FLOAT16:
    return sdo_f32_from_f16(sdo_f16_from_f32(v));
  default:
    return v;
  }
}

static float load_scalar(const void *p, int dtype, int64_t i) {
  switch (dtype) {
  case SDO_BFLOAT16:
    return sdo_f32_from_bf16(((const uint16_t *)p)[i]);
  case SDO_FLOAT16:
    return sdo_f32_from_f16(((const uint16_t *)p)[i]);
  default:
    return ((const float *)p)[i];
  }
}

static void store_scalar(void *p, int dtype, int64_t i, float v) {
  switch (dtype) {
  case SDO_BFLOAT16:
    ((uint16_t *)p)[i] = sdo_bf16_from_f32(v);
    break;
  case SDO_FLOAT16:
    ((uint16_t *)p)[i] = sdo_f16_from_f32(v);
    break;
  default:
    ((float *)p)[i] = v;
  }
}

/* std::max / std::min, argument order included (they keep the first
 * argument on ties). */
static float max_std(float a, float b) { return (a < b) ? b : a; }
static float min_std(float a, float b) { return (b < a) ? b : a; }

static int valid_layout(int64_t rows, int64_t cols, int group_size, int bits) {
  if (rows < 0 || cols <= 0) return 0;
  if (group_size != 32 && group_size != 64 && group_size != 128) return 0;
  if (bits != 2 && bits != 4 && bits != 8) return 0;
  if (cols % group_size != 0) return 0;
  return 1;
}

static int valid_dtype(int d) {
  return d == SDO_FLOAT32 || d == SDO_BFLOAT16 || d == SDO_FLOAT16;
}

/* ---- quantize (spec Q1-Q3) ---------------------------------------------- */

int sdo_quantize(const float *w, int64_t rows, int64_t cols, int group_size,
                 int bits, int store_dtype, uint32_t *wq, void *scales,
                 void *biases) {
  if (!valid_layout(rows, cols, group_size, bits) || !valid_dtype(store_dtype))
    return -1;
  const float n_bins = (float)((1 << bits) - 1);
  const float eps = 1e-7f;
  const int per_word = 32 / bits;
  const int64_t groups = cols / group_size;
  const int64_t words_per_row = cols / per_word;
  const int words_per_group = group_size / per_word;

  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t g = 0; g < groups; ++g) {
      const float *src = w + r * cols + g * group_size;
      float w_min = INFINITY, w_max = -INFINITY;
      for (int j = 0; j < group_size; ++j) {
        w_max = max_std(w_max, src[j]);
        w_min = min_std(w_min, src[j]);
      }
      int mask = fabsf(w_min) > fabsf(w_max);
      float scale = max_std((w_max - w_min) / n_bins, eps);
      scale = mask ? scale : -scale;
      float edge = mask ? w_min : w_max;
      float q0 = rintf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      uint32_t *dst = wq + r * words_per_row + g * words_per_group;
      for (int j = 0; j < words_per_group; ++j) {
        uint32_t word = 0;
        for (int e = 0; e < per_word; ++e) {
          float v = src[j * per_word + e];
          v = rintf((v - bias) / scale);
          v = min_std(max_std(v, 0.0f), n_bins);
          word |= (uint32_t)v << (e * bits);
        }
        dst[j] = word;
      }
      store_scalar(scales, store_dtype, r * groups + g, scale);
      store_scalar(biases, store_dtype, r * groups + g, bias);
    }
  }
  return 0;
}

/* ---- dequantize (spec D1) ----------------------------------------------- */

int sdo_dequantize(const uint32_t *wq, const void *scales, const void *biases,
                   int scale_dtype, int64_t rows, int64_t cols, int group_size,
                   int bits, float *out) {
  if (!valid_layout(rows, cols, group_size, bits) || !valid_dtype(scale_dtype))
    return -1;
  const int per_word = 32 / bits;
  const uint32_t code_mask = (1u << bits) - 1u;
  const int64_t groups = cols / group_size;
  const int64_t words_per_row = cols / per_word;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      uint32_t word = wq[r * words_per_row + c / per_word];
      uint32_t q = (word >> ((c % per_word) * bits)) & code_mask;
      float s = load_scalar(scales, scale_dtype, r * groups + c / group_size);
      float b = load_scalar(biases, scale_dtype, r * groups + c / group_size);
      float p = sdo_round_to((float)q * s, scale_dtype);
      out[r * cols + c] = sdo_round_to(p + b, scale_dtype);
    }
  }
  return 0;
}

/* ---- quantized matmul (spec M1) ----------------------------------------- */

static float dequant_one(const uint32_t *row_words, const float *row_s,
                         const float *row_b, int64_t k, int group_size,
                         int bits) {
  const int per_word = 32 / bits;
  uint32_t q = (row_words[k / per_word] >> ((k % per_word) * bits)) &
               ((1u << bits) - 1u);
  float p = (float)q * row_s[k / group_size];
  return p + row_b[k / group_size];
}

int sdo_qmatmul(const float *x, int64_t M, int64_t K, const uint32_t *wq,
                const float *scales, const float *biases, int64_t N,
                int group_size, int bits, float *y) {
  if (M < 0 || N < 0 || !valid_layout(N, K, group_size, bits)) return -1;
  const int64_t words_per_row = K * bits / 32;
  const int64_t groups = K / group_size;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      const uint32_t *rw = wq + n * words_per_row;
      float sum = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        float wv = dequant_one(rw, scales + n * groups, biases + n * groups, k,
                               group_size, bits);
        float t = x[m * K + k] * wv;
        sum = sum + t;
      }
      y[m * N + n] = sum;
    }
  }
  return 0;
}

int sdo_qmatmul_f64(const float *x, int64_t M, int64_t K, const uint32_t *wq,
                    const float *scales, const float *biases, int64_t N,
                    int group_size, int bits, double *y) {
  if (M < 0 || N < 0 || !valid_layout(N, K, group_size, bits)) return -1;
  const int64_t words_per_row = K * bits / 32;
  const int64_t groups = K / group_size;
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      const uint32_t *rw = wq + n * words_per_row;
      double sum = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        float wv = dequant_one(rw, scales + n * groups, biases + n * groups, k,
                               group_size, bits);
        sum += (double)x[m * K + k] * (double)wv;
      }
      y[m * N + n] = sum;
    }
  }
  return 0;
}

/* Blocked form of sdo_qmatmul: a block of NB weight rows is dequantized into
 * a k-major buffer, then every output of the block is accumulated over k in
 * order with separate multiplies and adds -- the same operations as the
 * scalar loop, so the same bits, but vectorizable across the block. */
#define OMP_NB 32
int sdo_qmatmul_omp(const float *x, int64_t M, int64_t K, const uint32_t *wq,
                    const float *scales, const float *biases, int64_t N,
                    int group_size, int bits, float *y, int threads) {
  if (M < 0 || N < 0 || !valid_layout(N, K, group_size, bits)) return -1;
  const int64_t words_per_row = K * bits / 32;
  const int64_t groups = K / group_size;
  const int64_t nblocks = (N + OMP_NB - 1) / OMP_NB;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
#pragma omp parallel
  {
    float *wt = (float *)malloc(sizeof(float) * (size_t)K * OMP_NB);
#pragma omp for schedule(dynamic, 1)
    for (int64_t nb = 0; nb < nblocks; ++nb) {
      const int64_t n0 = nb * OMP_NB;
      const int64_t nn = (N - n0) < OMP_NB ? (N - n0) : OMP_NB;
      for (int64_t j = 0; j < OMP_NB; ++j) {
        const int64_t n = n0 + (j < nn ? j : 0);
        const uint32_t *rw = wq + n * words_per_row;
        for (int64_t k = 0; k < K; ++k)
          wt[k * OMP_NB + j] = dequant_one(rw, scales + n * groups,
                                           biases + n * groups, k, group_size,
                                           bits);
      }
      int64_t m = 0;
      for (; m + 2 <= M; m += 2) {
        float a0[OMP_NB], a1[OMP_NB];
        for (int j = 0; j < OMP_NB; ++j) a0[j] = a1[j] = 0.0f;
        const float *x0 = x + m * K, *x1 = x + (m + 1) * K;
        for (int64_t k = 0; k < K; ++k) {
          const float *wk = wt + k * OMP_NB;
          const float xa = x0[k], xb = x1[k];
          for (int j = 0; j < OMP_NB; ++j) {
            float ta = xa * wk[j];
            float tb = xb * wk[j];
            a0[j] = a0[j] + ta;
            a1[j] = a1[j] + tb;
          }
        }
        for (int64_t j = 0; j < nn; ++j) {
          y[m * N + n0 + j] = a0[j];
          y[(m + 1) * N + n0 + j] = a1[j];
        }
      }
      for (; m < M; ++m) {
        float a0[OMP_NB];
        for (int j = 0; j < OMP_NB; ++j) a0[j] = 0.0f;
        const float *x0 = x + m * K;
        for (int64_t k = 0; k < K; ++k) {
          const float *wk = wt + k * OMP_NB;
          const float xa = x0[k];
          for (int j = 0; j < OMP_NB; ++j) {
            float ta = xa * wk[j];
            a0[j] = a0[j] + ta;
          }
        }
        for (int64_t j = 0; j < nn; ++j) y[m * N + n0 + j] = a0[j];
      }
    }
    free(wt);
  }
  return 0;
}

uint64_t sdo_resident_bytes(int64_t rows, int64_t cols, int group_size,
                            int bits) {
  /* mlx.rs:1981-1984: packed words at 4 bytes, scales and biases counted at
   * 4 bytes each. */
  uint64_t words = (uint64_t)rows * (uint64_t)cols * (uint64_t)bits / 32u;
  uint64_t groups = (uint64_t)rows * (uint64_t)(cols / group_size);
  return words * 4u + 2u * groups * 4u;
}

void sdo_gelu_approx(const float *x, float *y, size_t n) {
  /* mlx.rs:1041-1054, one rounded f32 op at a time in that order. */
  const float half = 0.5f;
  const float one = 1.0f;
  const float c = sqrtf(2.0f / 3.14159265358979323846f);
  const float k = 0.044715f;
  for (size_t i = 0; i < n; ++i) {
    float v = x[i];
    float sq = v * v;
    float cubed = sq * v;
    float t = cubed * k;
    float u = v + t;
    float inner = tanhf(u * c);
    float a = v * half;
    y[i] = a * (inner + one);
  }
}
