/*
 * sdq_oracle_block.c -- CPU restatement of the ops around the Flux block
 * linears.
 *
 * TEST INFRASTRUCTURE ONLY (see sdq_oracle.h): the checker for the HIP
 * norm, rotary and attention kernels, never linked into libsdq.so.
 *
 * Restates:
 *   layer norm, no affine or with weight/bias   mlx.rs:1059-1085 (MLX's fast
 *       layer_norm, not vendored: the textbook (x - mean) / sqrt(var + eps)
 *       with the biased variance, statistics in f64)
 *   RMS norm                                    mlx.rs:1095-1115, and Flux's
 *       qk_norm composition flux.rs:322-327 (x * rsqrt(mean(x^2) + eps) * w)
 *   norm_modulate                               flux.rs:255-275
 *   rotate (interleaved RoPE)                   flux.rs:165-205, f32 ops in
 *       the composition's order: e*cos - o*sin, e*sin + o*cos
 *   embed_nd (the rotary tables)                flux.rs:126-156, f64 angles
 *   scaled dot-product attention                mlx.rs:1119-1197 (MLX's fast
 *       sdpa: softmax(scale q k^T + mask) v, restated in f64)
 * Pinning (tests/test_oracle_block.py): closed forms and invariants (zero
 * mean and unit variance, hand-worked rows, rotation by 0 and pi/2, pair
 * norms, uniform attention for q = 0, a one-hot key, the causal first row,
 * permutation of keys) and numpy's own softmax on small cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "sdq_oracle.h"

void sdo_layer_norm(const float *x, int64_t rows, int64_t C, float eps, const float *w, const float *b,
                    float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * C;
    double mean = 0.0, var = 0.0;
    for (int64_t c = 0; c < C; ++c) mean += xr[c];
    mean /= (double)C;
    for (int64_t c = 0; c < C; ++c) var += (xr[c] - mean) * (xr[c] - mean);
    var /= (double)C;
    const double rstd = 1.0 / sqrt(var + (double)eps);
    for (int64_t c = 0; c < C; ++c) {
      double t = (xr[c] - mean) * rstd;
      if (w) t *= w[c];
      if (b) t += b[c];
      out[r * C + c] = (float)t;
    }
  }
}

void sdo_rms_norm(const float *x, int64_t rows, int64_t C, float eps, const float *w, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * C;
    double ms = 0.0;
    for (int64_t c = 0; c < C; ++c) ms += (double)xr[c] * xr[c];
    ms /= (double)C;
    const double rr = 1.0 / sqrt(ms + (double)eps);
    for (int64_t c = 0; c < C; ++c) out[r * C + c] = (float)(xr[c] * rr * (w ? w[c] : 1.0));
  }
}

void sdo_norm_modulate(const float *x, int64_t B, int64_t N, int64_t C, float eps, const float *shift,
                       const float *scale, float *out) {
  sdo_layer_norm(x, B * N, C, eps, NULL, NULL, out);
  for (int64_t b = 0; b < B; ++b)
    for (int64_t n = 0; n < N; ++n)
      for (int64_t c = 0; c < C; ++c) {
        float *o = out + (b * N + n) * C + c;
        *o = (float)((double)*o * (1.0 + scale[b * C + c]) + shift[b * C + c]);
      }
}

void sdo_rope(const float *x, int64_t rows, int64_t D, int64_t N, const float *cs, const float *sn, float *out) {
  const int64_t half = D / 2;
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t n = r % N;
    for (int64_t i = 0; i < half; ++i) {
      const float e = x[r * D + 2 * i], o = x[r * D + 2 * i + 1];
      const float c = cs[n * half + i], s = sn[n * half + i];
      const float ec = e * c, os = o * s, es = e * s, oc = o * c;
      out[r * D + 2 * i] = ec - os;
      out[r * D + 2 * i + 1] = es + oc;
    }
  }
}

int sdo_embed_nd(const float *ids, int64_t seq, const int64_t *axes_dim, int64_t n_axes, float theta, float *cs,
                 float *sn) {
  int64_t half_total = 0;
  for (int64_t a = 0; a < n_axes; ++a) {
    if (axes_dim[a] % 2 != 0) return -1;
    half_total += axes_dim[a] / 2;
  }
  int64_t offset = 0;
  for (int64_t a = 0; a < n_axes; ++a) {
    const int64_t dim = axes_dim[a], half = dim / 2;
    for (int64_t t = 0; t < seq; ++t) {
      const double pos = ids[t * n_axes + a];
      for (int64_t i = 0; i < half; ++i) {
        const double omega = 1.0 / pow((double)theta, 2.0 * (double)i / (double)dim);
        const double angle = pos * omega;
        cs[t * half_total + offset + i] = (float)cos(angle);
        sn[t * half_total + offset + i] = (float)sin(angle);
      }
    }
    offset += half;
  }
  return 0;
}

int sdo_sdpa(const float *q, const float *k, const float *v, int64_t B, int64_t Hq, int64_t Hk, int64_t Nq,
             int64_t Nk, int64_t D, float scale, int mode, int64_t causal_offset, const float *mask, int64_t m_sb,
             int64_t m_sh, int64_t m_sq, float *out) {
  if (Hk <= 0 || Hq % Hk != 0 || Nk <= 0) return -1;
  double *p = (double *)malloc((size_t)Nk * sizeof(double));
  if (!p) return -1;
  const int64_t group = Hq / Hk;
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h) {
      const float *qh = q + (b * Hq + h) * Nq * D;
      const float *kh = k + (b * Hk + h / group) * Nk * D;
      const float *vh = v + (b * Hk + h / group) * Nk * D;
      for (int64_t i = 0; i < Nq; ++i) {
        double mx = -INFINITY;
        for (int64_t j = 0; j < Nk; ++j) {
          double s = 0.0;
          for (int64_t d = 0; d < D; ++d) s += (double)qh[i * D + d] * kh[j * D + d];
          s *= scale;
          if (mode == 2) s += mask[b * m_sb + h * m_sh + i * m_sq + j];
          if (mode == 1 && j > i + causal_offset) s = -INFINITY;
          p[j] = s;
          if (s > mx) mx = s;
        }
        double sum = 0.0;
        for (int64_t j = 0; j < Nk; ++j) {
          p[j] = p[j] == -INFINITY ? 0.0 : exp(p[j] - mx);
          sum += p[j];
        }
        for (int64_t d = 0; d < D; ++d) {
          double acc = 0.0;
          for (int64_t j = 0; j < Nk; ++j) acc += p[j] * vh[j * D + d];
          out[((b * Hq + h) * Nq + i) * D + d] = (float)(acc / sum);
        }
      }
    }
  free(p);
  return 0;
}
