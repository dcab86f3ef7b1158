/*
 * sdq_oracle_gguf.c -- CPU restatement of the reference's GGUF block decoders.
 *
 * TEST INFRASTRUCTURE ONLY (see sdq_oracle.h): the checker the HIP GGUF
 * kernels are compared against, never linked into libsdq.so.
 *
 * Restates, value for value, crates/sd-tensor/src/mlx_gguf.rs:
 *   block sizes                 mlx_gguf.rs:27-40, 81-92
 *   type ids                    mlx_gguf.rs:61-79
 *   f16_to_f32 (arithmetic form) mlx_gguf.rs:302-318
 *   bf16_to_f32 (a shift)       mlx_gguf.rs:296-298
 *   dequant_q4_0                mlx_gguf.rs:324-335
 *   dequant_q8_0                mlx_gguf.rs:337-344
 *   scale_min_k4                mlx_gguf.rs:351-360
 *   dequant_q4_k                mlx_gguf.rs:362-383
 *   dequant_q5_k                mlx_gguf.rs:385-409
 *   dequant_q6_k                mlx_gguf.rs:411-438
 * Every product and difference is one f32 operation in the reference's order
 * (Rust does not contract a*b-c into a fused multiply-add, and this file is
 * built with -ffp-contract=off), so the decoded values are the reference's
 * bit for bit.  NaN halves decode to the reference's canonical f32 NaN, and
 * every NaN a block's arithmetic produces is that NaN as well: on the
 * reference's platform (Apple arm64, default-NaN propagation) a NaN operand
 * passes through as the positive quiet NaN and inf*0 gives it too, where
 * x86 would give its negative "indefinite" NaN for the latter.
 *
 * Pinning (tests/test_oracle_gguf.py): the f16 decode against numpy's
 * float16 -> float32 over all 65536 patterns (the reference's own exhaustive
 * test, mlx_gguf.rs:464-475) and against the bit-construction decoder
 * sdo_f32_from_f16; bf16 against the reference's known answers
 * (mlx_gguf.rs:504-530); each block type against hand-worked blocks whose
 * values are written out in the test, and against an encoder written in the
 * test from the llama.cpp block layouts (pack, the inverse direction).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "sdq_oracle.h"

static float f32_of_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

int sdo_gguf_block(int type, int64_t *values, int64_t *bytes) {
  int64_t v, b;
  switch (type) {
  case SDO_GGML_F32: v = 1; b = 4; break;
  case SDO_GGML_F16: v = 1; b = 2; break;
  case SDO_GGML_BF16: v = 1; b = 2; break;
  case SDO_GGML_Q4_0: v = 32; b = 18; break;
  case SDO_GGML_Q8_0: v = 32; b = 34; break;
  case SDO_GGML_Q4_K: v = 256; b = 144; break;
  case SDO_GGML_Q5_K: v = 256; b = 176; break;
  case SDO_GGML_Q6_K: v = 256; b = 210; break;
  default: return -1;
  }
  if (values) *values = v;
  if (bytes) *bytes = b;
  return 0;
}

/* mlx_gguf.rs:302-318: sign * frac * 2^-24 for subnormals, sign * (1 +
 * frac/1024) * 2^(exp-15) for normals; every step is exact in f32. */
float sdo_gguf_f16(uint16_t h) {
  const float sign = (h >> 15) == 1 ? -1.0f : 1.0f;
  const int exp = (h >> 10) & 0x1f;
  const float frac = (float)(h & 0x3ff);
  if (exp == 0) return sign * frac * ldexpf(1.0f, -24);
  if (exp == 0x1f) return frac == 0.0f ? sign * INFINITY : f32_of_bits(0x7fc00000u);
  return sign * (1.0f + frac / 1024.0f) * ldexpf(1.0f, exp - 15);
}

static float canon_nan(float v) { return v != v ? f32_of_bits(0x7fc00000u) : v; }

static float half_at(const uint8_t *p) { return sdo_gguf_f16((uint16_t)(p[0] | (p[1] << 8))); }

/* mlx_gguf.rs:351-360 */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

static void q4_0(const uint8_t *blk, float *out) {
  const float d = half_at(blk);
  for (int i = 0; i < 16; ++i) {
    const uint8_t byte = blk[2 + i];
    out[i] = canon_nan(d * (float)((int)(byte & 0x0f) - 8));
    out[i + 16] = canon_nan(d * (float)((int)(byte >> 4) - 8));
  }
}

static void q8_0(const uint8_t *blk, float *out) {
  const float d = half_at(blk);
  for (int i = 0; i < 32; ++i) out[i] = canon_nan(d * (float)(int8_t)blk[2 + i]);
}

static void qk_45(const uint8_t *blk, float *out, int five) {
  const float d = half_at(blk);
  const float dmin = half_at(blk + 2);
  const uint8_t *scales = blk + 4;
  const uint8_t *qh = blk + 16;
  const uint8_t *qs = five ? blk + 48 : blk + 16;
  for (int j = 0; j < 8; ++j) {
    uint8_t sc, m;
    scale_min_k4(j, scales, &sc, &m);
    const float d1 = d * (float)sc;
    const float m1 = dmin * (float)m;
    const int half_idx = j / 2, shift = (j % 2) ? 4 : 0;
    for (int i = 0; i < 32; ++i) {
      uint32_t q = (uint32_t)(qs[half_idx * 32 + i] >> shift) & 0x0fu;
      if (five) q |= (uint32_t)((qh[i] >> j) & 1) << 4;
      const float t = d1 * (float)q;
      out[j * 32 + i] = canon_nan(t - m1);
    }
  }
}

static void q6_k(const uint8_t *blk, float *out) {
  const float d = half_at(blk + 208);
  for (int n = 0; n < 2; ++n) {
    const uint8_t *ql = blk + n * 64;
    const uint8_t *qh = blk + 128 + n * 32;
    const int8_t *sc = (const int8_t *)(blk + 192 + n * 8);
    for (int l = 0; l < 32; ++l) {
      const int is = l / 16;
      const int q1 = ((ql[l] & 0x0f) | ((qh[l] & 3) << 4)) - 32;
      const int q2 = ((ql[l + 32] & 0x0f) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      float *o = out + n * 128 + l;
      /* `d * (sc as i8) as f32 * q as f32` evaluates left to right. */
      o[0] = canon_nan((d * (float)sc[is]) * (float)q1);
      o[32] = canon_nan((d * (float)sc[is + 2]) * (float)q2);
      o[64] = canon_nan((d * (float)sc[is + 4]) * (float)q3);
      o[96] = canon_nan((d * (float)sc[is + 6]) * (float)q4);
    }
  }
}

int sdo_gguf_dequantize(const uint8_t *raw, size_t raw_bytes, int type, int64_t n, float *out) {
  int64_t per, bpb;
  if (sdo_gguf_block(type, &per, &bpb) != 0 || n < 0 || n % per != 0) return -1;
  const int64_t blocks = n / per;
  if ((uint64_t)(blocks * bpb) != (uint64_t)raw_bytes) return -1;
  for (int64_t b = 0; b < blocks; ++b) {
    const uint8_t *blk = raw + b * bpb;
    float *o = out + b * per;
    switch (type) {
    case SDO_GGML_F32: {
      uint32_t u = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8) | ((uint32_t)blk[2] << 16) |
                   ((uint32_t)blk[3] << 24);
      o[0] = f32_of_bits(u);
      break;
    }
    case SDO_GGML_F16: o[0] = half_at(blk); break;
    case SDO_GGML_BF16: o[0] = f32_of_bits((uint32_t)(blk[0] | (blk[1] << 8)) << 16); break;
    case SDO_GGML_Q4_0: q4_0(blk, o); break;
    case SDO_GGML_Q8_0: q8_0(blk, o); break;
    case SDO_GGML_Q4_K: qk_45(blk, o, 0); break;
    case SDO_GGML_Q5_K: qk_45(blk, o, 1); break;
    case SDO_GGML_Q6_K: q6_k(blk, o); break;
    }
  }
  return 0;
}
