/*
 * sdq_oracle.h -- CPU restatement of the MLX-affine quantized linear.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (libsdq.so) never links,
 * loads or calls it, and has no CPU fallback of any kind.
 *
 * What it restates (reference paths relative to andreinknv/stable-diffusion.rs):
 *   - SeededRng: splitmix64 + Box-Muller, cos then sin, f64 math cast to f32
 *       crates/sd-tensor/src/lib.rs:105-145
 *   - QuantizedArray::quantize / dequantize / matmul, mode "affine"
 *       crates/sd-tensor/src/mlx.rs:1856-1975 (the arithmetic itself lives in
 *       MLX's CPU backend, which is not vendored; restated below)
 *   - QuantizedArray::resident_bytes   crates/sd-tensor/src/mlx.rs:1977-1985
 *   - Array::gelu_approx               crates/sd-tensor/src/mlx.rs:1041-1054
 *   - GGUF block decoders (F32, F16, BF16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K)
 *       crates/sd-tensor/src/mlx_gguf.rs:27-438 (sdq_oracle_gguf.c)
 *   - layer/RMS norm, norm_modulate, RoPE, the rotary tables and attention
 *       mlx.rs:1059-1197, sd-models/src/mlx/flux.rs:125-327 (sdq_oracle_block.c)
 *
 * Pinning status of each function is recorded beside it and in the tests
 * (tests/test_oracle.py).  Every function here is checked there against
 * known-answer vectors, closed forms or brute force; none is "unpinned" with
 * respect to the written specification.  Byte equality with real MLX cannot
 * be checked anywhere (MLX is absent), so the specification choices are
 * listed at the top of sdq_oracle.c.
 *
 * dtype codes are the positions of mlx_dtype (crates/sd-tensor/src/mlx.rs:100-104):
 *   3 = uint32, 9 = float16, 10 = float32, 12 = bfloat16.
 */
#ifndef SDQ_ORACLE_H
#define SDQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { SDO_UINT32 = 3, SDO_FLOAT16 = 9, SDO_FLOAT32 = 10, SDO_BFLOAT16 = 12 };

/* ---- SeededRng (lib.rs:105-145) ---------------------------------------- */
uint64_t sdo_rng_next_u64(uint64_t *state);
double sdo_rng_next_f64(uint64_t *state);
/* Fills out[0..n) exactly as SeededRng::normals(n) does and advances state. */
void sdo_rng_normals(uint64_t *state, float *out, size_t n);

/* ---- 16-bit float storage helpers (round to nearest even) -------------- */
uint16_t sdo_bf16_from_f32(float f);
float sdo_f32_from_bf16(uint16_t h);
uint16_t sdo_f16_from_f32(float f);
float sdo_f32_from_f16(uint16_t h);
/* Round an f32 value to the given storage dtype and widen it back. */
float sdo_round_to(float v, int dtype);

/* ---- the path -------------------------------------------------------- */
/* w [rows, cols] given as f32 values (already exact widenings when the
 * source is bf16/f16).  Writes wq [rows, cols*bits/32] uint32 and
 * scales/biases [rows, cols/group_size] in store_dtype (f32: float*,
 * bf16/f16: uint16_t*).  Returns 0, or -1 on an invalid argument. */
int sdo_quantize(const float *w, int64_t rows, int64_t cols, int group_size,
                 int bits, int store_dtype, uint32_t *wq, void *scales,
                 void *biases);

/* out[r, c] = round_T(round_T(q * s) + b) with T = scale_dtype, returned
 * widened to f32.  Returns 0, or -1 on an invalid argument. */
int sdo_dequantize(const uint32_t *wq, const void *scales, const void *biases,
                   int scale_dtype, int64_t rows, int64_t cols, int group_size,
                   int bits, float *out);

/* y[m, n] = sum_k x[m, k] * w[n, k], w the f32 dequantized weight,
 * accumulated in f32 in increasing k (the order of MLX's CPU qmm_t).
 * x, scales, biases are f32 (MLX promotes x and the scales to one type). */
int sdo_qmatmul(const float *x, int64_t M, int64_t K, const uint32_t *wq,
                const float *scales, const float *biases, int64_t N,
                int group_size, int bits, float *y);

/* The same sums in f64 (an accuracy reference, not MLX's order). */
int sdo_qmatmul_f64(const float *x, int64_t M, int64_t K, const uint32_t *wq,
                    const float *scales, const float *biases, int64_t N,
                    int group_size, int bits, double *y);

/* sdo_qmatmul blocked over N and parallel over `threads` OpenMP threads.
 * Each output is the same f32 sum in the same k order, so the result is
 * bit-identical to sdo_qmatmul.  This is the timed CPU baseline. */
int sdo_qmatmul_omp(const float *x, int64_t M, int64_t K, const uint32_t *wq,
                    const float *scales, const float *biases, int64_t N,
                    int group_size, int bits, float *y, int threads);

/* Bytes a quantized weight holds (mlx.rs:1977-1985): packed words * 4 plus
 * (scales + biases) * 4. */
uint64_t sdo_resident_bytes(int64_t rows, int64_t cols, int group_size,
                            int bits);

/* 0.5*x*(1+tanh(sqrt(2/pi)*(x+0.044715*x^3))) evaluated op by op in f32 in the
 * order of mlx.rs:1048-1053. */
void sdo_gelu_approx(const float *x, float *y, size_t n);

/* ---- GGUF block decoding (sdq_oracle_gguf.c; mlx_gguf.rs:27-438) -------- */
/* GGML type ids as written in a GGUF file (mlx_gguf.rs:61-79). */
enum {
  SDO_GGML_F32 = 0, SDO_GGML_F16 = 1, SDO_GGML_Q4_0 = 2, SDO_GGML_Q8_0 = 8,
  SDO_GGML_Q4_K = 12, SDO_GGML_Q5_K = 13, SDO_GGML_Q6_K = 14, SDO_GGML_BF16 = 30
};
/* (values per block, bytes per block) of a type; -1 for an unsupported id. */
int sdo_gguf_block(int type, int64_t *values, int64_t *bytes);
/* The reference's f16 decoder (mlx_gguf.rs:302-318), in its arithmetic form. */
float sdo_gguf_f16(uint16_t h);
/* Decodes n values of `type` from raw (exactly n/values*bytes bytes) into
 * out, as Gguf::dequantize does (mlx_gguf.rs:235-276).  Returns 0, or -1 on
 * an unsupported type or a size mismatch. */
int sdo_gguf_dequantize(const uint8_t *raw, size_t raw_bytes, int type, int64_t n, float *out);

/* ---- the ops around the Flux block linears (sdq_oracle_block.c) -------- */
/* x, out: [rows, C] f32; w, b: C values or NULL.  Statistics in f64. */
void sdo_layer_norm(const float *x, int64_t rows, int64_t C, float eps, const float *w, const float *b,
                    float *out);
void sdo_rms_norm(const float *x, int64_t rows, int64_t C, float eps, const float *w, float *out);
/* x [B, N, C]; shift, scale [B, C]: layer_norm(x) * (1 + scale) + shift. */
void sdo_norm_modulate(const float *x, int64_t B, int64_t N, int64_t C, float eps, const float *shift,
                       const float *scale, float *out);
/* Interleaved RoPE of x [rows, D], row r at position r % N; cs, sn [N, D/2]. */
void sdo_rope(const float *x, int64_t rows, int64_t D, int64_t N, const float *cs, const float *sn, float *out);
/* Rotary tables [seq, sum(axes_dim)/2] of ids [seq, n_axes] (flux.rs:126-156). */
int sdo_embed_nd(const float *ids, int64_t seq, const int64_t *axes_dim, int64_t n_axes, float theta, float *cs,
                 float *sn);
/* softmax(scale q k^T + mask) v in f64; q [B,Hq,Nq,D], k, v [B,Hk,Nk,D];
 * mode 0 none, 1 causal (key j > i + causal_offset masked), 2 additive f32
 * mask at b*m_sb + h*m_sh + i*m_sq + j.  Returns 0, or -1 on bad sizes. */
int sdo_sdpa(const float *q, const float *k, const float *v, int64_t B, int64_t Hq, int64_t Hk, int64_t Nq,
             int64_t Nk, int64_t D, float scale, int mode, int64_t causal_offset, const float *mask, int64_t m_sb,
             int64_t m_sh, int64_t m_sq, float *out);

#ifdef __cplusplus
}
#endif

#endif
