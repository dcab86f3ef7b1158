/*
 * sdq.h -- C ABI of libsdq, the MI355X (gfx950) backend for the MLX-affine
 * quantized linear of stable-diffusion.rs.
 *
 * The reference binds mlx-c by hand (crates/sd-tensor/src/mlx.rs:21-22,
 * 106-417) and reaches the quantized path through five groups of calls:
 * handles and dtypes, array lifecycle, streams/eval, the error handler, and
 * the three quantization ops.  Every entry point below replaces one of those
 * bindings one for one -- same argument order, same meaning, same
 * status/ownership rules -- so the Rust crate binds this header exactly as it
 * binds mlx-c today, with the prefix changed.  Each declaration cites the
 * binding it replaces.
 *
 * Conventions (mirroring mlx-c, as the reference relies on them):
 *   - handles are `struct { void* ctx; }` passed by value (mlx.rs:38-98);
 *   - ops return int status, 0 = success; on failure the message goes,
 *     synchronously and on the calling thread, to the handler installed with
 *     sdq_set_error_handler (mlx.rs:412-470), and the result is left as it was;
 *   - results come back through out-pointers; a result handle whose ctx is
 *     NULL gets a new array, an existing one is overwritten (mlx.rs:1923);
 *   - every handle returned is owned by the caller and released exactly once
 *     with its *_free (mlx.rs:1448-1452);
 *   - arrays live in device memory (HBM).  Ops are enqueued on the stream
 *     and run asynchronously; sdq_eval / sdq_synchronize / the data accessors
 *     are true device synchronisations, so MLX's lazy-then-eval semantics
 *     (mlx.rs:8-13, 1531-1544) hold for a caller;
 *   - there is no CPU backend.  A CPU stream is accepted as a handle (the
 *     reference creates one, mlx.rs:491-494) but every op submitted to it
 *     fails with a message; nothing silently falls back to host code.
 */
#ifndef SDQ_H
#define SDQ_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- handles: mlx.rs:38-98 ----------------------------------------------- */

/* replaces mlx_array (mlx.rs:38-42) */
typedef struct sdq_array_ {
  void *ctx;
} sdq_array;

/* replaces mlx_stream (mlx.rs:44-48) */
typedef struct sdq_stream_ {
  void *ctx;
} sdq_stream;

/* replaces mlx_vector_array (mlx.rs:50-54) */
typedef struct sdq_vector_array_ {
  void *ctx;
} sdq_vector_array;

/* replaces mlx_optional_int (mlx.rs:56-72): an int then a bool, by value */
typedef struct sdq_optional_int_ {
  int value;
  bool has_value;
} sdq_optional_int;

/* replaces mlx_optional_dtype (mlx.rs:74-80) */
typedef struct sdq_optional_dtype_ {
  int value;
  bool has_value;
} sdq_optional_dtype;

/* Positions are those of mlx_dtype (mlx.rs:100-104: INT32=7, FLOAT16=9,
 * FLOAT32=10), so the Rust constants carry over unchanged. */
typedef enum sdq_dtype_ {
  SDQ_BOOL = 0,
  SDQ_UINT8 = 1,
  SDQ_UINT16 = 2,
  SDQ_UINT32 = 3,
  SDQ_UINT64 = 4,
  SDQ_INT8 = 5,
  SDQ_INT16 = 6,
  SDQ_INT32 = 7,
  SDQ_INT64 = 8,
  SDQ_FLOAT16 = 9,
  SDQ_FLOAT32 = 10,
  SDQ_FLOAT64 = 11,
  SDQ_BFLOAT16 = 12,
  SDQ_COMPLEX64 = 13
} sdq_dtype;

/* ---- errors: mlx.rs:412-416 ------------------------------------------------ */

typedef void (*sdq_error_handler_func)(const char *msg, void *data);

/* replaces mlx_set_error_handler (mlx.rs:412-416).  Process-wide; NULL
 * restores the default handler (print to stderr).  The previous handler's
 * dtor, if any, is called on its data. */
void sdq_set_error_handler(sdq_error_handler_func handler, void *data,
                           void (*dtor)(void *));

/* ---- arrays: mlx.rs:106-121, 558-612 --------------------------------------- */

/* An empty handle (mlx-c's mlx_array_new). */
sdq_array sdq_array_new(void);
/* replaces mlx_array_new_data (mlx.rs:109-114): copies `data` (host memory,
 * row-major, shape[0..dim)) into a new device array.  On error the returned
 * ctx is NULL and the handler has the message (mlx.rs:572-577). */
sdq_array sdq_array_new_data(const void *data, const int *shape, int dim,
                             sdq_dtype dtype);
/* replaces mlx_array_new_float32 (mlx.rs:115): a 0-d f32 array. */
sdq_array sdq_array_new_float32(float val);
/* replaces mlx_array_free (mlx.rs:116) */
int sdq_array_free(sdq_array arr);
/* replaces mlx_array_size (mlx.rs:117) */
size_t sdq_array_size(sdq_array arr);
/* replaces mlx_array_ndim (mlx.rs:118) */
size_t sdq_array_ndim(sdq_array arr);
/* replaces mlx_array_shape (mlx.rs:119): valid while the array lives */
const int *sdq_array_shape(sdq_array arr);
/* replaces mlx_array_dtype (mlx.rs:120) */
sdq_dtype sdq_array_dtype(sdq_array arr);
size_t sdq_array_nbytes(sdq_array arr);
/* Waits for the work that produces `arr` (mlx-c's mlx_array_eval). */
int sdq_array_eval(sdq_array arr);
/* replaces mlx_array_data_float32 (mlx.rs:121): synchronises, copies the
 * contents to a host mirror owned by the array and returns it (valid until
 * the array is freed or written again).  NULL, with a message, if the dtype
 * is not float32. */
const float *sdq_array_data_float32(sdq_array arr);
/* The same for uint32 (packed weights) and for the 16-bit float types, whose
 * elements are returned as raw bit patterns. */
const uint32_t *sdq_array_data_uint32(sdq_array arr);
const uint16_t *sdq_array_data_bfloat16(sdq_array arr);
const uint16_t *sdq_array_data_float16(sdq_array arr);
/* Copies the contents to caller memory; nbytes must equal sdq_array_nbytes. */
int sdq_array_copy_to_host(void *dst, size_t nbytes, sdq_array arr);

/* ---- vectors of arrays: mlx.rs:341-342, 358-359, 398 ----------------------- */

sdq_vector_array sdq_vector_array_new(void);                     /* mlx.rs:342 */
sdq_vector_array sdq_vector_array_new_value(sdq_array val);      /* mlx.rs:341 */
int sdq_vector_array_append_value(sdq_vector_array vec, sdq_array val);
size_t sdq_vector_array_size(sdq_vector_array vec);              /* mlx.rs:358 */
int sdq_vector_array_get(sdq_array *res, sdq_vector_array vec,   /* mlx.rs:359 */
                         size_t index);
int sdq_vector_array_free(sdq_vector_array vec);                 /* mlx.rs:398 */

/* ---- streams and evaluation: mlx.rs:338-340, 399 ---------------------------- */

/* replaces mlx_default_gpu_stream_new (mlx.rs:338): a handle on the current
 * device's default HIP stream (one per device, created on first use, default
 * priority). */
sdq_stream sdq_default_gpu_stream_new(void);
/* replaces mlx_default_cpu_stream_new (mlx.rs:339).  See the note on the CPU
 * backend at the top of this file. */
sdq_stream sdq_default_cpu_stream_new(void);
/* A handle on a new HIP stream of its own on the current device. */
sdq_stream sdq_gpu_stream_new(void);
/* replaces mlx_stream_free (mlx.rs:340) */
int sdq_stream_free(sdq_stream s);
/* Blocks until everything enqueued on `s` has finished. */
int sdq_synchronize(sdq_stream s);
/* The hipStream_t behind a GPU stream (NULL for the CPU stream), for callers
 * that time or order work with HIP events of their own. */
void *sdq_stream_native(sdq_stream s);
/* replaces mlx_eval (mlx.rs:399): waits for the work producing each array. */
int sdq_eval(sdq_vector_array outputs);

/* ---- memory accounting: mlx.rs:405-411 ---------------------------------------- */

int sdq_get_active_memory(size_t *res);          /* mlx.rs:405 */
int sdq_get_peak_memory(size_t *res);            /* mlx.rs:406 */
int sdq_get_cache_memory(size_t *res);           /* mlx.rs:407 */
int sdq_reset_peak_memory(void);                 /* mlx.rs:408 */
int sdq_set_cache_limit(size_t *res, size_t limit); /* mlx.rs:410 */
int sdq_clear_cache(void);                       /* mlx.rs:411 */

/* ---- the quantized path: mlx.rs:361-397 -------------------------------------- */

/* replaces mlx_quantize (mlx.rs:363-371; called at mlx.rs:1871-1879).
 * w: [..., K] float32/bfloat16/float16, K % group_size == 0.
 * res: a vector of three arrays -- packed weight [..., K*bits/32] uint32,
 * scales and biases [..., K/group_size] in w's dtype.  group_size defaults to
 * 64 and may be 32, 64 or 128; bits defaults to 4 and may be 2, 4 or 8;
 * mode must be "affine" (or NULL); global_scale must be empty (ctx NULL). */
int sdq_quantize(sdq_vector_array *res, sdq_array w,
                 sdq_optional_int group_size, sdq_optional_int bits,
                 const char *mode, sdq_array global_scale, sdq_stream s);

/* replaces mlx_dequantize (mlx.rs:373-384; called at mlx.rs:1926-1940).
 * res: [..., K] in the scales' dtype, or in `dtype` when it has a value. */
int sdq_dequantize(sdq_array *res, sdq_array w, sdq_array scales,
                   sdq_array biases, sdq_optional_int group_size,
                   sdq_optional_int bits, const char *mode,
                   sdq_array global_scale, sdq_optional_dtype dtype,
                   sdq_stream s);

/* replaces mlx_quantized_matmul (mlx.rs:386-397; called at mlx.rs:1959-1970).
 * y = x @ dequantize(w).T for transpose == true (the only form the reference
 * uses, mlx.rs:1947-1951).  x: [..., K]; w [N, K*bits/32]; y: [..., N] in the
 * promotion of x's and the scales' dtypes.  transpose == false is rejected
 * with a message. */
int sdq_quantized_matmul(sdq_array *res, sdq_array x, sdq_array w,
                         sdq_array scales, sdq_array biases, bool transpose,
                         sdq_optional_int group_size, sdq_optional_int bits,
                         const char *mode, sdq_stream s);

/* Activations the matmul epilogue can apply. */
typedef enum sdq_activation_ {
  SDQ_ACT_NONE = 0,
  SDQ_ACT_GELU_APPROX = 1, /* Array::gelu_approx (mlx.rs:1041-1054) */
} sdq_activation;

/* quantized::linear's quantized branch (quantized.rs:293-318) with its bias
 * add, plus an optional activation, fused into the matmul's store:
 * y = act(x @ dequantize(w).T + bias).  It replaces the call sequence
 * mlx_quantized_matmul (quantized.rs:305-306) -> mlx_add (314-317) and, for
 * the Flux MLP, -> gelu_approx (flux.rs:400-413); the reference has no single
 * mlx-c call for it.  bias: a float array of N values, or a handle whose ctx
 * is NULL for none.  The sum and the activation are computed in f32 from the
 * f32 accumulator and rounded once to y's dtype (the unfused sequence rounds
 * after each op, so the two can differ by an output rounding step).  Other
 * arguments and errors as sdq_quantized_matmul with transpose = true. */
int sdq_quantized_linear(sdq_array *res, sdq_array x, sdq_array w,
                         sdq_array scales, sdq_array biases, sdq_array bias,
                         int activation, sdq_optional_int group_size,
                         sdq_optional_int bits, const char *mode, sdq_stream s);

/* How sdq_quantized_linear_combine merges the linear's output v with a
 * second [..., N] operand r (and an optional per-column gate g). */
typedef enum sdq_combine_ {
  SDQ_COMBINE_NONE = 0,
  SDQ_COMBINE_GATED_RESIDUAL = 1, /* y = r + g * v: Flux's x + gate * attn/mlp
                                   * (flux.rs:389-398, 414, 470); g = 1 if absent */
  SDQ_COMBINE_PRODUCT = 2,        /* y = v * r: T5's gelu(wi_0 x) * (wi_1 x)
                                   * (t5.rs:209-214), v being the wi_0 linear
                                   * with SDQ_ACT_GELU_APPROX */
} sdq_combine;

/* sdq_quantized_linear followed by the combine stage above:
 * it replaces the mlx_multiply / mlx_add calls the reference issues after the
 * linear at those call sites.  residual: the output's shape, any float
 * dtype; gate: N values or a NULL-ctx handle.  The whole epilogue runs in
 * the matmul's store (or in the reduction of split-K tiles): in the small-M
 * kernel (M <= 32, or up to 128 rows when N <= 4096 and K <= 3320) on the
 * f32 value; in the large-M kernel the combine stage takes v rounded to the
 * output dtype (as the unfused sequence does). */
int sdq_quantized_linear_combine(sdq_array *res, sdq_array x, sdq_array w,
                                 sdq_array scales, sdq_array biases,
                                 sdq_array bias, int activation,
                                 sdq_array residual, sdq_array gate,
                                 int combine, sdq_optional_int group_size,
                                 sdq_optional_int bits, const char *mode,
                                 sdq_stream s);

/* T5's gated feed-forward input, gelu_new(wi_0 x) * (wi_1 x) (t5.rs:201-214:
 * the two linears, gelu_approx and mlx_multiply), in one matmul launch over
 * both weights.  w/scales/biases: the two quantized weights with their rows
 * interleaved in blocks of eight (sdq_pair_rows on each of the three arrays):
 * 2 * N rows, N % 8 == 0.  y[..., N] = act(x @ gate.T + bias_g) * (x @ up.T +
 * bias_u), computed in f32 from the accumulators and rounded once to y's
 * dtype (the unfused sequence rounds after each of its four ops, so the two
 * differ by output rounding steps).  bias: 2 * N values in the paired row
 * order (sdq_pair_rows on the two biases), or a NULL-ctx handle; activation:
 * applied to the gate, SDQ_ACT_GELU_APPROX for T5.  No mlx-c counterpart. */
int sdq_quantized_linear_gated(sdq_array *res, sdq_array x, sdq_array w,
                               sdq_array scales, sdq_array biases,
                               sdq_array bias, int activation,
                               sdq_optional_int group_size,
                               sdq_optional_int bits, const char *mode,
                               sdq_stream s);

/* Rows of two equal-shaped arrays interleaved in blocks of eight: rows
 * 16 b .. 16 b + 7 of the result are gate's rows 8 b .. 8 b + 7 and rows
 * 16 b + 8 .. 16 b + 15 up's.  gate, up: the same shape [R, ...] (R a
 * positive multiple of 8) and dtype; res: [2 R, ...].  It builds the operands
 * of sdq_quantized_linear_gated once, at load time (packed weights, scales,
 * biases and the optional bias alike).  No mlx-c counterpart. */
int sdq_pair_rows(sdq_array *res, sdq_array gate, sdq_array up, sdq_stream s);

/* ---- elementwise ops the linear and its callers use ------------------------- */

/* replaces mlx_add (mlx.rs:124) for the shapes the quantized linear needs:
 * equal shapes, or b broadcast along the last axis of a (the bias add after
 * the matmul, quantized.rs:314-317). */
int sdq_add(sdq_array *res, sdq_array a, sdq_array b, sdq_stream s);
/* replaces mlx_multiply (mlx.rs:126), equal shapes (T5's gate, t5.rs:211) */
int sdq_multiply(sdq_array *res, sdq_array a, sdq_array b, sdq_stream s);
/* replaces mlx_astype (mlx.rs:149) between float32, bfloat16 and float16 */
int sdq_astype(sdq_array *res, sdq_array a, sdq_dtype dtype, sdq_stream s);
/* replaces mlx_contiguous (mlx.rs:150-155).  Arrays made here are always
 * row-major, so this is a copy. */
int sdq_contiguous(sdq_array *res, sdq_array a, bool allow_col_major,
                   sdq_stream s);
/* Array::gelu_approx (mlx.rs:1041-1054) as one fused op: the reference
 * composes it from mlx_multiply/add/tanh; the value is the same formula. */
int sdq_gelu_approx(sdq_array *res, sdq_array a, sdq_stream s);
/* a @ b.T with f32 accumulation: the dense linear `x @ w.T`
 * (sd-models/src/mlx/mod.rs:181-189), which the reference composes from
 * mlx_transpose_axes (mlx.rs:142) and mlx_matmul (mlx.rs:241).  a: [..., K],
 * b: [N, K]; result [..., N]. */
int sdq_matmul_nt(sdq_array *res, sdq_array a, sdq_array b, sdq_stream s);

/* ---- GGUF tensors: the quantized loader ------------------------------------ */

/* GGML type ids as a GGUF file writes them (mlx_gguf.rs:61-79). */
typedef enum sdq_ggml_type_ {
  SDQ_GGML_F32 = 0,
  SDQ_GGML_F16 = 1,
  SDQ_GGML_Q4_0 = 2,  /* 32 values: f16 d, 16 nibble bytes */
  SDQ_GGML_Q8_0 = 8,  /* 32 values: f16 d, 32 signed bytes */
  SDQ_GGML_Q4_K = 12, /* 256 values in 144 bytes */
  SDQ_GGML_Q5_K = 13, /* 256 values in 176 bytes */
  SDQ_GGML_Q6_K = 14, /* 256 values in 210 bytes */
  SDQ_GGML_BF16 = 30
} sdq_ggml_type;

/* replaces Gguf::dequantize (mlx_gguf.rs:235-276) followed by
 * Array::from_slice_f32 (quantized.rs:190-191): the block decoding runs on
 * the device.  raw: a uint8 array holding the tensor's bytes exactly as the
 * file stores them (the caller reads them at data_start + offset, as
 * mlx_gguf.rs:246-250 does); shape: the tensor's row-major shape (the file's
 * dimensions reversed, mlx_gguf.rs:97-104, 208).  res: float32 [shape], the
 * values of mlx_gguf.rs's decoders bit for bit.  Fails, naming the type, for
 * a type outside the set above, and when the element count is not a multiple
 * of the block size or the byte count does not match the shape. */
int sdq_gguf_dequantize(sdq_array *res, sdq_array raw, int ggml_type,
                        const int *shape, int ndim, sdq_stream s);

/* replaces the loader's sequence Gguf::dequantize -> Array::from_slice_f32
 * -> QuantizedArray::quantize (quantized.rs:190-196, 236-243): one kernel
 * decodes the blocks and quantizes the f32 values to the MLX-affine layout,
 * so the dense tensor is never written.  res: three arrays as sdq_quantize
 * returns them for a float32 matrix -- packed [..., K*bits/32] uint32, f32
 * scales and biases [..., K/group_size] -- equal to sdq_quantize of
 * sdq_gguf_dequantize's result.  Shape rules as sdq_quantize, type and size
 * rules as sdq_gguf_dequantize. */
int sdq_gguf_quantize(sdq_vector_array *res, sdq_array raw, int ggml_type,
                      const int *shape, int ndim, sdq_optional_int group_size,
                      sdq_optional_int bits, sdq_stream s);

/* ---- the ops around the linears in a Flux block ----------------------------- */

/* replaces mlx_fast_layer_norm (mlx.rs:219-227; Array::layer_norm,
 * mlx.rs:1059-1085): y = (x - mean) / sqrt(var + eps) [* weight] [+ bias]
 * over the last axis (at most 8192 values).  weight, bias: that many values
 * or a NULL-ctx handle.  y has x's dtype; statistics are f32. */
int sdq_fast_layer_norm(sdq_array *res, sdq_array x, sdq_array weight,
                        sdq_array bias, float eps, sdq_stream s);

/* replaces mlx_fast_rms_norm (mlx.rs:212-218; Array::rms_norm,
 * mlx.rs:1095-1115): y = x / sqrt(mean(x^2) + eps) [* weight]. */
int sdq_fast_rms_norm(sdq_array *res, sdq_array x, sdq_array weight,
                      float eps, sdq_stream s);

/* replaces mlx_fast_scaled_dot_product_attention (mlx.rs:228-238; Array::
 * sdpa / sdpa_causal / sdpa_masked, mlx.rs:1119-1197):
 * softmax(scale * q k^T [+ mask]) v.  queries [B, Hq, Nq, D], keys and
 * values [B, Hk, Nk, D] with Hq a multiple of Hk and D 64 or 128.
 * mask_mode "" or NULL: none; "causal": key j visible to query i when
 * j <= i + Nk - Nq; "array": mask_arr, a float additive mask broadcastable
 * to [B, Hq, Nq, Nk] over its leading axes.  sinks must be empty.  The
 * products run as bf16 MFMAs (inputs rounded to bf16) with f32 softmax and
 * accumulation; the result has the queries' dtype. */
int sdq_fast_scaled_dot_product_attention(sdq_array *res, sdq_array queries,
                                          sdq_array keys, sdq_array values,
                                          float scale, const char *mask_mode,
                                          sdq_array mask_arr, sdq_array sinks,
                                          sdq_stream s);

/* Flux's norm_modulate (flux.rs:255-275) as one pass:
 * y = layer_norm(x, eps) * (1 + scale) + shift, x [B, N, C] (C <= 8192),
 * shift and scale [B, 1, C] (a modulation triple's rows, flux.rs:279-299).
 * The reference composes mlx_fast_layer_norm, mlx_add and mlx_multiply; y
 * has x's dtype and is rounded once. */
int sdq_flux_norm_modulate(sdq_array *res, sdq_array x, sdq_array shift,
                           sdq_array scale, float eps, sdq_stream s);

/* Flux's interleaved rotary embedding `rotate` (flux.rs:165-205):
 * x [B, H, N, D], cos and sin [1, N, D/2] float32 (Rope, flux.rs:120-156);
 * pairs (x[2i], x[2i+1]) become (e cos - o sin, e sin + o cos).  y has x's
 * dtype. */
int sdq_flux_rope(sdq_array *res, sdq_array x, sdq_array cos, sdq_array sin,
                  sdq_stream s);

/* A Flux block's attention from its qkv linear output(s) to merged heads, as
 * one call: split_qkv -> qk_norm (RMS over each head, times the norm
 * scale) -> concat -> rotate -> sdpa -> merge_heads (flux.rs:300-327,
 * 352-381 for the double block, 446-461 for the single block).  qkv_a
 * [B, Na, >= 3*heads*128] holds q, k, v of each token in its first
 * 3*heads*128 columns ([3, heads, 128]); the single block passes linear1's
 * output, whose MLP columns follow.  qkv_b (NULL ctx for none) is the second
 * stream, appended after qkv_a along the tokens (the double block passes
 * text as a and image as b, flux.rs:375-379), with its own norm scales.
 * pe_cos/pe_sin: [1, Na+Nb, 64] float32.  Result [B, Na+Nb, heads*128] in
 * qkv_a's dtype.  q, k and v are rounded to bf16 for the attention's
 * MFMAs.  No mlx-c counterpart: the reference issues these as separate
 * calls. */
int sdq_flux_attention(sdq_array *res, sdq_array qkv_a, sdq_array q_norm_a,
                       sdq_array k_norm_a, sdq_array qkv_b, sdq_array q_norm_b,
                       sdq_array k_norm_b, sdq_array pe_cos, sdq_array pe_sin,
                       int heads, float scale, float eps, sdq_stream s);

/* The single block's linear1 through to linear2's input (flux.rs:440-465):
 * projected = linear1(x) (the quantized linear w/scales/biases plus bias);
 * its first 3*heads*128 columns go to the attention above (q/k norm, rope,
 * sdpa, merge_heads) and its remaining (MLP) columns through gelu_approx;
 * the result is concat([attention, gelu(mlp)], axis 2), [B, T, heads*128 +
 * mlp].  One matmul launch writes both parts (the MLP part straight into the
 * result, GELU applied in its epilogue to the f32 value, so it can differ
 * from the unfused sequence by one rounding), then the attention writes the
 * result's first columns.  x [B, T, hidden]; 3*heads*128 must be a multiple
 * of 256 (an even head count).  No mlx-c counterpart. */
int sdq_flux_single_linear1_attention(sdq_array *res, sdq_array x, sdq_array w,
                                      sdq_array scales, sdq_array biases, sdq_array bias,
                                      sdq_optional_int group_size, sdq_optional_int bits,
                                      const char *mode, sdq_array q_norm, sdq_array k_norm,
                                      sdq_array pe_cos, sdq_array pe_sin, int heads,
                                      float scale, float eps, sdq_stream s);

/* ---- raw-pointer entry point ------------------------------------------------- */

/* The kernel behind sdq_quantized_matmul on caller-owned device memory:
 * y[M, N] (y_dtype) = x[M, K] (x_dtype, row stride ldx elements) @
 * dequantize(w[N, K*bits/32], scales/biases[N, K/group_size] (s_dtype)).T,
 * enqueued on `hip_stream` (a hipStream_t; NULL = the default stream).  The
 * dtypes must be float32, bfloat16 or float16; y_dtype is free.  Scratch
 * memory, when a shape needs it, comes from the library's cache. */
int sdq_quantized_matmul_raw(void *y, int y_dtype, const void *x, int x_dtype,
                             int64_t ldx, const uint32_t *w,
                             const void *scales, const void *biases,
                             int s_dtype, int64_t M, int64_t N, int64_t K,
                             int group_size, int bits, void *hip_stream);

/* sdq_quantized_matmul_raw with sdq_quantized_linear's epilogue:
 * y = act(x @ dequantize(w).T + bias) on caller-owned device memory.  bias:
 * N values of bias_dtype (float32/bfloat16/float16), or NULL for none;
 * activation: an sdq_activation. */
int sdq_quantized_matmul_epilogue_raw(void *y, int y_dtype, const void *x,
                                      int x_dtype, int64_t ldx,
                                      const uint32_t *w, const void *scales,
                                      const void *biases, int s_dtype,
                                      int64_t M, int64_t N, int64_t K,
                                      int group_size, int bits,
                                      const void *bias, int bias_dtype,
                                      int activation, void *hip_stream);

/* sdq_quantized_matmul_epilogue_raw for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  It has no counterpart in the reference (MLX allocates
 * its own scratch).  Same arguments, validation and results to the north
 * star's tolerance; it calls no hipMalloc, hipFree or allocating library
 * routine.  The large-M kernel's split-K partial tiles live in a fixed
 * 16 MiB scratch array per GPU, held until the process ends; the launch
 * planner takes no split that would need more (so the summation order, and
 * the last bits of the result, may differ from the allocating entry point's
 * for some shapes).  All calls on one GPU share that array: calls that
 * overlap on one GPU (on different streams, or from several threads) race;
 * calls ordered on one stream do not. */
int sdq_quantized_matmul_noalloc(void *y, int y_dtype, const void *x, int x_dtype,
                                 int64_t ldx, const uint32_t *w, const void *scales,
                                 const void *biases, int s_dtype, int64_t M,
                                 int64_t N, int64_t K, int group_size, int bits,
                                 const void *bias, int bias_dtype, int activation,
                                 void *hip_stream);

/* sdq_quantized_matmul_epilogue_raw writing its output to two places:
 * columns [0, split) to y (row stride ldy elements, activation), columns
 * [split, N) to y2 (row stride ldy2, column n at y2 + (n - split),
 * activation2).  split is a multiple of 256 inside (0, N).  It replaces the
 * narrow / gelu_approx / concat calls after Flux's single-block linear1
 * (flux.rs:440-469: q, k, v columns to the attention, GELU'd MLP columns
 * into linear2's input after the attention output).  No mlx-c counterpart:
 * the reference issues those calls separately. */
int sdq_quantized_linear_split_raw(void *y, int64_t ldy, int activation, void *y2,
                                   int64_t ldy2, int activation2, int64_t split,
                                   int y_dtype, const void *x, int x_dtype, int64_t ldx,
                                   const uint32_t *w, const void *scales,
                                   const void *biases, int s_dtype, int64_t M,
                                   int64_t N, int64_t K, int group_size, int bits,
                                   const void *bias, int bias_dtype, void *hip_stream);

/* sdq_quantized_linear_gated on caller-owned device memory: y[M, N / 2] (row
 * stride ldy elements, 0 = N / 2) from the paired weight w[N, K*bits/32]
 * (N % 16 == 0, rows as sdq_pair_rows lays them out); bias: N values in the
 * paired order, or NULL.  Other arguments as
 * sdq_quantized_matmul_epilogue_raw. */
int sdq_quantized_linear_gated_raw(void *y, int64_t ldy, int y_dtype,
                                   const void *x, int x_dtype, int64_t ldx,
                                   const uint32_t *w, const void *scales,
                                   const void *biases, int s_dtype, int64_t M,
                                   int64_t N, int64_t K, int group_size,
                                   int bits, const void *bias, int bias_dtype,
                                   int activation, void *hip_stream);

/* tanh-GELU on caller-owned device memory (dtype float32/bfloat16/float16),
 * enqueued on `hip_stream`: the elementwise step between the two Flux MLP
 * linears (flux.rs:400-413) without an array handle. */
int sdq_gelu_approx_raw(void *out, const void *in, int dtype, int64_t n,
                        void *hip_stream);

/* The device address of an array's data (valid while the array lives), for
 * callers that pass it to the raw entry points or to other HIP code.  Has no
 * mlx-c counterpart: MLX arrays live in unified memory. */
void *sdq_array_device_ptr(sdq_array arr);

/* ---- library information ----------------------------------------------------- */

/* "sdq <version> gfx950" */
const char *sdq_version(void);
/* Number of HIP devices visible (0 when none); never fails. */
int sdq_device_count(void);

#ifdef __cplusplus
}
#endif

#endif /* SDQ_H */
