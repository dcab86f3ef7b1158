// launch.hpp -- host-side launchers of the gfx950 kernels.  Each validates
// the shape facts its kernel's indexing assumes (the op layer has already
// checked the user-facing contract) and throws sdq::Error on failure.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sdq.h"

namespace sdq {
namespace kern {

// w [rows, cols] (w_dtype) -> wq [rows, cols*bits/32], scales/biases
// [rows, cols/group_size] in w_dtype.  quant.hip.
void quantize(const void *w, int w_dtype, int64_t rows, int64_t cols,
              int group_size, int bits, uint32_t *wq, void *scales,
              void *biases, hipStream_t stream);

// out [rows, cols] (out_dtype) = round_T(round_T(q*s) + b), T = s_dtype.
// quant.hip.
void dequantize(const uint32_t *wq, const void *scales, const void *biases,
                int s_dtype, int64_t rows, int64_t cols, int group_size,
                int bits, void *out, int out_dtype, hipStream_t stream);

// GGUF tensors (gguf.hip).  `raw` holds the tensor's GGML blocks as the file
// stores them (16-byte aligned, raw_bytes = n / values * bytes).
// (values, bytes) per block of GGML type `type`; false if unsupported.
bool gguf_block(int type, int64_t *values, int64_t *bytes);
// out[0..n) = the decoded f32 values (mlx_gguf.rs:235-276).
void gguf_dequantize(const uint8_t *raw, int type, int64_t n, int64_t raw_bytes, float *out,
                     hipStream_t stream);
// The decoded [rows, cols] tensor quantized as quantize() would quantize its
// f32 values: wq [rows, cols*bits/32], f32 scales/biases [rows, cols/group_size].
void gguf_quantize(const uint8_t *raw, int type, int64_t rows, int64_t cols, int64_t raw_bytes,
                   int group_size, int bits, uint32_t *wq, float *scales, float *biases,
                   hipStream_t stream);

// Output epilogue of the matmul kernels, applied to each f32 result before
// the output's rounding:
//   v = act(acc + bias[n])                      (bias optional, act 0 or GELU)
//   y = v                                        combine 0
//   y = res[m, n] + gate[n] * v                  combine 1 (gate optional: 1)
//   y = v * res[m, n]                            combine 2
// `bias` and `gate` are device pointers to N values, `res` to an [M, N]
// tensor with row stride `ld_res` elements; each of float32, bfloat16 or
// float16.  It fuses the calls that follow a quantized linear in the models:
// the bias add (quantized.rs:314-317), the Flux MLP's GELU (flux.rs:400-413),
// the gated residual x + gate * y (flux.rs:389-398, 414, 470) and T5's
// gelu(wi_0 x) * (wi_1 x) (t5.rs:209-214).  The small-M kernel applies the
// combine stage to the f32 value in its store; the large-M kernel applies it
// in its store (or its reduction kernel) to v rounded to the output dtype, as
// the unfused sequence does.
//
// Output layout: y has row stride ldy (0: N).  With split > 0 (a multiple of
// 256, below N) columns [split, N) go instead to y2, row stride ldy2, column
// n at y2 + (n - split), with activation act2 (Flux's single block: linear1's
// q/k/v columns to one buffer, its GELU'd MLP columns into linear2's input
// after the attention output, flux.rs:440-469).  No combine stage with a
// split.
//
// Gated pair (pair = 1): the weight's rows come in blocks of 16, eight rows
// of a gate projection then the matching eight of an up projection
// (quantize_pair); output column 8 b + i (of N / 2) is
// act(v[16 b + i]) * v[16 b + 8 + i], v = acc + bias: T5's
// gelu(wi_0 x) * (wi_1 x) (t5.rs:209-214) in one launch.  No split or
// combine stage with a pair; ldy applies to the N / 2 output columns.
struct Epilogue {
  const void *bias = nullptr;
  int bias_dtype = 0;
  int act = 0;
  const void *res = nullptr;
  int res_dtype = 0;
  int64_t ld_res = 0;
  const void *gate = nullptr;
  int gate_dtype = 0;
  int combine = 0;
  int64_t ldy = 0;
  int64_t split = 0;
  void *y2 = nullptr;
  int64_t ldy2 = 0;
  int act2 = 0;
  int pair = 0;
};

inline bool epi_dtype_ok(int dt) {
  return dt == SDQ_FLOAT32 || dt == SDQ_BFLOAT16 || dt == SDQ_FLOAT16;
}

inline bool epilogue_ok(const Epilogue &ep) {
  if (ep.bias && !epi_dtype_ok(ep.bias_dtype)) return false;
  if (ep.act != 0 && ep.act != 1) return false;
  if (ep.ldy < 0) return false;
  if (ep.split != 0) {
    if (ep.split < 0 || ep.split % 256 != 0 || !ep.y2 || ep.ldy2 < 1) return false;
    if (ep.act2 != 0 && ep.act2 != 1) return false;
    if (ep.combine != 0) return false;
  }
  if (ep.pair != 0 && (ep.pair != 1 || ep.split != 0 || ep.combine != 0)) return false;
  if (ep.combine == 0) return true;
  if (ep.combine != 1 && ep.combine != 2) return false;
  if (!ep.res || !epi_dtype_ok(ep.res_dtype)) return false;
  if (ep.gate && (ep.combine != 1 || !epi_dtype_ok(ep.gate_dtype))) return false;
  return true;
}

// Workspace the large-M kernel uses when it splits K across blocks: f32
// partial tiles (added by a second kernel, or by the stream-K owner blocks)
// and, for stream-K, one flag per worker, zero between launches.
struct SplitWorkspace {
  float *partial = nullptr;
  int *flags = nullptr;
};

// Launch plan of the small-M kernel: each block owns `tiles_per_block`
// tiles of 16 weight rows and all of K; each tile is streamed by `waves`
// waves over contiguous K ranges, whose partial tiles are added in LDS.
struct QmvPlan {
  int tiles_per_block = 1; // T
  int waves = 4;           // S: K ranges per tile (the block has T * S waves)
  int row_blocks = 1;      // 16-token MFMA row blocks: 1 for M <= 16, 2 for M <= 32
  int xmode = 1;           // where x comes from: 0 read per chunk, 1 staged per
                           // wave, 2 staged once per block, 3 a K range
                           // staged per block (ranges > 1 blocks per tile)
  int ranges = 1;          // R: K ranges across blocks (xmode 3)
  int row_groups = 1;      // blocks per tile group, each 16 rows of x (xmode 2,
                           // row_blocks 1; x of all M rows too large to stage)
  int lds_bytes = 0;       // dynamic LDS of one block
  size_t partial_floats = 0; // workspace for the ranges' partial tiles
};

// y [M, N] = x [M, K] @ dequantize(w).T for M <= 32 (up to 128 in row groups,
// see qmv_takes).  qmv.hip.  With
// allow_split false the plan needs no workspace (ranges == 1).
// Whether the small-M kernel takes an M x K activation against N weight
// rows: M <= 32, or up to 128 rows in row groups of 16 when 16 rows of x fit
// one block's stage and N is small (the large-M kernel has few tiles there).
bool qmv_takes(int64_t M, int64_t N, int64_t K);
QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int bits, int cus,
                 bool allow_split = true);
// partial: plan.partial_floats floats of workspace when plan.ranges > 1.
void qmv(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, const QmvPlan &plan, const Epilogue &ep, hipStream_t stream,
         float *partial = nullptr);

// Tile and split-K plan of one qmm launch (a pure function of the shape and
// the CU count).
struct QmmPlan {
  int bm = 256;             // rows per block tile (64, 128 or 256); tiles are bm x 256
  int tiles_n = 0;          // tiles along N
  int tiles = 0;            // all tiles, M-tile major
  int dp_tiles = 0;         // tiles [0, dp_tiles) are computed whole
  int splits = 1;           // K ranges of each later tile
  int steps_per_split = 0;  // 64-wide K steps per range
  int sk_workers = 0;       // > 0: stream-K over this many blocks (one per CU)
  int blocks = 0;           // grid size
  int tiles_m = 0;          // tiles along M
  int group_m = 1;          // tile order: groups of group_m tile rows, column by column
  int xcds = 1;             // L2 domains the hardware deals blocks to, round robin
  size_t partial_floats = 0; // workspace needed (0 without split tiles)
};

// y [M, N] = x [M, K] @ dequantize(w).T for any M.  qmm.hip.
// max_partial_floats caps the split-K workspace the plan may use (the
// no-allocation entry point's fixed scratch); a split that would need more
// is not taken.
QmmPlan plan_qmm(int64_t M, int64_t N, int64_t K, int bits, int cus,
                 size_t max_partial_floats = ~size_t(0), bool allow_stream_k = true);
// Zeroes `bytes` (a multiple of 4) at `p` with a kernel on `stream`.
void fill_zero(void *p, size_t bytes, hipStream_t stream);
void qmm(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, const QmmPlan &plan, const SplitWorkspace &ws, const Epilogue &ep,
         hipStream_t stream);

// Fused attention (attention.hip): out = softmax(scale q k^T [+ mask]) v.
// q, k: bf16 [B, H(k: H/group), N, D] rows of D contiguous elements (row
// strides q_sn / k_sn, head and batch strides *_sh / *_sb); vt: bf16 V^T
// [B, H/group, D, v_sd] with keys contiguous, v_sd a multiple of 64 and the
// padding keys zero; o: [B, H, Nq, D] by its strides, in the launch's output
// dtype.  mode 0: no mask; 1: causal (key <= query + causal_offset); 2: an
// additive mask of mask_dtype indexed [b * m_sb + h * m_sh + q * m_sq + key].
struct AttnArgs {
  const uint16_t *q = nullptr;
  const uint16_t *k = nullptr;
  const uint16_t *vt = nullptr;
  void *o = nullptr;
  int64_t q_sb = 0, q_sh = 0, q_sn = 0;
  int64_t k_sb = 0, k_sh = 0, k_sn = 0;
  int64_t v_sb = 0, v_sh = 0, v_sd = 0;
  int64_t o_sb = 0, o_sh = 0, o_sn = 0;
  int B = 0, H = 0, group = 1, Nq = 0, Nk = 0, D = 0;
  float scale_log2 = 0.0f; // scale * log2(e)
  int mode = 0;
  int causal_offset = 0;
  const void *mask = nullptr;
  int mask_dtype = 0;
  int64_t m_sb = 0, m_sh = 0, m_sq = 0;
  int q_blocks = 0; // set by attention()
};
void attention(const AttnArgs &a, int o_dtype, hipStream_t stream);
// The V^T row length attention() needs for nk keys.
int64_t attention_vt_stride(int64_t nk);
// V [bh, n, d] (float dtype, row stride ld, head stride v_sbh) -> bf16 V^T
// [bh, d, ldt] (head stride vt_sbh), keys [n, ldt) zero-filled.
void transpose_v(const void *v, int v_dtype, int64_t bh, int64_t n, int64_t d, int64_t v_sbh, int64_t ld,
                 uint16_t *vt, int64_t vt_sbh, int64_t ldt, hipStream_t stream);

// Row normalisations and the rotary embedding (norm.hip).  x, y: [rows, C]
// row-major (float32/bfloat16/float16); parameters of p_dtype.
// y = (x - mean) * rsqrt(var + eps) [* w] [+ b]   (w, b: C values or NULL)
void layer_norm(const void *x, int x_dtype, void *y, int y_dtype, int64_t rows, int C, float eps, const void *w,
                const void *b, int p_dtype, hipStream_t stream);
// y = x * rsqrt(mean(x^2) + eps) [* w]
void rms_norm(const void *x, int x_dtype, void *y, int y_dtype, int64_t rows, int C, float eps, const void *w,
              int p_dtype, hipStream_t stream);
// y = layer_norm(x) * (1 + scale[g]) + shift[g], g = row / rows_per_group;
// shift, scale: [groups, C].
void norm_modulate(const void *x, int x_dtype, void *y, int y_dtype, int64_t rows, int C, float eps,
                   const void *shift, const void *scale, int p_dtype, int64_t rows_per_group, hipStream_t stream);
// Interleaved rotary embedding of x [rows, D] whose row r is position
// r % N: pairs (x[2i], x[2i+1]) rotated by (cos, sin)[n, i]; cs, sn: [N, D/2] f32.
void rope(const void *x, int x_dtype, void *y, int64_t rows, int D, int N, const float *cs, const float *sn,
          hipStream_t stream);
// One source of the Flux attention input: qkv rows [B, n, >= 3*H*128]
// (token stride ld, batch stride sb, elements) and the q/k RMSNorm scales.
struct FluxPrepSrc {
  const void *qkv = nullptr;
  int64_t ld = 0, sb = 0;
  const void *qn = nullptr;
  const void *kn = nullptr;
};
// Tokens [0, na) from a, [na, na + nb) from b: q, k = rope(rms_norm(.) * scale)
// as bf16 [B, H, na + nb, 128]; v as bf16 V^T [B, H, 128, ldt] (ldt a multiple
// of 64, padding zero).  cs, sn: [na + nb, 64] f32.
void flux_attention_prep(const FluxPrepSrc &a, const FluxPrepSrc &b, int x_dtype, int w_dtype, int na, int nb, int B,
                         int H, float eps, const float *cs, const float *sn, uint16_t *q, uint16_t *k, uint16_t *vt,
                         int64_t ldt, hipStream_t stream);

// Elementwise helpers (elementwise.hip).  n = element count.
void astype(const void *a, int a_dtype, void *out, int out_dtype, int64_t n,
            hipStream_t stream);
// out = a + b; b has n elements (equal shapes) or `inner` elements broadcast
// along the last axis of a (inner = the last dimension).
void add(const void *a, int a_dtype, const void *b, int b_dtype, void *out,
         int out_dtype, int64_t n, int64_t b_n, hipStream_t stream);
void multiply(const void *a, int a_dtype, const void *b, int b_dtype,
              void *out, int out_dtype, int64_t n, hipStream_t stream);
void gelu_approx(const void *a, int dtype, void *out, int64_t n,
                 hipStream_t stream);

// y [M, N] = a [M, K] @ b [N, K].T, f32 accumulate; y in the promotion of
// the two dtypes.  dense.hip.
void matmul_nt(const void *a, int a_dtype, const void *b, int b_dtype, void *y,
               int64_t M, int64_t N, int64_t K, hipStream_t stream);

} // namespace kern
} // namespace sdq
