// qmv.hip -- y = x @ dequantize(w).T for few rows of x (M <= 32): the
// bandwidth-bound decode/modulation shape of mlx_quantized_matmul
// (crates/sd-tensor/src/mlx.rs:386-397, 1947-1975; callers e.g. the Flux
// modulation linears at M = 1, sd-models/src/mlx/flux.rs:279-299, 437).
//
// Time here is the packed weight stream, so the kernel is built to keep VALU
// work per weight element small enough that HBM stays the bound:
//
//   * Codes are never dequantized element by element.  For one 64-wide step
//     of K (one group at group size 64; half a group at 128) the MFMA
//     computes t[m][n] = sum_k x[m,k] * c_k with c_k = q_k + OFF held EXACTLY
//     in bf16 (4-bit: OFF = 128 and the bf16 pattern 0x4300|q is built with
//     one byte-permute and one and-or per pair; 8-bit: OFF = 0, q converted).
//     Then y += s * t + (b - OFF*s) * X, where X[m] = sum_k x[m,k] over the
//     step.  That is the affine dequantization applied once per group per
//     output instead of once per weight, and it is more accurate than
//     rounding each dequantized weight to bf16.
//   * One wave owns 32 weight rows (the MFMA's N side) and walks K in 64-wide
//     steps; a block's four waves interleave the steps of the block's K range
//     and are summed through LDS.  When there are too few 32-row tiles to
//     fill the chip, K is split across blocks as well and the last block of a
//     tile (found with an atomic counter) adds the partial sums in split
//     order, so the result is deterministic.
//   * MFMA v_mfma_f32_32x32x16_bf16 with the tokens on the M side (rows
//     >= M are zero).  Lane (r, h) = (lane % 32, lane / 32) feeds token r and
//     weight row r; its eight K elements of k-step i are
//     k = 64*step + 32*h + 8*i + e, so each lane's weight bytes for a step
//     are one contiguous 16 B (4-bit) or 32 B (8-bit) load and its
//     activations one contiguous 64 B run.
#include <algorithm>

#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kThreads = 256;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Eight 4-bit codes of `wd`, in element order, as bf16 (128 + q): exact.
__device__ __forceinline__ u32x4 codes4_plus128(uint32_t wd) {
  const uint32_t s4 = wd >> 4;
  u32x4 r;
  // byte 0 <- wd.byte[d] (low nibble q[2d]), byte 2 <- s4.byte[d] (low
  // nibble q[2d+1]), bytes 1 and 3 <- 0; then keep the nibbles and set the
  // bf16 exponent of 128.
  r[0] = (__builtin_amdgcn_perm(s4, wd, 0x0C040C00u) & 0x000F000Fu) | 0x43004300u;
  r[1] = (__builtin_amdgcn_perm(s4, wd, 0x0C050C01u) & 0x000F000Fu) | 0x43004300u;
  r[2] = (__builtin_amdgcn_perm(s4, wd, 0x0C060C02u) & 0x000F000Fu) | 0x43004300u;
  r[3] = (__builtin_amdgcn_perm(s4, wd, 0x0C070C03u) & 0x000F000Fu) | 0x43004300u;
  return r;
}

// Eight 8-bit codes (two words), in element order, as bf16 q: exact.
__device__ __forceinline__ u32x4 codes8(uint32_t w0, uint32_t w1) {
  u32x4 r;
  r[0] = pack_bf16x2(float(w0 & 0xffu), float((w0 >> 8) & 0xffu));
  r[1] = pack_bf16x2(float((w0 >> 16) & 0xffu), float(w0 >> 24));
  r[2] = pack_bf16x2(float(w1 & 0xffu), float((w1 >> 8) & 0xffu));
  r[3] = pack_bf16x2(float((w1 >> 16) & 0xffu), float(w1 >> 24));
  return r;
}

template <int BITS, int XDT, int SDT> struct Stage {
  u32x4 w[BITS / 4]; // this lane's half-row of the step: 16 B or 32 B
  float s, b;
  u32x4 x[4];        // bf16 activations of the four k-steps
};

template <int BITS, int XDT, int SDT, int ODT, int MROWS, int GS>
__global__ __launch_bounds__(kThreads) void qmv_kernel(
    typename Elem<ODT>::T *__restrict__ y, const typename Elem<XDT>::T *__restrict__ x,
    int64_t ldx, const uint32_t *__restrict__ w,
    const typename Elem<SDT>::T *__restrict__ scales,
    const typename Elem<SDT>::T *__restrict__ biases, int M, int N, int K,
    int steps_per_split, float *__restrict__ partial, unsigned *__restrict__ counters) {
  using XT = typename Elem<XDT>::T;
  using ST = typename Elem<SDT>::T;
  constexpr float kOff = BITS == 4 ? 128.0f : 0.0f;
  constexpr int kWordsPerStep = 64 * BITS / 32; // 8 or 16
  constexpr int kHalfWords = kWordsPerStep / 2;
  constexpr int kAcc = MROWS / 2; // accumulator entries holding rows < MROWS

  const int steps = K / 64;
  const int groups = K / GS;
  const int tile = blockIdx.x;
  const int split = blockIdx.y;
  const int nsplit = gridDim.y;
  const int s_begin = split * steps_per_split;
  const int s_end = min(steps, s_begin + steps_per_split);
  const int ns = s_end - s_begin;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 31;
  const int h = lane >> 5;

  extern __shared__ float smem[];
  float *xsum = smem;                 // [ns][MROWS]
  float *red = smem + ns * MROWS;     // [4][MROWS][32]

  // 1. Per-step activation sums over this block's K range, of the bf16
  //    values the MFMA multiplies (dot2 against (1, 1)).
  {
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
    for (int p = tid; p < ns * M; p += kThreads) {
      const int sl = p / M;
      const int m = p - sl * M;
      const XT *src = x + int64_t(m) * ldx + int64_t(s_begin + sl) * 64;
      float sum = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const u32x4 v = Load8<XDT>::get(src + 8 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // Copy the element out first: bit-casting a vector-element
          // expression directly reinterprets element 0 instead.
          const uint32_t pair = v[j];
          sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), ones, sum, false);
        }
      }
      xsum[sl * MROWS + m] = sum;
    }
    for (int p = tid; p < ns * (MROWS - M); p += kThreads) {
      const int sl = p / (MROWS - M);
      xsum[sl * MROWS + M + (p - sl * (MROWS - M))] = 0.0f;
    }
  }
  __syncthreads();

  // 2. This wave's steps.
  const int n = tile * 32 + r;
  const int nrow = n < N ? n : N - 1; // rows past N are read, never stored
  const uint32_t *wrow = w + int64_t(nrow) * (int64_t(K) * BITS / 32) + h * kHalfWords;
  const ST *srow = scales + int64_t(nrow) * groups;
  const ST *brow = biases + int64_t(nrow) * groups;
  const bool xvalid = r < M;
  const XT *xrow = x + int64_t(xvalid ? r : 0) * ldx + 32 * h;

  auto load_stage = [&](int step, Stage<BITS, XDT, SDT> &st) {
    const uint32_t *wp = wrow + int64_t(step) * kWordsPerStep;
#pragma unroll
    for (int v = 0; v < BITS / 4; ++v) st.w[v] = *reinterpret_cast<const u32x4 *>(wp + 4 * v);
    const int gi = (step * 64) / GS;
    st.s = Elem<SDT>::load(srow[gi]);
    st.b = Elem<SDT>::load(brow[gi]);
    if (xvalid) {
#pragma unroll
      for (int i = 0; i < 4; ++i) st.x[i] = Load8<XDT>::get(xrow + int64_t(step) * 64 + 8 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) st.x[i] = u32x4{0u, 0u, 0u, 0u};
    }
  };

  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

  auto compute = [&](const Stage<BITS, XDT, SDT> &st, int sl) {
    floatx16 t;
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 bq;
      if constexpr (BITS == 4) {
        bq = codes4_plus128(st.w[0][i]);
      } else {
        bq = codes8(st.w[i / 2][(i % 2) * 2], st.w[i / 2][(i % 2) * 2 + 1]);
      }
      t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(st.x[i]), as_bf16x8(bq), t, 0, 0, 0);
    }
    const float cv = st.b - kOff * st.s;
    const float *xs_step = xsum + sl * MROWS;
#pragma unroll
    for (int j = 0; j < kAcc / 4; ++j) {
      const floatx4 xs = *reinterpret_cast<const floatx4 *>(xs_step + 8 * j + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[4 * j + e] = fmaf(st.s, t[4 * j + e], acc[4 * j + e]);
        acc[4 * j + e] = fmaf(cv, xs[e], acc[4 * j + e]);
      }
    }
  };

  int sl = wave;
  if (sl < ns) {
    Stage<BITS, XDT, SDT> cur;
    load_stage(s_begin + sl, cur);
    for (; sl < ns; sl += 4) {
      Stage<BITS, XDT, SDT> nxt;
      const bool more = sl + 4 < ns;
      if (more) load_stage(s_begin + sl + 4, nxt);
      compute(cur, sl);
      if (more) cur = nxt;
    }
  }

  // 3. Sum the four waves.  Accumulator entry i of lane (r, h) is row
  //    8*(i/4) + 4*h + i%4, column r.
#pragma unroll
  for (int i = 0; i < kAcc; ++i) {
    const int m = 8 * (i / 4) + 4 * h + (i % 4);
    red[(wave * MROWS + m) * 32 + r] = acc[i];
  }
  __syncthreads();
  for (int o = tid; o < MROWS * 32; o += kThreads) {
    const int m = o >> 5;
    const int c = o & 31;
    const int nn = tile * 32 + c;
    if (m < M && nn < N) {
      const float v = ((red[(0 * MROWS + m) * 32 + c] + red[(1 * MROWS + m) * 32 + c]) +
                       red[(2 * MROWS + m) * 32 + c]) +
                      red[(3 * MROWS + m) * 32 + c];
      if (nsplit == 1)
        y[int64_t(m) * N + nn] = Elem<ODT>::store(v);
      else
        partial[(int64_t(split) * M + m) * N + nn] = v;
    }
  }
  if (nsplit == 1) return;

  // 4. K was split: the last block to finish this tile adds the partial
  //    sums in split order and resets the tile's counter for the next call.
  __shared__ unsigned s_last;
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = (atomicAdd(&counters[tile], 1u) == unsigned(nsplit - 1)) ? 1u : 0u;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int o = tid; o < MROWS * 32; o += kThreads) {
    const int m = o >> 5;
    const int c = o & 31;
    const int nn = tile * 32 + c;
    if (m < M && nn < N) {
      float v = 0.0f;
      for (int sp = 0; sp < nsplit; ++sp) v += partial[(int64_t(sp) * M + m) * N + nn];
      y[int64_t(m) * N + nn] = Elem<ODT>::store(v);
    }
  }
  if (tid == 0) counters[tile] = 0u;
}

template <int BITS, int XDT, int SDT, int ODT, int MROWS, int GS>
void launch_qmv_t(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K,
                  const kern::QmvPlan &plan, const kern::SplitWorkspace &ws,
                  hipStream_t st) {
  const dim3 grid((N + 31) / 32, plan.splits);
  const size_t lds = (size_t(plan.groups_per_split) * MROWS + 4 * MROWS * 32) * sizeof(float);
  qmv_kernel<BITS, XDT, SDT, ODT, MROWS, GS><<<grid, kThreads, lds, st>>>(
      static_cast<typename Elem<ODT>::T *>(y), static_cast<const typename Elem<XDT>::T *>(x), ldx,
      w, static_cast<const typename Elem<SDT>::T *>(s),
      static_cast<const typename Elem<SDT>::T *>(b), M, N, K, plan.groups_per_split,
      ws.partial, ws.counters);
}

template <int BITS, int XDT, int SDT, int ODT>
void launch_qmv_m(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K, int gs,
                  const kern::QmvPlan &plan, const kern::SplitWorkspace &ws,
                  hipStream_t st) {
  if (gs == 64) {
    if (M <= 16)
      launch_qmv_t<BITS, XDT, SDT, ODT, 16, 64>(y, x, ldx, w, s, b, M, N, K, plan, ws, st);
    else
      launch_qmv_t<BITS, XDT, SDT, ODT, 32, 64>(y, x, ldx, w, s, b, M, N, K, plan, ws, st);
  } else {
    if (M <= 16)
      launch_qmv_t<BITS, XDT, SDT, ODT, 16, 128>(y, x, ldx, w, s, b, M, N, K, plan, ws, st);
    else
      launch_qmv_t<BITS, XDT, SDT, ODT, 32, 128>(y, x, ldx, w, s, b, M, N, K, plan, ws, st);
  }
}

#define SDQ_QMV_CASE(XD, SD, OD)                                                      \
  if (x_dtype == XD && s_dtype == SD && y_dtype == OD) {                              \
    if (bits == 4)                                                                    \
      launch_qmv_m<4, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K), \
                                  group_size, plan, ws, stream);                      \
    else                                                                              \
      launch_qmv_m<8, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K), \
                                  group_size, plan, ws, stream);                      \
    hip_check(hipGetLastError(), "qmv launch");                                       \
    return;                                                                           \
  }

} // namespace

namespace kern {

QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int cus) {
  (void)group_size;
  QmvPlan p;
  const int64_t steps = K / 64;
  const int64_t tiles = (N + 31) / 32;
  const int64_t target_blocks = 2 * int64_t(cus > 0 ? cus : 256);
  int64_t splits = (target_blocks + tiles - 1) / tiles;
  // At least two 64-wide steps per wave (eight per block) ...
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, steps / 8));
  // ... and at most 256 steps per block, so the sums fit in LDS.
  splits = std::max<int64_t>(splits, (steps + 255) / 256);
  if (splits < 1) splits = 1;
  int64_t sps = (steps + splits - 1) / splits;
  splits = (steps + sps - 1) / sps;
  p.splits = int(splits);
  p.groups_per_split = int(sps);
  p.partial_floats = splits > 1 ? size_t(splits) * size_t(M) * size_t(N) : 0;
  p.counters = int(tiles);
  return p;
}

void qmv(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, const QmvPlan &plan, const SplitWorkspace &ws,
         hipStream_t stream) {
  if (M < 1 || M > 32) fail("qmv: M must be in [1, 32]");
  if (N < 1 || K < 64 || K % 64 != 0) fail("qmv: bad N or K");
  if (group_size != 64 && group_size != 128) fail("qmv: group size must be 64 or 128");
  if (K % group_size != 0) fail("qmv: K % group_size != 0");
  if (bits != 4 && bits != 8) fail("qmv: bits must be 4 or 8");
  if (ldx < K || ldx % 8 != 0) fail("qmv: row stride of x must be >= K and a multiple of 8");
  if (plan.splits > 1 && (!ws.partial || !ws.counters)) fail("qmv: split without workspace");
  SDQ_QMV_CASE(SDQ_BFLOAT16, SDQ_FLOAT32, SDQ_FLOAT32)
  SDQ_QMV_CASE(SDQ_BFLOAT16, SDQ_BFLOAT16, SDQ_BFLOAT16)
  SDQ_QMV_CASE(SDQ_FLOAT32, SDQ_FLOAT32, SDQ_FLOAT32)
  SDQ_QMV_CASE(SDQ_BFLOAT16, SDQ_FLOAT32, SDQ_BFLOAT16)
  SDQ_QMV_CASE(SDQ_FLOAT16, SDQ_FLOAT16, SDQ_FLOAT16)
  SDQ_QMV_CASE(SDQ_FLOAT16, SDQ_FLOAT32, SDQ_FLOAT32)
  SDQ_QMV_CASE(SDQ_FLOAT32, SDQ_BFLOAT16, SDQ_FLOAT32)
  SDQ_QMV_CASE(SDQ_FLOAT32, SDQ_FLOAT16, SDQ_FLOAT32)
  SDQ_QMV_CASE(SDQ_BFLOAT16, SDQ_FLOAT16, SDQ_FLOAT32)
  SDQ_QMV_CASE(SDQ_FLOAT16, SDQ_BFLOAT16, SDQ_FLOAT32)
  fail(std::string("qmv: unsupported dtype combination x=") + dtype_name(x_dtype) +
       " scales=" + dtype_name(s_dtype) + " y=" + dtype_name(y_dtype));
}

} // namespace kern
} // namespace sdq
