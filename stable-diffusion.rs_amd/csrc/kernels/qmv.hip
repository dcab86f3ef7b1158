// qmv.hip -- y = x @ dequantize(w).T for few rows of x (M <= 32): the
// bandwidth-bound decode/modulation shape of mlx_quantized_matmul
// (crates/sd-tensor/src/mlx.rs:386-397, 1947-1975; callers e.g. the Flux
// modulation linears at M = 1, sd-models/src/mlx/flux.rs:279-299, 437, and the
// T5 FFN at few tokens, t5.rs:209-214).
//
// Time here is the packed weight stream, so the kernel keeps VALU work per
// weight element small and many weight bytes in flight:
//
//   * Codes are never dequantized element by element.  For one 64-wide step
//     of K (one group at group size 64; half a group at 128) the MFMA
//     computes t[m][n] = sum_k x[m,k] * c_k with c_k = q_k + OFF held EXACTLY
//     in bf16 (4-bit: OFF = 128 and the bf16 pattern 0x4300|q is built with
//     one byte-permute and one and-or per pair; 8-bit: OFF = 0, q converted).
//     Then y += s * t + (b - OFF*s) * X, where X[m] = sum_k x[m,k] over the
//     step.  The affine dequantization is applied once per group per output
//     instead of once per weight, and is more accurate than rounding each
//     dequantized weight to bf16.
//   * A block of eight waves owns 32 weight rows (the MFMA's N side) and a
//     range of K.  It first stages its rows of x (bf16) and their per-step
//     sums in LDS, so that the only global traffic of the main loop is the
//     weight stream: each wave keeps a queue of kDepth steps of packed codes,
//     scales and biases in registers, loaded unconditionally so every wait
//     covers exactly one queue slot.
//   * When there are too few 32-row tiles to fill the chip, K is split across
//     blocks.  Partial sums are written with agent-scope (L2-bypassing)
//     stores; after they complete, the block bumps the tile's counter; the
//     last block reads the partials back with agent-scope loads and adds them
//     in split order, so the result is deterministic and no cache-wide
//     writeback or invalidate is needed.
//   * MFMA v_mfma_f32_32x32x16_bf16 with the tokens on the M side.  Lane
//     (r, h) = (lane % 32, lane / 32) feeds token r and weight row r; its
//     eight K elements of k-step i are k = 64*step + 32*h + 8*i + e, so each
//     lane's weight bytes for a step are one contiguous 16 B (4-bit) or 32 B
//     (8-bit) load.  Token rows r >= M read row M - 1; their results are
//     never stored.
#include <algorithm>

#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kDepth = 8;            // weight steps in flight per wave
constexpr int kXBudget = 48 * 1024;  // LDS bytes for the staged rows of x

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

template <int BITS> struct Stage {
  u32x4 w[BITS / 4]; // this lane's half-row of the step: 16 B or 32 B
  float s, b;
};

// Row stride, in bf16 elements, of the staged x: 16 bytes of padding keep
// consecutive rows on different LDS banks.
__host__ __device__ constexpr int x_stride(int steps) { return steps * 64 + 8; }

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
  const int ns = s_end - s_begin; // >= 1 by construction of the plan
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 31;
  const int h = lane >> 5;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int xs_stride = x_stride(ns);
  uint16_t *xl = reinterpret_cast<uint16_t *>(smem);                         // [M][xs_stride] bf16
  float *xsum = reinterpret_cast<float *>(smem + size_t(M) * xs_stride * 2);  // [ns][MROWS]
  float *red = reinterpret_cast<float *>(smem);                               // [kWaves][MROWS][32], after the loop

  // 1. This wave's weight queue goes out first, so its latency overlaps the
  //    staging of x below.  The wave's steps are local steps wave,
  //    wave + kWaves, ...
  const int n = tile * 32 + r;
  const int nrow = n < N ? n : N - 1; // rows past N are read, never stored
  const uint32_t *wrow = w + int64_t(nrow) * (int64_t(K) * BITS / 32) + h * kHalfWords;
  const ST *srow = scales + int64_t(nrow) * groups;
  const ST *brow = biases + int64_t(nrow) * groups;
  const uint16_t *arow = xl + (r < M ? r : M - 1) * xs_stride + 32 * h;

  auto load_stage = [&](int sl, Stage<BITS> &st) {
    const int step = s_begin + sl;
    const uint32_t *wp = wrow + int64_t(step) * kWordsPerStep;
#pragma unroll
    for (int v = 0; v < BITS / 4; ++v) st.w[v] = *reinterpret_cast<const u32x4 *>(wp + 4 * v);
    const int gi = (step * 64) / GS;
    st.s = Elem<SDT>::load(srow[gi]);
    st.b = Elem<SDT>::load(brow[gi]);
  };

  // A queue of kDepth steps in registers: slot d holds this wave's step
  // base + d; after computing it, the slot is refilled with step
  // base + d + kDepth.  Slots past the last step hold a valid (wasted) step
  // computed with zero weight, so the body is straight-line and the queue
  // stays in issue order.
  const int my_steps = ns > wave ? (ns - wave + kWaves - 1) / kWaves : 0;
  auto local_step = [&](int i) {
    const int sl = wave + kWaves * i;
    return sl < ns ? sl : ns - 1;
  };
  Stage<BITS> q[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth; ++d) load_stage(local_step(d), q[d]);
  // 2. Stage x[0:M, K range] as bf16, 16-byte chunks.
  {
    const int chunks_per_row = ns * 8;
    for (int c = tid; c < M * chunks_per_row; c += kThreads) {
      const int m = c / chunks_per_row;
      const int q = c - m * chunks_per_row;
      const u32x4 v = Load8<XDT>::get(x + int64_t(m) * ldx + int64_t(s_begin) * 64 + 8 * q);
      *reinterpret_cast<u32x4 *>(xl + m * xs_stride + 8 * q) = v;
    }
  }
  __syncthreads();
  // 3. Per-step sums of the staged values (dot2 against (1, 1)); rows >= M
  //    are zero.
  {
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
    for (int p = tid; p < ns * MROWS; p += kThreads) {
      const int sl = p / MROWS;
      const int m = p - sl * MROWS;
      float sum = 0.0f;
      if (m < M) {
        const uint16_t *src = xl + m * xs_stride + sl * 64;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const u32x4 v = *reinterpret_cast<const u32x4 *>(src + 8 * c);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            // Copy the element out first: bit-casting a vector-element
            // expression directly reinterprets element 0 instead.
            const uint32_t pair = v[j];
            sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), ones, sum, false);
          }
        }
      }
      xsum[p] = sum;
    }
  }
  __syncthreads();

  // 4. The queue's steps.
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

  auto compute = [&](const Stage<BITS> &st, int sl, float weight) {
    const uint16_t *ap = arow + sl * 64;
    floatx16 t;
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 a = *reinterpret_cast<const u32x4 *>(ap + 8 * i);
      u32x4 bq;
      if constexpr (BITS == 4) {
        bq = codes4_plus128(st.w[0][i]);
      } else {
        bq = codes8(st.w[i / 2][(i % 2) * 2], st.w[i / 2][(i % 2) * 2 + 1]);
      }
      t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(bq), t, 0, 0, 0);
    }
    const float sv = st.s * weight;
    const float cv = (st.b - kOff * st.s) * weight;
    const float *xs_step = xsum + sl * MROWS;
#pragma unroll
    for (int j = 0; j < kAcc / 4; ++j) {
      const floatx4 xs = *reinterpret_cast<const floatx4 *>(xs_step + 8 * j + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[4 * j + e] = fmaf(sv, t[4 * j + e], acc[4 * j + e]);
        acc[4 * j + e] = fmaf(cv, xs[e], acc[4 * j + e]);
      }
    }
  };

  for (int base = 0; base < my_steps; base += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int i = base + d;
      compute(q[d], local_step(i), i < my_steps ? 1.0f : 0.0f);
      __builtin_amdgcn_sched_barrier(0);
      load_stage(local_step(i + kDepth), q[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // 5. Sum the waves.  Accumulator entry i of lane (r, h) is row
  //    8*(i/4) + 4*h + i%4, column r.  `red` reuses the staging space.
  __syncthreads();
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
      float v = red[m * 32 + c];
#pragma unroll
      for (int wv = 1; wv < kWaves; ++wv) v += red[(wv * MROWS + m) * 32 + c];
      if (nsplit == 1)
        y[int64_t(m) * N + nn] = Elem<ODT>::store(v);
      else
        __hip_atomic_store(&partial[(int64_t(split) * M + m) * N + nn], v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (nsplit == 1) return;

  // 6. K was split.  The partials went out as agent-scope stores, which do
  //    not stay in this XCD's L2; wait until they have completed, then count
  //    this split in.  The last block to arrive reads every split's partial
  //    with agent-scope loads, adds them in split order and re-arms the
  //    counter for the next call.
  __shared__ unsigned s_last;
  __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this wave's stores are done
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == unsigned(nsplit - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  for (int o = tid; o < MROWS * 32; o += kThreads) {
    const int m = o >> 5;
    const int c = o & 31;
    const int nn = tile * 32 + c;
    if (m < M && nn < N) {
      float v = 0.0f;
      for (int sp = 0; sp < nsplit; ++sp)
        v += __hip_atomic_load(&partial[(int64_t(sp) * M + m) * N + nn], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      y[int64_t(m) * N + nn] = Elem<ODT>::store(v);
    }
  }
  if (tid == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t qmv_lds_bytes(int M, int mrows, int steps_per_split) {
  const size_t staged = size_t(M) * x_stride(steps_per_split) * 2 + size_t(steps_per_split) * mrows * 4;
  const size_t reduce = size_t(kWaves) * mrows * 32 * 4;
  return std::max(staged, reduce);
}

template <int BITS, int XDT, int SDT, int ODT, int MROWS, int GS>
void launch_qmv_t(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K,
                  const kern::QmvPlan &plan, const kern::SplitWorkspace &ws,
                  hipStream_t st) {
  const dim3 grid((N + 31) / 32, plan.splits);
  const size_t lds = qmv_lds_bytes(M, MROWS, plan.groups_per_split);
  if (lds > 64 * 1024) fail("qmv: plan exceeds the LDS budget");
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
  const int64_t mrows = M <= 16 ? 16 : 32;
  // Split K only when there are fewer 32-row tiles than CUs: a split adds a
  // round trip (partials, counter, reload) that these short kernels feel.
  const int64_t target_blocks = int64_t(cus > 0 ? cus : 256);
  int64_t splits = (target_blocks + tiles - 1) / tiles;
  // At least one step per wave ...
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, steps / kWaves));
  // ... and a K range whose rows of x fit the LDS budget.
  int64_t max_steps = (kXBudget / (2 * M) - 8) / 64;
  max_steps = std::max<int64_t>(1, std::min<int64_t>(max_steps, 1024));
  while (size_t(M) * x_stride(int(max_steps)) * 2 + size_t(max_steps) * mrows * 4 > size_t(kXBudget) + 8192 &&
         max_steps > 1)
    --max_steps;
  splits = std::max<int64_t>(splits, (steps + max_steps - 1) / max_steps);
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
  if (plan.splits < 1 || plan.groups_per_split < 1 ||
      int64_t(plan.splits) * plan.groups_per_split < K / 64 ||
      int64_t(plan.splits - 1) * plan.groups_per_split >= K / 64)
    fail("qmv: inconsistent plan");
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
