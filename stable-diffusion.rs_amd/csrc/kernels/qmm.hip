// qmm.hip -- y = x @ dequantize(w).T for many rows of x: the prefill-shaped,
// MFMA-bound side of mlx_quantized_matmul (crates/sd-tensor/src/mlx.rs:386-397,
// 1947-1975; e.g. every Flux block linear at 4096+512 tokens,
// sd-models/src/mlx/flux.rs:333-471).
//
// Block tile BM x 256, four waves.  Wave v owns output columns
// [64v, 64v + 64) of the tile and all BM rows, i.e. BM/32 x 2 MFMA tiles of
// 32 x 32 (v_mfma_f32_32x32x16_bf16, fp32 accumulate).  Per 64-wide K step:
//   * the block stages the BM x 64 activation tile into LDS as bf16
//     (double-buffered, 16-byte chunks XOR-swizzled by row so the MFMA
//     operand reads are conflict-free); every wave reads all of it;
//   * each wave loads only ITS weight rows -- 16 B (4-bit) or 32 B (8-bit)
//     per lane per 32-row block -- and dequantizes them in registers,
//     scale * q + bias in f32, straight into the bf16 B operand.  A weight
//     element is dequantized once per block and used for BM rows, which is
//     what keeps the unpack cost under the MFMA time.
// Lane (r, h) = (lane % 32, lane / 32) feeds its eight K elements of k-step i
// from k = 64*step + 32*h + 8*i + e for both operands.
#include <algorithm>
#include <type_traits>

#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kThreads = 256;
constexpr int kTileN = 256;

__device__ __forceinline__ float byte_f(uint32_t v, int b) {
  return float((v >> (8 * b)) & 0xffu);
}

// Eight dequantized weights of k-step i, in element order, as bf16.
template <int BITS>
__device__ __forceinline__ u32x4 dequant8(const u32x4 (&wr)[BITS / 4], int i, float s, float b);

template <>
__device__ __forceinline__ u32x4 dequant8<4>(const u32x4 (&wr)[1], int i, float s, float b) {
  const uint32_t wd = wr[0][i];
  const uint32_t lo = opaque(wd & 0x0F0F0F0Fu);        // codes 0, 2, 4, 6
  const uint32_t hi = opaque((wd >> 4) & 0x0F0F0F0Fu); // codes 1, 3, 5, 7
  u32x4 r;
#pragma unroll
  for (int d = 0; d < 4; ++d)
    r[d] = pack_bf16x2(fmaf(byte_f(lo, d), s, b), fmaf(byte_f(hi, d), s, b));
  return r;
}

template <>
__device__ __forceinline__ u32x4 dequant8<8>(const u32x4 (&wr)[2], int i, float s, float b) {
  const uint32_t w0 = wr[i / 2][(i % 2) * 2];
  const uint32_t w1 = wr[i / 2][(i % 2) * 2 + 1];
  u32x4 r;
  r[0] = pack_bf16x2(fmaf(byte_f(w0, 0), s, b), fmaf(byte_f(w0, 1), s, b));
  r[1] = pack_bf16x2(fmaf(byte_f(w0, 2), s, b), fmaf(byte_f(w0, 3), s, b));
  r[2] = pack_bf16x2(fmaf(byte_f(w1, 0), s, b), fmaf(byte_f(w1, 1), s, b));
  r[3] = pack_bf16x2(fmaf(byte_f(w1, 2), s, b), fmaf(byte_f(w1, 3), s, b));
  return r;
}

// Work assignment of one launch.  Tiles are numbered M-tile major; tiles
// [0, dp_tiles) are computed whole, one block each; each tile after that is
// split into `splits` K ranges of `steps_per_split` 64-wide steps, one block
// per range, reduced through `partial` and `counters`.
struct QmmWork {
  int tiles_n;
  int dp_tiles;
  int splits;
  int steps_per_split;
  float *partial;
  unsigned *counters;
};

template <int BITS, int XDT, int SDT, int ODT, int BM, int GS>
__global__ __launch_bounds__(kThreads, 1) void qmm_kernel(
    typename Elem<ODT>::T *__restrict__ y, const typename Elem<XDT>::T *__restrict__ x,
    int64_t ldx, const uint32_t *__restrict__ w,
    const typename Elem<SDT>::T *__restrict__ scales,
    const typename Elem<SDT>::T *__restrict__ biases, int M, int N, int K, QmmWork wk) {
  using XT = typename Elem<XDT>::T;
  using ST = typename Elem<SDT>::T;
  constexpr int MB = BM / 32;           // 32-row MFMA blocks per wave
  constexpr int kWordsPerStep = 2 * BITS; // 64 codes of one row
  constexpr int kHalfWords = BITS;        // this lane half's share
  constexpr int kWV = BITS / 4;           // u32x4 per lane per 32-row block
  // Three stages of BM rows x 64 bf16 (128 B = 32 words per row).
  constexpr int kStage = BM * 32;
  __shared__ __attribute__((aligned(16))) uint32_t xs[3 * kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 31;
  const int h = lane >> 5;
  const int steps = K / 64;
  const int groups = K / GS;
  const int bid = blockIdx.x;
  int tile = bid, split = 0, k_begin = 0, k_end = steps;
  if (bid >= wk.dp_tiles) {
    const int j = bid - wk.dp_tiles;
    tile = wk.dp_tiles + j / wk.splits;
    split = j % wk.splits;
    k_begin = split * wk.steps_per_split;
    k_end = min(steps, k_begin + wk.steps_per_split);
  }
  const int m0 = (tile / wk.tiles_n) * BM;
  const int nw = (tile % wk.tiles_n) * kTileN + wave * 64;
  const int k_last = k_end - 1;

  // Buffer windows (byte offsets fit in 32 bits: checked on the host).
  const Rsrc rx = make_rsrc(x, uint32_t((int64_t(M - 1) * ldx + K) * sizeof(XT)));
  const Rsrc rw = make_rsrc(w, uint32_t(int64_t(N) * K * BITS / 8));
  const Rsrc rs = make_rsrc(scales, uint32_t(int64_t(N) * groups * sizeof(ST)));
  const Rsrc rb = make_rsrc(biases, uint32_t(int64_t(N) * groups * sizeof(ST)));

  uint32_t woff[2], soff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = nw + 32 * j + r;
    const int nrow = n < N ? n : N - 1; // rows past N are read, never stored
    woff[j] = uint32_t((int64_t(nrow) * (int64_t(K) * BITS / 32) + h * kHalfWords) * 4);
    soff[j] = uint32_t(int64_t(nrow) * groups * sizeof(ST));
  }

  // Staging: thread t moves 16-byte chunk (t % 8) of rows t/8 + 32q.  Rows
  // past M re-read row M - 1 (their products are never stored), so every
  // load is unconditional and each wait counts exactly the loads it needs.
  const int sc = tid & 7;
  const int sr = tid >> 3;
  uint32_t xoff[MB];
#pragma unroll
  for (int q = 0; q < MB; ++q)
    xoff[q] = uint32_t((int64_t(min(m0 + sr + 32 * q, M - 1)) * ldx + 8 * sc) * sizeof(XT));
  auto stage_load = [&](int step, u32x4 (&xr)[MB]) {
    const uint32_t so = uint32_t(step) * 64 * sizeof(XT);
#pragma unroll
    for (int q = 0; q < MB; ++q) xr[q] = BLoad8<XDT>::get(rx, xoff[q], so);
  };
  // Chunk c of row `row` sits at chunk c ^ ((row >> 1) & 7) of that row, so
  // the MFMA operand reads below hit all 64 banks without conflicts.
  auto stage_store = [&](uint32_t *dst, const u32x4 (&xr)[MB]) {
#pragma unroll
    for (int q = 0; q < MB; ++q) {
      const int row = sr + 32 * q;
      *reinterpret_cast<u32x4 *>(&dst[row * 32 + ((sc ^ ((row >> 1) & 7)) * 4)]) = xr[q];
    }
  };
  // A fragment of 32-row block mb for k-step i.
  auto read_a = [&](const uint32_t *src, int i, int mb) {
    const int chunk = (4 * h + i) ^ ((r >> 1) & 7);
    return *reinterpret_cast<const u32x4 *>(&src[(mb * 32 + r) * 32 + chunk * 4]);
  };
  struct WStep {
    u32x4 q[2][kWV];
    float s[2], b[2];
  };
  auto load_w = [&](int step, WStep &ws) {
    const uint32_t wso = uint32_t(step) * kWordsPerStep * 4;
    const uint32_t sso = uint32_t((step * 64) / GS) * sizeof(ST);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int v = 0; v < kWV; ++v) ws.q[j][v] = bload16(rw, woff[j] + 16 * v, wso);
      ws.s[j] = BLoadScalar<SDT>::get(rs, soff[j], sso);
      ws.b[j] = BLoadScalar<SDT>::get(rb, soff[j], sso);
    }
  };
  auto dequant = [&](const WStep &ws, int i, u32x4 (&dst)[2]) {
    dst[0] = dequant8<BITS>(ws.q[0], i, ws.s[0], ws.b[0]);
    dst[1] = dequant8<BITS>(ws.q[1], i, ws.s[1], ws.b[1]);
  };

  floatx16 acc[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mb][j][e] = 0.0f;

  // Software pipeline, per 64-wide step s of this block's K range:
  //   * weights: codes, scales and biases of step s + 2 are loaded at the top
  //     of step s (a three-deep register queue);
  //   * activations: the tile of step s + 2 arrives in registers during step
  //     s - 1 and is written to LDS stage (s + 2) % 3 halfway through step s,
  //     when the tile of step s + 3 is requested; one barrier per step makes
  //     it visible;
  //   * operands: the A fragments and dequantized B fragments of k-step i + 1
  //     are prepared while the MFMAs of k-step i run -- across the step
  //     boundary too, since stage (s + 1) % 3 is complete before step s ends.
  // Steps past the range re-read its last step, never used, so the body has
  // no branches.
  WStep w0, w1, w2;
  u32x4 xr[MB];
  stage_load(k_begin, xr);
  stage_store(xs, xr);
  stage_load(min(k_begin + 1, k_last), xr);
  stage_store(xs + kStage, xr);
  stage_load(min(k_begin + 2, k_last), xr);
  load_w(k_begin, w0);
  load_w(min(k_begin + 1, k_last), w1);
  __syncthreads();

  u32x4 a[MB];
  u32x4 bq[2][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) a[mb] = read_a(xs, 0, mb);
  dequant(w0, 0, bq[0]);

  int st0 = 0; // LDS stage of step s; s + 1 and s + 2 follow cyclically
  for (int step = k_begin; step < k_end; ++step) {
    const int st1 = st0 == 2 ? 0 : st0 + 1;
    const int st2 = st1 == 2 ? 0 : st1 + 1;
    load_w(min(step + 2, k_last), w2);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = i & 1;
      if (i == 1) {
        stage_store(xs + st2 * kStage, xr);
        stage_load(min(step + 3, k_last), xr);
      }
      if (i < 3)
        dequant(w0, i + 1, bq[c ^ 1]);
      else
        dequant(w1, 0, bq[c ^ 1]);
      // Each A fragment is refilled for the next k-step (the next step's
      // first k-step after the last) as soon as its two MFMAs are issued.
      const uint32_t *nsrc = xs + (i < 3 ? st0 : st1) * kStage;
      const int ni = i < 3 ? i + 1 : 0;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        acc[mb][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[mb]), as_bf16x8(bq[c][0]), acc[mb][0], 0, 0, 0);
        acc[mb][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[mb]), as_bf16x8(bq[c][1]), acc[mb][1], 0, 0, 0);
        a[mb] = read_a(nsrc, ni, mb);
      }
      // One MFMA at a time, with the next k-step's LDS reads, dequant VALU
      // and (halfway) the staging traffic threaded between them.
#pragma unroll
      for (int g = 0; g < MB; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
        if (i == 1) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0); // DS write
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0); // VALU
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
        if (i == 1) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // VMEM read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0); // VALU
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    w0 = w1;
    w1 = w2;
    st0 = st1;
    __syncthreads();
  }

  if (bid >= wk.dp_tiles) {
    // A K range of a split tile.  Its accumulators go out as agent-scope
    // (L2-bypassing) stores, register-major so that each store instruction
    // writes 256 consecutive floats; once they have completed the block
    // counts itself in.  The last block of the tile to arrive reads every
    // range's partial back with agent-scope loads (its own from registers),
    // adds them in range order -- the same order whichever block is last, so
    // the result is deterministic -- re-arms the counter and stores the tile.
    const int sk = tile - wk.dp_tiles;
    constexpr int kRegs = MB * 2 * 16;
    float *base = wk.partial + int64_t(sk) * wk.splits * (kRegs * kThreads) + tid;
    float *mine = base + int64_t(split) * (kRegs * kThreads);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          __hip_atomic_store(mine + ((mb * 2 + j) * 16 + e) * kThreads, acc[mb][j][e],
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __shared__ unsigned s_last;
    __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this wave's stores are done
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&wk.counters[sk], 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == unsigned(wk.splits - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const floatx16 own = acc[mb][j];
        floatx16 sum;
        for (int p = 0; p < wk.splits; ++p) {
          floatx16 t;
          if (p == split) {
            t = own;
          } else {
            const float *src = base + int64_t(p) * (kRegs * kThreads);
#pragma unroll
            for (int e = 0; e < 16; ++e)
              t[e] = __hip_atomic_load(src + ((mb * 2 + j) * 16 + e) * kThreads, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
          }
          sum = p == 0 ? t : sum + t;
        }
        acc[mb][j] = sum;
      }
    }
    if (tid == 0)
      __hip_atomic_store(&wk.counters[sk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Accumulator entry e of lane (r, h) in tile (mb, j) is row
  // 32*mb + 8*(e/4) + 4*h + e%4, column 32*j + r of the wave's slab.
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = nw + 32 * j + r;
      if (col >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + 32 * mb + 8 * (e / 4) + 4 * h + (e % 4);
        if (row < M) y[int64_t(row) * N + col] = Elem<ODT>::store(acc[mb][j][e]);
      }
    }
  }
}

template <int BITS, int XDT, int SDT, int ODT, int BM>
void launch_qmm_t(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K, int gs,
                  const kern::QmmPlan &plan, const kern::SplitWorkspace &ws, hipStream_t st) {
  const QmmWork wk{plan.tiles_n, plan.dp_tiles, plan.splits, plan.steps_per_split, ws.partial,
                   ws.counters};
  const dim3 grid(plan.blocks);
  auto *yp = static_cast<typename Elem<ODT>::T *>(y);
  auto *xp = static_cast<const typename Elem<XDT>::T *>(x);
  auto *sp = static_cast<const typename Elem<SDT>::T *>(s);
  auto *bp = static_cast<const typename Elem<SDT>::T *>(b);
  if (gs == 64)
    qmm_kernel<BITS, XDT, SDT, ODT, BM, 64><<<grid, kThreads, 0, st>>>(yp, xp, ldx, w, sp, bp, M, N, K, wk);
  else
    qmm_kernel<BITS, XDT, SDT, ODT, BM, 128><<<grid, kThreads, 0, st>>>(yp, xp, ldx, w, sp, bp, M, N, K, wk);
}

template <int BITS, int XDT, int SDT, int ODT>
void launch_qmm_bm(void *y, const void *x, int64_t ldx, const uint32_t *w,
                   const void *s, const void *b, int M, int N, int K, int gs,
                   const kern::QmmPlan &plan, const kern::SplitWorkspace &ws, hipStream_t st) {
  if (plan.bm == 128)
    launch_qmm_t<BITS, XDT, SDT, ODT, 128>(y, x, ldx, w, s, b, M, N, K, gs, plan, ws, st);
  else
    launch_qmm_t<BITS, XDT, SDT, ODT, 256>(y, x, ldx, w, s, b, M, N, K, gs, plan, ws, st);
}

#define SDQ_QMM_CASE(XD, SD, OD)                                                         \
  if (x_dtype == XD && s_dtype == SD && y_dtype == OD) {                                 \
    if (bits == 4)                                                                       \
      launch_qmm_bm<4, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K),  \
                                   group_size, plan, ws, stream);                        \
    else                                                                                 \
      launch_qmm_bm<8, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K),  \
                                   group_size, plan, ws, stream);                        \
    hip_check(hipGetLastError(), "qmm launch");                                          \
    return;                                                                              \
  }

} // namespace

namespace kern {

QmmPlan plan_qmm(int64_t M, int64_t N, int64_t K, int cus) {
  QmmPlan p;
  p.bm = M <= 128 ? 128 : 256;
  p.tiles_n = int((N + kTileN - 1) / kTileN);
  const int64_t tiles_m = (M + p.bm - 1) / p.bm;
  p.tiles = int(tiles_m * p.tiles_n);
  const int64_t steps = K / 64;
  const int64_t slots = cus > 0 ? cus : 256; // one block per CU at a time
  const int64_t rounds = p.tiles / slots;
  const int64_t rem = p.tiles % slots;
  // The last, partly filled round of whole tiles costs as much as a full
  // one.  Its tiles can instead be split along K into ranges that run side
  // by side; each range then costs its length in steps, plus about one step
  // per range for writing and re-reading its partial tile.
  p.dp_tiles = p.tiles;
  p.splits = 1;
  p.steps_per_split = int(steps);
  if (rem > 0) {
    int64_t best = steps;
    for (int64_t s = 2; s <= 16 && rem * s <= slots; ++s) {
      const int64_t sps = (steps + s - 1) / s;
      if (sps < 4) break;
      const int64_t ranges = (steps + sps - 1) / sps;
      const int64_t cost = sps + ranges;
      if (cost < best) {
        best = cost;
        p.splits = int(ranges);
        p.steps_per_split = int(sps);
      }
    }
    if (p.splits > 1) p.dp_tiles = int(p.tiles - rem);
  }
  const int64_t sk_tiles = p.tiles - p.dp_tiles;
  p.blocks = int(p.dp_tiles + sk_tiles * p.splits);
  p.partial_floats = size_t(sk_tiles) * size_t(p.splits) * size_t(p.bm) * kTileN;
  p.counters = int(sk_tiles);
  return p;
}

void qmm(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, const QmmPlan &plan, const SplitWorkspace &ws, hipStream_t stream) {
  if (M < 1 || N < 1 || K < 64 || K % 64 != 0) fail("qmm: bad M, N or K");
  if (M > (int64_t(1) << 30) || N > (int64_t(1) << 30) || K > (int64_t(1) << 30))
    fail("qmm: dimension too large");
  if (group_size != 64 && group_size != 128) fail("qmm: group size must be 64 or 128");
  if (K % group_size != 0) fail("qmm: K % group_size != 0");
  if (bits != 4 && bits != 8) fail("qmm: bits must be 4 or 8");
  if (ldx < K || ldx % 8 != 0) fail("qmm: row stride of x must be >= K and a multiple of 8");
  // The kernel addresses x, the codes, scales and biases through 32-bit
  // buffer windows.
  const int64_t lim = int64_t(1) << 31;
  if ((int64_t(M - 1) * ldx + K) * dtype_size(x_dtype) >= lim || N * K * bits / 8 >= lim ||
      N * (K / group_size) * dtype_size(s_dtype) >= lim)
    fail("qmm: x, the packed weight, scales and biases must each be under 2 GiB");
  // The launch must be exactly the plan for this shape: the grid, the
  // per-range K bounds and the workspace all follow from it.
  const QmmPlan want = plan_qmm(M, N, K, 0);
  if (plan.bm != want.bm || plan.tiles_n != want.tiles_n || plan.tiles != want.tiles ||
      plan.splits < 1 || plan.steps_per_split < 1 || plan.dp_tiles < 0 || plan.dp_tiles > plan.tiles ||
      plan.blocks != plan.dp_tiles + (plan.tiles - plan.dp_tiles) * plan.splits ||
      (plan.dp_tiles < plan.tiles &&
       (int64_t(plan.splits - 1) * plan.steps_per_split >= K / 64 ||
        int64_t(plan.splits) * plan.steps_per_split < K / 64)))
    fail("qmm: inconsistent launch plan");
  if (plan.dp_tiles < plan.tiles && (!ws.partial || !ws.counters))
    fail("qmm: split-K launch without a workspace");
  SDQ_QMM_CASE(SDQ_BFLOAT16, SDQ_FLOAT32, SDQ_FLOAT32)
  SDQ_QMM_CASE(SDQ_BFLOAT16, SDQ_BFLOAT16, SDQ_BFLOAT16)
  SDQ_QMM_CASE(SDQ_FLOAT32, SDQ_FLOAT32, SDQ_FLOAT32)
  SDQ_QMM_CASE(SDQ_BFLOAT16, SDQ_FLOAT32, SDQ_BFLOAT16)
  SDQ_QMM_CASE(SDQ_FLOAT16, SDQ_FLOAT16, SDQ_FLOAT16)
  SDQ_QMM_CASE(SDQ_FLOAT16, SDQ_FLOAT32, SDQ_FLOAT32)
  SDQ_QMM_CASE(SDQ_FLOAT32, SDQ_BFLOAT16, SDQ_FLOAT32)
  SDQ_QMM_CASE(SDQ_FLOAT32, SDQ_FLOAT16, SDQ_FLOAT32)
  SDQ_QMM_CASE(SDQ_BFLOAT16, SDQ_FLOAT16, SDQ_FLOAT32)
  SDQ_QMM_CASE(SDQ_FLOAT16, SDQ_BFLOAT16, SDQ_FLOAT32)
  fail(std::string("qmm: unsupported dtype combination x=") + dtype_name(x_dtype) +
       " scales=" + dtype_name(s_dtype) + " y=" + dtype_name(y_dtype));
}

} // namespace kern
} // namespace sdq
