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

template <int BITS, int XDT, int SDT, int ODT, int BM, int GS>
__global__ __launch_bounds__(kThreads, 1) void qmm_kernel(
    typename Elem<ODT>::T *__restrict__ y, const typename Elem<XDT>::T *__restrict__ x,
    int64_t ldx, const uint32_t *__restrict__ w,
    const typename Elem<SDT>::T *__restrict__ scales,
    const typename Elem<SDT>::T *__restrict__ biases, int M, int N, int K) {
  using XT = typename Elem<XDT>::T;
  using ST = typename Elem<SDT>::T;
  constexpr int MB = BM / 32;           // 32-row MFMA blocks per wave
  constexpr int kWordsPerStep = 2 * BITS; // 64 codes of one row
  constexpr int kHalfWords = BITS;        // this lane half's share
  constexpr int kWV = BITS / 4;           // u32x4 per lane per 32-row block
  // Two stages of BM rows x 64 bf16 (128 B = 32 words per row).
  __shared__ __attribute__((aligned(16))) uint32_t xs[2][BM * 32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 31;
  const int h = lane >> 5;
  const int m0 = blockIdx.y * BM;
  const int nw = blockIdx.x * kTileN + wave * 64;
  const int steps = K / 64;
  const int groups = K / GS;

  const uint32_t *wrow[2];
  const ST *srow[2];
  const ST *brow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = nw + 32 * j + r;
    const int nrow = n < N ? n : N - 1; // rows past N are read, never stored
    wrow[j] = w + int64_t(nrow) * (int64_t(K) * BITS / 32) + h * kHalfWords;
    srow[j] = scales + int64_t(nrow) * groups;
    brow[j] = biases + int64_t(nrow) * groups;
  }

  // Staging: thread t moves 16-byte chunk (t % 8) of rows t/8 + 32q.
  const int sc = tid & 7;
  const int sr = tid >> 3;
  auto stage_load = [&](int step, u32x4 (&xr)[MB]) {
#pragma unroll
    for (int q = 0; q < MB; ++q) {
      const int gm = m0 + sr + 32 * q;
      if (gm < M)
        xr[q] = Load8<XDT>::get(x + int64_t(gm) * ldx + int64_t(step) * 64 + 8 * sc);
      else
        xr[q] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto stage_store = [&](int buf, const u32x4 (&xr)[MB]) {
#pragma unroll
    for (int q = 0; q < MB; ++q) {
      const int row = sr + 32 * q;
      *reinterpret_cast<u32x4 *>(&xs[buf][row * 32 + ((sc ^ ((row >> 1) & 7)) * 4)]) = xr[q];
    }
  };
  auto load_w = [&](int step, u32x4 (&wr)[2][kWV], float (&s)[2], float (&b)[2]) {
    const int gi = (step * 64) / GS;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t *wp = wrow[j] + int64_t(step) * kWordsPerStep;
#pragma unroll
      for (int v = 0; v < kWV; ++v) wr[j][v] = *reinterpret_cast<const u32x4 *>(wp + 4 * v);
      s[j] = Elem<SDT>::load(srow[j][gi]);
      b[j] = Elem<SDT>::load(brow[j][gi]);
    }
  };

  floatx16 acc[MB][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mb][j][e] = 0.0f;

  u32x4 wc[2][kWV];
  float scur[2], bcur[2];
  {
    u32x4 xr[MB];
    stage_load(0, xr);
    stage_store(0, xr);
    load_w(0, wc, scur, bcur);
  }
  __syncthreads();

  for (int step = 0; step < steps; ++step) {
    const int buf = step & 1;
    // The next step's loads are issued unconditionally (the last iteration
    // reloads its own step into the idle buffer), so the loop body has no
    // branch and each wait counts only the loads it needs.
    const int next = step + 1 < steps ? step + 1 : step;
    u32x4 xr[MB];
    u32x4 wn[2][kWV];
    float sn[2], bn[2];
    stage_load(next, xr);
    load_w(next, wn, sn, bn);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t *xb = xs[buf];
    // Operand fragments are double-buffered across the four k-steps: the
    // LDS reads and the dequantization of k-step i + 1 are issued before the
    // MFMAs of k-step i, so their latency hides under the matrix work.
    u32x4 a[2][MB];
    u32x4 bq[2][2];
    auto read_a = [&](int i, u32x4 (&dst)[MB]) {
      const int chunk = (4 * h + i) ^ ((r >> 1) & 7);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        dst[mb] = *reinterpret_cast<const u32x4 *>(&xb[(mb * 32 + r) * 32 + chunk * 4]);
    };
    read_a(0, a[0]);
    bq[0][0] = dequant8<BITS>(wc[0], 0, scur[0], bcur[0]);
    bq[0][1] = dequant8<BITS>(wc[1], 0, scur[1], bcur[1]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cur = i & 1;
      if (i < 3) {
        read_a(i + 1, a[cur ^ 1]);
        bq[cur ^ 1][0] = dequant8<BITS>(wc[0], i + 1, scur[0], bcur[0]);
        bq[cur ^ 1][1] = dequant8<BITS>(wc[1], i + 1, scur[1], bcur[1]);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        acc[mb][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[cur][mb]), as_bf16x8(bq[cur][0]), acc[mb][0], 0, 0, 0);
        acc[mb][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[cur][mb]), as_bf16x8(bq[cur][1]), acc[mb][1], 0, 0, 0);
      }
    }
    // Issue order for the region above: the first k-step's operands, then
    // for each k-step one MFMA at a time with the next k-step's LDS reads
    // and dequantization threaded between them, so the matrix pipe never
    // waits on a whole batch of reads or VALU work.
    __builtin_amdgcn_sched_group_barrier(0x100, MB, 0); // DS reads of k-step 0
    __builtin_amdgcn_sched_group_barrier(0x002, 24, 0); // part of its dequant
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
      for (int g = 0; g < MB; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0); // VALU
      }
#pragma unroll
      for (int g = 0; g < MB; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      }
    }
#pragma unroll
    for (int g = 0; g < 2 * MB; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    stage_store(buf ^ 1, xr);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int v = 0; v < kWV; ++v) wc[j][v] = wn[j][v];
      scur[j] = sn[j];
      bcur[j] = bn[j];
    }
    __syncthreads();
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
                  hipStream_t st) {
  const dim3 grid((N + kTileN - 1) / kTileN, (M + BM - 1) / BM);
  auto *yp = static_cast<typename Elem<ODT>::T *>(y);
  auto *xp = static_cast<const typename Elem<XDT>::T *>(x);
  auto *sp = static_cast<const typename Elem<SDT>::T *>(s);
  auto *bp = static_cast<const typename Elem<SDT>::T *>(b);
  if (gs == 64)
    qmm_kernel<BITS, XDT, SDT, ODT, BM, 64><<<grid, kThreads, 0, st>>>(yp, xp, ldx, w, sp, bp, M, N, K);
  else
    qmm_kernel<BITS, XDT, SDT, ODT, BM, 128><<<grid, kThreads, 0, st>>>(yp, xp, ldx, w, sp, bp, M, N, K);
}

template <int BITS, int XDT, int SDT, int ODT>
void launch_qmm_bm(void *y, const void *x, int64_t ldx, const uint32_t *w,
                   const void *s, const void *b, int M, int N, int K, int gs,
                   hipStream_t st) {
  if (M <= 128)
    launch_qmm_t<BITS, XDT, SDT, ODT, 128>(y, x, ldx, w, s, b, M, N, K, gs, st);
  else
    launch_qmm_t<BITS, XDT, SDT, ODT, 256>(y, x, ldx, w, s, b, M, N, K, gs, st);
}

#define SDQ_QMM_CASE(XD, SD, OD)                                                         \
  if (x_dtype == XD && s_dtype == SD && y_dtype == OD) {                                 \
    if (bits == 4)                                                                       \
      launch_qmm_bm<4, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K),  \
                                   group_size, stream);                                  \
    else                                                                                 \
      launch_qmm_bm<8, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K),  \
                                   group_size, stream);                                  \
    hip_check(hipGetLastError(), "qmm launch");                                          \
    return;                                                                              \
  }

} // namespace

namespace kern {

void qmm(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, hipStream_t stream) {
  if (M < 1 || N < 1 || K < 64 || K % 64 != 0) fail("qmm: bad M, N or K");
  if (M > (int64_t(1) << 30) || N > (int64_t(1) << 30) || K > (int64_t(1) << 30))
    fail("qmm: dimension too large");
  if (group_size != 64 && group_size != 128) fail("qmm: group size must be 64 or 128");
  if (K % group_size != 0) fail("qmm: K % group_size != 0");
  if (bits != 4 && bits != 8) fail("qmm: bits must be 4 or 8");
  if (ldx < K || ldx % 8 != 0) fail("qmm: row stride of x must be >= K and a multiple of 8");
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
