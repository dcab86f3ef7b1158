// qmv.hip -- the launch planner and dtype dispatch of the small-M kernel
// (qmv_kernel.hpp holds the kernel; qmv_inst.hip instantiates it per dtype
// combination): the bandwidth-bound side of mlx_quantized_matmul
// (crates/sd-tensor/src/mlx.rs:386-397, 1947-1975).
#include <algorithm>
#include <string>

#include "launch.hpp"
#include "qmv_lds.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace qmv_detail {

template <int XD, int SD, int OD>
void qmv_combo(int bits, void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s,
               const void *b, int M, int N, int K, int gs, const kern::QmvPlan &plan,
               const kern::Epilogue &ep, hipStream_t st, float *partial);

} // namespace qmv_detail

namespace {

constexpr int64_t kStageXMax = 104 * 1024; // x bytes staged once per block at most
constexpr int kLdsMax = 150 * 1024;       // of the CU's 160 KB

#define SDQ_QMV_CASE(XD, SD, OD)                                                              \
  if (x_dtype == XD && s_dtype == SD && y_dtype == OD) {                                      \
    qmv_detail::qmv_combo<XD, SD, OD>(bits, y, x, ldx, w, scales, biases, int(M), int(N), int(K), \
                                      group_size, plan, ep, stream, partial);                 \
    hip_check(hipGetLastError(), "qmv launch");                                               \
    return;                                                                                   \
  }

} // namespace

namespace kern {

constexpr int kern_xblock() { return qmv_detail::kXBlock; }

// 32 < M <= 128 in 3-8 row groups against the large-M kernel, measured at
// K = 2048-3072: 3072->3072 30-45 % faster (M = 33-64: 15.1-17.6 -> 9.5-10.8
// us, M = 65-128: 19.4-23.5 -> 11.0-15.9 us; the tile kernel has 12 tiles to
// split), 2048->1024 about 2x, 3072->4096 even; 3072->9216 and wider 5-60 %
// slower.
bool qmv_takes(int64_t M, int64_t N, int64_t K) {
  return M <= 32 || (M <= 128 && N <= 4096 && 16 * (K + 8) * 2 <= kStageXMax);
}

QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int bits, int cus, bool allow_split) {
  using namespace qmv_detail;
  QmvPlan p;
  p.row_blocks = M <= 16 ? 1 : 2;
  const int64_t tiles = (N + 15) / 16;
  const int64_t ncu = cus > 0 ? cus : 256;
  const int64_t nchunk = (K + 127) / 128;
  // About a dozen waves per CU in all (four K ranges per tile at the Flux
  // and T5 widths measured best); at least two chunks per wave where K has
  // four or more (3072->3072, 192 tiles: 12 waves per tile instead of 16,
  // 11-17 % faster at M = 1-16; 768->3072 4-7 %).
  auto waves_for = [&](int64_t T, int max_waves) {
    int64_t s = (12 * ncu + tiles - 1) / tiles;
    s = std::min<int64_t>(s, max_waves / T);
    s = std::min<int64_t>(s, nchunk >= 4 ? nchunk / 2 : nchunk);
    return int(std::max<int64_t>(s, 1));
  };
  auto fits = [&](int xmode, int64_t T, int S) {
    const QmvLds l = qmv_lds(xmode, int(M), int(K), group_size, int(T), S, p.row_blocks);
    return l.total <= kLdsMax ? l.total : 0;
  };
  // M <= 4: each wave stages its own slice of x (no block-wide barrier).
  if (M <= 4) {
    // More waves per tile when that brings each wave's slice of x within
    // what it stages (long K over many tiles, e.g. T5's paired wi).
    int S = waves_for(1, kMaxWaves[kXWave]);
    while (S < kMaxWaves[kXWave] && S < nchunk && (nchunk + S - 1) / S > kXWaveMaxChunks) ++S;
    const QmvLds l = qmv_lds(kXWave, int(M), int(K), group_size, 1, S, p.row_blocks);
    if (l.cmax <= kXWaveMaxChunks && l.total <= kLdsMax) {
      p.xmode = kXWave;
      p.tiles_per_block = 1;
      p.waves = S;
      p.lds_bytes = l.total;
      return p;
    }
  }
  // A small x is staged once per block; blocks take several tiles when that
  // keeps the grid within one block per CU (x is then staged once per CU).
  if (M <= 32 && M * (K + 8) * 2 <= kStageXMax) {
    const int64_t T = std::min<int64_t>((tiles + ncu - 1) / ncu, 8);
    const int S = waves_for(T, kMaxWaves[kXBlock]);
    if (const int bytes = fits(kXBlock, T, S)) {
      p.xmode = kXBlock;
      p.tiles_per_block = int(T);
      p.waves = S;
      p.lds_bytes = bytes;
      return p;
    }
  }
  // 16 < M <= 128 with 16 rows of x small enough: 2-8 row groups, each block
  // staging 16 rows of x for its T tiles; the blocks of a tile group
  // read its codes from HBM once (one XCD's L2 serves the second) and no
  // partial tiles are written.  Measured 0-25 % faster than K ranges at
  // K = 3072 (M = 17-32; N = 3072-21504).
  if (M > 16 && 16 * (K + 8) * 2 <= kStageXMax) {
    const int RG = int((M + 15) / 16);
    // Fewer tiles per block when the block's waves would not fit the LDS.
    for (int64_t T = std::min<int64_t>((tiles * RG + ncu - 1) / ncu, 8); T >= 1; --T) {
      int64_t S = (12 * ncu + tiles * RG - 1) / (tiles * RG);
      S = std::max<int64_t>(1, std::min<int64_t>({S, kMaxWaves[kXBlock] / T, nchunk}));
      const QmvLds l = qmv_lds(kXBlock, 16, int(K), group_size, int(T), int(S), 1);
      if (l.total <= kLdsMax) {
        p.xmode = kXBlock;
        p.row_blocks = 1;
        p.row_groups = RG;
        p.tiles_per_block = int(T);
        p.waves = int(S);
        p.lds_bytes = l.total;
        return p;
      }
    }
  }
  // More than 32 rows only in row groups (the kernel's row blocks cover 32).
  if (M > 32) fail("qmv: no row-group plan fits for M = " + std::to_string(M) + ", K = " + std::to_string(K));
  // A large x: K in R ranges, each staged once per block of T tiles.  The
  // shape is chosen by an estimate of the busiest CU's time, in 128-wide
  // chunks of one tile's codes: its blocks' code chunks, their x slices
  // (read from L2, weighted 1/4) and partial tiles, slowed in proportion
  // when fewer than eight waves stream on it.  R: the fewest ranges whose
  // slice of x fits, or one more.  Up to 8 rows the waves read x directly
  // instead (kXDirect below: no partial tiles, no second kernel), measured
  // 2-16 % faster at M = 5-8 on Flux's fc2 and T5's wo; from 12 rows the
  // ranges are 7-40 % faster.
  if (allow_split && M > 8) {
    double best_cost = 0.0;
    int bestR = 0, bestT = 0, bestS = 0;
    int rmin = 0;
    for (int R = 2; R <= kMaxRanges && R <= nchunk; ++R) {
      const int64_t nb = (nchunk + R - 1) / R;
      if (M * (nb * 128 + 8) * 2 > kStageXMax) continue;
      if (!rmin) rmin = R;
      if (R > rmin + 1) break;
      for (int T = 16; T >= 1; --T) {
        for (int S = 1; T * S <= kMaxWaves[kXSplit] && S <= nb; ++S) {
          const QmvLds l = qmv_lds(kXSplit, int(M), int(K), group_size, T, S, p.row_blocks, R);
          if (l.total > kLdsMax) break;
          const int64_t blocks = (tiles + T - 1) / T * R;
          const int64_t per_cu = std::min<int64_t>(kLdsMax / l.total, 32 / (T * S));
          const int64_t load = (blocks + ncu - 1) / ncu; // blocks on the busiest CU
          const int64_t active = std::min(per_cu, load) * T * S;
          const double x_chunks = 0.25 * double(M) / bits;       // per chunk of K, per block
          const double part = double(R) * M * 16 * 8 / (256.0 * bits); // per tile
          const double cost = double(load) * (double(nb) * (T + x_chunks) + T * part) *
                              std::max(1.0, 8.0 / double(active));
          if (!bestR || cost < best_cost - 1e-9) {
            best_cost = cost;
            bestR = R;
            bestT = T;
            bestS = S;
          }
        }
      }
    }
    if (bestR) {
      p.xmode = kXSplit;
      p.ranges = bestR;
      p.tiles_per_block = bestT;
      p.waves = bestS;
      p.lds_bytes = qmv_lds(kXSplit, int(M), int(K), group_size, bestT, bestS, p.row_blocks, bestR).total;
      p.partial_floats = size_t(bestR) * size_t(tiles) * size_t(p.row_blocks) * 64 * 4;
      return p;
    }
  }
  p.xmode = kXDirect;
  p.tiles_per_block = 1;
  p.waves = waves_for(1, kMaxWaves[kXDirect]);
  p.lds_bytes = fits(kXDirect, 1, p.waves);
  if (!p.lds_bytes) fail("qmv: no launch shape fits the LDS");
  return p;
}

void qmv(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, const QmvPlan &plan, const Epilogue &ep, hipStream_t stream, float *partial) {
  if (M < 1 || !qmv_takes(M, N, K))
    fail("qmv: M must be in [1, 32], or [1, 128] when N <= 4096 and 16 rows of x fit a block");
  if (N < 1 || K < 64 || K % 64 != 0) fail("qmv: bad N or K");
  if (group_size != 64 && group_size != 128) fail("qmv: group size must be 64 or 128");
  if (K % group_size != 0) fail("qmv: K % group_size != 0");
  if (bits != 4 && bits != 8) fail("qmv: bits must be 4 or 8");
  if (ldx < K || ldx % 8 != 0) fail("qmv: row stride of x must be >= K and a multiple of 8");
  // The kernel addresses the codes, x, scales and biases through 32-bit
  // buffer windows, and uses 2^31 as its out-of-range offset.
  const int64_t lim = int64_t(1) << 31;
  if (N * K * bits / 8 >= lim || (M - 1) * ldx * int64_t(dtype_size(x_dtype)) + K * 4 >= lim ||
      N * (K / group_size) * int64_t(dtype_size(s_dtype)) >= lim)
    fail("qmv: x, the packed weight, scales and biases must each be under 2 GiB");
  if (plan.row_groups < 1 || plan.row_groups > 8 || (plan.row_groups > 1 && plan.xmode != kern_xblock()))
    fail("qmv: bad row groups");
  if (plan.row_groups > 1 ? plan.row_blocks != 1 || plan.row_groups != (M + 15) / 16
                          : M > 32 || plan.row_blocks != (M <= 16 ? 1 : 2))
    fail("qmv: plan's row blocks do not cover M");
  using namespace qmv_detail;
  if ((K / 128 + 1) * int64_t(std::max(plan.waves, kMaxRanges) + 1) >= lim)
    fail("qmv: K too large for the chunk arithmetic");
  if (plan.xmode < kXDirect || plan.xmode > kXSplit || plan.tiles_per_block < 1 || plan.waves < 1 ||
      plan.tiles_per_block * plan.waves > kMaxWaves[plan.xmode] ||
      (plan.xmode != kXBlock && plan.xmode != kXSplit && plan.tiles_per_block != 1) ||
      (plan.xmode == kXWave && M > 4) || plan.ranges < 1 || plan.ranges > kMaxRanges ||
      (plan.xmode != kXSplit && plan.ranges != 1) || plan.ranges > (K + 127) / 128)
    fail("qmv: inconsistent plan");
  const int64_t tiles = (N + 15) / 16;
  if (plan.ranges > 1) {
    if (!partial) fail("qmv: a plan with K ranges needs its partial-tile workspace");
    if (plan.partial_floats < size_t(plan.ranges) * size_t(tiles) * size_t(plan.row_blocks) * 256)
      fail("qmv: the plan's workspace is too small for its partial tiles");
  }
  const QmvLds l = qmv_lds(plan.xmode, plan.row_groups > 1 ? 16 : int(M), int(K), group_size,
                           plan.tiles_per_block, plan.waves, plan.row_blocks, plan.ranges);
  if (plan.xmode == kXWave && l.cmax > kXWaveMaxChunks) fail("qmv: a wave's x slice is too long to stage");
  if (l.total != plan.lds_bytes || l.total > kLdsMax) fail("qmv: plan's LDS size is wrong or too large");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) fail("qmv: x must be 16-byte aligned");
  if (!epilogue_ok(ep)) fail("qmv: bad epilogue (bias dtype or activation)");
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
