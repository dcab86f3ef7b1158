// qmm.hip -- the launch planner and dtype dispatch of the large-M tile kernel
// (qmm_kernel.hpp holds the kernel; qmm_inst.hip instantiates it per dtype
// combination): the MFMA-bound side of mlx_quantized_matmul
// (crates/sd-tensor/src/mlx.rs:386-397, 1947-1975).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <string>

#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace qmm_detail {

constexpr int kTileN = 256;

// One activation/scale/output dtype combination of the tile kernel, for 4 or
// 8 bits: instantiated once per combination in its own translation unit
// (qmm_inst.hip, compiled once per combination) so the build runs in parallel.
template <int XD, int SD, int OD>
void qmm_combo(int bits, void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s,
               const void *b, int M, int N, int K, int gs, const kern::QmmPlan &plan,
               const kern::SplitWorkspace &ws, const kern::Epilogue &ep, hipStream_t st);

} // namespace qmm_detail

namespace {
#define SDQ_QMM_CASE(XD, SD, OD)                                                           \
  if (x_dtype == XD && s_dtype == SD && y_dtype == OD) {                                   \
    qmm_detail::qmm_combo<XD, SD, OD>(bits, y, x, ldx, w, scales, biases, int(M), int(N),  \
                                      int(K), group_size, plan, ws, ep, stream);           \
    hip_check(hipGetLastError(), "qmm launch");                                            \
    return;                                                                                \
  }

} // namespace

namespace kern {

namespace {

// The plan for tiles of `bm` rows, and its estimated cost (`*cost`, in
// thousandths of one block's 64-wide K step at that tile height).
QmmPlan plan_qmm_bm(int64_t M, int64_t N, int64_t K, int bits, int cus, size_t max_partial_floats,
                    bool allow_stream_k, int bm, int64_t *cost) {
  QmmPlan p;
  p.bm = bm;
  p.tiles_n = int((N + qmm_detail::kTileN - 1) / qmm_detail::kTileN);
  const int64_t tiles_m = (M + p.bm - 1) / p.bm;
  p.tiles_m = int(tiles_m);
  p.tiles = int(tiles_m * p.tiles_n);
  const int64_t steps = K / 64;
  // One block per CU at a time.  (Two 64-row blocks fit on a CU, but a CU
  // runs two at about half the speed each: measured, no gain in throughput.)
  const int64_t slots = cus > 0 ? cus : 256;
  const int64_t rem = p.tiles % slots;
  const size_t tile_floats = size_t(p.bm) * qmm_detail::kTileN;
  // Costs in thousandths of one block's 64-wide K step.
  // Data-parallel: whole tiles in rounds of `slots`.  The last, partly filled
  // round costs as much as a full one; its tiles can instead be split along
  // K into ranges that run side by side: a range costs its length, plus a
  // fixed part (writing its partial tile, and the reduction kernel's
  // launch), plus its share of the reduction kernel, which reads every
  // partial tile once at roughly HBM speed.
  constexpr int64_t kSplitFixed = 4000;
  // (A 64-row partial tile is half the bytes of the 128-row tiles the
  // constant was measured on.)
  const int64_t kReducePerRange = p.bm == 64 ? 23 : 45;
  p.dp_tiles = p.tiles;
  p.splits = 1;
  p.steps_per_split = int(steps);
  int64_t dp_cost = (p.tiles + slots - 1) / slots * steps * 1000;
  if (rem > 0) {
    int64_t best = steps * 1000;
    for (int64_t s = 2; s <= 16 && rem * s <= slots; ++s) {
      const int64_t sps = (steps + s - 1) / s;
      if (sps < 2) break;
      const int64_t ranges = (steps + sps - 1) / sps;
      if (size_t(rem * ranges) * tile_floats > max_partial_floats) continue;
      const int64_t cost = sps * 1000 + kSplitFixed + rem * ranges * kReducePerRange;
      if (cost < best) {
        best = cost;
        p.splits = int(ranges);
        p.steps_per_split = int(sps);
      }
    }
    if (p.splits > 1) {
      p.dp_tiles = int(p.tiles - rem);
      dp_cost = p.dp_tiles / slots * steps * 1000 + best;
    }
  }
  // Stream-K: one block per CU, each taking an equal share of the
  // tiles x steps iterations.  A tile cut between blocks costs the
  // contributor a coherent partial-tile write and its owner one coherent
  // read per contributor, plus a second pipeline fill; measured on MI355X
  // at about 9 steps of a 256-row tile per partial moved (fc1 at M = 1024:
  // 36 steps of work ran 54 step-times), so stream-K pays only for long K
  // (Flux's fc2 and linear2 at 4096+ tokens: 5-10 % over whole tiles).
  constexpr int64_t kSkPerPartial = 9000;
  const int64_t T = int64_t(p.tiles) * steps;
  const int64_t G = std::min<int64_t>(slots, T / 4);
  if (allow_stream_k && p.bm == 256 && G >= 2 && rem > 0) {
    const int64_t share = (T + G - 1) / G;
    const int64_t contributors = (steps + share - 1) / share; // per cut tile, at most
    // Every piece after a block's first refills the pipeline (~2 steps).
    const int64_t pieces = share / steps + 2;
    const int64_t sk_cost = share * 1000 + (1 + contributors) * kSkPerPartial + (pieces - 1) * 2000;
    const size_t need = size_t(G) * tile_floats;
    if (sk_cost < dp_cost && need <= max_partial_floats) {
      p.dp_tiles = p.tiles;
      p.splits = 1;
      p.steps_per_split = int(steps);
      p.sk_workers = int(G);
      p.blocks = int(G);
      p.partial_floats = need;
      *cost = sk_cost;
      return p;
    }
  }
  const int64_t sk_tiles = p.tiles - p.dp_tiles;
  p.blocks = int(p.dp_tiles + sk_tiles * p.splits);
  p.partial_floats = size_t(sk_tiles) * size_t(p.splits) * tile_floats;
  // Data-parallel launches run in XCD order (MI355X: 8 XCDs of 32 CUs, each
  // with its own L2), each XCD taking a contiguous run of the tile order.
  // The group height makes one XCD's run a near-square block of tiles,
  // weighted by the bytes a tile row shares (its activation panel, BM rows)
  // against a tile column (its weight panel, 256 rows of codes): rows / cols
  // ~ weight bytes / activation bytes = bits / (8 * 2) * 256 / BM.
  p.xcds = slots % 8 == 0 && slots >= 64 ? 8 : 1;
  {
    const double per_xcd = std::max(1.0, double(p.tiles) / p.xcds);
    const double ratio = double(bits) / 16.0 * 256.0 / p.bm;
    const int64_t gm = int64_t(std::lround(std::sqrt(per_xcd * ratio)));
    p.group_m = int(std::clamp<int64_t>(gm, 1, tiles_m));
  }
  *cost = dp_cost;
  return p;
}

} // namespace

QmmPlan plan_qmm(int64_t M, int64_t N, int64_t K, int bits, int cus, size_t max_partial_floats,
                 bool allow_stream_k) {
  int64_t cost = 0;
  // 64-row tiles for M <= 64: half the MFMAs and activation staging of a
  // 128-row tile, the same weight stream (measured 10-15 % faster at
  // M = 33-64 on the Flux and T5 shapes).
  if (M <= 64) return plan_qmm_bm(M, N, K, bits, cus, max_partial_floats, allow_stream_k, 64, &cost);
  if (M <= 128) return plan_qmm_bm(M, N, K, bits, cus, max_partial_floats, allow_stream_k, 128, &cost);
  // Above 128 rows both heights are priced.  A 256-row step costs about 1.3-
  // 1.4 times a 128-row one (measured: T5's paired wi at M = 384, one round
  // of 64 steps either way, 100 vs 76 us), so 128-row tiles win where they
  // fill the CUs with fewer split ranges (M = 192-640 on several Flux and T5
  // shapes: 5-24 % faster); 256-row tiles everywhere else (M >= 768 at the
  // Flux widths).  At 1.4 the choice matched the faster height at 20 of 24
  // measured points, the others within 5 %.
  int64_t c128 = 0, c256 = 0;
  const QmmPlan p128 = plan_qmm_bm(M, N, K, bits, cus, max_partial_floats, allow_stream_k, 128, &c128);
  const QmmPlan p256 = plan_qmm_bm(M, N, K, bits, cus, max_partial_floats, allow_stream_k, 256, &c256);
  return c128 * 10 < c256 * 14 ? p128 : p256;
}

void qmm(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, const QmmPlan &plan, const SplitWorkspace &ws, const Epilogue &ep,
         hipStream_t stream) {
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
  const QmmPlan want = plan_qmm(M, N, K, bits, 0);
  if (plan.bm != want.bm || plan.tiles_n != want.tiles_n || plan.tiles != want.tiles ||
      plan.tiles_m != want.tiles_m || plan.group_m < 1 || plan.group_m > plan.tiles_m || plan.xcds < 1)
    fail("qmm: inconsistent launch plan");
  if (plan.sk_workers > 0) {
    if (plan.blocks != plan.sk_workers || int64_t(plan.sk_workers) > int64_t(plan.tiles) * (K / 64) ||
        plan.dp_tiles != plan.tiles)
      fail("qmm: inconsistent stream-K plan");
    if (!ws.partial || !ws.flags) fail("qmm: stream-K launch without a workspace");
  } else {
    if (plan.splits < 1 || plan.steps_per_split < 1 || plan.dp_tiles < 0 || plan.dp_tiles > plan.tiles ||
        plan.blocks != plan.dp_tiles + (plan.tiles - plan.dp_tiles) * plan.splits ||
        (plan.dp_tiles < plan.tiles &&
         (int64_t(plan.splits - 1) * plan.steps_per_split >= K / 64 ||
          int64_t(plan.splits) * plan.steps_per_split < K / 64)))
      fail("qmm: inconsistent launch plan");
    if (plan.dp_tiles < plan.tiles && !ws.partial) fail("qmm: split-K launch without a workspace");
  }
  if (!kern::epilogue_ok(ep)) fail("qmm: bad epilogue (bias dtype or activation)");
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
