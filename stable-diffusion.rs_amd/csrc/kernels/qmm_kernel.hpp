// qmm_kernel.hpp -- y = x @ dequantize(w).T for many rows of x: the prefill-shaped,
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

#pragma once

namespace sdq {
namespace qmm_detail {

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

// Tile order: tile t lies in group t / (group_m * tiles_n) of group_m tile
// rows (fewer in the last group), which it walks column by column, so that
// consecutive tiles share activation row panels (down a column) and weight
// column panels (along a row).
__device__ __forceinline__ void tile_rc(int tile, int tiles_m, int tiles_n, int group_m, int &tm, int &tn) {
  const int per_group = group_m * tiles_n;
  const int grp = tile / per_group;
  const int first = grp * group_m;
  const int rows = min(group_m, tiles_m - first);
  const int within = tile - grp * per_group;
  tm = first + within % rows;
  tn = within / rows;
}

// The hardware deals the blocks of a launch to its L2 domains (XCDs) round
// robin: block b runs on XCD b % xcds.  This renumbers them so that each XCD
// takes one contiguous run of the work order (a bijection on [0, G)), and
// the tiles that share operands share that XCD's L2.
__device__ __forceinline__ int xcd_order(int b, int G, int xcds) {
  if (xcds <= 1) return b;
  const int xcd = b % xcds, idx = b / xcds;
  const int q = G / xcds, r = G % xcds;
  return xcd * q + min(xcd, r) + idx;
}

// Work assignment of one launch.  Tiles are numbered in tile_rc's order.
// Data-parallel (sk_workers == 0): tiles [0, dp_tiles) are computed whole,
// one block each; each tile after that is split into `splits` K ranges of
// `steps_per_split` 64-wide steps, one block per range, each writing its f32
// partial tile to `partial` ([split tile][range][BM][256]);
// qmm_reduce_kernel adds them.  Stream-K (sk_workers = G > 0): G blocks share
// the tiles * K/64 iterations evenly (see the kernel); `partial` has G slots
// and `flags` G ints, zero between launches.
struct QmmWork {
  int tiles_m;
  int group_m;
  int xcds;
  int tiles_n;
  int tiles;
  int dp_tiles;
  int splits;
  int steps_per_split;
  int sk_workers;
  float *partial;
  int *flags;
};

template <int BITS, int XDT, int SDT, int ODT, int BM, int GS, bool SCH, bool SKM>
__global__ __launch_bounds__(kThreads, BM <= 64 ? 2 : 1) void qmm_kernel(
    typename Elem<ODT>::T *__restrict__ y, const typename Elem<XDT>::T *__restrict__ x,
    int64_t ldx, const uint32_t *__restrict__ w,
    const typename Elem<SDT>::T *__restrict__ scales,
    const typename Elem<SDT>::T *__restrict__ biases, int M, int N, int K, QmmWork wk,
    kern::Epilogue ep) {
  using XT = typename Elem<XDT>::T;
  using ST = typename Elem<SDT>::T;
  constexpr int MB = BM / 32;           // 32-row MFMA blocks per wave
  constexpr int kWordsPerStep = 2 * BITS; // 64 codes of one row
  constexpr int kHalfWords = BITS;        // this lane half's share
  constexpr int kWV = BITS / 4;           // u32x4 per lane per 32-row block
  // Three stages of BM rows x 64 bf16 (128 B = 32 words per row).
  constexpr int kStage = BM * 32;
  // The output staging reuses the LDS, 32 rows of a wave's 64 columns at a
  // time (padded rows): at 64-row tiles that can exceed the three stages.
  constexpr int kOutWords = 4 * 32 * (64 * int(sizeof(typename Elem<ODT>::T)) + 16) / 4;
  constexpr int kLdsWords = 3 * kStage > kOutWords ? 3 * kStage : kOutWords;
  __shared__ __attribute__((aligned(16))) uint32_t xs[kLdsWords];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 31;
  const int h = lane >> 5;
  const int steps = K / 64;
  const int groups = K / GS;
  int m0 = 0, nw = 0;
  floatx16 acc[MB][2];
  // The product of tile `tile` over the K steps [k_begin, k_end), into acc.
  auto run = [&](const int tile, const int k_begin, const int k_end) __attribute__((always_inline)) {
  {
    int tm, tn;
    tile_rc(tile, wk.tiles_m, wk.tiles_n, wk.group_m, tm, tn);
    m0 = tm * BM;
    nw = tn * kTileN + wave * 64;
  }
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

  // Scale and bias chunks (SCH): a 16-byte load brings kCG consecutive
  // groups of one row, so each row's scales and biases cost one load per
  // kCG groups instead of one per step -- a load instruction's cost is set
  // by the distinct cache lines it touches (32 rows here), not its bytes.
  // Needs 16-byte aligned scale rows; the host picks SCH accordingly.
  constexpr int kCG = 16 / int(sizeof(ST));
  auto chunk_of = [&](int step) { return ((step * 64) / GS) / kCG; };
  auto load_chunk = [&](int c, u32x4 (&cs)[2], u32x4 (&cb)[2]) {
    const uint32_t off = uint32_t(c) * 16;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      cs[j] = bload16(rs, soff[j], off);
      cb[j] = bload16(rb, soff[j], off);
    }
  };
  auto pick = [&](const u32x4 &v, int e) -> float {
    if constexpr (sizeof(ST) == 4) {
      const uint32_t wv = e == 0 ? v[0] : e == 1 ? v[1] : e == 2 ? v[2] : v[3];
      return __uint_as_float(wv);
    } else {
      const int d = e >> 1;
      const uint32_t wv = d == 0 ? v[0] : d == 1 ? v[1] : d == 2 ? v[2] : v[3];
      return Elem<SDT>::load(typename Elem<SDT>::T((e & 1) ? (wv >> 16) : (wv & 0xffffu)));
    }
  };

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
  //     s - 1 and is written to LDS stage (s + 2) % 3 in the third k-step of
  //     step s, when the tile of step s + 3 is requested; one barrier per
  //     step makes it visible;
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
  // SCH: one chunk in registers, always the one holding step s + 1 at the
  // top of step s.  That step's scale and bias are picked from it there (the
  // weight queue entry of step s + 1 was loaded without them), then the chunk
  // of step s + 2 is loaded if it differs -- a full step before its first
  // pick, and with no register copy that would wait for the load.
  u32x4 cs[2], cb[2];
  int c_cur = 0;
  if constexpr (SCH) {
    c_cur = chunk_of(min(k_begin + 1, k_last));
    load_chunk(c_cur, cs, cb);
  }
  __syncthreads();

  u32x4 a[MB];
  u32x4 bq[2][2];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) a[mb] = read_a(xs, 0, mb);
  dequant(w0, 0, bq[0]);

  // Dequantization of one k-step for both 32-row blocks of weights, cut into
  // pieces that are spread over the MFMA slots below (block j's pieces are
  // numbered j * kPieces + piece).  4-bit: piece 0 splits the word into even
  // and odd codes, pieces 1-4 each produce one packed bf16 pair.  8-bit:
  // pieces 0-3 each produce one pair.
  constexpr int kPieces = BITS == 4 ? 5 : 4;
  constexpr int kSlots = 2 * MB;    // MFMAs per k-step
  // Slots between an A fragment's last MFMA and its refill (with two or four
  // MFMAs per k-step every fragment is refilled for the next k-step at once).
  constexpr int kRefillLag = kSlots >= 8 ? 4 : 0;
  uint32_t lo[2], hi[2];
  auto dq_piece = [&](const WStep &ws, int i, int j, int piece, u32x4 &dst) {
    const float sc_ = ws.s[j], bi_ = ws.b[j];
    if constexpr (BITS == 4) {
      if (piece == 0) {
        const uint32_t wd = ws.q[j][0][i];
        lo[j] = opaque(wd & 0x0F0F0F0Fu);        // codes 0, 2, 4, 6
        hi[j] = opaque((wd >> 4) & 0x0F0F0F0Fu); // codes 1, 3, 5, 7
      } else {
        const int d = piece - 1;
        dst[d] = pack_bf16x2(fmaf(byte_f(lo[j], d), sc_, bi_), fmaf(byte_f(hi[j], d), sc_, bi_));
      }
    } else {
      const uint32_t wd = ws.q[j][i / 2][(i % 2) * 2 + piece / 2];
      const int e = 2 * (piece % 2);
      dst[piece] = pack_bf16x2(fmaf(byte_f(wd, e), sc_, bi_), fmaf(byte_f(wd, e + 1), sc_, bi_));
    }
  };

  int st0 = 0; // LDS stage of step s; s + 1 and s + 2 follow cyclically
  for (int step = k_begin; step < k_end; ++step) {
    const int st1 = st0 == 2 ? 0 : st0 + 1;
    const int st2 = st1 == 2 ? 0 : st1 + 1;
    const int wstep = min(step + 2, k_last);
    const int xstep = min(step + 3, k_last);
    if constexpr (SCH) {
      const int e1 = (min(step + 1, k_last) * 64) / GS - c_cur * kCG;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        w1.s[j] = pick(cs[j], e1);
        w1.b[j] = pick(cb[j], e1);
      }
      const int c2 = chunk_of(wstep);
      if (c2 != c_cur) {
        c_cur = c2;
        load_chunk(c2, cs, cb);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // Issue order is fixed by hand: every MFMA is followed by one small
    // piece of other work -- a slice of the next k-step's dequantization, an
    // LDS read refilling an A fragment, in k-step 0 the weight loads and in
    // k-step 2 the staging store and the next activation load -- so that the
    // matrix pipe and the VALU work side by side, global loads are spread
    // over the step, and no wait blocks a whole batch.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = i & 1;
      const WStep &wsrc = i < 3 ? w0 : w1;
      const int di = i < 3 ? i + 1 : 0;
      const uint32_t *csrc = xs + st0 * kStage;                 // this k-step's stage
      const uint32_t *nsrc = xs + (i < 3 ? st0 : st1) * kStage; // the next k-step's
#pragma unroll
      for (int t = 0; t < kSlots; ++t) {
        const int mb = t >> 1, j = t & 1;
        acc[mb][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[mb]), as_bf16x8(bq[c][j]), acc[mb][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        // Dequantization pieces of the next k-step, spread evenly.
#pragma unroll
        for (int pc = 0; pc < 2 * kPieces; ++pc)
          if ((pc * kSlots) / (2 * kPieces) == t)
            dq_piece(wsrc, di, pc / kPieces, pc % kPieces, bq[c ^ 1][pc / kPieces]);
        // A fragment m is refilled kRefillLag slots after its second MFMA,
        // once that MFMA has surely read it; the last fragments of a k-step
        // are refilled early in the next one, before their own use.
        if (j == 1) {
          const int m = (((t - kRefillLag - 1) % kSlots + kSlots) % kSlots) >> 1;
          if (t >= kRefillLag + 1)
            a[m] = read_a(nsrc, i < 3 ? i + 1 : 0, m); // used in the next k-step
          else
            a[m] = read_a(csrc, i, m);                 // used later in this one
        }
        if (i == 2) {
          const int q = mb;
          if (j == 0) {
            const int row = sr + 32 * q;
            *reinterpret_cast<u32x4 *>(&xs[st2 * kStage + row * 32 + ((sc ^ ((row >> 1) & 7)) * 4)]) = xr[q];
          } else {
            xr[q] = BLoad8<XDT>::get(rx, xoff[q], uint32_t(xstep) * 64 * sizeof(XT));
          }
        }
        if (i == 0 && t >= kSlots - 2) {
          // This step's share of the weight queue: step s + 2, one 32-row
          // block per slot.
          const int jj = t - (kSlots - 2);
          const uint32_t wso = uint32_t(wstep) * kWordsPerStep * 4;
          const uint32_t sso = uint32_t((wstep * 64) / GS) * sizeof(ST);
#pragma unroll
          for (int v = 0; v < kWV; ++v) w2.q[jj][v] = bload16(rw, woff[jj] + 16 * v, wso);
          if constexpr (!SCH) {
            w2.s[jj] = BLoadScalar<SDT>::get(rs, soff[jj], sso);
            w2.b[jj] = BLoadScalar<SDT>::get(rb, soff[jj], sso);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    w0 = w1;
    w1 = w2;
    st0 = st1;
    __syncthreads();
  }
  };

  // Output.  Accumulator entry e of lane (r, h) in tile (mb, j) is row
  // 32*mb + 8*(e/4) + 4*h + e%4, column 32*j + r of the wave's slab: one
  // store per element would write 2-byte pieces of two rows per instruction,
  // and the cost of a store is per instruction.  So each wave stages its
  // slab through its own part of the (now idle) LDS, a few 32-row blocks at
  // a time, and writes whole 128-byte row pieces with 16-byte stores (single
  // elements where the output rows are not 16-byte aligned).
  using OT = typename Elem<ODT>::T;
  constexpr int kChunkElems = 16 / int(sizeof(OT));
  constexpr int kCpr = 64 / kChunkElems;                 // 16-byte chunks per slab row
  constexpr int kRowBytes = 64 * int(sizeof(OT)) + 16;   // padded: no bank conflicts
  constexpr int kWaveLds = kLdsWords;                    // LDS bytes per wave (a quarter)
  constexpr int kPassMB = (kWaveLds / kRowBytes) / 32 >= 4 && MB % 4 == 0 ? 4
                          : (kWaveLds / kRowBytes) / 32 >= 2 && MB % 2 == 0 ? 2 : 1;
  static_assert(kPassMB * 32 * kRowBytes <= kWaveLds, "output staging exceeds the LDS");
  // The combine stage (gated residual or product) runs on the 16-byte
  // pieces as they leave the LDS, on values already rounded to the output
  // dtype (as the unfused add/multiply after the linear sees them).
  const bool comb = ep.combine != 0;
  auto a16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool comb_vec = comb && a16(ep.res) && (ep.ld_res * int64_t(dtype_size_dev(ep.res_dtype))) % 16 == 0 &&
                        (!ep.gate || a16(ep.gate));
  // PAIR (kern::Epilogue::pair): `produce` leaves each gate column's
  // product in the gate lanes; the pieces of up columns are not stored and a
  // gate piece goes to output column (c / 16) * 8 + c % 8 of the wave's 32.
  auto store_tile = [&](auto produce, auto pairc) {
    constexpr bool PAIR = decltype(pairc)::value;
    // Output layout (kern::Epilogue): a tile lies wholly on one side of the
    // split (a multiple of 256).
    const bool hi = ep.split > 0 && nw - wave * 64 >= ep.split;
    OT *const ybase = hi ? static_cast<OT *>(ep.y2) : y;
    const int nout = PAIR ? N / 2 : N;
    const int64_t ldo = hi ? ep.ldy2 : (ep.ldy > 0 ? ep.ldy : int64_t(nout));
    const int col0 = hi ? int(ep.split) : 0;
    const bool vec = nout % kChunkElems == 0 && a16(ybase) && (ldo * int64_t(sizeof(OT))) % 16 == 0;
    uint8_t *wl = reinterpret_cast<uint8_t *>(xs) + wave * kWaveLds;
#pragma unroll
    for (int p0 = 0; p0 < MB; p0 += kPassMB) {
#pragma unroll
      for (int mb = p0; mb < p0 + kPassMB; ++mb) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          float v[16];
          produce(mb, j, v);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int row = 32 * (mb - p0) + 8 * (e / 4) + 4 * h + (e % 4);
            *reinterpret_cast<OT *>(wl + row * kRowBytes + (32 * j + r) * int(sizeof(OT))) =
                Elem<ODT>::store(v[e]);
          }
        }
      }
      // The slab is read back by other lanes of this wave only.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // Piece `it` of the slab back from the LDS to y; with the combine
      // stage (CB) the pieces go one at a time (a loop, not unrolled: the
      // stage's dtype cases would otherwise be copied into every piece).
      auto readback = [&](const int it, auto cb) {
        const int idx = it * 64 + lane;
        const int row = idx / kCpr, chunk = idx % kCpr;
        u32x4 v = *reinterpret_cast<const u32x4 *>(wl + row * kRowBytes + chunk * 16);
        const int grow = m0 + 32 * p0 + row;
        int gcol = nw + chunk * kChunkElems;
        if constexpr (PAIR) {
          const int c = chunk * kChunkElems; // slab column of the piece's first element
          if ((c & 8) != 0) return;          // an up piece
          gcol = nw / 2 + (c >> 4) * 8 + (c & 7);
        }
        if (grow >= M) return;
        OT *dst = ybase + int64_t(grow) * ldo + (gcol - col0);
        if constexpr (decltype(cb)::value) {
          if (gcol < nout) {
            // Whole chunk in range (vec) or the ragged last one (elementwise).
            float f[kChunkElems];
#pragma unroll
            for (int q = 0; q < kChunkElems; ++q) {
              const uint32_t word = v[(q * int(sizeof(OT))) / 4];
              f[q] = sizeof(OT) == 4 ? __uint_as_float(word)
                                     : Elem<ODT>::load(OT((q & 1) ? (word >> 16) : (word & 0xffffu)));
            }
            if (vec && comb_vec) {
              epi_combine_n<kChunkElems>(ep, grow, gcol, true, f);
            } else {
#pragma unroll
              for (int q = 0; q < kChunkElems; ++q)
                if (gcol + q < nout) f[q] = epi_combine(ep, f[q], grow, gcol + q);
            }
#pragma unroll
            for (int q = 0; q < kChunkElems; ++q) {
              const uint32_t bits = sizeof(OT) == 4 ? __float_as_uint(f[q]) : uint32_t(Elem<ODT>::store(f[q]));
              if constexpr (sizeof(OT) == 4) {
                v[q] = bits;
              } else {
                const int wi = q >> 1;
                v[wi] = (q & 1) ? ((v[wi] & 0xffffu) | (bits << 16)) : ((v[wi] & 0xffff0000u) | bits);
              }
            }
          }
        }
        if (vec) {
          if (gcol < nout) *reinterpret_cast<u32x4 *>(dst) = v;
        } else {
          // Rows not 16-byte aligned, or a ragged last chunk: element stores.
#pragma unroll
          for (int q = 0; q < kChunkElems; ++q) {
            if (gcol + q < nout) {
              const uint32_t word = v[(q * int(sizeof(OT))) / 4];
              if constexpr (sizeof(OT) == 4)
                dst[q] = __builtin_bit_cast(OT, word);
              else
                dst[q] = OT((q & 1) ? (word >> 16) : (word & 0xffffu));
            }
          }
        }
      };
      constexpr int kPieces = kPassMB * 32 * kCpr / 64;
      if (!PAIR && comb) {
#pragma unroll 1
        for (int it = 0; it < kPieces; ++it) readback(it, std::integral_constant<bool, !PAIR>{});
      } else {
#pragma unroll
        for (int it = 0; it < kPieces; ++it) readback(it, std::integral_constant<bool, false>{});
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  };

  // A K range's f32 accumulators in a workspace slot of BM x 256 floats:
  // 16-byte pieces, register-major -- entries 4q..4q+3 of MFMA tile (mb, j)
  // of thread t at float4 ((mb*2 + j)*4 + q)*256 + t -- so each store
  // instruction writes 1 KB contiguous per wave.  Rows past M are written too
  // and never used.
  // Partial tiles of the data-parallel split go through ordinary stores (the
  // reduction kernel reads them after this kernel ends).  Stream-K partials
  // are read by another block of this kernel, possibly on another XCD, whose
  // L2 is not this one's: they are written and read with device-coherent
  // (sc1) accesses, which go to the memory side instead of an XCD's L2, so
  // no L2 write-back or invalidation is needed around the flag (both would
  // cost every block on the XCD its cached tiles).
  const Rsrc rp = make_rsrc(wk.partial, 0x7ffffff0u);
  constexpr int kCoherent = 16; // the sc1 cache-policy bit
  auto part_off = [&](int64_t slot, int reg4) {
    return uint32_t(slot * (BM * kTileN * 4) + (int64_t(reg4) * kThreads + tid) * 16);
  };
  auto write_partial = [&](int64_t slot, bool coherent) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x4 v = {__float_as_uint(acc[mb][j][4 * q]), __float_as_uint(acc[mb][j][4 * q + 1]),
                           __float_as_uint(acc[mb][j][4 * q + 2]), __float_as_uint(acc[mb][j][4 * q + 3])};
          const uint32_t off = part_off(slot, (mb * 2 + j) * 4 + q);
          if (coherent)
            __builtin_amdgcn_raw_buffer_store_b128(v, rp, off, 0, kCoherent);
          else
            __builtin_amdgcn_raw_buffer_store_b128(v, rp, off, 0, 0);
        }
  };
  // Loads go out in batches of 16 (64 registers, free once the K loop is
  // done): one at a time, each would wait a full trip to the memory side.
  auto add_partial = [&](int64_t slot) {
    constexpr int kPieces4 = MB * 2 * 4, kBatch = 16;
#pragma unroll
    for (int b0 = 0; b0 < kPieces4; b0 += kBatch) {
      u32x4 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, part_off(slot, b0 + u), 0, kCoherent));
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int reg4 = b0 + u, mb = reg4 >> 3, j = (reg4 >> 2) & 1, q = reg4 & 3;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[mb][j][4 * q + c] += __uint_as_float(v[u][c]);
      }
    }
  };

  // The epilogue needs only the column's bias: one value per lane per 32-row
  // block of weights.  The activation is chosen once for the whole tile: a
  // per-element branch would end each element's LDS write in a wait.
  auto finish_tile = [&]() __attribute__((always_inline)) {
    float bcol[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) bcol[j] = epi_bias(ep, min(nw + 32 * j + r, N - 1));
    // PAIR: lane r holds gate column r when (r & 8) == 0 and the matching up
    // column in lane r + 8 (rows interleaved in blocks of eight).
    auto finish = [&](auto act, auto pairc) {
      store_tile([&](int mb, int j, float (&v)[16]) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float t = acc[mb][j][e] + bcol[j];
          const float a = decltype(act)::value ? gelu_approx_f(t) : t;
          if constexpr (decltype(pairc)::value)
            v[e] = a * __shfl_xor(t, 8);
          else
            v[e] = a;
        }
      }, pairc);
    };
    const bool hi = ep.split > 0 && nw - wave * 64 >= ep.split;
    const bool gelu = (hi ? ep.act2 : ep.act) == 1;
    if (ep.pair) {
      if (gelu)
        finish(std::integral_constant<bool, true>{}, std::integral_constant<bool, true>{});
      else
        finish(std::integral_constant<bool, false>{}, std::integral_constant<bool, true>{});
    } else if (gelu) {
      finish(std::integral_constant<bool, true>{}, std::integral_constant<bool, false>{});
    } else {
      finish(std::integral_constant<bool, false>{}, std::integral_constant<bool, false>{});
    }
  };

  // Data-parallel launch (sk_workers == 0): block b computes tile b whole,
  // or (b past dp_tiles) one K range of a split tile, whose partial the
  // reduction kernel that follows on the stream adds.
  //
  // Stream-K launch: worker g (this block) owns the iterations [lo(g),
  // lo(g+1)) of the tile-major sequence of (tile, K step), lo(g) = g*T/G.
  // Its range is at most three kinds of piece, done in this order:
  //   1. the tail: a tile's K prefix that goes on in worker g+1's range --
  //      a partial, stored in slot g, then flag g is raised;
  //   2. the whole tiles in between, stored directly;
  //   3. the head: the end of a tile begun by lower workers -- it waits for
  //      their flags (raised by pieces they did first), adds their partials
  //      in worker order (so the sum does not depend on timing) and stores
  //      the tile.
  // Waits point only to lower block indices, which the hardware dispatches
  // first, so no wait depends on a block not yet running; each wait is
  // bounded all the same (a flag that never comes leaves the tile without
  // that partial rather than hanging).  The three kinds are three inlined
  // copies of the K loop: a loop over mixed pieces keeps too much alive.
  if constexpr (!SKM) {
    // Whole tiles and split ranges are renumbered separately: the whole
    // tiles come first in dispatch order (the first round of the launch)
    // and must stay there, ahead of the split ranges.
    const int b = int(blockIdx.x);
    const int g = b < wk.dp_tiles ? xcd_order(b, wk.dp_tiles, wk.xcds)
                                  : wk.dp_tiles + xcd_order(b - wk.dp_tiles, int(gridDim.x) - wk.dp_tiles, wk.xcds);
    // Data-parallel launch: block b computes tile b whole, or (b past
    // dp_tiles) one K range of a split tile, whose partial the reduction
    // kernel that follows on the stream adds.  (An instantiation of its own:
    // the stream-K piece structure costs this loop ~9 % in register
    // allocation.)
    int tile = g, kb = 0, ke = steps;
    int64_t slot = -1;
    if (g >= wk.dp_tiles) {
      const int jb = g - wk.dp_tiles;
      tile = wk.dp_tiles + jb / wk.splits;
      const int split = jb % wk.splits;
      kb = split * wk.steps_per_split;
      ke = min(steps, kb + wk.steps_per_split);
      slot = int64_t(tile - wk.dp_tiles) * wk.splits + split;
    }
    run(tile, kb, ke);
    if (slot >= 0) {
      write_partial(slot, false);
      return;
    }
    finish_tile();
    return;
  }
  // Stream-K keeps the dispatch order: its waits point to lower block
  // indices, which must be dispatched first.
  const int g = blockIdx.x;
  const bool sk = true;
  int tail_tile = -1, tail_kb = 0, tail_ke = 0; // a partial piece, stored in slot g
  int64_t tail_slot = 0;
  int full_begin = 0, full_end = 0;             // whole tiles [full_begin, full_end)
  int head_tile = -1, head_kb = 0;              // the end of a tile begun by lower workers
  const int G = wk.sk_workers;
  const int64_t T = int64_t(wk.tiles) * steps;
  auto lo_of = [&](int gg) { return int64_t(gg) * T / G; };
  {
    const int64_t lo = lo_of(g);
    const int64_t hi = lo_of(g + 1);
    // Tiles touched: [t_first, t_last]; the head is t_first when lo is
    // inside it, the tail t_last when hi is inside it (possibly one tile).
    const int t_first = int(lo / steps), t_last = int((hi - 1) / steps);
    const int kb_first = int(lo - int64_t(t_first) * steps);
    const int ke_last = int(hi - int64_t(t_last) * steps);
    if (ke_last < steps) {
      tail_tile = t_last;
      tail_kb = t_first == t_last ? kb_first : 0;
      tail_ke = ke_last;
      tail_slot = g;
    }
    if (kb_first > 0 && !(tail_tile >= 0 && t_first == t_last)) {
      head_tile = t_first;
      head_kb = kb_first;
    }
    full_begin = t_first + (kb_first > 0 ? 1 : 0);
    full_end = t_last + (ke_last < steps ? 0 : 1);
  }
  bool ran = false;
  if (tail_tile >= 0) {
    run(tail_tile, tail_kb, tail_ke);
    write_partial(tail_slot, sk);
    if (sk) {
      // Every thread's coherent stores complete (s_waitcnt 0: all counters
      // drained) before the block's flag goes up.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (tid == 0) __hip_atomic_store(wk.flags + g, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    ran = true;
  }
  for (int tile = full_end - 1; tile >= full_begin; --tile) {
    if (ran) __syncthreads(); // the previous piece's output staging used the LDS
    run(tile, 0, steps);
    finish_tile();
    ran = true;
  }
  if (head_tile >= 0) {
    if (ran) __syncthreads();
    run(head_tile, head_kb, steps);
    const int64_t tile_lo = int64_t(head_tile) * steps;
    int from = g - 1;
    while (from > 0 && lo_of(from) > tile_lo) --from;
    for (int gg = from; gg < g; ++gg) {
      if (tid == 0) {
        int spins = 0;
        // Coherent (sc1) polls: the flag is read at the memory side.
        while (__hip_atomic_load(wk.flags + gg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0 &&
               ++spins < (1 << 22))
          __builtin_amdgcn_s_sleep(2);
        __hip_atomic_store(wk.flags + gg, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // The partial's loads are issued only after the flag was seen (the
      // barrier follows the poll), and read it coherently as well.
      __syncthreads();
      add_partial(gg);
    }
    finish_tile();
  }
}

// Sum of the K ranges of the split tiles, in range order (so the result does
// not depend on which block finished first), with the epilogue, converted to
// the output type.  Thread i of the launch takes float4 i of the partial
// layout: four consecutive rows of one column (accumulator entries 4q..4q+3
// of one MFMA tile of one tile-kernel thread).
template <int ODT>
__global__ __launch_bounds__(256) void qmm_reduce_kernel(typename Elem<ODT>::T *__restrict__ y,
                                                         const float *__restrict__ partial,
                                                         int M, int N, int bm, int tiles_m, int tiles_n,
                                                         int group_m, int dp_tiles, int splits,
                                                         kern::Epilogue ep) {
  const int per_tile = bm * (kTileN / 4); // float4 pieces of one partial tile
  const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int sk = int(idx / per_tile);
  const int within = int(idx % per_tile);
  const int reg4 = within / kThreads;      // (mb*2 + j)*4 + q
  const int t = within % kThreads;         // the tile kernel's thread
  const int lane = t & 63, wave = t >> 6;
  const int mb = reg4 >> 3, j = (reg4 >> 2) & 1, q = reg4 & 3;
  const int row = 32 * mb + 8 * q + 4 * (lane >> 5);  // first of four rows
  const int col = wave * 64 + 32 * j + (lane & 31);
  const int tile = dp_tiles + sk;
  int tm, tn;
  tile_rc(tile, tiles_m, tiles_n, group_m, tm, tn);
  const int grow = tm * bm + row;
  const int gcol = tn * kTileN + col;
  if (grow >= M || gcol >= N) return;
  // Gated pair: the thread of a gate column also sums the matching up column
  // (eight columns on: the partial layout's thread t + 8); up columns' threads
  // have nothing to store.
  if (ep.pair && (gcol & 8)) return;
  auto sum_of = [&](int64_t w) {
    const float4 *src = reinterpret_cast<const float4 *>(partial) + int64_t(sk) * splits * per_tile + w;
    float4 sum = src[0];
    for (int p0 = 1; p0 < splits; p0 += 4) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (p0 + u < splits) v[u] = src[int64_t(p0 + u) * per_tile];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (p0 + u < splits) {
          sum.x += v[u].x;
          sum.y += v[u].y;
          sum.z += v[u].z;
          sum.w += v[u].w;
        }
    }
    return sum;
  };
  const float4 sum = sum_of(within);
  const float b = epi_bias(ep, gcol);
  const float s4[4] = {sum.x, sum.y, sum.z, sum.w};
  if (ep.pair) {
    const float4 up = sum_of(within + 8);
    const float bu = epi_bias(ep, gcol + 8);
    const float u4[4] = {up.x, up.y, up.z, up.w};
    const int ocol = (gcol >> 4) * 8 + (gcol & 7);
    const int64_t ldo = ep.ldy > 0 ? ep.ldy : int64_t(N / 2);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (grow + u < M)
        y[int64_t(grow + u) * ldo + ocol] = Elem<ODT>::store(epi_apply(ep, s4[u], b) * (u4[u] + bu));
    return;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u)
    if (grow + u < M) {
      float v = Elem<ODT>::round(epi_apply_col(ep, s4[u], b, gcol));
      // The combine stage on the value rounded to the output dtype, as in the
      // tile kernel's store.
      if (ep.combine) v = epi_combine(ep, v, grow + u, gcol);
      *epi_dst(ep, y, N, grow + u, gcol) = Elem<ODT>::store(v);
    }
}

template <int BITS, int XDT, int SDT, int ODT, int BM>
void launch_qmm_t(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K, int gs,
                  const kern::QmmPlan &plan, const kern::SplitWorkspace &ws,
                  const kern::Epilogue &ep, hipStream_t st) {
  const QmmWork wk{plan.tiles_m, plan.group_m, plan.xcds, plan.tiles_n, plan.tiles, plan.dp_tiles, plan.splits, plan.steps_per_split, plan.sk_workers,
                   ws.partial, ws.flags};
  const dim3 grid(plan.blocks);
  auto *yp = static_cast<typename Elem<ODT>::T *>(y);
  auto *xp = static_cast<const typename Elem<XDT>::T *>(x);
  auto *sp = static_cast<const typename Elem<SDT>::T *>(s);
  auto *bp = static_cast<const typename Elem<SDT>::T *>(b);
  // Chunked scale loads need every scale row 16-byte aligned.
  const size_t srow_bytes = size_t(K / gs) * sizeof(typename Elem<SDT>::T);
  const bool sch = srow_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(s) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(b) % 16 == 0;
#define SDQ_QMM_LAUNCH(G, C)                                                                               \
  do {                                                                                                     \
    if (plan.sk_workers > 0) {                                                                             \
      if constexpr (BM == 256)                                                                             \
        qmm_kernel<BITS, XDT, SDT, ODT, BM, G, C, true>                                                    \
            <<<grid, kThreads, 0, st>>>(yp, xp, ldx, w, sp, bp, M, N, K, wk, ep);                          \
      else                                                                                                 \
        fail("qmm: stream-K plans use 256-row tiles");                                                     \
    } else {                                                                                               \
      qmm_kernel<BITS, XDT, SDT, ODT, BM, G, C, false>                                                     \
          <<<grid, kThreads, 0, st>>>(yp, xp, ldx, w, sp, bp, M, N, K, wk, ep);                            \
    }                                                                                                      \
  } while (0)
  if (gs == 64) {
    if (sch) SDQ_QMM_LAUNCH(64, true);
    else SDQ_QMM_LAUNCH(64, false);
  } else {
    if (sch) SDQ_QMM_LAUNCH(128, true);
    else SDQ_QMM_LAUNCH(128, false);
  }
#undef SDQ_QMM_LAUNCH
  const int sk_tiles = plan.sk_workers ? 0 : plan.tiles - plan.dp_tiles;
  if (sk_tiles > 0) {
    hip_check(hipGetLastError(), "qmm launch");
    const int64_t threads = int64_t(sk_tiles) * BM * (kTileN / 4);
    qmm_reduce_kernel<ODT><<<dim3(unsigned(threads / 256)), 256, 0, st>>>(
        yp, ws.partial, M, N, BM, plan.tiles_m, plan.tiles_n, plan.group_m, plan.dp_tiles, plan.splits, ep);
  }
}

template <int BITS, int XDT, int SDT, int ODT>
void launch_qmm_bm(void *y, const void *x, int64_t ldx, const uint32_t *w,
                   const void *s, const void *b, int M, int N, int K, int gs,
                   const kern::QmmPlan &plan, const kern::SplitWorkspace &ws,
                   const kern::Epilogue &ep, hipStream_t st) {
  if (plan.bm == 64)
    launch_qmm_t<BITS, XDT, SDT, ODT, 64>(y, x, ldx, w, s, b, M, N, K, gs, plan, ws, ep, st);
  else if (plan.bm == 128)
    launch_qmm_t<BITS, XDT, SDT, ODT, 128>(y, x, ldx, w, s, b, M, N, K, gs, plan, ws, ep, st);
  else
    launch_qmm_t<BITS, XDT, SDT, ODT, 256>(y, x, ldx, w, s, b, M, N, K, gs, plan, ws, ep, st);
}

// One activation/scale/output dtype combination of the tile kernel, for 4 or
// 8 bits: instantiated once per combination in its own translation unit
// (qmm_inst.hip, compiled once per combination) so the build runs in parallel.
template <int XD, int SD, int OD>
void qmm_combo(int bits, void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s,
               const void *b, int M, int N, int K, int gs, const kern::QmmPlan &plan,
               const kern::SplitWorkspace &ws, const kern::Epilogue &ep, hipStream_t st);

template <int XD, int SD, int OD>
void qmm_combo(int bits, void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s,
               const void *b, int M, int N, int K, int gs, const kern::QmmPlan &plan,
               const kern::SplitWorkspace &ws, const kern::Epilogue &ep, hipStream_t st) {
  if (bits == 4)
    launch_qmm_bm<4, XD, SD, OD>(y, x, ldx, w, s, b, M, N, K, gs, plan, ws, ep, st);
  else
    launch_qmm_bm<8, XD, SD, OD>(y, x, ldx, w, s, b, M, N, K, gs, plan, ws, ep, st);
}

} // namespace qmm_detail
} // namespace sdq
