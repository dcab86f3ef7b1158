// qmv_kernel.hpp -- y = x @ dequantize(w).T for few rows of x (M <= 32, up to
// 128 in row groups of 16): the
// bandwidth-bound decode/modulation shape of mlx_quantized_matmul
// (crates/sd-tensor/src/mlx.rs:386-397, 1947-1975; callers e.g. the Flux
// modulation linears at M = 1, sd-models/src/mlx/flux.rs:279-299, 437, and the
// T5 FFN at few tokens, t5.rs:209-214).
//
// Time here is the packed weight stream, so the kernel is laid out as a
// stream with little work per byte and nothing serialised behind it:
//
//   * A block owns T tiles of 16 weight rows (output columns) and all of K.
//     Its T*S waves each stream one tile over one of S contiguous K ranges;
//     at the end the S waves of a tile add their partial tiles through LDS in
//     range order (deterministic) and the first applies the epilogue and
//     stores.  No partial result leaves the block and there is no second pass.
//   * Each wave stages the scales and biases of its 16 rows and K range in
//     its own LDS region, as (s, b - OFF*s) pairs, and -- at M <= 4 -- its
//     slice of x as bf16 (XMode kXWave): no block-wide barrier stands between
//     a wave and its stream.  For larger M with a small x the block stages x
//     once for all its tiles (kXBlock).  When x is too large for that, K is
//     cut into R ranges, one per block (kXSplit): a block stages its range
//     of x once for its T tiles and stores partial tiles, which
//     qmv_reduce_kernel adds in range order and finishes with the epilogue.
//     Otherwise each wave reads its activation fragments per chunk from
//     global memory (kXDirect).
//   * MFMA v_mfma_f32_16x16x32_bf16 with the weight rows on its N side and
//     the tokens on its M side (16 rows per MFMA row block, two blocks for
//     M <= 32).  Lane (n, h) = (lane % 16, lane / 16) supplies weight row n
//     and token row n of the row block.  Codes are loaded 16 bytes per lane,
//     16 rows x 64 bytes per load instruction, in chunks of 128 K:
//       4-bit: one load per chunk; lane h holds K [32h, 32h + 32) as four
//       words.  A 4 x 4 transpose of words across the four lane groups
//       (v_permlane32_swap, then v_permlane16_swap) leaves word i of lane h
//       holding K [32i + 8h, 32i + 8h + 8), so MFMA i of the chunk covers K
//       [32i, 32i + 32) -- inside group i / 2.
//       8-bit: two loads per chunk (one per group); MFMA i takes words
//       2i, 2i + 1, i.e. K [64(i/2) + 16h + 8(i%2), +8).
//   * Codes are never dequantized element by element.  The MFMA multiplies x
//     by c_k = q_k + OFF held EXACTLY in bf16 (4-bit: OFF = 128, the pattern
//     0x43nn built by byte permutes; 8-bit: OFF = 0, q converted), giving
//     t[m][n] = sum_k x[m,k] c_k per group, and a second MFMA against ones
//     gives the group sums X[m] = sum_k x[m,k] in the same lane layout.  Then
//     y += s t + (b - OFF s) X: the affine dequantization is applied once per
//     group per output, in f32, which is more accurate than rounding each
//     dequantized weight to bf16.
//   * kDepth chunks of loads are in flight per wave.  Chunks past a wave's
//     range are addressed beyond the buffer's end: such loads return zeros
//     without touching memory.
#pragma once

#include <algorithm>

#include "device_common.hpp"
#include "launch.hpp"
#include "qmv_lds.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace qmv_detail {

using namespace dev;

constexpr int kDepth = 2;       // 128-wide chunks in flight per wave (default)
constexpr uint32_t kOob = 0x80000000u; // an offset past every buffer (all are < 2 GiB)

// v_permlane32_swap: lanes 32-63 of a trade places with lanes 0-31 of b.
__device__ __forceinline__ void perm32_swap(uint32_t &a, uint32_t &b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

// v_permlane16_swap: the odd 16-lane rows of a trade places with the even
// rows of b.
__device__ __forceinline__ void perm16_swap(uint32_t &a, uint32_t &b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

// MFMA B operand for eight 4-bit codes (one word, first code in the low bits)
// in natural K order, each as the exact bf16 value 128 + q (pattern 0x43nn):
// split into even and odd codes, interleave them back into code order, then
// pair each code byte with the constant exponent byte 0x43.
__device__ __forceinline__ u32x4 codes4_b(uint32_t wd) {
  const uint32_t lo = wd & 0x0F0F0F0Fu;        // c0 c2 c4 c6
  const uint32_t hi = (wd >> 4) & 0x0F0F0F0Fu; // c1 c3 c5 c7
  const uint32_t m0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u); // c0 c1 c2 c3
  const uint32_t m1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u); // c4 c5 c6 c7
  const uint32_t k43 = 0x43434343u;
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(k43, m0, 0x04010400u); // (c0, c1)
  r[1] = __builtin_amdgcn_perm(k43, m0, 0x04030402u); // (c2, c3)
  r[2] = __builtin_amdgcn_perm(k43, m1, 0x04010400u); // (c4, c5)
  r[3] = __builtin_amdgcn_perm(k43, m1, 0x04030402u); // (c6, c7)
  return r;
}

// The same eight codes without the interleave: bf16 pairs (c0, c2), (c4, c6),
// (c1, c3), (c5, c7) -- K slots in the order x_perm8 gives the activations.
__device__ __forceinline__ u32x4 codes4_b_split(uint32_t wd) {
  const uint32_t lo = wd & 0x0F0F0F0Fu;        // c0 c2 c4 c6
  const uint32_t hi = (wd >> 4) & 0x0F0F0F0Fu; // c1 c3 c5 c7
  const uint32_t k43 = 0x43434343u;
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(k43, lo, 0x04010400u); // (c0, c2)
  r[1] = __builtin_amdgcn_perm(k43, lo, 0x04030402u); // (c4, c6)
  r[2] = __builtin_amdgcn_perm(k43, hi, 0x04010400u); // (c1, c3)
  r[3] = __builtin_amdgcn_perm(k43, hi, 0x04030402u); // (c5, c7)
  return r;
}

// Eight activations (bf16 pairs (x0, x1) .. (x6, x7)) reordered to the K
// slots of codes4_b_split: (x0, x2), (x4, x6), (x1, x3), (x5, x7).  Applied
// once when x is staged, it saves two permutes per code word in the stream.
__device__ __forceinline__ u32x4 x_perm8(const u32x4 &v) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);
  r[2] = __builtin_amdgcn_perm(v[1], v[0], 0x07060302u);
  r[3] = __builtin_amdgcn_perm(v[3], v[2], 0x07060302u);
  return r;
}

// Eight 8-bit codes (two words), in element order, as exact bf16 values q.
__device__ __forceinline__ u32x4 codes8_b(uint32_t w0, uint32_t w1) {
  const uint32_t a = opaque(w0), b = opaque(w1);
  u32x4 r;
  r[0] = pack_bf16x2(float(a & 0xffu), float((a >> 8) & 0xffu));
  r[1] = pack_bf16x2(float((a >> 16) & 0xffu), float(a >> 24));
  r[2] = pack_bf16x2(float(b & 0xffu), float((b >> 8) & 0xffu));
  r[3] = pack_bf16x2(float((b >> 16) & 0xffu), float(b >> 24));
  return r;
}

__device__ __forceinline__ floatx4 mfma16(const u32x4 &a, const u32x4 &b, const floatx4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// K offset, within a 128-wide chunk, of lane group h's eight slots of MFMA i.
template <int BITS> __device__ __forceinline__ int slot_k(int i, int h) {
  return BITS == 4 ? 32 * i + 8 * h : 64 * (i >> 1) + 16 * h + 8 * (i & 1);
}

// One chunk's loads: the lane's codes and, when x is read directly, its
// activation fragments (MFMA i of row block mb).
template <int BITS, int MB, bool XD> struct Chunk {
  u32x4 q[BITS / 4];
  u32x4 a[XD ? MB : 1][XD ? 4 : 1];
};

// The epilogue of one 16-row block of a tile: accumulator entry e of lane
// (n, h) = (lane % 16, lane / 16) is token 16 mb + 4 h + e, output column
// 16 tile + n; m0 offsets the rows (row groups).  Every lane of the wave
// takes part (the gated pair trades values between lanes n and n ^ 8).
template <int ODT>
__device__ __forceinline__ void qmv_store_rows(typename Elem<ODT>::T *__restrict__ y, const kern::Epilogue &ep,
                                               const floatx4 &a, int mb, int M, int N, int tile, int lane,
                                               int m0 = 0) {
  const int ln = lane & 15, lh = lane >> 4;
  const int n = tile * 16 + ln;
  const float bn = epi_bias(ep, min(n, N - 1));
  if (ep.pair) {
    // Gated pair (kern::Epilogue::pair, N % 16 == 0): column ln < 8 of the
    // tile is a gate, ln + 8 (lane ^ 8) its up column; output column
    // 8 tile + ln of N / 2.
    const int64_t ldo = ep.ldy > 0 ? ep.ldy : int64_t(N / 2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float up = __shfl_xor(a[e] + bn, 8);
      const int m = mb * 16 + 4 * lh + e;
      if (ln < 8 && m < M) y[(m0 + m) * ldo + tile * 8 + ln] = Elem<ODT>::store(epi_apply(ep, a[e], bn) * up);
    }
    return;
  }
  if (n >= N) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = mb * 16 + 4 * lh + e;
    if (m < M)
      *epi_dst(ep, y, N, m0 + m, n) = Elem<ODT>::store(epi_combine(ep, epi_apply_col(ep, a[e], bn, n), m0 + m, n));
  }
}

// MB: 16-token MFMA row blocks (M <= 16 * MB).  GS: group size (64 or 128).
// XM: where x comes from (XMode).  Launch: grid = ceil(tiles / T) (times R
// for kXSplit, range-major), T * S waves.  partial (kXSplit, R > 1): R x
// tiles x MB x 64 float4, the range's accumulators of each tile.
template <int BITS, int XDT, int SDT, int ODT, int MB, int GS, int XM, int DEPTH = kDepth>
__global__ __launch_bounds__(64 * kMaxWaves[XM]) void qmv_kernel(
    typename Elem<ODT>::T *__restrict__ y, const typename Elem<XDT>::T *__restrict__ x,
    int64_t ldx, const uint32_t *__restrict__ w,
    const typename Elem<SDT>::T *__restrict__ scales,
    const typename Elem<SDT>::T *__restrict__ biases, int M, int N, int K, int T, int S,
    kern::Epilogue ep, int R, float *__restrict__ partial, int RG) {
  using XT = typename Elem<XDT>::T;
  using ST = typename Elem<SDT>::T;
  constexpr bool kXD = XM == kXDirect;
  constexpr float kOff = BITS == 4 ? 128.0f : 0.0f;
  constexpr int kChunkBytes = 128 * BITS / 8; // one row's codes per chunk
  constexpr int kGpc = 128 / GS;              // groups per chunk (1 or 2)

  // The wave index, and everything derived from it (tile, K range, chunk
  // offsets), is uniform across the wave: readfirstlane tells the compiler,
  // so the chunk offsets go to the loads' scalar offset.  (Derived from
  // threadIdx.x alone it counts as divergent, and every buffer load with
  // such a scalar offset becomes a loop over the distinct values.)
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int lane = int(threadIdx.x) & 63;
  const int ln = lane & 15;
  const int lh = lane >> 4;
  const int tl = wave / S;      // tile of this block
  const int rs = wave - tl * S; // K range of the tile
  const int tiles = (N + 15) / 16;
  // kXSplit: block b takes K range rr = b / ntb of tile group tb = b % ntb.
  constexpr bool kSplit = XM == kXSplit;
  const int ntb = (tiles + T - 1) / T;
  const int rr = kSplit ? int(blockIdx.x) / ntb : 0;
  // Row groups (kXBlock, RG > 1): block b takes rows [16 MB rg, +16 MB) of
  // tile group tbx; the RG blocks of a tile group are 8 apart, so they run
  // on one XCD close in time and read the group's codes from HBM once, then
  // from that XCD's L2.  Blocks past the last tile group have no live tile.
  int rg = 0, tbx = int(blockIdx.x);
  if (RG > 1) {
    rg = (tbx >> 3) % RG;
    tbx = (tbx / (8 * RG)) * 8 + (tbx & 7);
  }
  const int m0 = rg * 16 * MB;           // first row of this block
  const int Mlay = RG > 1 ? 16 * MB : M; // rows the LDS layout is sized for
  if (RG > 1) {
    x += int64_t(m0) * ldx;
    M = min(M - m0, 16 * MB);
  }
  const int tb = kSplit ? int(blockIdx.x) - rr * ntb : tbx;
  const int tile = tb * T + tl;
  const bool live = tile < tiles;
  const int n = tile * 16 + ln;
  const int nrow = min(n, N - 1); // rows past N are read, never stored
  const int groups = K / GS;

  // The block's chunks [b0, b1) of the 128-wide chunks (all of K but for
  // kXSplit), this wave's [c0, c1) and groups [g0, g1); the last chunk is
  // half when K % 128 == 64 (group size 64).
  const int nchunk = (K + 127) / 128;
  // 32-bit products: nchunk * max(S, R) < 2^31 (checked on the host).
  const int b0 = kSplit ? int(uint32_t(nchunk * rr) / uint32_t(R)) : 0;
  const int nb = (kSplit ? int(uint32_t(nchunk * (rr + 1)) / uint32_t(R)) : nchunk) - b0;
  const int c0 = b0 + int(uint32_t(nb * rs) / uint32_t(S));
  const int c1 = b0 + int(uint32_t(nb * (rs + 1)) / uint32_t(S));
  const int ncs = live ? c1 - c0 : 0;
  const bool half_tail = (K & 127) != 0;
  const int g0 = c0 * kGpc;
  const int gw = min(c1 * kGpc, groups) - g0;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const QmvLds L = qmv_lds(XM, Mlay, K, GS, T, S, MB, R);
  constexpr bool kStaged = XM == kXBlock || XM == kXSplit; // x staged once per block
  unsigned char *wreg = smem + L.wave + wave * L.wave_bytes;
  float2 *sbw = reinterpret_cast<float2 *>(wreg);                 // [16][L.gws]
  uint16_t *xl = reinterpret_cast<uint16_t *>(kStaged ? smem + L.x : wreg + L.wsb);
  floatx4 *red = reinterpret_cast<floatx4 *>(smem + L.red);

  // Buffer windows: byte offsets fit in 32 bits (checked on the host).
  const Rsrc rw = make_rsrc(w, uint32_t(int64_t(N) * K * BITS / 8));
  const uint32_t woff = uint32_t(int64_t(nrow) * K * BITS / 8) + uint32_t(16 * lh);
  const Rsrc rx = make_rsrc(x, uint32_t((int64_t(M - 1) * ldx + K) * sizeof(XT)));
  const Rsrc rs_ = make_rsrc(scales, uint32_t(int64_t(N) * groups * sizeof(ST)));
  const Rsrc rb_ = make_rsrc(biases, uint32_t(int64_t(N) * groups * sizeof(ST)));
  uint32_t xoff[MB];
  int xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    xrow[mb] = min(mb * 16 + ln, M - 1); // rows past M repeat row M - 1, never stored
    xoff[mb] = uint32_t(int64_t(xrow[mb]) * ldx * sizeof(XT));
  }

  auto load = [&](int i, Chunk<BITS, MB, kXD> &q) {
    // Local chunk i of this wave; past the range every load is out of bounds.
    const bool in = i < ncs;
    const int c = c0 + i;
    const uint32_t cw = in ? uint32_t(c) * kChunkBytes : kOob;
#pragma unroll
    for (int v = 0; v < BITS / 4; ++v) q.q[v] = bload16(rw, woff + 64 * v, cw);
    if constexpr (kXD) {
      const uint32_t cx = in ? uint32_t(c) * 128 * uint32_t(sizeof(XT)) : kOob;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          q.a[mb][j] = BLoad8<XDT>::get(rx, xoff[mb] + slot_k<BITS>(j, lh) * uint32_t(sizeof(XT)), cx);
    }
  };

  // 1. Staging.  Order matters, for two reasons.
  //    * The load counter retires in issue order: staging loads (x, the
  //      scale/bias pairs) go out before the code loads, so the waits for the
  //      staging do not include the codes, which keep streaming.
  //    * The compiler counts the loads in flight per register.  A load under
  //      a branch issued between a code load and its use makes it assume the
  //      worst and wait for every load.  So everything conditional (rows
  //      m < M, the scale form, long ranges) comes first, then the code
  //      loads, unconditionally, then the stores of the staged values.
  //    Few load instructions go out before the codes: the memory pipeline's
  //    cost is per instruction, not per byte.
  // Staged 4-bit: x is stored in the K-slot order of codes4_b_split.
  constexpr bool kXPerm = BITS == 4 && !kXD;
  Chunk<BITS, MB, kXD> ring[DEPTH + 1];
  {
    const uint32_t sbase = uint32_t(int64_t(nrow) * groups * sizeof(ST));
    const uint32_t soff0 = uint32_t(g0) * uint32_t(sizeof(ST));
    auto put = [&](int g, float sc, float bi) {
      if (g < gw) sbw[ln * L.gws + g] = make_float2(sc, fmaf(-kOff, sc, bi));
    };
    auto pick_e = [&](const u32x4 &v, int e) -> float {
      if constexpr (sizeof(ST) == 4) {
        return __uint_as_float(v[e]);
      } else {
        const uint32_t wv = v[e >> 1];
        return Elem<SDT>::load(typename Elem<SDT>::T((e & 1) ? (wv >> 16) : (wv & 0xffffu)));
      }
    };

    // (a) kXBlock, kXSplit: the block stages x (kXSplit: columns of its K
    //     range), eight values per piece, for its T tiles.  The first round
    //     of loads is held in registers and stored after the code loads;
    //     further rounds (large x) are loaded and stored here.
    constexpr int kXLoads = 8;
    const int tid = int(threadIdx.x);
    const int nthreads = int(blockDim.x);
    const int kx0 = b0 * 128;                         // first staged column
    const int per_row = (min((b0 + nb) * 128, K) - kx0) / 8;
    const int x_pieces = M * per_row;
    // Row of piece e: a float estimate corrected once (exact: the estimate
    // is off by at most one for these sizes).
    const float inv_per_row = 1.0f / float(per_row);
    auto x_row = [&](int e) {
      int m = int(float(e) * inv_per_row);
      m -= m * per_row > e;
      m += (m + 1) * per_row <= e;
      return m;
    };
    auto xb_load = [&](int base, u32x4 (&v)[kXLoads]) {
#pragma unroll
      for (int j = 0; j < kXLoads; ++j) {
        const int e = min(base + j * nthreads + tid, x_pieces - 1);
        const int m = x_row(e);
        v[j] = Load8<XDT>::get(x + int64_t(m) * ldx + kx0 + 8 * (e - m * per_row));
      }
    };
    auto xb_store = [&](int base, const u32x4 (&v)[kXLoads]) {
#pragma unroll
      for (int j = 0; j < kXLoads; ++j) {
        const int e = base + j * nthreads + tid;
        if (e < x_pieces) {
          const int m = x_row(e);
          *reinterpret_cast<u32x4 *>(xl + m * L.xstride + 8 * (e - m * per_row)) = kXPerm ? x_perm8(v[j]) : v[j];
        }
      }
    };
    u32x4 xb[kStaged ? kXLoads : 1];
    if constexpr (kStaged) {
      for (int base = kXLoads * nthreads; base < x_pieces; base += kXLoads * nthreads) {
        u32x4 v[kXLoads];
        xb_load(base, v);
        xb_store(base, v);
      }
      xb_load(0, xb);
    }

    // (b) kXWave: the wave's slice of x, rows m < M (M <= 4) of columns
    //     [128 c0, 128 c1), eight per piece.
    constexpr int kXIter = kXWaveMaxChunks * 16 / 64; // x pieces per lane and row
    u32x4 xv[XM == kXWave ? 4 : 1][kXIter];
    if constexpr (XM == kXWave) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= M) break;
#pragma unroll
        for (int j = 0; j < kXIter; ++j) {
          const int pc = lane + 64 * j;
          const uint32_t off = pc < ncs * 16 ? uint32_t((int64_t(m) * ldx + c0 * 128 + 8 * pc) * sizeof(XT)) : kOob;
          xv[m][j] = BLoad8<XDT>::get(rx, off, 0);
        }
      }
    }

    // (c) Scale and bias pieces.  Vector form (rows and the wave's first
    //     group 16-byte aligned): lane (r, p) loads groups [kE p, kE p + kE)
    //     of row r (plus 4 kE per further batch), kE = 16 / sizeof(ST), so
    //     one instruction covers 16 rows x 4 kE groups.  Scalar form: one
    //     group per lane, groups p + 4i.  Lanes past the range read zeros.
    //     The first kMaxBatch batches (16 groups in scalar form) are held in
    //     registers and stored after the code loads; further ones (long
    //     ranges) are loaded and stored here.
    constexpr int kE = 16 / int(sizeof(ST));
    constexpr int kMaxBatch = 2;
    const bool vec_sb = (groups * int(sizeof(ST))) % 16 == 0 && soff0 % 16 == 0;
    const int nbatch = vec_sb ? (gw + 4 * kE - 1) / (4 * kE) : (gw + 15) / 16;
    auto sb_off = [&](int g) { return g < gw ? sbase + uint32_t(g) * uint32_t(sizeof(ST)) : kOob; };
    u32x4 sq[kMaxBatch], bq[kMaxBatch];
    float sv[4], bv[4];
    if (vec_sb) {
      for (int bt = kMaxBatch; bt < nbatch; ++bt) {
        const int g = bt * 4 * kE + kE * lh;
        const u32x4 a = bload16(rs_, sb_off(g), soff0), b = bload16(rb_, sb_off(g), soff0);
#pragma unroll
        for (int e = 0; e < kE; ++e) put(g + e, pick_e(a, e), pick_e(b, e));
      }
#pragma unroll
      for (int bt = 0; bt < kMaxBatch; ++bt) {
        if (bt >= nbatch) break;
        const int g = bt * 4 * kE + kE * lh;
        sq[bt] = bload16(rs_, sb_off(g), soff0);
        bq[bt] = bload16(rb_, sb_off(g), soff0);
      }
    } else {
      for (int gb = 16; gb < gw; gb += 16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = gb + lh + 4 * i;
          put(g, BLoadScalar<SDT>::get(rs_, sb_off(g), soff0), BLoadScalar<SDT>::get(rb_, sb_off(g), soff0));
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[i] = BLoadScalar<SDT>::get(rs_, sb_off(lh + 4 * i), soff0);
        bv[i] = BLoadScalar<SDT>::get(rb_, sb_off(lh + 4 * i), soff0);
      }
    }

    // (d) The code loads of the first DEPTH chunks, unconditionally.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(d, ring[d]);
    __builtin_amdgcn_sched_barrier(0);

    // (e) Stores of the staged values.  The scale form is re-read through an
    //     opaque copy, so the compiler cannot merge this branch with (c) and
    //     move these stores (and their waits) above the code loads.
    if constexpr (kStaged) xb_store(0, xb);
    if constexpr (XM == kXWave) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= M) break;
#pragma unroll
        for (int j = 0; j < kXIter; ++j) {
          const int pc = lane + 64 * j;
          if (pc < ncs * 16) *reinterpret_cast<u32x4 *>(xl + m * L.xstride + 8 * pc) = kXPerm ? x_perm8(xv[m][j]) : xv[m][j];
        }
      }
    }
    int vec2 = __builtin_amdgcn_readfirstlane(int(vec_sb));
    asm volatile("" : "+s"(vec2));
    if (vec2) {
#pragma unroll
      for (int bt = 0; bt < kMaxBatch; ++bt) {
        if (bt >= nbatch) break;
#pragma unroll
        for (int e = 0; e < kE; ++e) put(bt * 4 * kE + kE * lh + e, pick_e(sq[bt], e), pick_e(bq[bt], e));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) put(lh + 4 * i, sv[i], bv[i]);
    }
    if constexpr (kStaged) {
      __syncthreads();
    } else {
      // The stage is this wave's own: a wave-scope fence orders it.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }

  // 2. Stream the chunks.
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  floatx4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = zero;
  const float2 *sbrow = sbw + ln * L.gws;
  // Column of chunk c's K range within the staged x rows.
  const int xcol0 = kStaged ? b0 * 128 : c0 * 128;

  // One chunk's math: chunk i (local) of the range, codes in q.
  auto process = [&](const int i, const Chunk<BITS, MB, kXD> &q) __attribute__((always_inline)) {
    const int c = c0 + i;
    u32x4 bq[4];
    if constexpr (BITS == 4) {
      uint32_t w0 = q.q[0][0], w1 = q.q[0][1], w2 = q.q[0][2], w3 = q.q[0][3];
      perm32_swap(w0, w2);
      perm32_swap(w1, w3);
      perm16_swap(w0, w1);
      perm16_swap(w2, w3);
      if constexpr (kXPerm) {
        bq[0] = codes4_b_split(w0);
        bq[1] = codes4_b_split(w1);
        bq[2] = codes4_b_split(w2);
        bq[3] = codes4_b_split(w3);
      } else {
        bq[0] = codes4_b(w0);
        bq[1] = codes4_b(w1);
        bq[2] = codes4_b(w2);
        bq[3] = codes4_b(w3);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) bq[j] = codes8_b(q.q[j >> 1][2 * (j & 1)], q.q[j >> 1][2 * (j & 1) + 1]);
    }
    // The chunk's MFMAs, group by group: t = sum x c, xs = sum x.
    const bool two = !(half_tail && c == nchunk - 1); // second half of the chunk exists
#pragma unroll
    for (int gg = 0; gg < kGpc; ++gg) {
      if (gg == 1 && !two) break;
      constexpr int kPer = 4 / kGpc; // MFMAs per group in this chunk
      floatx4 t[MB], xs[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
          const int mi = gg * kPer + j;
          u32x4 a;
          if constexpr (kXD) {
            a = q.a[mb][mi];
          } else {
            a = *reinterpret_cast<const u32x4 *>(xl + xrow[mb] * L.xstride + c * 128 - xcol0 +
                                                 slot_k<BITS>(mi, lh));
          }
          t[mb] = mfma16(a, bq[mi], j == 0 ? zero : t[mb]);
          xs[mb] = mfma16(a, ones, j == 0 ? zero : xs[mb]);
        }
      }
      const float2 sc = sbrow[i * kGpc + gg];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // Entry e of lane (n, h) is token 16 mb + 4 h + e: for M <= 4 only
          // e < M holds a token on any lane (a uniform test).
          if (M > 4 || e < M) {
            acc[mb][e] = fmaf(sc.x, t[mb][e], acc[mb][e]);
            acc[mb][e] = fmaf(sc.y, xs[mb][e], acc[mb][e]);
          }
        }
    }
  };
  {
    // Ring of DEPTH + 1 slots: the load of chunk i + DEPTH goes out before
    // chunk i is processed (into the slot chunk i - 1 left), so the math of
    // a chunk does not delay the stream.  Every load is unconditional (past
    // the range it reads zeros without touching memory): the compiler then
    // counts the loads in flight exactly and each chunk waits only for its
    // own; a load under a branch would make it wait for all of them.
    // Ranges of up to kStraight chunks run as straight-line code: at a loop
    // header the compiler merges the states of entry and back edge and waits
    // for every load in flight.
    constexpr int kRing = DEPTH + 1;
    constexpr int kStraight = 8;
    if (ncs <= kStraight) {
#pragma unroll
      for (int i = 0; i < kStraight; ++i) {
        if (i >= ncs) break;
        load(i + DEPTH, ring[(i + DEPTH) % kRing]);
        process(i, ring[i % kRing]);
      }
    } else {
      for (int base = 0; base < ncs; base += kRing) {
#pragma unroll
        for (int d = 0; d < kRing; ++d) {
          const int i = base + d;
          if (i >= ncs) break;
          load(i + DEPTH, ring[(d + DEPTH) % kRing]);
          process(i, ring[d]);
        }
      }
    }
  }

  // 3. The S partial tiles of each tile are added in range order.
  if (S > 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) red[(wave * MB + mb) * 64 + lane] = acc[mb];
    __syncthreads();
    if (rs != 0) return;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      floatx4 sum = red[((tl * S) * MB + mb) * 64 + lane];
      for (int v = 1; v < S; ++v) {
        const floatx4 p = red[((tl * S + v) * MB + mb) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) sum[e] += p[e];
      }
      acc[mb] = sum;
    }
  }

  if (!live) return;
  if constexpr (kSplit) {
    if (R > 1) {
      // The range's accumulators, 1 KB per wave and row block, for
      // qmv_reduce_kernel (the next kernel on the stream).
      floatx4 *dst = reinterpret_cast<floatx4 *>(partial) + ((int64_t(rr) * tiles + tile) * MB) * 64 + lane;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) dst[mb * 64] = acc[mb];
      return;
    }
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) qmv_store_rows<ODT>(y, ep, acc[mb], mb, M, N, tile, lane, m0);
}

// The sum of kXSplit's R partial tiles in range order (so the result does
// not depend on which block finished first), with the epilogue.  One wave
// per tile and row block: lane l adds float4 l of each range's slot.
template <int ODT, int MB>
__global__ __launch_bounds__(256) void qmv_reduce_kernel(typename Elem<ODT>::T *__restrict__ y,
                                                         const float *__restrict__ partial, int M, int N, int R,
                                                         kern::Epilogue ep) {
  const int tiles = (N + 15) / 16;
  const int lane = int(threadIdx.x) & 63;
  const int64_t wv = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 6; // tile * MB + mb
  if (wv >= int64_t(tiles) * MB) return;                              // whole waves
  const int tile = int(wv / MB), mb = int(wv % MB);
  const floatx4 *src = reinterpret_cast<const floatx4 *>(partial) + wv * 64 + lane;
  const int64_t stride = int64_t(tiles) * MB * 64;
  floatx4 v[kMaxRanges];
#pragma unroll
  for (int r = 0; r < kMaxRanges; ++r)
    if (r < R) v[r] = src[r * stride];
  floatx4 sum = v[0];
#pragma unroll
  for (int r = 1; r < kMaxRanges; ++r)
    if (r < R)
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[e] += v[r][e];
  qmv_store_rows<ODT>(y, ep, sum, mb, M, N, tile, lane);
}

template <int BITS, int XDT, int SDT, int ODT, int MB, int GS, int XM, int DEPTH = kDepth>
void launch_qmv_t(void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s,
                  const void *b, int M, int N, int K, const kern::QmvPlan &plan,
                  const kern::Epilogue &ep, hipStream_t st, float *partial) {
  const int tiles = (N + 15) / 16;
  const int T = plan.tiles_per_block;
  const int R = XM == kXSplit ? plan.ranges : 1;
  const int RG = XM == kXBlock ? plan.row_groups : 1;
  const QmvLds l = qmv_lds(XM, RG > 1 ? 16 * MB : M, K, GS, T, plan.waves, MB, R);
  const int ntb = (tiles + T - 1) / T;
  const dim3 grid(unsigned(RG > 1 ? (ntb + 7) / 8 * 8 * RG : ntb * R));
  qmv_kernel<BITS, XDT, SDT, ODT, MB, GS, XM, DEPTH><<<grid, 64 * T * plan.waves, l.total, st>>>(
      static_cast<typename Elem<ODT>::T *>(y), static_cast<const typename Elem<XDT>::T *>(x), ldx,
      w, static_cast<const typename Elem<SDT>::T *>(s), static_cast<const typename Elem<SDT>::T *>(b),
      M, N, K, T, plan.waves, ep, R, partial, RG);
  if (R > 1) {
    const int64_t threads = int64_t(tiles) * MB * 64;
    qmv_reduce_kernel<ODT, MB><<<dim3(unsigned((threads + 255) / 256)), 256, 0, st>>>(
        static_cast<typename Elem<ODT>::T *>(y), partial, M, N, R, ep);
  }
}

// One activation/scale/output dtype combination of the kernel, for 4 or 8
// bits: instantiated once per combination in its own translation unit
// (qmv_inst.hip, compiled once per combination) so the build runs in parallel.
template <int XD, int SD, int OD>
void qmv_combo(int bits, void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s,
               const void *b, int M, int N, int K, int gs, const kern::QmvPlan &plan,
               const kern::Epilogue &ep, hipStream_t st, float *partial);

template <int BITS, int XD, int SD, int OD, int XM>
void qmv_xm(void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s, const void *b,
            int M, int N, int K, int gs, const kern::QmvPlan &plan, const kern::Epilogue &ep,
            hipStream_t st, float *partial) {
  if (gs == 64) {
    if (plan.row_blocks == 1)
      launch_qmv_t<BITS, XD, SD, OD, 1, 64, XM>(y, x, ldx, w, s, b, M, N, K, plan, ep, st, partial);
    else
      launch_qmv_t<BITS, XD, SD, OD, 2, 64, XM>(y, x, ldx, w, s, b, M, N, K, plan, ep, st, partial);
  } else {
    if (plan.row_blocks == 1)
      launch_qmv_t<BITS, XD, SD, OD, 1, 128, XM>(y, x, ldx, w, s, b, M, N, K, plan, ep, st, partial);
    else
      launch_qmv_t<BITS, XD, SD, OD, 2, 128, XM>(y, x, ldx, w, s, b, M, N, K, plan, ep, st, partial);
  }
}

template <int BITS, int XD, int SD, int OD>
void qmv_bits(void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s, const void *b,
              int M, int N, int K, int gs, const kern::QmvPlan &plan, const kern::Epilogue &ep,
              hipStream_t st, float *partial) {
  if (plan.xmode == kXWave)
    qmv_xm<BITS, XD, SD, OD, kXWave>(y, x, ldx, w, s, b, M, N, K, gs, plan, ep, st, partial);
  else if (plan.xmode == kXBlock)
    qmv_xm<BITS, XD, SD, OD, kXBlock>(y, x, ldx, w, s, b, M, N, K, gs, plan, ep, st, partial);
  else if (plan.xmode == kXSplit)
    qmv_xm<BITS, XD, SD, OD, kXSplit>(y, x, ldx, w, s, b, M, N, K, gs, plan, ep, st, partial);
  else
    qmv_xm<BITS, XD, SD, OD, kXDirect>(y, x, ldx, w, s, b, M, N, K, gs, plan, ep, st, partial);
}

template <int XD, int SD, int OD>
void qmv_combo(int bits, void *y, const void *x, int64_t ldx, const uint32_t *w, const void *s,
               const void *b, int M, int N, int K, int gs, const kern::QmvPlan &plan,
               const kern::Epilogue &ep, hipStream_t st, float *partial) {
  if (bits == 4)
    qmv_bits<4, XD, SD, OD>(y, x, ldx, w, s, b, M, N, K, gs, plan, ep, st, partial);
  else
    qmv_bits<8, XD, SD, OD>(y, x, ldx, w, s, b, M, N, K, gs, plan, ep, st, partial);
}

} // namespace qmv_detail
} // namespace sdq
