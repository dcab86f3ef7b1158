// attention.hip -- fused scaled dot-product attention for gfx950.
//
// Replaces mlx_fast_scaled_dot_product_attention (crates/sd-tensor/src/mlx.rs:
// 228-238, called by Array::sdpa / sdpa_causal / sdpa_masked at 1119-1197):
//   out = softmax(scale * q @ k^T [+ mask]) @ v   over [batch, heads, seq, head_dim]
// for every attention of the Flux blocks (sd-models/src/mlx/flux.rs:381, 461),
// CLIP's causal text tower and T5's additive position bias.
//
// One pass over the keys with an online softmax (the score matrix never
// leaves registers).  Block = 8 waves, 256 queries; each wave owns 32
// queries (one MFMA column tile); the block walks the keys 64 at a time
// through a double-buffered LDS stage shared by its waves.  A wave needs
// under 256 registers, so two waves share each SIMD and one wave's softmax
// (VALU, exp) runs under the other's MFMAs.
//
// Layout trick.  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16_bf16: a lane's accumulator column is ONE query and its
// 16 entries are keys, so the softmax statistics of a query live in one lane
// and its partner lane (lane ^ 32) -- one cross-lane exchange per row
// maximum, none for the rescale.  The output is kept transposed as well,
// O^T = V^T P^T, whose B operand (P^T) is the score accumulator itself,
// rounded to bf16 in place: the K rows are staged in a permuted order chosen
// so that accumulator entries 8s..8s+7 of lane half h are the consecutive
// keys 16s + 8h .. +7, exactly the eight keys the next MFMA's B operand
// wants from that lane.  V arrives transposed (V^T, keys contiguous per
// head-dim row) so the A operand is one 16-byte LDS read.
//
// Numerics: q, k, v enter the MFMAs as bf16 (rounded to nearest even by
// the caller's conversion), P is rounded to bf16, every product and sum
// accumulates in f32, exp is exp2 of log2(e)-scaled scores.  The kernel
// is built with contraction on (the score scaling is an explicit fma).
#include <cmath>
#include <type_traits>

#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;
using kern::AttnArgs;

// QT 32-query column tiles per wave and 8 / QT waves per block: every
// block owns kBQ = 256 queries.  QT = 1 keeps a wave's registers under 256,
// so two waves share each SIMD and one's softmax overlaps the other's MFMAs.
constexpr int kBQ = 256;           // queries per block
constexpr int kBK = 64;            // keys per iteration
template <int QT> struct Shape {
  static constexpr int kWaves = 8 / QT;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kQW = 32 * QT;  // queries per wave
};
constexpr int kQT = 1;

enum { MODE_NONE = 0, MODE_CAUSAL = 1, MODE_ARRAY = 2 };

__device__ __forceinline__ floatx16 mfma32(const u32x4 &a, const u32x4 &b, const floatx16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// 16-byte chunk c of LDS row `row` (ROW_BYTES long) as stored.  The LDS
// serves a 16-byte read for 16 lanes per cycle across 256 bytes of banks;
// the MFMA operand reads have lanes 0-15 on 16 consecutive rows, same chunk,
// so the chunk is XOR-swizzled by row to put those rows on distinct banks:
// by the row within 16 for 256-byte rows, and by the row pair within 8 for
// 128-byte rows (two rows share one 256-byte bank line).
template <int ROW_BYTES> __device__ __forceinline__ int swz(int row, int c) {
  static_assert(ROW_BYTES == 128 || ROW_BYTES == 256, "row length");
  if constexpr (ROW_BYTES == 256)
    return c ^ (row & 15);
  else
    return c ^ ((row >> 1) & 7);
}

// LDS row of key `w` (0..63) of a tile: the MFMA row whose accumulator entry
// holds it (see the layout note above).
__device__ __forceinline__ int k_row(int w) {
  const int kt = w >> 5, u = w & 31, s = u >> 4, h = (u >> 3) & 1, i = u & 7;
  return 32 * kt + 16 * s + (i < 4 ? 4 * h + i : 8 + 4 * h + (i - 4));
}

template <int D, int ODT, int MODE, int MDT, int QT>
__global__ __launch_bounds__(Shape<QT>::kThreads, 1) void flash_attn_kernel(AttnArgs a) {
  constexpr int kThreads = Shape<QT>::kThreads;
  constexpr int kQW = Shape<QT>::kQW;
  constexpr int kCK = D / 8;         // 16-byte chunks per K row
  constexpr int kKS = D / 16;        // MFMA k-steps of the score product
  constexpr int kDT = D / 32;        // 32-row tiles of head_dim in O^T
  constexpr int kKBytes = kBK * D * 2;
  constexpr int kVBytes = D * kBK * 2;
  constexpr int kStage = kKBytes + kVBytes;
  constexpr int kLoads = kStage / 16 / kThreads;  // 16-byte global loads per thread per tile
  static_assert(kStage % (16 * kThreads) == 0, "tile must split evenly over the block");
  extern __shared__ __align__(16) uint8_t lds[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, h = lane >> 5;

  // Block -> (batch*head, query block).  Blocks of one head share its K and
  // V, so they are kept on one XCD (blocks are dealt to the 8 XCDs round
  // robin by linear id) when the grid divides evenly.
  int lin = blockIdx.x;
  const int total = gridDim.x;
  if (total % 8 == 0) lin = (lin % 8) * (total / 8) + lin / 8;
  const int bh = lin / a.q_blocks, qb = lin % a.q_blocks;
  const int b = bh / a.H, hh = bh % a.H;
  const int hk = hh / a.group;  // grouped-query heads share a K/V head

  const uint16_t *qp = a.q + int64_t(b) * a.q_sb + int64_t(hh) * a.q_sh;
  const uint16_t *kp = a.k + int64_t(b) * a.k_sb + int64_t(hk) * a.k_sh;
  const uint16_t *vp = a.vt + int64_t(b) * a.v_sb + int64_t(hk) * a.v_sh;

  const int q0 = qb * kBQ + wave * kQW;  // first query of this wave

  // Q^T operands: lane (r, h) of column tile qt holds query q0 + 32qt + r,
  // head-dim elements 16ks + 8h .. +7.
  u32x4 qreg[QT][kKS];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + 32 * qt + r;
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      if (qi < a.Nq)
        qreg[qt][ks] = *reinterpret_cast<const u32x4 *>(qp + int64_t(qi) * a.q_sn + 16 * ks + 8 * h);
      else
        qreg[qt][ks] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  // Wait for the Q operands here, once: otherwise the wait for them is
  // re-inserted inside the key loop, where it would also wait for every tile
  // load in flight.
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) asm volatile("" : "+v"(qreg[qt][ks]));

  floatx16 oacc[kDT][QT];
#pragma unroll
  for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[dt][qt][e] = 0.0f;
  float m[QT], l[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.0f;
  }

  // Keys this block needs: all, or (causal) up to its last query's diagonal.
  int k_end = a.Nk;
  if constexpr (MODE == MODE_CAUSAL) {
    const int last_q = min(qb * kBQ + kBQ, a.Nq) - 1;
    k_end = min(a.Nk, last_q + a.causal_offset + 1);
  }
  const int n_tiles = (k_end + kBK - 1) / kBK;

  // Staging of tile t: thread i moves 16-byte pieces p = i + 256j; pieces
  // [0, kKBytes/16) are K (row w = p / kCK, chunk c = p % kCK), the rest V^T
  // (row d, chunk c of 8 keys).
  u32x4 stage_regs[kLoads];
  auto load_tile = [&](int t) {
    const int k0 = t * kBK;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int p = threadIdx.x + j * kThreads;
      if (p < kKBytes / 16) {
        const int w = p / kCK, c = p % kCK;
        const int key = k0 + w;
        stage_regs[j] = key < a.Nk ? *reinterpret_cast<const u32x4 *>(kp + int64_t(key) * a.k_sn + 8 * c)
                                   : u32x4{0u, 0u, 0u, 0u};
      } else {
        const int pv = p - kKBytes / 16;
        const int d = pv / (kBK / 8), c = pv % (kBK / 8);
        // V^T rows are padded to a multiple of kBK keys, zero-filled.
        stage_regs[j] = *reinterpret_cast<const u32x4 *>(vp + int64_t(d) * a.v_sd + k0 + 8 * c);
      }
    }
  };
  auto store_tile = [&](int buf) {
    uint8_t *base = lds + buf * kStage;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int p = threadIdx.x + j * kThreads;
      if (p < kKBytes / 16) {
        const int w = p / kCK, c = p % kCK;
        const int row = k_row(w);
        *reinterpret_cast<u32x4 *>(base + row * (D * 2) + (swz<D * 2>(row, c) * 16)) = stage_regs[j];
      } else {
        const int pv = p - kKBytes / 16;
        const int d = pv / (kBK / 8), c = pv % (kBK / 8);
        *reinterpret_cast<u32x4 *>(base + kKBytes + d * (kBK * 2) + (swz<kBK * 2>(d, c) * 16)) = stage_regs[j];
      }
    }
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    const uint8_t *kl = lds + buf * kStage;
    const uint8_t *vl = kl + kKBytes;
    const int k0 = t * kBK;
    if (t + 1 < n_tiles) load_tile(t + 1);

    // S^T = K Q^T for the 64 keys of this tile.
    floatx16 sacc[2][QT];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[kt][qt][e] = 0.0f;
    // Operands are read one k-step ahead of the MFMAs that use them, so an
    // LDS read's latency hides under the previous step's MFMAs.
    auto k_operand = [&](int ks, int kt) {
      const int row = 32 * kt + r;
      return *reinterpret_cast<const u32x4 *>(kl + row * (D * 2) + swz<D * 2>(row, 2 * ks + h) * 16);
    };
    u32x4 ka[2][2];
    ka[0][0] = k_operand(0, 0);
    ka[0][1] = k_operand(0, 1);
#pragma unroll
    for (int ks = 0; ks < kKS; ++ks) {
      if (ks + 1 < kKS) {
        ka[(ks + 1) & 1][0] = k_operand(ks + 1, 0);
        ka[(ks + 1) & 1][1] = k_operand(ks + 1, 1);
      }
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) sacc[kt][qt] = mfma32(ka[ks & 1][kt], qreg[qt][ks], sacc[kt][qt]);
    }

    // Online softmax in the log2 domain: entry e of key tile kt is key
    // k0 + 32kt + 16(e/8) + 8h + (e%8) for query q0 + 32qt + r.  Keys are
    // masked only in tiles that need it (past the last key, or past the
    // causal diagonal of the wave's first query): a wave-uniform test.
    // The running maximum is raised lazily -- only when some query's tile
    // maximum exceeds it by more than 2^8 -- so the accumulators are
    // rescaled in the first few tiles and rarely after; until then a
    // probability is at most 2^8, exact enough in bf16 and f32.
    // Entry e's key offset within the tile, less 8h, is the constant
    // c(e) = 32kt + 16(e/8) + e%8; it is masked when c(e) >= lim.  Tiles
    // that need no mask get a limit no entry reaches.
    const bool need_mask = k0 + kBK > a.Nk ||
                           (MODE == MODE_CAUSAL && k0 + kBK - 1 > q0 + a.causal_offset);
    const int lim_keys = need_mask ? a.Nk - k0 - 8 * h : kBK;
    u32x4 pb[2][2][QT];  // [kt][s][qt]: P^T operands
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int qi = q0 + 32 * qt + r;
      float sv[2][16];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float v = sacc[kt][qt][e];
          const int key = k0 + 32 * kt + 16 * (e >> 3) + 8 * h + (e & 7);
          if constexpr (MODE == MODE_ARRAY) {
            const typename Elem<MDT>::T *mrow =
                static_cast<const typename Elem<MDT>::T *>(a.mask) + int64_t(b) * a.m_sb +
                int64_t(hh) * a.m_sh + int64_t(min(qi, a.Nq - 1)) * a.m_sq;
            v = fmaf(v, a.scale_log2, (key < a.Nk ? Elem<MDT>::load(mrow[key]) : 0.0f) * 1.4426950408889634f);
          }
          const int ce = 32 * kt + 16 * (e >> 3) + (e & 7);
          if constexpr (MODE == MODE_CAUSAL) {
            // keys past the diagonal too: key <= qi + offset
            const int lim = min(lim_keys, need_mask ? qi + a.causal_offset + 1 - k0 - 8 * h : kBK);
            v = ce >= lim ? -INFINITY : v;
          } else {
            v = ce >= lim_keys ? -INFINITY : v;
          }
          sv[kt][e] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // Raw scores are scaled by the positive scale_log2 after the maximum.
      if constexpr (MODE != MODE_ARRAY) mx = mx * a.scale_log2;
      if (__builtin_amdgcn_ballot_w64(mx > m[qt] + 8.0f) != 0) {
        const float m_new = fmaxf(m[qt], mx);
        const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[qt] - m_new);
        m[qt] = m_new;
        l[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[dt][qt][e] *= alpha;
      }
      // A query with no unmasked key yet keeps its state at zero.
      const float m_use = m[qt] == -INFINITY ? 0.0f : m[qt];
      float sum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        float p[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float t = MODE == MODE_ARRAY ? sv[kt][e] - m_use : fmaf(sv[kt][e], a.scale_log2, -m_use);
          p[e] = __builtin_amdgcn_exp2f(t);
          sum += p[e];
        }
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int w = 0; w < 4; ++w) pb[kt][s][qt][w] = pack_bf16x2(p[8 * s + 2 * w], p[8 * s + 2 * w + 1]);
      }
      l[qt] += sum;
    }

    // O^T += V^T P^T, operands again read one step ahead.
    auto v_operand = [&](int i) {  // i = (dt, kt, s) flattened
      const int dt = i >> 2, kt = (i >> 1) & 1, s = i & 1;
      const int row = 32 * dt + r;
      return *reinterpret_cast<const u32x4 *>(vl + row * (kBK * 2) + swz<kBK * 2>(row, 4 * kt + 2 * s + h) * 16);
    };
    constexpr int kVSteps = kDT * 4;
    u32x4 va[2];
    va[0] = v_operand(0);
#pragma unroll
    for (int i = 0; i < kVSteps; ++i) {
      if (i + 1 < kVSteps) va[(i + 1) & 1] = v_operand(i + 1);
      const int dt = i >> 2, kt = (i >> 1) & 1, s = i & 1;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) oacc[dt][qt] = mfma32(va[i & 1], pb[kt][s][qt], oacc[dt][qt]);
    }
    // The next tile's K and V^T go to the other stage last, leaving the
    // whole iteration for their global loads.
    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  // out[q, d] = O^T[d, q] / l; entry e of d-tile dt is d = 32dt + 8(e/4) + 4h + e%4.
  using OT = typename Elem<ODT>::T;
  OT *op = static_cast<OT *>(a.o) + int64_t(b) * a.o_sb + int64_t(hh) * a.o_sh;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int qi = q0 + 32 * qt + r;
    const float lt = l[qt] + __shfl_xor(l[qt], 32);
    const float inv = 1.0f / lt;
    if (qi >= a.Nq) continue;
    OT *orow = op + int64_t(qi) * a.o_sn;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * h;
        if constexpr (ODT == SDQ_FLOAT32) {
          *reinterpret_cast<floatx4 *>(orow + d) =
              floatx4{oacc[dt][qt][4 * g] * inv, oacc[dt][qt][4 * g + 1] * inv, oacc[dt][qt][4 * g + 2] * inv,
                      oacc[dt][qt][4 * g + 3] * inv};
        } else {
          u32x2 w;
#pragma unroll
          for (int i = 0; i < 2; ++i)
            w[i] = uint32_t(Elem<ODT>::store(oacc[dt][qt][4 * g + 2 * i] * inv)) |
                   (uint32_t(Elem<ODT>::store(oacc[dt][qt][4 * g + 2 * i + 1] * inv)) << 16);
          *reinterpret_cast<u32x2 *>(orow + d) = w;
        }
      }
    }
  }
}

// V [.., N, D] (any float dtype, row stride ld) -> V^T bf16 [.., D, ldt],
// keys [N, ldt) zero.  One block moves a 64-key x 64-dim tile through LDS.
template <int IDT>
__global__ __launch_bounds__(256) void transpose_v_kernel(const typename Elem<IDT>::T *__restrict__ v,
                                                          int64_t v_sbh, int64_t ld, uint16_t *__restrict__ vt,
                                                          int64_t vt_sbh, int64_t ldt, int N, int D) {
  __shared__ uint16_t tile[64][65];
  const int bh = blockIdx.z;
  const int n0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const typename Elem<IDT>::T *src = v + int64_t(bh) * v_sbh;
  uint16_t *dst = vt + int64_t(bh) * vt_sbh;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int n = i / 64, d = i % 64;
    const int gn = n0 + n, gd = d0 + d;
    const float x = (gn < N && gd < D) ? Elem<IDT>::load(src[int64_t(gn) * ld + gd]) : 0.0f;
    tile[n][d] = f32_to_bf16_bits(x);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int d = i / 64, n = i % 64;
    const int gn = n0 + n, gd = d0 + d;
    if (gd < D && gn < ldt) dst[int64_t(gd) * ldt + gn] = tile[n][d];
  }
}

template <int D, int ODT, int MODE, int MDT> void launch_d(const AttnArgs &a, hipStream_t st) {
  constexpr int kStage = kBK * D * 2 * 2;
  const int blocks = a.q_blocks * a.B * a.H;
  hipLaunchKernelGGL((flash_attn_kernel<D, ODT, MODE, MDT, kQT>), dim3(blocks), dim3(Shape<kQT>::kThreads),
                     2 * kStage, st, a);
}

template <int D, int ODT, int MODE> void launch_mdt(const AttnArgs &a, hipStream_t st) {
  if constexpr (MODE != MODE_ARRAY) {
    launch_d<D, ODT, MODE, SDQ_FLOAT32>(a, st);
  } else {
    switch (a.mask_dtype) {
    case SDQ_FLOAT32: launch_d<D, ODT, MODE, SDQ_FLOAT32>(a, st); break;
    case SDQ_BFLOAT16: launch_d<D, ODT, MODE, SDQ_BFLOAT16>(a, st); break;
    case SDQ_FLOAT16: launch_d<D, ODT, MODE, SDQ_FLOAT16>(a, st); break;
    default: fail("attention: the mask must be float32, bfloat16 or float16");
    }
  }
}

template <int D, int ODT> void launch_mode(const AttnArgs &a, hipStream_t st) {
  switch (a.mode) {
  case MODE_NONE: launch_mdt<D, ODT, MODE_NONE>(a, st); break;
  case MODE_CAUSAL: launch_mdt<D, ODT, MODE_CAUSAL>(a, st); break;
  case MODE_ARRAY: launch_mdt<D, ODT, MODE_ARRAY>(a, st); break;
  default: fail("attention: unknown mask mode");
  }
}

template <int D> void launch_odt(const AttnArgs &a, int odt, hipStream_t st) {
  switch (odt) {
  case SDQ_FLOAT32: launch_mode<D, SDQ_FLOAT32>(a, st); break;
  case SDQ_BFLOAT16: launch_mode<D, SDQ_BFLOAT16>(a, st); break;
  case SDQ_FLOAT16: launch_mode<D, SDQ_FLOAT16>(a, st); break;
  default: fail("attention: unsupported output dtype");
  }
}

} // namespace

namespace kern {

int64_t attention_vt_stride(int64_t nk) { return (nk + kBK - 1) / kBK * kBK; }

void transpose_v(const void *v, int v_dtype, int64_t bh, int64_t n, int64_t d, int64_t v_sbh, int64_t ld,
                 uint16_t *vt, int64_t vt_sbh, int64_t ldt, hipStream_t stream) {
  if (bh == 0 || d == 0 || ldt == 0) return;
  if (ldt < n || ldt % kBK != 0) fail("attention: bad V^T stride");
  const dim3 grid(unsigned(ldt / 64), unsigned((d + 63) / 64), unsigned(bh));
  switch (v_dtype) {
  case SDQ_FLOAT32:
    transpose_v_kernel<SDQ_FLOAT32><<<grid, 256, 0, stream>>>(static_cast<const float *>(v), v_sbh, ld, vt, vt_sbh,
                                                               ldt, int(n), int(d));
    break;
  case SDQ_BFLOAT16:
    transpose_v_kernel<SDQ_BFLOAT16><<<grid, 256, 0, stream>>>(static_cast<const uint16_t *>(v), v_sbh, ld, vt,
                                                                vt_sbh, ldt, int(n), int(d));
    break;
  case SDQ_FLOAT16:
    transpose_v_kernel<SDQ_FLOAT16><<<grid, 256, 0, stream>>>(static_cast<const uint16_t *>(v), v_sbh, ld, vt,
                                                               vt_sbh, ldt, int(n), int(d));
    break;
  default: fail("attention: unsupported V dtype");
  }
  hip_check(hipGetLastError(), "transpose_v launch");
}

void attention(const AttnArgs &args, int o_dtype, hipStream_t stream) {
  AttnArgs a = args;
  if (a.B == 0 || a.H == 0 || a.Nq == 0) return;
  if (a.Nk <= 0) fail("attention: no keys");
  if (a.D != 64 && a.D != 128) fail("attention: head_dim must be 64 or 128");
  if (a.group < 1 || a.H % a.group != 0) fail("attention: heads must be a multiple of the K/V heads");
  if (a.v_sd % kBK != 0 || a.v_sd < a.Nk) fail("attention: V^T rows must be padded to 64 keys");
  const uintptr_t align = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.k) |
                          reinterpret_cast<uintptr_t>(a.vt);
  if (align % 16 != 0 || a.q_sn % 8 != 0 || a.k_sn % 8 != 0)
    fail("attention: q, k and V^T must be 16-byte aligned rows");
  if (o_dtype == SDQ_FLOAT32 ? (reinterpret_cast<uintptr_t>(a.o) % 16 != 0 || a.o_sn % 4 != 0)
                             : (reinterpret_cast<uintptr_t>(a.o) % 8 != 0 || a.o_sn % 4 != 0))
    fail("attention: output rows must be aligned");
  a.q_blocks = int((a.Nq + kBQ - 1) / kBQ);
  if (int64_t(a.q_blocks) * a.B * a.H > 0x7fffffff) fail("attention: grid too large");
  if (a.D == 128)
    launch_odt<128>(a, o_dtype, stream);
  else
    launch_odt<64>(a, o_dtype, stream);
  hip_check(hipGetLastError(), "attention launch");
}

} // namespace kern
} // namespace sdq
