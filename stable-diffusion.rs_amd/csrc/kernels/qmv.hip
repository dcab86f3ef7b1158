// qmv.hip -- y = x @ dequantize(w).T for few rows of x (M <= 32): the
// bandwidth-bound decode/modulation shape of mlx_quantized_matmul
// (crates/sd-tensor/src/mlx.rs:386-397, 1947-1975; callers e.g. the Flux
// modulation linears at M = 1, sd-models/src/mlx/flux.rs:279-299, 437, and the
// T5 FFN at few tokens, t5.rs:209-214).
//
// Time here is the packed weight stream, so everything is arranged to keep
// many whole cache lines of codes in flight and little other work per byte:
//
//   * A block is four waves; wave v owns one 32-row tile of weights (the MFMA
//     N side) over the block's range of K.  K is split so that the grid is
//     about two blocks per CU, all resident at once.
//   * Codes stream in row chunks of 128 bytes (four 64-wide steps at 4 bits,
//     two at 8): each load instruction brings eight whole rows' chunks, i.e.
//     eight full cache lines (a load's cost is set by the cache lines it
//     touches), with kDepth chunks in flight per wave.  A small wave-private
//     LDS buffer turns them around into the MFMA operand layout.
//   * Codes are never dequantized element by element.  For one 64-wide step
//     of K the MFMA computes t[m][n] = sum_k x[m,k] * c_k with c_k = q_k + OFF
//     held EXACTLY in bf16 (4-bit: OFF = 128, the bf16 pattern 0x4300|q built
//     by byte permutes; 8-bit: OFF = 0, q converted).  Then
//     y += s * t + (b - OFF*s) * X, where X[m] = sum_k x[m,k] over the step:
//     the affine dequantization is applied once per group per output, and is
//     more accurate than rounding each dequantized weight to bf16.
//   * x[0:M, range] (bf16, zero past the range), its per-step sums and the
//     tiles' scales and biases for the range are staged in LDS once per
//     block with coalesced loads, so the loop's only global traffic is codes.
//   * When K is split across blocks, each wave writes its partial tile with
//     agent-scope (L2-bypassing) stores and counts itself in; the last wave
//     to arrive for a tile adds the partials in split order (deterministic)
//     and re-arms the counter.
//   * MFMA v_mfma_f32_32x32x16_bf16 with the tokens on the M side.  Lane
//     (r, h) = (lane % 32, lane / 32) feeds token r and weight row r; its
//     eight K elements of k-step i are k = 64*step + 32*h + 8*i + e.  Token
//     rows r >= M read row M - 1; their results are never stored.
#include <algorithm>

#include "device_common.hpp"
#include "launch.hpp"

#include "../sdq_internal.hpp"

namespace sdq {
namespace {

using namespace dev;

constexpr int kWRow = 144;         // LDS bytes per staged weight row (128 + pad)
constexpr int kWBuf = 32 * kWRow;  // one wave's chunk buffer
constexpr int kLdsBudget = 64 * 1024;

__host__ __device__ constexpr int chunk_steps(int bits) { return bits == 4 ? 4 : 2; }

// Eight 4-bit codes of `wd` as bf16 (128 + q), exact, in the order
// q0 q2 q4 q6 q1 q3 q5 q7: each pair is one byte permute of the even or odd
// codes with the constant exponent byte 0x43 (bf16 0x43nn = 128 + nn for
// nn < 128).  The staged x uses the same order within each eight elements.
__device__ __forceinline__ u32x4 codes4_plus128(uint32_t wd) {
  const uint32_t lo = wd & 0x0F0F0F0Fu;         // codes 0, 2, 4, 6
  const uint32_t hi = (wd >> 4) & 0x0F0F0F0Fu;  // codes 1, 3, 5, 7
  const uint32_t c43 = 0x43434343u;
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(c43, lo, 0x04010400u); // (q0, q2)
  r[1] = __builtin_amdgcn_perm(c43, lo, 0x04030402u); // (q4, q6)
  r[2] = __builtin_amdgcn_perm(c43, hi, 0x04010400u); // (q1, q3)
  r[3] = __builtin_amdgcn_perm(c43, hi, 0x04030402u); // (q5, q7)
  return r;
}

// Eight bf16 values e0..e7 reordered to e0 e2 e4 e6 e1 e3 e5 e7.
__device__ __forceinline__ u32x4 even_odd(const u32x4 &v) {
  const uint32_t v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(v1, v0, 0x05040100u); // (e0, e2)
  o[1] = __builtin_amdgcn_perm(v3, v2, 0x05040100u); // (e4, e6)
  o[2] = __builtin_amdgcn_perm(v1, v0, 0x07060302u); // (e1, e3)
  o[3] = __builtin_amdgcn_perm(v3, v2, 0x07060302u); // (e5, e7)
  return o;
}

// Eight 8-bit codes (two words), in element order, as bf16 q: exact.
__device__ __forceinline__ u32x4 codes8(uint32_t w0, uint32_t w1) {
  const uint32_t a = opaque(w0), b = opaque(w1);
  u32x4 r;
  r[0] = pack_bf16x2(float(a & 0xffu), float((a >> 8) & 0xffu));
  r[1] = pack_bf16x2(float((a >> 16) & 0xffu), float(a >> 24));
  r[2] = pack_bf16x2(float(b & 0xffu), float((b >> 8) & 0xffu));
  r[3] = pack_bf16x2(float((b >> 16) & 0xffu), float(b >> 24));
  return r;
}

// Row stride, in bf16 elements, of the staged x: 16 bytes of padding keep
// consecutive rows on different LDS banks.
__host__ __device__ constexpr int x_stride(int steps) { return steps * 64 + 8; }

// LDS layout of one block of `waves` waves (bytes): staged x, per-step
// sums, scales and biases, the waves' chunk buffers.
struct QmvLds {
  int x, xsum, sb, wbuf, total;
};

__host__ __device__ inline QmvLds qmv_lds(int waves, int M, int mrows, int steps_pad,
                                          int groups_range) {
  QmvLds l;
  l.x = 0;
  l.xsum = (M * x_stride(steps_pad) * 2 + 15) & ~15;
  l.sb = l.xsum + steps_pad * mrows * 4;
  l.wbuf = (l.sb + waves * 32 * groups_range * 8 + 15) & ~15;
  l.total = l.wbuf + waves * kWBuf;
  return l;
}

// WAVES waves per block (4 when K is split into short ranges, 1 when each
// wave streams a long range), DEPTH code chunks in flight per wave.
template <int BITS, int XDT, int SDT, int ODT, int MROWS, int GS, int WAVES, int DEPTH>
__global__ __launch_bounds__(64 * WAVES) void qmv_kernel(
    typename Elem<ODT>::T *__restrict__ y, const typename Elem<XDT>::T *__restrict__ x,
    int64_t ldx, const uint32_t *__restrict__ w,
    const typename Elem<SDT>::T *__restrict__ scales,
    const typename Elem<SDT>::T *__restrict__ biases, int M, int N, int K,
    int steps_per_split, int groups_range, float *__restrict__ partial,
    unsigned *__restrict__ counters, kern::Epilogue ep) {
  constexpr int kWaves = WAVES;
  constexpr int kThreads = 64 * WAVES;
  constexpr int kDepth = DEPTH;
  constexpr float kOff = BITS == 4 ? 128.0f : 0.0f;
  constexpr int kC = chunk_steps(BITS);      // steps per 128-byte row chunk
  constexpr int kStepBytes = 64 * BITS / 8;  // one row's codes per step
  constexpr int kAcc = MROWS / 2;            // accumulator entries holding rows < MROWS

  const int steps = K / 64;
  const int groups = K / GS;
  const int tiles = (N + 31) / 32;
  const int split = blockIdx.y;
  const int nsplit = gridDim.y;
  const int s0 = split * steps_per_split;
  const int s1 = min(steps, s0 + steps_per_split);
  const int ns = s1 - s0;                               // >= 1 by the plan
  const int nchunks = (ns + kC - 1) / kC;
  const int spad = (steps_per_split + kC - 1) / kC * kC; // staged steps, as laid out
  const int g0 = (s0 * 64) / GS;
  const int gr = groups_range;                          // groups staged per row
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane & 31;
  const int h = lane >> 5;
  const int tile = blockIdx.x * kWaves + wave;
  const bool live = tile < tiles;
  const int tl = live ? tile : tiles - 1; // idle waves shadow the last tile, store nothing

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const QmvLds L = qmv_lds(kWaves, M, MROWS, spad, gr);
  const int xs_stride = x_stride(spad);
  uint16_t *xl = reinterpret_cast<uint16_t *>(smem + L.x);     // [M][xs_stride] bf16
  float *xsum = reinterpret_cast<float *>(smem + L.xsum);     // [spad][MROWS]
  float *sbl = reinterpret_cast<float *>(smem + L.sb);        // [waves][32][gr][2]
  unsigned char *wbuf = smem + L.wbuf + wave * kWBuf;         // this wave's chunk buffer

  // Code chunks: lane L of load i brings bytes 16*(L%8) .. +16 of row
  // 8*i + L/8's chunk, eight whole lines per load.  Chunks past the range
  // are addressed beyond the buffer's end: such loads return zeros without
  // touching memory, and their slots are never computed.
  const Rsrc rw = make_rsrc(w, uint32_t(int64_t(N) * K * BITS / 8));
  uint32_t woff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = tl * 32 + 8 * i + (lane >> 3);
    woff[i] = uint32_t(int64_t(n < N ? n : N - 1) * (int64_t(K) * BITS / 8) + 16 * (lane & 7));
  }
  auto load_chunk = [&](int c, u32x4 (&dst)[4]) {
    const uint32_t so = c < nchunks ? uint32_t(s0 + c * kC) * kStepBytes : 0x80000000u;
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = bload16(rw, woff[i], so);
  };
  u32x4 q[kDepth][4];

  // 1. Stage x[0:M, s0*64 : (s0+spad)*64] as bf16, zero past the range (at
  //    4 bits each eight elements in the codes' even/odd order), and the
  //    waves' scales and biases.  Every staging load goes out in one batch,
  //    before the wave's first kDepth code chunks, and is stored after them:
  //    the wait for the staging then does not include the chunks (loads
  //    complete in issue order for the counter), which keep streaming into
  //    the loop below.  The plan keeps a range short enough for one batch:
  //    kXB 16-byte pieces of x and kSB scale/bias pairs per thread.
  constexpr int kXB = MROWS / 2;
  constexpr int kSB = 8;
  const int chunks_per_row = spad * 8; // 16-byte chunks of x
  const int xtotal = M * chunks_per_row;
  const int stotal = kWaves * 32 * gr;
  u32x4 xv[kXB];
  float2 sv[kSB];
  // Pieces past the range or past x are loaded from a valid address and
  // replaced by zeros, so every load is unconditional.
#pragma unroll
  for (int j = 0; j < kXB; ++j) {
    const int c = min(tid + j * kThreads, xtotal - 1);
    const int m = c / chunks_per_row;
    const int qk = min(c - m * chunks_per_row, ns * 8 - 1);
    xv[j] = Load8<XDT>::get(x + int64_t(m) * ldx + int64_t(s0) * 64 + 8 * qk);
  }
  // Consecutive threads read consecutive groups of a row; groups past the
  // last one repeat it (their x is zero).
#pragma unroll
  for (int j = 0; j < kSB; ++j) {
    const int e = min(tid + j * kThreads, stotal - 1);
    const int wv = e / (32 * gr);
    const int rem = e - wv * 32 * gr;
    const int row = rem / gr;
    const int g = min(g0 + (rem - row * gr), groups - 1);
    int n = (blockIdx.x * kWaves + wv) * 32 + row;
    n = n < N ? n : N - 1;
    const int64_t gi = int64_t(n) * groups + g;
    sv[j].x = Elem<SDT>::load(scales[gi]);
    sv[j].y = Elem<SDT>::load(biases[gi]);
  }
#pragma unroll
  for (int d = 0; d < kDepth; ++d) load_chunk(d, q[d]);
#pragma unroll
  for (int j = 0; j < kXB; ++j) {
    const int c = tid + j * kThreads;
    const int m = c / chunks_per_row;
    const int qk = c - m * chunks_per_row;
    if (c < xtotal) {
      const u32x4 v = qk < ns * 8 ? xv[j] : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4 *>(xl + m * xs_stride + 8 * qk) = BITS == 4 ? even_odd(v) : v;
    }
  }
#pragma unroll
  for (int j = 0; j < kSB; ++j) {
    const int e = tid + j * kThreads;
    if (e < stotal) *reinterpret_cast<float2 *>(sbl + 2 * e) = sv[j];
  }
  __syncthreads();
  // 2. Per-step sums of the staged values (dot2 against (1, 1)); rows >= M
  //    are zero.
  {
    const bf16x2 ones = __builtin_bit_cast(bf16x2, 0x3F803F80u);
    for (int p = tid; p < spad * MROWS; p += kThreads) {
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
  if (!live) return; // no further block-wide synchronisation

  // 3. Stream the chunks.
  const uint16_t *arow = xl + (r < M ? r : M - 1) * xs_stride + 32 * h;
  const float *sbrow = sbl + 2 * (wave * 32 + r) * gr;
  floatx16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

  auto compute_chunk = [&](const u32x4 (&cq)[4], int c) {
    // Turn the chunk around through the wave's buffer: written as eight
    // rows per load, read back as this lane's row r, half h.
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<u32x4 *>(wbuf + (8 * i + (lane >> 3)) * kWRow + 16 * (lane & 7)) = cq[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    u32x4 bw[kC][BITS / 4];
#pragma unroll
    for (int u = 0; u < kC; ++u)
#pragma unroll
      for (int v = 0; v < BITS / 4; ++v)
        bw[u][v] = *reinterpret_cast<const u32x4 *>(wbuf + r * kWRow + u * kStepBytes +
                                                    h * (kStepBytes / 2) + 16 * v);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // The kC steps' products are independent: their MFMAs are interleaved so
    // that none waits for the previous one's result.
    floatx16 t[kC];
#pragma unroll
    for (int u = 0; u < kC; ++u)
#pragma unroll
      for (int e = 0; e < 16; ++e) t[u][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int u = 0; u < kC; ++u) {
        // Local step c*kC + u; past the range the staged x is zero.
        const u32x4 a = *reinterpret_cast<const u32x4 *>(arow + (c * kC + u) * 64 + 8 * i);
        u32x4 bq;
        if constexpr (BITS == 4) {
          bq = codes4_plus128(bw[u][0][i]);
        } else {
          bq = codes8(bw[u][i / 2][(i % 2) * 2], bw[u][i / 2][(i % 2) * 2 + 1]);
        }
        t[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(bq), t[u], 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < kC; ++u) {
      const int sl = c * kC + u;
      const int g = min(((s0 + sl) * 64) / GS - g0, gr - 1);
      const float2 sb = *reinterpret_cast<const float2 *>(sbrow + 2 * g);
      const float sv = sb.x;
      const float cv = sb.y - kOff * sb.x;
      const float *xs_step = xsum + sl * MROWS;
#pragma unroll
      for (int j = 0; j < kAcc / 4; ++j) {
        const floatx4 xs = *reinterpret_cast<const floatx4 *>(xs_step + 8 * j + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[4 * j + e] = fmaf(sv, t[u][4 * j + e], acc[4 * j + e]);
          acc[4 * j + e] = fmaf(cv, xs[e], acc[4 * j + e]);
        }
      }
    }
  };

  // Each slot is refilled with the chunk kDepth later as soon as it has been
  // used.
  for (int base = 0; base < nchunks; base += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int c = base + d;
      if (c < nchunks) compute_chunk(q[d], c);
      __builtin_amdgcn_sched_barrier(0);
      load_chunk(c + kDepth, q[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // 4. Accumulator entry i of lane (r, h) is token 8*(i/4) + 4*h + i%4,
  //    weight row r of the tile.
  const int n = tile * 32 + r;
  if (nsplit == 1) {
    const float bn = epi_bias(ep, min(n, N - 1));
#pragma unroll
    for (int i = 0; i < kAcc; ++i) {
      const int m = 8 * (i / 4) + 4 * h + (i % 4);
      if (m < M && n < N)
        y[int64_t(m) * N + n] = Elem<ODT>::store(epi_combine(ep, epi_apply(ep, acc[i], bn), m, n));
    }
    return;
  }
  // K was split: this wave's partial tile goes out as agent-scope stores,
  // which do not stay in this XCD's L2; once they have completed the wave
  // counts itself in, and the last wave of the tile adds every split's
  // partial in split order and re-arms the counter.
  float *mine = partial + ((int64_t(split) * tiles + tile) * MROWS) * 32;
#pragma unroll
  for (int i = 0; i < kAcc; ++i) {
    const int m = 8 * (i / 4) + 4 * h + (i % 4);
    __hip_atomic_store(mine + m * 32 + r, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): this wave's stores are done
  unsigned prev = 0;
  if (lane == 0)
    prev = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __builtin_amdgcn_readfirstlane(prev);
  if (prev != unsigned(nsplit - 1)) return;
  // The partials of kSplitBatch splits are loaded together (one round trip
  // per batch rather than per value), then added in split order.
  constexpr int kSplitBatch = 4;
  float v[kAcc];
#pragma unroll
  for (int i = 0; i < kAcc; ++i) v[i] = 0.0f;
  for (int sp0 = 0; sp0 < nsplit; sp0 += kSplitBatch) {
    float t[kSplitBatch][kAcc];
#pragma unroll
    for (int j = 0; j < kSplitBatch; ++j) {
      const int sp = min(sp0 + j, nsplit - 1);
      const float *src = partial + ((int64_t(sp) * tiles + tile) * MROWS) * 32 + r;
#pragma unroll
      for (int i = 0; i < kAcc; ++i)
        t[j][i] = __hip_atomic_load(src + (8 * (i / 4) + 4 * h + (i % 4)) * 32, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int j = 0; j < kSplitBatch; ++j)
      if (sp0 + j < nsplit)
#pragma unroll
        for (int i = 0; i < kAcc; ++i) v[i] += t[j][i];
  }
  const float bn = epi_bias(ep, min(n, N - 1));
#pragma unroll
  for (int i = 0; i < kAcc; ++i) {
    const int m = 8 * (i / 4) + 4 * h + (i % 4);
    if (m < M && n < N)
      y[int64_t(m) * N + n] = Elem<ODT>::store(epi_combine(ep, epi_apply(ep, v[i], bn), m, n));
  }
  if (lane == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Groups a range of `steps` 64-wide steps can touch (one more when a
// 128-group range starts mid-group).
__host__ __device__ inline int range_groups(int steps, int gs) { return (steps * 64) / gs + 1; }

// Longest K range (64-wide steps, a multiple of both chunk sizes) whose
// staging fits the kernel's single batch: at most 16 steps of x and 16
// groups of scales and biases per row.
inline int max_range_steps(int gs) { return gs == 64 ? 12 : 16; }

template <int BITS, int XDT, int SDT, int ODT, int MROWS, int GS, int WAVES, int DEPTH>
void launch_qmv_w(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K,
                  const kern::QmvPlan &plan, const kern::SplitWorkspace &ws,
                  const kern::Epilogue &ep, hipStream_t st) {
  const int tiles = (N + 31) / 32;
  const dim3 grid((tiles + WAVES - 1) / WAVES, plan.splits);
  const int sps = plan.groups_per_split;
  const int spad = (sps + chunk_steps(BITS) - 1) / chunk_steps(BITS) * chunk_steps(BITS);
  const int gr = range_groups(spad, GS);
  const QmvLds l = qmv_lds(WAVES, M, MROWS, spad, gr);
  if (l.total > kLdsBudget) fail("qmv: plan exceeds the LDS budget");
  // The staging is one batch per thread: MROWS/2 pieces of x, 8 scale pairs.
  if (spad > 16 || M * spad * 8 > (MROWS / 2) * 64 * WAVES || WAVES * 32 * gr > 8 * 64 * WAVES)
    fail("qmv: K range too long for the staging batch");
  qmv_kernel<BITS, XDT, SDT, ODT, MROWS, GS, WAVES, DEPTH><<<grid, 64 * WAVES, l.total, st>>>(
      static_cast<typename Elem<ODT>::T *>(y), static_cast<const typename Elem<XDT>::T *>(x), ldx,
      w, static_cast<const typename Elem<SDT>::T *>(s),
      static_cast<const typename Elem<SDT>::T *>(b), M, N, K, sps, gr, ws.partial, ws.counters, ep);
}

template <int BITS, int XDT, int SDT, int ODT, int MROWS, int GS>
void launch_qmv_t(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K,
                  const kern::QmvPlan &plan, const kern::SplitWorkspace &ws,
                  const kern::Epilogue &ep, hipStream_t st) {
  if (plan.waves != 4) fail("qmv: plan must use four waves per block");
  launch_qmv_w<BITS, XDT, SDT, ODT, MROWS, GS, 4, 4>(y, x, ldx, w, s, b, M, N, K, plan, ws, ep, st);
}

template <int BITS, int XDT, int SDT, int ODT>
void launch_qmv_m(void *y, const void *x, int64_t ldx, const uint32_t *w,
                  const void *s, const void *b, int M, int N, int K, int gs,
                  const kern::QmvPlan &plan, const kern::SplitWorkspace &ws,
                  const kern::Epilogue &ep, hipStream_t st) {
  // MROWS: the token rows the kernel keeps (the accumulator holds MROWS / 2
  // entries per lane).
  if (gs == 64) {
    if (M <= 8)
      launch_qmv_t<BITS, XDT, SDT, ODT, 8, 64>(y, x, ldx, w, s, b, M, N, K, plan, ws, ep, st);
    else if (M <= 16)
      launch_qmv_t<BITS, XDT, SDT, ODT, 16, 64>(y, x, ldx, w, s, b, M, N, K, plan, ws, ep, st);
    else
      launch_qmv_t<BITS, XDT, SDT, ODT, 32, 64>(y, x, ldx, w, s, b, M, N, K, plan, ws, ep, st);
  } else {
    if (M <= 8)
      launch_qmv_t<BITS, XDT, SDT, ODT, 8, 128>(y, x, ldx, w, s, b, M, N, K, plan, ws, ep, st);
    else if (M <= 16)
      launch_qmv_t<BITS, XDT, SDT, ODT, 16, 128>(y, x, ldx, w, s, b, M, N, K, plan, ws, ep, st);
    else
      launch_qmv_t<BITS, XDT, SDT, ODT, 32, 128>(y, x, ldx, w, s, b, M, N, K, plan, ws, ep, st);
  }
}

#define SDQ_QMV_CASE(XD, SD, OD)                                                      \
  if (x_dtype == XD && s_dtype == SD && y_dtype == OD) {                              \
    if (bits == 4)                                                                    \
      launch_qmv_m<4, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K), \
                                  group_size, plan, ws, ep, stream);                  \
    else                                                                              \
      launch_qmv_m<8, XD, SD, OD>(y, x, ldx, w, scales, biases, int(M), int(N), int(K), \
                                  group_size, plan, ws, ep, stream);                  \
    hip_check(hipGetLastError(), "qmv launch");                                       \
    return;                                                                           \
  }

} // namespace

namespace kern {

QmvPlan plan_qmv(int64_t M, int64_t N, int64_t K, int group_size, int bits, int cus) {
  QmvPlan p;
  const int64_t steps = K / 64;
  const int64_t tiles = (N + 31) / 32;
  const int mrows = M <= 8 ? 8 : M <= 16 ? 16 : 32;
  const int c = chunk_steps(bits);
  const int64_t ncu = cus > 0 ? cus : 256;
  auto fits = [&](int waves, int64_t s) {
    const int pad = int((s + c - 1) / c * c);
    return qmv_lds(waves, int(M), mrows, pad, range_groups(pad, group_size)).total <= kLdsBudget;
  };
  auto finish = [&](int waves, int64_t sps) {
    sps = std::min<int64_t>(sps, steps);
    const int64_t splits = (steps + sps - 1) / sps;
    p.waves = waves;
    p.splits = int(splits);
    p.groups_per_split = int(sps);
    p.partial_floats = splits > 1 ? size_t(splits) * size_t(tiles) * size_t(mrows) * 32 : 0;
    p.counters = int(tiles);
    return p;
  };
  // Four waves per block and K split so that there are about two blocks per
  // CU, in ranges of whole chunks that fit the LDS: many short ranges keep
  // more bytes in flight than a few long ones, which outweighs the partial
  // round trips at the end.
  // (Rounded down: a grid just over two blocks per CU would need a second
  // round wherever a third block does not fit.)
  const int64_t tile_groups = (tiles + 3) / 4;
  const int64_t target = 2 * ncu;
  int64_t splits = std::max<int64_t>(1, target / tile_groups);
  int64_t sps = (steps + splits - 1) / splits;
  sps = (sps + c - 1) / c * c;
  sps = std::min<int64_t>(sps, max_range_steps(group_size));
  while (sps > c && !fits(4, sps)) sps -= c;
  return finish(4, sps);
}

void qmv(void *y, int y_dtype, const void *x, int x_dtype, int64_t ldx,
         const uint32_t *w, const void *scales, const void *biases,
         int s_dtype, int64_t M, int64_t N, int64_t K, int group_size,
         int bits, const QmvPlan &plan, const SplitWorkspace &ws,
         const Epilogue &ep, hipStream_t stream) {
  if (M < 1 || M > 32) fail("qmv: M must be in [1, 32]");
  if (N < 1 || K < 64 || K % 64 != 0) fail("qmv: bad N or K");
  if (group_size != 64 && group_size != 128) fail("qmv: group size must be 64 or 128");
  if (K % group_size != 0) fail("qmv: K % group_size != 0");
  if (bits != 4 && bits != 8) fail("qmv: bits must be 4 or 8");
  if (ldx < K || ldx % 8 != 0) fail("qmv: row stride of x must be >= K and a multiple of 8");
  if (N * K * bits / 8 >= (int64_t(1) << 31)) fail("qmv: the packed weight must be under 2 GiB");
  if (plan.splits < 1 || plan.groups_per_split < 1 ||
      int64_t(plan.splits) * plan.groups_per_split < K / 64 ||
      int64_t(plan.splits - 1) * plan.groups_per_split >= K / 64)
    fail("qmv: inconsistent plan");
  if (plan.splits > 1 && (!ws.partial || !ws.counters)) fail("qmv: split without workspace");
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
