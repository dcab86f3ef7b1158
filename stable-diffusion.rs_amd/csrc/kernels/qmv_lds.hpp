// qmv_lds.hpp -- block shape limits and LDS layout of the small-M kernel,
// shared by its planner (qmv.hip) and the kernel (qmv_kernel.hpp).
#pragma once

#include <hip/hip_runtime.h>

namespace sdq {
namespace qmv_detail {

// Where the kernel's activation operands come from.
enum XMode {
  kXDirect = 0, // read per chunk from global memory (large x)
  kXWave = 1,   // each wave stages its own slice of x in LDS (M <= 4)
  kXBlock = 2,  // the block stages all of x in LDS once (x shared by T tiles)
  kXSplit = 3,  // K is cut into R ranges, one per block; the block stages its
                // range of x once for T tiles and writes partial tiles that a
                // second kernel adds (x too large for one block's LDS)
};

constexpr int kMaxWaves[4] = {8, 16, 16, 16}; // waves per block, by XMode
constexpr int kMaxRanges = 8;                 // R of kXSplit, at most
constexpr int kXWaveMaxChunks = 8;        // chunks per wave a kXWave stage holds

// LDS layout of one block (bytes): [kXBlock, kXSplit: x][per wave:
// scale/bias pairs, kXWave: x slice][partial tiles of the waves, S > 1].
struct QmvLds {
  int x, wave, red, total;
  int wave_bytes; // one wave's region
  int nb;         // most 128-wide chunks of K one block covers
  int cmax;       // most 128-wide chunks of K one wave streams
  int gw;         // groups of K one wave's scale region holds
  int gws;        // its row stride in float2: gw made odd, so that the 16 rows
                  // of a per-group read sit on distinct LDS banks
  int xstride;    // bf16 elements per staged x row (block or wave)
  int wsb;        // byte offset of the wave's x slice within its region
};

__host__ __device__ inline QmvLds qmv_lds(int xmode, int M, int K, int gs, int T, int S, int MB, int R = 1) {
  QmvLds l;
  const int nchunk = (K + 127) / 128;
  l.nb = xmode == kXSplit ? (nchunk + R - 1) / R : nchunk;
  l.cmax = (l.nb + S - 1) / S;
  l.gw = l.cmax * (128 / gs);
  l.gws = l.gw | 1;
  // x rows are padded by 16 bytes so that the 16 rows an MFMA operand read
  // touches sit on distinct LDS banks.
  l.xstride = xmode == kXBlock ? K + 8 : xmode == kXSplit ? l.nb * 128 + 8 : l.cmax * 128 + 8;
  l.x = 0;
  l.wave = xmode == kXBlock || xmode == kXSplit ? (M * l.xstride * 2 + 15) & ~15 : 0;
  l.wsb = (16 * l.gws * 8 + 15) & ~15;
  l.wave_bytes = l.wsb + (xmode == kXWave ? (M * l.xstride * 2 + 15) & ~15 : 0);
  l.red = l.wave + T * S * l.wave_bytes;
  l.total = l.red + (S > 1 ? T * S * MB * 64 * 16 : 0);
  return l;
}

} // namespace qmv_detail
} // namespace sdq
