// Host-side view of the single-launch skinny RMSNorm -> linear (skl.hpp):
// arguments, shape constants for planning and the instantiation accessor.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace mtp {

constexpr int kSklGammaMax = 8192;  // k of one split whose gamma is staged in LDS (32 KB)

struct SklArgs {
  const void *x;        // [M, K] in the compute type, row-major
  const float *gamma;   // [K] fp32 or null
  const void *w;        // [N, K] fp8 or the compute type
  const float *wscale;  // [N] or null
  const void *bias;     // [N] or null
  int bias_dt;
  void *y;              // [M, N] compute type
  int M, N, K, norm;
  float eps, scale;
  int G, S, kb_per, nkb;  // column tiles, K-splits, stages per split, stages
  int xg;                 // 1: the splits of a tile on one XCD (split_tile_of)
  int tw;                 // output columns per workgroup (<= 32 waves, a multiple of 4)
  float *part;            // split-K partial tiles [G * S][tile] (S > 1)
  float *part_ss;         // split-K partial sums of squares [G * S][64] (S > 1)
  unsigned *ticket;       // [G] arrival tickets (S > 1)
};

typedef void (*SklKernel)(SklArgs);
// Kernel for x dtype ct (BF16 / F16), W dtype wt (FP8E4M3 or ct), mt 32-row
// tiles of x (1 or 2), nw waves (4 or 8: 32 nw columns per workgroup) and
// gamma present, or null.
SklKernel skl_pick(int ct, int wt, int mt, int nw, bool gam);
// The same per x dtype (one translation unit each).
SklKernel skl_pick_bf16(int wt, int mt, int nw, bool gam);
SklKernel skl_pick_f16(int wt, int mt, int nw, bool gam);

// Columns per workgroup for nw waves.
constexpr int skl_bn(int nw) { return 32 * nw; }
// Bytes of one workgroup's split-K partial tile.
constexpr size_t skl_tile_bytes(int mt, int nw) { return (size_t)32 * nw * 32 * mt * 4; }

}  // namespace mtp
