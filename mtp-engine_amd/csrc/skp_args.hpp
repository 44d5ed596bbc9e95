// Host-side view of the x-resident skinny RMSNorm -> linear kernel
// (skp.hpp): launch arguments and instantiation accessor.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/mtp_hip.h"

namespace mtp {

constexpr int kSkpWaves = 4;                 // waves per workgroup (one per SIMD)
constexpr int kSkpStageBytes = 128;          // W bytes per row per step
constexpr int kSkpXMaxBytes = 128 * 1024;    // LDS for the workgroup's x blocks
constexpr int kSkpStaging = kSkpWaves * 2048;  // LDS for the waves' W staging
constexpr int kSkpGammaLoads = 4;  // 16-byte gamma loads per thread: a split's k <= 4096

struct SkpArgs {
  const void *x;        // [M, K] compute type (bf16 / f16), row-major
  const float *gamma;   // [K] fp32 or null
  const void *w;        // [N, K] fp8 or compute type
  const float *wscale;  // [N] or null
  const void *bias;     // [N] or null
  int bias_dt;
  void *y;              // [M, N] compute type
  int M, N, K;
  int norm;
  float eps, scale;
  int G, S;             // column tiles, K-splits
  int kb_per, nkb;      // steps per split, steps in K
  int xg;               // 1: the splits of a tile on one XCD (split_tile_of)
  int tw;               // output columns per workgroup (<= 64 TA, a multiple of 4)
  float *part;          // [G][S][waves][TA][MT][64] f32x4 (S > 1)
  float *part_ss;       // [G][S][64]
  unsigned *ticket;     // [G]
};

typedef void (*SkpKernel)(SkpArgs);
// Instantiations per x type (skp_bf16.hip, skp_f16.hip): W type fp8 or the
// same 16-bit type, 16-row x tiles mt 1..4, A tiles per wave ta 1 / 2 / 4,
// gamma; null for anything else.
// h8: the compact form for at most 8 rows (mt 1): x blocks keep only the
// parts holding rows 0 .. 7.
SkpKernel skp_pick_bf16(int wt, int mt, int ta, bool gam, bool h8);
SkpKernel skp_pick_f16(int wt, int mt, int ta, bool gam, bool h8);
inline SkpKernel skp_pick(int ct, int wt, int mt, int ta, bool gam, bool h8) {
  if (ct == MTP_BF16) return skp_pick_bf16(wt, mt, ta, gam, h8);
  if (ct == MTP_F16) return skp_pick_f16(wt, mt, ta, gam, h8);
  return nullptr;
}
// Dynamic LDS bytes of a launch with `steps` steps (of uk k) per split:
// x blocks, W staging, gamma of the split's k in whole 1 KB pieces (the
// copy writes whole pieces).
// xp: 1 KB parts kept per x block (ks, or 8 rows' worth in the compact form).
inline size_t skp_lds_bytes(int mt, int xp, int steps, int uk, bool gam) {
  const size_t g = gam ? ((size_t)steps * uk * 4 + 1023) / 1024 * 1024 : 0;
  return (size_t)mt * xp * steps * 1024 + kSkpStaging + g;
}

}  // namespace mtp
