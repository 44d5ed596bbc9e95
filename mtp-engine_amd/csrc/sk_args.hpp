// Host-side view of the skinny weight-streaming GEMM (sk.hpp): arguments,
// shape constants for planning and the instantiation accessors.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace mtp {

constexpr int kSkBN = 64;   // output columns per workgroup
constexpr int kSkUB = 128;  // W bytes per row per stage
constexpr int kSkMaxK = 16384;    // K at most (the prep's slices cover 16 x 1024 k)
constexpr int kSkPrepMaxSlices = 16;  // K-slices of the 8-row prep (row sums per slice)

struct SkPrepArgs {
  const void *x;       // [M, K] in the compute type
  const float *gamma;  // [K] or null
  void *xf;            // xn blocks: [ceil(M / 32) tiles][K / UK stages][k-steps][64 lanes] x 16 B
  int M, K, norm;
  float eps;
};

struct SkArgs {
  const void *xf;       // xn blocks written by the prep
  const void *x;        // raw x rows [M, K] (the prep-free form, no gamma)
  int norm;             // raw form: apply rs
  float eps;
  float *part_ss;       // raw form with split-K: sums of squares [G][S][64]
  const void *w;        // [N, K] fp8 or compute type
  const float *wscale;  // [N] or null
  const void *bias;     // [N] or null
  int bias_dt;
  void *y;              // [M, N] compute type
  int M, N, K;
  float scale;
  int G, S, kb_per, nkb;  // column tiles, K-splits, stages per split, stages
  float *part;            // split-K partials
  unsigned *ticket;       // [G] arrival tickets (S > 1)
  const float *pss;       // prep form: the prep's row sums of squares [nsl][64]
  int nsl;                // prep form: the prep's K-slices
};

typedef void (*SkKernel)(SkArgs);
typedef void (*SkPrep8Kernel)(SkPrepArgs, float *);
// 8-row prep for x dtype ct, the k-slot order of W dtype wt, gamma present,
// 256 ch k per slice (ch 1, 2 or 4), or null.
SkPrep8Kernel sk_prep8_pick(int ct, int wt, bool gam, int ch);
// GEMM for x dtype ct (BF16 / F16), W dtype wt (FP8E4M3 or ct), mt 32-row
// tiles of x (1 or 2), reading the prep's xn blocks or (xr) raw x, or null.
SkKernel sk_pick(int ct, int wt, int mt, bool xr);

// Bytes of the xn blocks for m rows of x and k columns.
constexpr size_t sk_xf_bytes(int64_t m, int64_t k) {
  return (size_t)((m + 31) / 32) * 32 * (size_t)k * 2;
}
// Bytes of one workgroup's split-K partial tile.
constexpr size_t sk_tile_bytes(int mt) { return (size_t)2 * mt * 4 * 64 * 16; }

}  // namespace mtp
