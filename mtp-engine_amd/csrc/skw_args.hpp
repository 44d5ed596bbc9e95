// Host-side view of the wave-specialised skinny RMSNorm -> linear GEMM
// (skw.hpp): arguments and the instantiation accessor. It reads the xn
// blocks and row sums that sk.hpp's prep launch writes.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace mtp {

struct SkwArgs {
  const void *xf;       // xn blocks of the prep: [tiles][stages][k-steps][64 lanes] x 16 B
  const float *pss;     // the prep's row sums of squares [nsl][64]
  int nsl;              // the prep's K-slices
  int norm;
  float eps;
  const void *w;        // [N, K] fp8 or the compute type
  const float *wscale;  // [N] or null
  const void *bias;     // [N] or null
  int bias_dt;
  void *y;              // [M, N] compute type
  int M, N, K;
  float scale;
  int nst;              // stages: 128 bytes of every W row each
  int tw;               // output columns per workgroup (8 .. 64, a multiple of 4)
};

typedef void (*SkwKernel)(SkwArgs);
// GEMM for x dtype ct (BF16 / F16), W dtype wt (FP8E4M3 or ct), mt 32-row
// tiles of x (1 or 2), or null.
SkwKernel skw_pick(int ct, int wt, int mt);

}  // namespace mtp
