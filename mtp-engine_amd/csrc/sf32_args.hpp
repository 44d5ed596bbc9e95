// Arguments and launch of the small fp32 RMSNorm -> linear kernel (sf32.hpp),
// shared by its instantiation unit and the host planner.
#pragma once

#include <hip/hip_runtime.h>

namespace mtp {

struct Sf32Args {
  const float *x;      // [M, K]
  const float *gamma;  // [K] or null
  const float *w;      // [N, K]
  const void *bias;    // [N] or null
  int bias_dt;
  float *y;            // [M, N]
  int M, N, K;
  int norm;
  float eps, scale;
};

constexpr int kSf32MaxK = 1024;  // k per launch: kSf32Waves waves x KPW k, all staged in LDS
// waves per workgroup, each KPW = kSf32MaxK / kSf32Waves k (4 and 8
// measured 6.7 and 6.9 us per call at M 16, K 1024, N 4096; 16 waves' LDS
// areas and sums do not fit the 160 KB)
constexpr int kSf32Waves = 4;

// Streaming form (sf32s_kernel) for kSf32MaxK < K <= kSf32StreamMaxK: each
// of kSf32sWaves waves streams its K-range in 64-k blocks (4 KB of W, 4 KB
// of x) through an LDS ring of kSf32Ring blocks. Fewer bytes in flight per
// wave and more waves measured faster (us per call, 8 waves x 1 block /
// 8 x 2 / 4 x 4: fp32 8 x 4096 x 4096 14.0 / 14.0 / 16.0, 8 x 14336 x 4096
// 42.8 / 48.0 / 53.9, 16 x 4096 x 2048 8.9 / 9.5 / 9.7; 16 waves x 1 block
// 16.2 at 8 x 4096 x 4096; a deeper W ring than x ring was slower still).
constexpr int kSf32StreamMaxK = 65536;
constexpr int kSf32Ring = 1;
constexpr int kSf32sWaves = 8;

// Launch for fp32 x and W, 1 <= M <= 32 (more than 16 rows or K past
// kSf32MaxK: the streaming form), 16 <= K <= kSf32StreamMaxK with
// K % 16 == 0, 16-byte aligned x / W / gamma / y (MTP_ERR_SHAPE otherwise).
int launch_sf32(const Sf32Args &a, hipStream_t st);

}  // namespace mtp
