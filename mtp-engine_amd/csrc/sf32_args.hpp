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
// wave streams its K-range in 64-k blocks through an LDS ring of
// kSf32Ring blocks (8 KB of x and W each, 32 KB per wave in flight).
constexpr int kSf32StreamMaxK = 65536;
constexpr int kSf32Ring = 4;

// Launch for fp32 x and W, 1 <= M <= 16, 16 <= K <= kSf32StreamMaxK with
// K % 16 == 0, 16-byte aligned x / W / gamma / y (MTP_ERR_SHAPE otherwise).
int launch_sf32(const Sf32Args &a, hipStream_t st);

}  // namespace mtp
