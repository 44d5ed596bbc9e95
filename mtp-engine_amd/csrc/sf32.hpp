// Small fp32 RMSNorm -> linear for gfx950 (TF32 off): at most 16 rows of
// fp32 x, fp32 W, K <= 1024, one launch, one round trip of loads.
//
//   y[m, n] = (rs[m] * sum_k (x[m, k] gamma[k]) W[n, k] + bias[n]) * scale,
//   rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) (norm) or 1
//
// The shape (the fp32 RMSNorm+linear configuration: x [16, 1024],
// W [4096, 1024]) moves 16.8 MB and is bound by launch latency and the
// first round trip, not by sustained bandwidth. So every workgroup takes
// only 16 columns (N / 16 workgroups: 256 for N = 4096, every CU), and
// every load of the launch goes out at once: wave w of the NW covers
// k = KPW w .. KPW w + KPW - 1 (KPW = 1024 / NW); lane l = 16 g + r holds,
// for each of its loads i, W[n0 + r] and x[r] (and gamma) at k = KPW w +
// 16 i + 4 g .. + 3, which is exactly its slot of 4 consecutive
// v_mfma_f32_16x16x4_f32 (A = W rows, B = x rows, k-slot g): no LDS
// staging. Each load instruction reads 64 contiguous bytes of 16 rows.
// x * gamma is formed in fp32 registers and the squares of x are summed on
// the way; the waves' 16x16 sums and row squares meet in LDS in a fixed
// order.
#pragma once

#include "mtp_common.hpp"
#include "sf32_args.hpp"
#include "wstream.hpp"

namespace mtp {

template <bool GAM, int NW>
__global__ void __launch_bounds__(64 * NW, 1) sf32_kernel(const Sf32Args a) {
  constexpr int KPW = kSf32MaxK / NW;  // k per wave
  constexpr int CPW = KPW / 16;        // 16-k chunks (4 MFMA k-slots x 4) per wave
  __shared__ f32x4 s_acc[NW][64];
  __shared__ float s_ss[NW][16];
  __shared__ f32x4 s_g[NW][64];
  const int th = threadIdx.x, lane = th & 63;
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int n0 = blockIdx.x * 16;
  const int K = a.K;
  // rows past M / N and k past K read 0 through the descriptors' range
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(a.w + (int64_t)n0 * K, (uint32_t)(min(16, a.N - n0) * K) * 4u);
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)(a.M * K) * 4u);
  const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.gamma, GAM ? (uint32_t)K * 4u : 0u);
  // Load order: gamma first (every MFMA needs it), then W and x of chunk i
  // side by side, so the MFMAs of chunk i start as soon as its two loads are
  // back instead of after the whole round trip.
  // gamma of the wave's KPW k: one load (lane L < KPW / 4: k KPW w + 4 L ..
  // + 3), then each lane reads its CPW chunks back from LDS (lanes of one
  // group read the same address)
  f32x4 gl = f32x4{1.f, 1.f, 1.f, 1.f};
  if constexpr (GAM)
    gl = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                   grs, lane < KPW / 4 ? (uint32_t)(KPW * wave + 4 * lane) * 4u : kOOB, 0, 0));
  // float offset of load i: row r, k = KPW w + 16 i + 4 g; chunks at or past
  // K (K % 16 == 0) use an out-of-range offset
  f32x4 wv[CPW], xv[CPW], gv[CPW];
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int k = KPW * wave + 16 * i + 4 * g;
    const bool live = KPW * wave + 16 * i < K;
    const uint32_t ro = live ? (uint32_t)(r * K + k) * 4u : kOOB;
    wv[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, ro, 0, 2));
    xv[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, ro, 0, 0));
  }
  if constexpr (GAM) {
    s_g[wave][lane] = gl;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < CPW; ++i) gv[i] = s_g[wave][4 * i + g];
  }
  // epilogue factors of the lane's outputs: columns n0 + 4 g + e
  float cws[4], cbi[4];
  load_col_factors<1>(nullptr, a.bias, a.bias_dt, a.N, n0 + 4 * g, 4, cws, cbi);

  // four independent accumulators (one per e), so consecutive MFMAs do not
  // wait for each other's results; summed in a fixed order below
  float ss = 0.f;
  f32x4 ac[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) ac[e] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xe = xv[i][e];
      ss = __builtin_fmaf(xe, xe, ss);
      const float b = GAM ? xe * gv[i][e] : xe;
      ac[e] = mfma16_f32(wv[i][e], b, ac[e]);
    }
  }
  const f32x4 acc = ((ac[0] + ac[1]) + ac[2]) + ac[3];
  // row squares: the 4 lane groups of row r, then the waves in order
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  if (g == 0) s_ss[wave][r] = ss;
  s_acc[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  // lane holds D[n = 4 g + e][m = r]; the waves' sums in wave order
  f32x4 t = s_acc[0][lane];
  float sq = s_ss[0][r];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    t += s_acc[w][lane];
    sq += s_ss[w][r];
  }
  const float rs = a.norm ? 1.0f / sqrtf(sq / (float)K + a.eps) : 1.0f;
  const int m = r;
  if (m >= a.M) return;
  const int n = n0 + 4 * g;
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = (a.bias ? t[e] * rs + cbi[e] : t[e] * rs) * a.scale;
  float *yr = a.y + (int64_t)m * a.N;
  if (n + 3 < a.N && (a.N & 3) == 0) {
    *(f32x4 *)(yr + n) = f32x4{o[0], o[1], o[2], o[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < a.N) yr[n + e] = o[e];
  }
}

}  // namespace mtp
