// Straightforward kernels for argument shapes the tiled kernels do not take
// (K not a multiple of the 16-byte vector width, unaligned pointers, mixed
// float dtypes). Same arithmetic contract: fp32 products of the upcast
// operands, fp32 accumulation, row statistic applied per row.
#pragma once

#include "mtp_common.hpp"

namespace mtp {

__device__ __forceinline__ float load_w_as_f32(const void *w, int wt, int64_t i) {
  if (wt == MTP_FP8E4M3) {
    const uint32_t b = ((const uint8_t *)w)[i];
    return __builtin_amdgcn_cvt_f32_fp8(b, 0);
  }
  return load_as_f32(w, wt, i);
}

// Block reduction (sum) for 256 threads.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// One block per (row m, 256 columns). Weight decode covers float, fp8 and
// packed INT4 (nibble_mode >= 0, group size `group`, scales in scale_dt).
__global__ void __launch_bounds__(256)
generic_rmsnorm_linear_kernel(const void *x, int xt, const void *w, int wt,
                              const float *wscale, const void *i4scale,
                              int i4scale_dt, int group, int nibble_mode,
                              const void *gamma, int gt, const void *bias,
                              int bt, void *y, int yt, int M, int N, int K,
                              float eps, float scale, int norm) {
  (void)M;  // the grid's y extent is M
  __shared__ float red[4];
  const int m = blockIdx.y;
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int64_t xo = (int64_t)m * K;
  float ss = 0.f;
  for (int k = threadIdx.x; k < K; k += 256) {
    const float v = load_as_f32(x, xt, xo + k);
    ss += v * v;
  }
  ss = block_sum_256(ss, red);
  const float rs = norm ? 1.0f / sqrtf(ss / (float)K + eps) : 1.0f;
  if (n >= N) return;
  float acc = 0.f;
  if (nibble_mode >= 0) {
    const uint8_t *pk = (const uint8_t *)w + (int64_t)n * (K / 2);
    const int ng = (K + group - 1) / group;
    for (int g = 0; g < ng; ++g) {
      const float sc = load_as_f32(i4scale, i4scale_dt, (int64_t)n * ng + g);
      float part = 0.f;
      const int k1 = min(K, (g + 1) * group);
      for (int k = g * group; k < k1; ++k) {
        const int nib = (pk[k >> 1] >> (4 * (k & 1))) & 0xF;
        const int q = nibble_mode == MTP_NIBBLE_OFFSET8 ? nib - 8 : (nib ^ 8) - 8;
        float xv = load_as_f32(x, xt, xo + k);
        if (gamma) xv *= load_as_f32(gamma, gt, k);
        part += xv * (float)q;
      }
      acc += part * sc;
    }
  } else {
    const int64_t wo = (int64_t)n * K;
    for (int k = 0; k < K; ++k) {
      float xv = load_as_f32(x, xt, xo + k);
      if (gamma) xv *= load_as_f32(gamma, gt, k);
      acc += xv * load_w_as_f32(w, wt, wo + k);
    }
  }
  float t = K > 0 ? acc * rs : 0.f;  // empty rows: mean is 0/0 but x_norm is empty
  if (wscale) t *= wscale[n];
  if (bias) t += load_as_f32(bias, bt, n);
  store_from_f32(y, yt, (int64_t)m * N + n, t * scale);
}

}  // namespace mtp
