// Weight / activation quantizers of the hot path on gfx950: fp8-e4m3
// (per tensor and per output channel) and grouped INT4, with their
// dequantizers. Element-wise and row-reduction work: HBM-bound, one pass
// over the input, no MFMA.
//
// Numerics follow the reference's torch expressions: the max of |x| keeps
// NaN (torch.max propagates it), the scale is amax / 448 (fp8) or amax / 7
// (INT4) when amax > 0 and 1 otherwise (NaN > 0 is false), x / scale is an
// IEEE fp32 division, INT4 rounds half to even (torch.round) before the
// clamp to [-8, 7], fp8 is the OCP e4m3fn round-to-nearest-even conversion
// of the value clamped to +-448.
#pragma once

#include "mtp_common.hpp"

namespace mtp {

// max(|a|, b) that keeps NaN, like torch.max over a tensor holding NaN.
__device__ __forceinline__ float amax_acc(float m, float v) {
  const float a = fabsf(v);
  return (a != a || a > m) ? a : m;
}
__device__ __forceinline__ float amax_merge(float m, float o) {
  return (o != o || o > m) ? o : m;
}

// clamp that keeps NaN, like torch.clamp.
__device__ __forceinline__ float clamp_nan(float v, float lo, float hi) {
  return v != v ? v : fminf(fmaxf(v, lo), hi);
}

// Two floats (each within +-448 or NaN) to two OCP e4m3fn bytes, round to
// nearest even.
__device__ __forceinline__ uint32_t f32x2_to_fp8x2(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// Block-wide NaN-keeping max of 256 threads.
__device__ __forceinline__ float block_amax_256(float m, float *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = amax_merge(m, __shfl_xor(m, o, 64));
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = m;
  __syncthreads();
  m = red[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) m = amax_merge(m, red[i]);
  __syncthreads();
  return m;
}

// Per-tensor amax: each block reduces a strided slice, the last block to
// arrive reduces the block maxima in block order and writes the fp32 scale.
__global__ void __launch_bounds__(256)
fp8_tensor_scale_kernel(const void *x, int dt, int64_t n, float *part, unsigned *ticket,
                        float *scale) {
  __shared__ float red[4];
  __shared__ int s_last;
  float m = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    m = amax_acc(m, load_as_f32(x, dt, i));
  m = block_amax_256(m, red);
  if (threadIdx.x == 0) {
    pub_f32(part + blockIdx.x, m);
    wait_stores();
    s_last = ticket_add(ticket) == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last || threadIdx.x != 0) return;
  float am = 0.f;
  for (unsigned b = 0; b < gridDim.x; ++b) am = amax_merge(am, get_f32(part + b));
  scale[0] = am > 0.f ? am / 448.0f : 1.0f;
  ticket_reset(ticket);
}

// x -> fp8(clamp(x / scale, +-448)); scale is one value (per tensor) or one
// per row of `row_len` elements (per channel).
__global__ void __launch_bounds__(256)
fp8_quantize_kernel(const void *x, int dt, int64_t n, int64_t row_len, const float *scale,
                    int per_row, uint8_t *q) {
  const int64_t pairs = (n + 1) / 2;
  for (int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x; p < pairs;
       p += (int64_t)gridDim.x * 256) {
    const int64_t i = 2 * p;
    const float s0 = scale[per_row ? i / row_len : 0];
    const float v0 = clamp_nan(load_as_f32(x, dt, i) / s0, -448.0f, 448.0f);
    if (i + 1 < n) {
      const float s1 = scale[per_row ? (i + 1) / row_len : 0];
      const float v1 = clamp_nan(load_as_f32(x, dt, i + 1) / s1, -448.0f, 448.0f);
      *(uint16_t *)(q + i) = (uint16_t)f32x2_to_fp8x2(v0, v1);
    } else {
      q[i] = (uint8_t)(f32x2_to_fp8x2(v0, 0.f) & 0xffu);
    }
  }
}

// Per-row scale amax / 448 (0 -> 1): one block per row.
__global__ void __launch_bounds__(256)
fp8_row_scale_kernel(const void *w, int dt, int64_t K, float *wscale) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float m = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += 256) m = amax_acc(m, load_as_f32(w, dt, row * K + k));
  m = block_amax_256(m, red);
  if (threadIdx.x == 0) wscale[row] = m > 0.f ? m / 448.0f : 1.0f;
}

// fp8 -> fp32 * scale (one scale, or one per row of row_len elements).
__global__ void __launch_bounds__(256)
fp8_dequantize_kernel(const uint8_t *q, int64_t n, int64_t row_len, const float *scale,
                      int per_row, float *out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const f32x2 v = fp8x2_to_f32((uint32_t)q[i], false);
    out[i] = v[0] * scale[per_row ? i / row_len : 0];
  }
}

// Per-channel fp8 in one pass: one 256-thread block per row, the row held
// in registers (NV chunks of 8 elements per thread, all loads issued before
// the reduction), the block amax, then the row is scaled and written as
// 8-byte stores. Rows of K = 8 c elements with c <= 256 NV, 16-byte aligned.
// The same arithmetic as fp8_row_scale_kernel + fp8_quantize_kernel.
template <int DT, int NV>
__global__ void __launch_bounds__(256)
fp8_rows_vec_kernel(const void *w, int64_t K, uint8_t *q, float *wscale) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int64_t kc = K / 8;
  float v[NV][8];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = threadIdx.x + 256 * i;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = 0.f;
    if (c < kc) {
      if constexpr (DT == MTP_F32) {
        const f32x4 *p = (const f32x4 *)w + 2 * (row * kc + c);
        const f32x4 a = p[0], b = p[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[i][e] = a[e];
          v[i][4 + e] = b[e];
        }
      } else {
        const u32x4 u = ((const u32x4 *)w)[row * kc + c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f32x2 t = unpack2<DT>(u[e]);
          v[i][2 * e] = t[0];
          v[i][2 * e + 1] = t[1];
        }
      }
    }
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) m = amax_acc(m, v[i][e]);
  m = block_amax_256(m, red);
  const float s = m > 0.f ? m / 448.0f : 1.0f;
  if (threadIdx.x == 0) wscale[row] = s;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t c = threadIdx.x + 256 * i;
    if (c >= kc) continue;
    uint32_t b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      b[e] = f32x2_to_fp8x2(clamp_nan(v[i][2 * e] / s, -448.0f, 448.0f),
                            clamp_nan(v[i][2 * e + 1] / s, -448.0f, 448.0f));
    uint2 o;
    o.x = b[0] | (b[1] << 16);
    o.y = b[2] | (b[3] << 16);
    ((uint2 *)q)[row * kc + c] = o;
  }
}

// Grouped INT4: one thread per (row, group). scale = amax / 7 (0 -> 1),
// q = clamp(rint(x / scale), -8, 7), byte k / 2 holds q[k] & 0xF in its low
// nibble for even k and q[k + 1] & 0xF in its high nibble.
__global__ void __launch_bounds__(256)
int4_quantize_kernel(const void *w, int dt, int64_t N, int64_t K, int64_t group, uint8_t *packed,
                     float *scales) {
  const int64_t ng = (K + group - 1) / group;
  const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (id >= N * ng) return;
  const int64_t row = id / ng, g = id - (id / ng) * ng;
  const int64_t c0 = g * group, c1 = min(c0 + group, K);
  const int64_t base = row * K;
  float m = 0.f;
  for (int64_t k = c0; k < c1; ++k) m = amax_acc(m, load_as_f32(w, dt, base + k));
  const float s = m > 0.f ? m / 7.0f : 1.0f;
  scales[row * ng + g] = s;
  for (int64_t k = c0; k < c1; k += 2) {
    const float q0 = clamp_nan(rintf(load_as_f32(w, dt, base + k) / s), -8.f, 7.f);
    const uint32_t lo = (uint32_t)(int)q0 & 0xFu;
    uint32_t hi = 0;
    if (k + 1 < c1) {
      const float q1 = clamp_nan(rintf(load_as_f32(w, dt, base + k + 1) / s), -8.f, 7.f);
      hi = ((uint32_t)(int)q1 & 0xFu) << 4;
    }
    packed[row * (K / 2) + k / 2] = (uint8_t)(lo | hi);
  }
}

// Grouped INT4, vector form (groups of 8 L elements with L a power of two
// <= 64, K a multiple of the group, 16-byte aligned rows): lane c takes the
// 8 consecutive elements of chunk c (one or two 16-byte loads), the L lanes
// of a group meet by shuffles for the amax, and each lane writes its 4
// packed bytes. The same arithmetic as int4_quantize_kernel (the maximum of
// |x| does not depend on the order it is taken in), so the same bytes and
// scales, from loads that all go out at once.
template <int DT, int U>
__global__ void __launch_bounds__(256)
int4_quantize_vec_kernel(const void *w, int64_t N, int64_t K, int L, uint8_t *packed,
                         float *scales) {
  // each wave takes 64 U consecutive chunks, load u at chunk 64 u + lane
  const int64_t c0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 64 * U + (threadIdx.x & 63);
  const int64_t nch = N * K / 8;
  float v[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t c = c0 + 64 * u;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[u][e] = 0.f;
    if (c < nch) {
      if constexpr (DT == MTP_F32) {
        const f32x4 a = ((const f32x4 *)w)[2 * c], b = ((const f32x4 *)w)[2 * c + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[u][e] = a[e];
          v[u][4 + e] = b[e];
        }
      } else {
        const u32x4 q = ((const u32x4 *)w)[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f32x2 t = unpack2<DT>(q[e]);
          v[u][2 * e] = t[0];
          v[u][2 * e + 1] = t[1];
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = amax_acc(m, v[u][e]);
    // groups are L consecutive lanes starting at a multiple of L (K / 8 and
    // 64 are multiples of L), so every lane of a group is in this wave
    for (int off = 1; off < L; off <<= 1) m = amax_merge(m, __shfl_xor(m, off, 64));
    const int64_t c = c0 + 64 * u;
    if (c >= nch) continue;
    const float s = m > 0.f ? m / 7.0f : 1.0f;
    // rows hold whole groups, so chunk c is in group c / L of the
    // row-major [N, K / group] scale matrix
    if ((c & (L - 1)) == 0) scales[c >> __builtin_ctz(L)] = s;
    uint32_t out = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = clamp_nan(rintf(v[u][e] / s), -8.f, 7.f);
      out |= ((uint32_t)(int)q & 0xFu) << (4 * e);
    }
    ((uint32_t *)packed)[c] = out;  // bytes 4 c .. 4 c + 3 = elements 8 c .. 8 c + 7
  }
}

// INT4 -> fp32: (nibble - 8) * scales[row, k / group] (the reference decoder).
__global__ void __launch_bounds__(256)
int4_dequantize_kernel(const uint8_t *packed, const void *scales, int sdt, int64_t N, int64_t K,
                       int64_t group, float *out) {
  const int64_t ng = (K + group - 1) / group;
  const int64_t half = K / 2;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < N * K;
       i += (int64_t)gridDim.x * 256) {
    const int64_t row = i / K, k = i - (i / K) * K;
    const uint32_t byte = packed[row * half + k / 2];
    const int nib = (int)((k & 1) ? (byte >> 4) & 0xFu : byte & 0xFu) - 8;
    out[i] = (float)nib * load_as_f32(scales, sdt, row * ng + k / group);
  }
}

}  // namespace mtp
