// Grouped INT4 weight-only GEMM for gfx950 (the INT4 RMSNorm -> linear path):
//   y[m, n] = omul[m] * cmul[n] * sum_k xn[m, k] * ((nib(n, k) - 8) * scale'[n, k / group])
//
// Two launches:
//  1. int4_prep_kernel. One block per row of x (rows padded to whole tiles):
//     xn = fp16(x * r * gamma * 2^-e * d(k)) with r = rstd (norm) or 1, 2^e
//     the power of two that brings max_k |x * r * gamma| into [2^14, 2^15]
//     (omul[m] = 2^e restores the row exactly; fp16 then keeps 11 bits for
//     every entry down to 2^-25 of the row maximum; padded rows are zero),
//     and d(k) = 1/16 for odd k, 1 for even k (the decode below yields 16
//     times the weight at odd k, so the product is unchanged and exact).
//     xn is written fragment-major (xfrag_piece): for each 32-row tile and
//     unit of 128 k, eight 1 KB blocks, one per MFMA k-step, each laid out
//     lane by lane as the B operand of v_mfma_f32_32x32x16_f16. A run of 8 k
//     inside a lane's 16 bytes is permuted to (0, 4, 1, 5, 2, 6, 3, 7), the
//     order in which the weight decode below produces k.
//     The remaining blocks transpose the scales, [N, ng] in any float
//     dtype, to fp16 [ng, ldst], so that the scales of the 32 weight rows a
//     load instruction serves are 64 contiguous bytes. Each column n is
//     first normalised by an exact power of two, 2^-c(n), that brings its
//     largest |scale| into [2^7, 2^8): the decoded weights (at most 128
//     times a scale) then stay below 2^15, far from the fp16 limit, and every
//     scale down to 2^-21 of the column's largest stays a normal fp16 number
//     (11 bits), whatever the scales' own magnitude (cmul[n] = 2^c(n) undoes
//     it in the fp32 epilogue). A column whose largest |scale| is inf or NaN
//     is left as it is (c = 0), so the non-finite value reaches its outputs.
//  2. int4_gemm_kernel<MT, NA>: 4 waves; wave w owns 32 NA weight rows
//     (NA 32-row A subtiles) against all 32 MT rows of x of the workgroup
//     (MT 32-row B tiles); the workgroup covers 128 NA columns of y.
//     K advances by units of 128 (64 bytes of a weight row). Per unit, the
//     x tile (MT x 8 KB), the weight tile (128 NA rows x 64 bytes) and the
//     fp16 scales of the rows are copied to LDS by buffer loads with the
//     LDS bit (no register staging), into one of three LDS stages, two
//     units ahead of the MFMAs; the copies are spread over the k-steps of
//     the current unit. Each lane reads 32 bytes (64 nibbles) of each of
//     its A rows from LDS and decodes them in registers, per dword w of 8
//     nibbles n_0 .. n_7 (n_i at bit 4 i):
//           v = w, then w >> 8:
//             v & 0x000F000F | 0x64006400 -> fp16 pair (1024 + n_j, 1024 + n_j+4)
//             v & 0x00F000F0 | 0x64006400 -> fp16 pair (1024 + 16 n_j+1, 1024 + 16 n_j+5)
//           (pair - 1032) * s or (pair - 1152) * s -> (n - 8) or 16 (n - 8),
//           exact, times s rounded once
//         giving one fp16x8 A fragment per k-step of 16;
//       - 8 k-steps of NA x MT v_mfma_f32_32x32x16_f16, fp32 accumulation.
//     One barrier per unit: it publishes the unit's LDS stage and retires
//     the stage that the next copy overwrites.
//  The row groups of a column group sit on one XCD (workgroups b, b + 8,
//  b + 16, ... are dispatched to the same XCD), so every read of a weight
//  tile after the first tends to hit that XCD's L2.
//  Precision: each scale is rounded once to fp16 (11 bits) after the exact
//  column normalisation; a scale below 2^-21 of its column's largest loses
//  bits (fp16 subnormal), a relative contribution already under 2^-21.
#pragma once

#include <type_traits>

#include "int4g_args.hpp"
#include "wstream.hpp"

namespace mtp {

typedef __attribute__((ext_vector_type(2))) _Float16 h2;
typedef __attribute__((ext_vector_type(8))) _Float16 h8;
typedef __attribute__((ext_vector_type(16))) float f32x16;

// Slot of k-offset i inside an aligned run of 8: the decode yields k in the
// slot order (0, 4, 1, 5, 2, 6, 3, 7).
__device__ __forceinline__ int slot8(int i) { return i < 4 ? 2 * i : 2 * (i - 4) + 1; }

// 16-byte piece of xn holding k = 8q .. 8q + 7 of row m (U units of 128 k):
// tile m / 32, unit q / 16, k-step q % 8, lane 32 * ((q / 8) % 2) + m % 32.
__device__ __forceinline__ int64_t xfrag_piece(int64_t m, int64_t q, int64_t U) {
  const int64_t u = q >> 4, r = q & 15;
  const int64_t lane = ((r >> 3) << 5) + (m & 31);
  return ((((m >> 5) * U + u) * 8 + (r & 7)) << 6) + lane;
}

// Eight consecutive elements p[i .. i + 7] (i % 8 == 0, 16-byte aligned
// rows) as fp32, with one or two vector loads.
template <int DT>
__device__ __forceinline__ void load8_f32(const void *p, int64_t i, float (&v)[8]) {
  if constexpr (DT == MTP_F32) {
    const float4 a = ((const float4 *)p)[i / 4], b = ((const float4 *)p)[i / 4 + 1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const u32x4 w = ((const u32x4 *)p)[i / 8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x2 t = unpack2<DT>(w[j]);
      v[2 * j] = t[0];
      v[2 * j + 1] = t[1];
    }
  }
}

// scales[n0 .. n0 + 63][0 .. ng) (dtype SDT) -> scT[g][n] fp16, n < N.
// Eight loads are issued before their conversions and stores.
template <int SDT>
__device__ __forceinline__ void transpose_scales_t(const void *__restrict__ scales, int64_t N,
                                                   int64_t ng, int64_t ldst, int64_t n0,
                                                   uint16_t *__restrict__ scT, const float *inv) {
  const int64_t total = 64 * ng;
  for (int64_t i0 = threadIdx.x; i0 < total; i0 += 8 * 256) {
    uint32_t raw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t i = i0 + 256 * j;
      const int64_t n = n0 + (i & 63), g = i >> 6;
      raw[j] = 0;
      if (i < total && n < N) {
        if constexpr (SDT == MTP_F32) raw[j] = ((const uint32_t *)scales)[n * ng + g];
        else raw[j] = ((const uint16_t *)scales)[n * ng + g];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t i = i0 + 256 * j;
      const int64_t n = n0 + (i & 63), g = i >> 6;
      if (i < total && n < N) {
        float f;
        if constexpr (SDT == MTP_F32) f = __builtin_bit_cast(float, raw[j]);
        else if constexpr (SDT == MTP_BF16) f = __builtin_bit_cast(float, raw[j] << 16);
        else f = (float)__builtin_bit_cast(_Float16, (uint16_t)raw[j]);
        scT[g * ldst + n] = __builtin_bit_cast(uint16_t, (_Float16)(f * inv[n - n0]));
      }
    }
  }
}
// The same with one 16-byte load per lane (EPC groups of one row) when the
// rows are whole 16-byte chunks: lane n of a wave takes row n0 + n, the
// waves take the chunks in turn, and every store of a wave writes 64
// consecutive rows of one group (128 contiguous bytes).
template <int SDT>
__device__ __forceinline__ void transpose_scales_v(const void *__restrict__ scales, int64_t N,
                                                   int64_t ng, int64_t ldst, int64_t n0,
                                                   uint16_t *__restrict__ scT, const float *inv) {
  constexpr int EPC = SDT == MTP_F32 ? 4 : 8;  // groups per 16-byte chunk
  const int64_t nch = ng / EPC;
  const int64_t n = n0 + (threadIdx.x & 63);
  if (n >= N) return;
  // the whole [N, ng] matrix through one descriptor (< 2 GiB: the host
  // limits ng * ldst * 2); chunks past the row load with an out-of-range
  // offset (zeros, never stored)
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales, (uint32_t)(N * nch * 16));
  for (int64_t c0 = threadIdx.x >> 6; c0 < nch; c0 += 4 * 4) {
    u32x4 raw[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = c0 + 4 * u;
      raw[u] = bload16(rs, c < nch ? (uint32_t)((n * nch + c) * 16) : kOOB);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t c = c0 + 4 * u;
      if (c >= nch) break;
      float f[EPC];
      if constexpr (SDT == MTP_F32) {
        const f32x4 v = __builtin_bit_cast(f32x4, raw[u]);
        f[0] = v[0];
        f[1] = v[1];
        f[2] = v[2];
        f[3] = v[3];
      } else {
        const uint32_t d[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t h = (e & 1) ? d[e >> 1] >> 16 : d[e >> 1] & 0xffffu;
          f[e] = SDT == MTP_BF16 ? __builtin_bit_cast(float, h << 16)
                                 : (float)__builtin_bit_cast(_Float16, (uint16_t)h);
        }
      }
      const float iv = inv[n - n0];
#pragma unroll
      for (int e = 0; e < EPC; ++e)
        scT[(c * EPC + e) * ldst + n] = __builtin_bit_cast(uint16_t, (_Float16)(f[e] * iv));
    }
  }
}
// |scale| of element i of [N, ng] as the bits of a non-negative float (they
// order like the values; inf and NaN sort above every finite value).
__device__ __forceinline__ uint32_t scale_abs_bits(const void *scales, int sdt, int64_t i) {
  if (sdt == MTP_F32) return ((const uint32_t *)scales)[i] & 0x7fffffffu;
  const uint32_t h = ((const uint16_t *)scales)[i];
  const float f = sdt == MTP_BF16 ? __builtin_bit_cast(float, h << 16)
                                  : (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  return __builtin_bit_cast(uint32_t, f) & 0x7fffffffu;
}

// Normalising exponent of a column whose largest |scale| has bits mb: c
// with max * 2^-c in [2^7, 2^8) (0 for an all-zero, inf or NaN column).
__device__ __forceinline__ int scale_norm_exp(uint32_t mb) {
  int e = 0;
  if (mb != 0u && mb < 0x7f800000u) {
    int ex;
    frexpf(__builtin_bit_cast(float, mb), &ex);  // 2^(ex-1) <= max < 2^ex
    e = min(max(ex - 8, -100), 100);
  }
  return e;
}

constexpr int kI4ScaleTileG = 128;  // groups of the one-pass transpose tile
constexpr int kI4ScaleRow = 68;     // fp16 per LDS tile row (64 columns + pad)

// Columns n0 .. n0 + 63 in one pass (16-byte aligned [N, ng] scales with
// whole 16-byte chunks per row, ng <= kI4ScaleTileG): every chunk is loaded
// once, coalesced (consecutive threads take consecutive chunks of a row),
// into registers; the row maxima meet in LDS; the normalised fp16 values go
// through an LDS tile [g][n] and leave as 128-byte runs of scT rows.
// LDS of the scale transposes (one object for every dtype's path)
struct I4ScaleLds {
  uint32_t mx[64];
  float inv[64];
  __attribute__((aligned(16))) uint16_t t[kI4ScaleTileG * kI4ScaleRow];
};

template <int SDT>
__device__ __forceinline__ void transpose_scales_1p(const void *scales, int64_t N, int64_t ng,
                                                    int64_t ldst, int64_t n0, uint16_t *scT,
                                                    float *cmul, I4ScaleLds &sl) {
  constexpr int EPC = SDT == MTP_F32 ? 4 : 8;  // groups per chunk
  constexpr int CPT = 64 * (kI4ScaleTileG / EPC) / 256;  // chunks per thread at most
  uint32_t *const s_mx = sl.mx;
  float *const s_inv = sl.inv;
  uint16_t *const s_t = sl.t;
  const int th = threadIdx.x;
  const int nch = (int)(ng / EPC);
  const int tot = 64 * nch;
  if (th < 64) s_mx[th] = 0u;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales, (uint32_t)(N * nch * 16));
  u32x4 raw[CPT];
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int i = th + 256 * u;
    const int r = i / nch, c = i - (i / nch) * nch;
    raw[u] = bload16(rs, i < tot && n0 + r < N ? (uint32_t)(((n0 + r) * nch + c) * 16) : kOOB);
  }
  __syncthreads();  // s_mx cleared
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int i = th + 256 * u;
    if (i >= tot) break;
    uint32_t mx = 0u;
    // the dwords as an array (indexing the vector with the loop counter
    // read element 0 for every e here)
    const uint32_t d[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      uint32_t b;
      if constexpr (SDT == MTP_F32) {
        b = d[e];
      } else {
        const uint32_t h = (e & 1) ? d[e >> 1] >> 16 : d[e >> 1] & 0xffffu;
        b = SDT == MTP_BF16 ? h << 16
                            : __builtin_bit_cast(uint32_t, (float)__builtin_bit_cast(_Float16, (uint16_t)h));
      }
      mx = max(mx, b & 0x7fffffffu);
    }
    atomicMax(&s_mx[i / nch], mx);
  }
  __syncthreads();
  if (th < 64) {
    const int e = scale_norm_exp(s_mx[th]);
    s_inv[th] = ldexpf(1.0f, -e);
    if (n0 + th < N) cmul[n0 + th] = ldexpf(1.0f, e);
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int i = th + 256 * u;
    if (i >= tot) break;
    const int r = i / nch, c = i - (i / nch) * nch;
    const float iv = s_inv[r];
    const uint32_t d[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      float f;
      if constexpr (SDT == MTP_F32) {
        f = __builtin_bit_cast(float, d[e]);
      } else {
        const uint32_t h = (e & 1) ? d[e >> 1] >> 16 : d[e >> 1] & 0xffffu;
        f = SDT == MTP_BF16 ? __builtin_bit_cast(float, h << 16)
                            : (float)__builtin_bit_cast(_Float16, (uint16_t)h);
      }
      s_t[(c * EPC + e) * kI4ScaleRow + r] = __builtin_bit_cast(uint16_t, (_Float16)(f * iv));
    }
  }
  __syncthreads();
  // row g of the tile -> scT[g][n0 .. n0 + 63]: 8 pieces of 8 columns
  for (int j = th; j < ng * 8; j += 256) {
    const int g = j >> 3, p = j & 7;
    const uint32_t *src = (const uint32_t *)(s_t + g * kI4ScaleRow + 8 * p);
    const int64_t n = n0 + 8 * p;
    uint16_t *dst = scT + g * ldst + n;
    if (n + 7 < N) {
      *(u32x4 *)dst = u32x4{src[0], src[1], src[2], src[3]};
    } else {
      for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = s_t[g * kI4ScaleRow + 8 * p + e];
    }
  }
}

// Columns n0 .. n0 + 63: the normalising powers of two (cmul), then the
// transpose of the normalised scales to fp16.
__device__ __forceinline__ void transpose_scales(const void *scales, int sdt, int64_t N,
                                                 int64_t ng, int64_t ldst, int64_t n0,
                                                 uint16_t *scT, float *cmul, I4ScaleLds &sl) {
  {
    const int epc = sdt == MTP_F32 ? 4 : 8;
    if ((((uintptr_t)scales) & 15) == 0 && ng % epc == 0 && ng <= kI4ScaleTileG) {
      if (sdt == MTP_F32) transpose_scales_1p<MTP_F32>(scales, N, ng, ldst, n0, scT, cmul, sl);
      else if (sdt == MTP_BF16) transpose_scales_1p<MTP_BF16>(scales, N, ng, ldst, n0, scT, cmul, sl);
      else transpose_scales_1p<MTP_F16>(scales, N, ng, ldst, n0, scT, cmul, sl);
      return;
    }
  }
  uint32_t *const s_mx = sl.mx;
  float *const s_inv = sl.inv;
  const int c = threadIdx.x & 63;
  const int64_t n = n0 + c;
  if (threadIdx.x < 64) s_mx[c] = 0u;
  __syncthreads();
  if (n < N) {
    // thread (c, q) takes groups q, q + 4, ...; eight loads go out together
    uint32_t mx = 0u;
    for (int64_t g0 = threadIdx.x >> 6; g0 < ng; g0 += 4 * 8) {
      uint32_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t g = g0 + 4 * j;
        v[j] = g < ng ? scale_abs_bits(scales, sdt, n * ng + g) : 0u;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = max(mx, v[j]);
    }
    atomicMax(&s_mx[c], mx);
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int e = scale_norm_exp(s_mx[c]);
    s_inv[c] = ldexpf(1.0f, -e);
    if (n < N) cmul[n] = ldexpf(1.0f, e);
  }
  __syncthreads();
  const int epc = sdt == MTP_F32 ? 4 : 8;
  if ((((uintptr_t)scales) & 15) == 0 && ng % epc == 0) {
    if (sdt == MTP_F32) transpose_scales_v<MTP_F32>(scales, N, ng, ldst, n0, scT, s_inv);
    else if (sdt == MTP_BF16) transpose_scales_v<MTP_BF16>(scales, N, ng, ldst, n0, scT, s_inv);
    else transpose_scales_v<MTP_F16>(scales, N, ng, ldst, n0, scT, s_inv);
    return;
  }
  if (sdt == MTP_F32) transpose_scales_t<MTP_F32>(scales, N, ng, ldst, n0, scT, s_inv);
  else if (sdt == MTP_BF16) transpose_scales_t<MTP_BF16>(scales, N, ng, ldst, n0, scT, s_inv);
  else transpose_scales_t<MTP_F16>(scales, N, ng, ldst, n0, scT, s_inv);
}

// Row statistics of the prep: the workgroup's sums (sum of x^2, max
// |x * gamma|) reduced, rstd r (norm) or 1, the power of two 2^e that brings
// max |x * r * gamma| into [2^14, 2^15] (omul[row] = 2^e); returns r 2^-e.
__device__ __forceinline__ float int4_row_stats(float ss, float mx, float (&red)[2][4], int64_t K,
                                                float eps, int norm, float *omul, int64_t row) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ss += __shfl_xor(ss, o, 64);
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = ss;
    red[1][threadIdx.x >> 6] = mx;
  }
  __syncthreads();
  ss = red[0][0] + red[0][1] + red[0][2] + red[0][3];
  mx = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
  const float r = norm ? 1.0f / sqrtf(ss / (float)K + eps) : 1.0f;
  const float top = mx * r;
  int e = 0;
  if (top > 0.f && top <= 3.0e38f) {
    int ex;
    frexpf(top, &ex);  // top <= 2^ex < 2 top
    e = min(max(ex - 15, -100), 100);
  }
  if (threadIdx.x == 0) omul[row] = ldexpf(1.0f, e);
  return ldexpf(r, -e);
}

// 16-byte xn piece of 8 consecutive k (first even): x * mul * gamma, odd k
// times 1/16, rounded to fp16, in the decode's slot order.
template <int GDT>
__device__ __forceinline__ u32x4 int4_xpiece(const float (&v)[8], const float (&g)[8], float mul) {
  _Float16 hv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float t = v[i] * ((i & 1) ? mul * 0.0625f : mul);
    if constexpr (GDT >= 0) t *= g[i];
    hv[slot8(i)] = (_Float16)t;
  }
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    o[j] = (uint32_t)__builtin_bit_cast(uint16_t, hv[2 * j]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, hv[2 * j + 1]) << 16);
  return o;
}

// Blocks [0, rows): row m of x -> xn (fp16, fragment-major), omul[m]; rows
// m >= M are zero. Blocks [rows, rows + ceil(N / 64)): scales -> scT, cmul.
// XDT: dtype of x; GDT: dtype of gamma, or -1 without gamma.
template <int XDT, int GDT>
__global__ void __launch_bounds__(256)
int4_prep_kernel(const void *x, int64_t M, int64_t K, const void *gamma, float eps, int norm,
                 void *xfv, float *omul, int64_t rows, const void *scales, int sdt, int64_t N,
                 int64_t ng, int64_t ldst, uint16_t *scT, float *cmul) {
  __shared__ float red[2][4];
  __shared__ I4ScaleLds sl;
  u32x4 *xf = (u32x4 *)xfv;
  if ((int64_t)blockIdx.x >= rows) {
    transpose_scales(scales, sdt, N, ng, ldst, ((int64_t)blockIdx.x - rows) * 64, scT, cmul, sl);
    return;
  }
  // The 8 rows whose pieces share the 128-byte lines of xn (rows 8 g .. 8 g
  // + 7) go to blocks b with one value of b mod 8, i.e. one XCD when blocks
  // are dealt to the XCDs in turn: their 16-byte stores then meet in one L2
  // and leave as whole lines (prep 8.2 -> 7.4 us at 256 rows). Any block
  // order gives the same result.
  int64_t row = blockIdx.x;
  if (rows % 64 == 0) {
    const int64_t xq = row & 7, y = row >> 3;
    row = 8 * (8 * (y >> 3) + xq) + (y & 7);
  }
  const int64_t U = K / 128, nq = K / 8;
  if (row >= M) {
    for (int64_t q = threadIdx.x; q < nq; q += 256)
      xf[xfrag_piece(row, q, U)] = u32x4{0u, 0u, 0u, 0u};
    if (threadIdx.x == 0) omul[row] = 0.f;
    return;
  }
  const int64_t base = row * K;
  float ss = 0.f, mx = 0.f;  // sum of x^2, max |x * gamma|
  if (nq <= 4 * 256) {
    // K <= 8192: the row (and gamma) stay in registers, one round trip
    float v[4][8], g[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t q = threadIdx.x + 256 * u;
      if (q < nq) {
        load8_f32<XDT>(x, base + 8 * q, v[u]);
        if constexpr (GDT >= 0) load8_f32<GDT>(gamma, 8 * q, g[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (threadIdx.x + 256 * u >= nq) break;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ss += v[u][i] * v[u][i];
        mx = fmaxf(mx, fabsf(GDT >= 0 ? v[u][i] * g[u][i] : v[u][i]));
      }
    }
    const float mul = int4_row_stats(ss, mx, red, K, eps, norm, omul, row);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t q = threadIdx.x + 256 * u;
      if (q >= nq) break;
      xf[xfrag_piece(row, q, U)] = int4_xpiece<GDT>(v[u], g[u], mul);
    }
    return;
  }
#pragma unroll 4
  for (int64_t q = threadIdx.x; q < nq; q += 256) {
    float v[8], g[8];
    load8_f32<XDT>(x, base + 8 * q, v);
    if constexpr (GDT >= 0) load8_f32<GDT>(gamma, 8 * q, g);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ss += v[i] * v[i];
      mx = fmaxf(mx, fabsf(GDT >= 0 ? v[i] * g[i] : v[i]));
    }
  }
  const float mul = int4_row_stats(ss, mx, red, K, eps, norm, omul, row);
#pragma unroll 4
  for (int64_t q = threadIdx.x; q < nq; q += 256) {
    float v[8], g[8];
    load8_f32<XDT>(x, base + 8 * q, v);
    if constexpr (GDT >= 0) load8_f32<GDT>(gamma, 8 * q, g);
    xf[xfrag_piece(row, q, U)] = int4_xpiece<GDT>(v, g, mul);
  }
}

// 16 bytes per lane from a buffer straight into LDS (lane i writes bytes
// 16 i .. 16 i + 15 after `lds`). The body exists only in the device pass:
// the host pass cannot form the LDS address-space pointer, and an invalid
// expression there would silently drop the host stubs of the kernels.
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, unsigned char *lds,
                                           uint32_t voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, soff, 0, 0);
#else
  (void)r; (void)lds; (void)voff; (void)soff;
#endif
}

// Chunk swizzle of the weight rows in LDS (16-byte chunks of a 64-byte row).
__device__ __forceinline__ int i4_swz(int r) { return (r >> 2) & 3; }

// (a & m) | c in one v_and_or_b32 (m, c in registers).
__device__ __forceinline__ uint32_t and_or_u32(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(m), "v"(c));
  return d;
}
// A constant the compiler keeps in a VGPR (it cannot fold it back into a
// literal operand).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  uint32_t d;
  asm volatile("v_mov_b32 %0, %1" : "=v"(d) : "s"(v));
  return d;
}

template <int MT, int NA, int NWV, bool KH, bool TWOS>
__global__ void __launch_bounds__(64 * NWV, 1)
int4_gemm_kernel(const I4Args a) {
  // KH: waves split each unit's k-steps in halves (wave = row group + RQ
  // k-half); the halves' sums meet in LDS at the end. RQ row groups of NA
  // 32-row A subtiles each: 8 waves x NA 2 (two waves per SIMD), or 4 waves
  // x NA 4 (one wave per SIMD, 256 accumulators: half the x reads per MFMA)
  constexpr int RQ = KH ? NWV / 2 : NWV;  // row groups
  constexpr int KSW = KH ? 4 : 8;         // k-steps per wave per unit
  constexpr int BN = 32 * NA * RQ, UK = 128;
  constexpr int TILE = 8 * 1024;          // bytes of one 32-row x tile per unit
  constexpr int XST = MT * TILE;          // x bytes of one LDS stage
  constexpr int WST = BN * 64;            // weight bytes of one LDS stage (64 per row)
  constexpr int SST = 4 * 1024;           // scale bytes of one LDS stage (4 runs of 32 k)
  constexpr int STAGE = XST + WST + SST;
  constexpr int NS = 3;                   // LDS stages (copies run two units ahead)
  constexpr int ND = 8 * MT / NWV;        // x copies per wave per unit
  constexpr int NWL = BN / 16 / NWV;      // weight copies per wave per unit (16 rows each)
  static_assert(NWV == 4 || NWV == 8, "4 or 8 waves");
  static_assert((8 * MT) % NWV == 0 && (BN / 16) % NWV == 0, "copies divide among the waves");
  static_assert(!KH || RQ * NA * MT * 4 * 1024 <= 3 * (MT * 8 * 1024 + BN * 64 + 4 * 1024),
                "k-half merge fits the LDS stages");
  // scale copy of a unit: KH with 8 waves, two waves per run (half the rows
  // each); otherwise one wave per run
  constexpr int SPARTS = KH ? NWV / 4 : 1;
  constexpr int NV = NWL + 1 + ND;        // vector-memory instructions per wave per unit
  // one LDS object (a second one makes the compiler wait for every LDS-DMA
  // copy before each LDS read of the main loop): the stages, then the
  // workgroup's column factors cmul
  __shared__ __attribute__((aligned(1024))) unsigned char xs[NS * STAGE + BN * 4];
  float *const s_cm = (float *)(xs + NS * STAGE);

  const int th = threadIdx.x;
  const int lane = th & 63;
  // the wave index is uniform: readfirstlane keeps the scale copy's scalar
  // offset (which depends on it) in scalar registers, without a waterfall
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int rq = KH ? wave % RQ : wave;  // row group: A tiles NA rq .. NA rq + NA - 1
  const int kh = KH ? wave / RQ : 0;     // k-half (k-steps 4 kh .. 4 kh + 3)

  // blockIdx -> (column group, row group): the row groups of column group
  // c are workgroups with b % 8 == c % 8 (one XCD).
  int cg, rg;
  {
    const int b = blockIdx.x;
    const int sb = b >> 3;
    const int q = sb / a.gm;
    cg = q * 8 + (b & 7);
    rg = sb - q * a.gm;
  }
  if (cg >= a.gn) return;
  const int n0 = cg * BN;
  // row factors of the epilogue, loaded now so that their latency hides
  // behind the main loop (rows past the padded tile read 0 and are not stored)
  float omr[MT];
  {
    const __amdgpu_buffer_rsrc_t ors = make_rsrc(a.omul, (uint32_t)a.M * 4u);
#pragma unroll
    for (int j = 0; j < MT; ++j)
      omr[j] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(
                     ors, (uint32_t)(rg * MT * 32 + 32 * j + (threadIdx.x & 31)) * 4u, 0, 0));
  }
  {
    // columns past N read 0 (never stored); the main loop's barriers order
    // these stores before the epilogue's reads
    const __amdgpu_buffer_rsrc_t crs = make_rsrc(a.cmul, (uint32_t)a.N * 4u);
    for (int i = th; i < BN; i += 64 * NWV)
      s_cm[i] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(crs, (uint32_t)(n0 + i) * 4u, 0, 0));
  }
  const int nunits = a.K / UK;

  // Weights: per unit the workgroup's BN rows x 64 bytes are copied to LDS,
  // 64 bytes per row, 16 rows x 64 bytes per copy (copy c = wave + NWV i);
  // the 16-byte chunk j of row r sits at chunk j ^ i4_swz(r) of the row's
  // 64 bytes, so lane L (LDS chunk L % 4 of row 16 c + L / 4) loads that
  // row's chunk (L % 4) ^ i4_swz(row). The MFMA A operand of subtile t is
  // read back per lane: row wcol[t], chunks 2 h, 2 h + 1 (one per k-half):
  // the 16 lanes of a read take 16 consecutive rows at one chunk, which the
  // swizzle spreads over all 64 banks (row-major they would hit 16 banks).
  const uint32_t ldw = (uint32_t)a.K / 2;
  const int nrows = min(BN, a.N - n0);
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(a.packed + (int64_t)n0 * ldw, (uint32_t)nrows * ldw);
  uint32_t wvo[NWL];
#pragma unroll
  for (int i = 0; i < NWL; ++i)
    wvo[i] = (uint32_t)(16 * (wave + NWV * i) + (lane >> 2)) * ldw +
             16u * (uint32_t)((lane & 3) ^ i4_swz(16 * (wave + NWV * i) + (lane >> 2)));
  int wcol[NA];  // row of the lane inside the workgroup's BN
#pragma unroll
  for (int t = 0; t < NA; ++t) wcol[t] = 32 * (NA * rq + t) + l32;
  // fp16 scales, transposed: scale of row n, group g at scT[g * ldst + n].
  // Per unit the scales of the 4 k-runs (k = 128 u + 32 r .. + 31) for the
  // BN rows go to LDS run by run (1 KB each, BN * 2 bytes used). 4 waves:
  // wave w copies run w, lanes 0 .. BN / 8 - 1 16 bytes each, the others
  // read past the descriptor into the unused part of the run. 8 waves: wave
  // w copies half w / 4 (rows BN / 2 * (w / 4) ..) of run w % 4 with lanes
  // 0 .. BN / 16 - 1 only (the other lanes are masked off: their zeros would
  // land on the other half).
  const __amdgpu_buffer_rsrc_t srs =
      make_rsrc((const uint16_t *)a.scales + n0, (uint32_t)(a.ng * a.ldst - n0) * 2u);
  const int srun = wave & 3;
  // a group of a multiple of 128 k covers the whole unit: its four runs
  // share one scale per row, so only run 0 is copied and read (the other
  // copies go to the zero-byte descriptor, keeping the per-unit count of
  // vector-memory instructions of every wave)
  const bool one_run = a.group % 128 == 0;
  const bool scopy = !one_run || srun == 0;
  const uint32_t shalf = (uint32_t)(wave >> 2) * (BN / SPARTS) * 2u;  // bytes
  const uint32_t svo = lane < BN / 8 ? (uint32_t)lane * 16u + shalf : kOOB;
  const uint32_t ldst2 = (uint32_t)a.ldst * 2u;
  // x tiles of this workgroup: MT consecutive 32-row tiles of the
  // fragment-major copy; tile T, unit u starts at byte (T * U + u) * TILE.
  const unsigned char *xbase = (const unsigned char *)a.xn + (int64_t)rg * MT * nunits * TILE;
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(xbase, (uint32_t)(MT * nunits) * TILE);
  // x copy c of a unit (c = wave + NWV i): tile c / 8, k-step c % 8; the
  // unit goes in the scalar offset, the per-lane part is fixed.
  uint32_t xvo[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) {
    const int c = wave + NWV * i;
    xvo[i] = (uint32_t)((c >> 3) * nunits * TILE + (c & 7) * 1024 + lane * 16);
  }

  // Vector-memory instruction v (0 <= v < NV) of unit `unit` into LDS
  // stage `slot`: weight copies first, then the scale copy, then x copies.
  // Units past the last one copy through a descriptor of zero bytes: every
  // offset is out of range, so zeros and no memory access (chosen with
  // scalar selects, not per-lane offsets).
  const __amdgpu_buffer_rsrc_t nrs = make_rsrc(a.packed, 0u);
  auto issue = [&](auto vc, int unit, int slot) __attribute__((always_inline)) {
    constexpr int v = decltype(vc)::value;
    const bool live = unit < nunits;
    const int su = live ? unit : 0;
    if constexpr (v < NWL) {
      lds_copy16(live ? wrs : nrs, xs + slot * STAGE + XST + (wave + NWV * v) * 1024, wvo[v],
                 su * 64);
    } else if constexpr (v == NWL) {
      const int k = su * UK + 32 * srun;
      const int g = a.glog >= 0 ? k >> a.glog : k / a.group;
      unsigned char *dst = xs + slot * STAGE + XST + WST + srun * 1024 + shalf;
      if constexpr (SPARTS > 1) {
        if (lane < BN / 8 / SPARTS)
          lds_copy16(live && scopy ? srs : nrs, dst, svo, (int)((uint32_t)g * ldst2));
      } else {
        lds_copy16(live && scopy ? srs : nrs, dst, svo, (int)((uint32_t)g * ldst2));
      }
    } else {
      const int i = v - NWL - 1;
      const int c = wave + NWV * i;
      lds_copy16(live ? xrs : nrs, xs + slot * STAGE + (c >> 3) * TILE + (c & 7) * 1024, xvo[i],
                 su * TILE);
    }
  };

  f32x16 acc[NA][MT];
#pragma unroll
  for (int t = 0; t < NA; ++t)
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[t][j][e] = 0.f;

  // decode constants in registers: v_and_or_b32 takes no literal operand
  // (VOP3), and with them it masks and ORs in one instruction
  const uint32_t klo = opaque_u32(0x000F000Fu), khi = opaque_u32(0x00F000F0u),
                 kmag = opaque_u32(0x64006400u);
  const h2 m1032 = h2{(_Float16)(-1032.0f), (_Float16)(-1032.0f)};
  const h2 m1152 = h2{(_Float16)(-1152.0f), (_Float16)(-1152.0f)};
  // One unit: 8 k-steps, software-pipelined one step deep (the LDS reads
  // and the weight decode of step s + 1 are issued before the MFMAs of s).
  // The NV vector-memory instructions of unit `nunit` (two units ahead) are
  // spread over the k-steps so that the memory pipeline's queues never fill
  // and block the in-order issue of the MFMAs behind them.
  auto compute = [&](int slot, int nunit, int nslot) __attribute__((always_inline)) {
    const unsigned char *sx = xs + slot * STAGE + lane * 16;
    const unsigned char *sw = xs + slot * STAGE + XST;
    const unsigned char *ss = xs + slot * STAGE + XST + WST;
    // the wave's 16-byte halves of its A rows (both, or its k-half's) and
    // the scales of their 32-k runs
    constexpr int NE = KH ? 1 : 2;
    u32x4 wr[NA][NE];
#pragma unroll
    for (int t = 0; t < NA; ++t)
#pragma unroll
      for (int e = 0; e < NE; ++e)
        wr[t][e] = *(const u32x4 *)(sw + wcol[t] * 64 +
                                    16 * ((2 * h + (KH ? kh : e)) ^ i4_swz(wcol[t])));
    h2 s2[NA][NE];
#pragma unroll
    for (int t = 0; t < NA; ++t)
#pragma unroll
      for (int g = 0; g < NE; ++g) {
        const int run = one_run ? 0 : 2 * h + (KH ? kh : g);
        const _Float16 f = *(const _Float16 *)(ss + run * 1024 + wcol[t] * 2);
        s2[t][g] = h2{f, f};
      }
    // wave k-step s (0 .. KSW - 1) is k-step 4 kh + s of the unit
    auto decode = [&](h8 (&af)[NA], int s) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < NA; ++t) {
        uint32_t w = wr[t][KH ? 0 : s >> 2][s & 3];
        if constexpr (TWOS) w ^= 0x88888888u;  // two's complement -> offset-8
        const uint32_t w8 = w >> 8;
        const h2 sv = s2[t][KH ? 0 : s >> 2];
        const uint32_t q0 = and_or_u32(w, klo, kmag);
        const uint32_t q1 = and_or_u32(w, khi, kmag);
        const uint32_t q2 = and_or_u32(w8, klo, kmag);
        const uint32_t q3 = and_or_u32(w8, khi, kmag);
        u32x4 o;
        o[0] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, q0) + m1032) * sv);
        o[1] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, q1) + m1152) * sv);
        o[2] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, q2) + m1032) * sv);
        o[3] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(h2, q3) + m1152) * sv);
        af[t] = __builtin_bit_cast(h8, o);
      }
    };
    auto read_b = [&](h8 (&bv)[MT], int s) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < MT; ++j) bv[j] = *(const h8 *)(sx + j * TILE + (4 * kh + s) * 1024);
    };
    h8 af[2][NA], bv[2][MT];
    read_b(bv[0], 0);
    decode(af[0], 0);
    static_for<0, KSW>([&](auto sc_) {
      constexpr int s = decltype(sc_)::value;
      static_for<s * NV / KSW, (s + 1) * NV / KSW>([&](auto vc) { issue(vc, nunit, nslot); });
      if constexpr (s + 1 < KSW) {
        read_b(bv[(s + 1) & 1], s + 1);
        decode(af[(s + 1) & 1], s + 1);
      }
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int t = 0; t < NA; ++t)
          acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s & 1][t], bv[s & 1][j],
                                                             acc[t][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Pipeline: units u + 1 and u + 2 are in flight while unit u computes.
  // The loop is unrolled by the ring length so that stage r's offsets are
  // compile-time constants. Copies are issued for every u + 2, also past
  // the last unit: such a copy writes zeros into a stage that is never
  // computed on, so the count of instructions behind the copies of unit u
  // is always NV.
  static_for<0, NV>([&](auto vc) { issue(vc, 0, 0); });
  __builtin_amdgcn_sched_barrier(0);  // every copy of unit 0 before any of unit 1
  static_for<0, NV>([&](auto vc) { issue(vc, 1, 1); });
  auto step = [&](auto rc, int u) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::value;
    __builtin_amdgcn_sched_barrier(0);
    // this wave's copies of unit u have landed once at most the NV
    // instructions of unit u + 1 are outstanding; the barrier makes every
    // wave's copies visible and retires the stage of unit u - 1, which the
    // copies of unit u + 2 overwrite
    wait_vmcnt_barrier<NV>();
    __builtin_amdgcn_sched_barrier(0);
    compute(r, u + 2, (r + 2) % 3);
  };
  int u = 0;
  for (; u + 3 <= nunits; u += 3) {
    step(std::integral_constant<int, 0>{}, u);
    step(std::integral_constant<int, 1>{}, u + 1);
    step(std::integral_constant<int, 2>{}, u + 2);
  }
  if (u < nunits) step(std::integral_constant<int, 0>{}, u);
  if (u + 1 < nunits) step(std::integral_constant<int, 1>{}, u + 1);
  // no copy into LDS may still be in flight when the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // k-halves: the waves of half 1 hand their sums to those of half 0
  // through LDS (the stages are free now)
  // ([rq][t][j][quad][lane] of f32x4: 16 lanes touch 256 contiguous bytes)
  f32x4 *red = (f32x4 *)xs;
  if constexpr (KH) {
    __syncthreads();
    if (kh == 1) {
#pragma unroll
      for (int t = 0; t < NA; ++t)
#pragma unroll
        for (int j = 0; j < MT; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            red[(((rq * NA + t) * MT + j) * 4 + g) * 64 + lane] =
                f32x4{acc[t][j][4 * g], acc[t][j][4 * g + 1], acc[t][j][4 * g + 2],
                      acc[t][j][4 * g + 3]};
    }
    __syncthreads();
    if (kh == 1) return;
  }

  // epilogue: acc[t][j][e] (plus the other k-half's red entry) = y[m][n]
  // with m = m0 + 32 j + l32 and n = n0 + wcol[t] - l32 + 8 (e / 4) + 4 h + e % 4.
  const int m0 = rg * MT * 32;
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const int m = m0 + 32 * j + l32;
    if (m >= a.M) continue;
    const float om = omr[j];
#pragma unroll
    for (int t = 0; t < NA; ++t) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wcol[t] - l32 + 8 * g + 4 * h;
        const int64_t base = (int64_t)m * a.N + n;
        float r4[4] = {acc[t][j][4 * g], acc[t][j][4 * g + 1], acc[t][j][4 * g + 2],
                       acc[t][j][4 * g + 3]};
        if constexpr (KH) {
          const f32x4 o = red[(((rq * NA + t) * MT + j) * 4 + g) * 64 + lane];
#pragma unroll
          for (int e = 0; e < 4; ++e) r4[e] += o[e];
        }
        const float *cm = s_cm + (n - n0);
        const float v0 = r4[0] * cm[0] * om, v1 = r4[1] * cm[1] * om, v2 = r4[2] * cm[2] * om,
                    v3 = r4[3] * cm[3] * om;
        if (n + 3 < a.N && a.yvec) {
          uint2 pk;
          if (a.ydt == MTP_BF16) {
            pk.x = pack2<MTP_BF16>(v0, v1);
            pk.y = pack2<MTP_BF16>(v2, v3);
          } else {
            pk.x = pack2<MTP_F16>(v0, v1);
            pk.y = pack2<MTP_F16>(v2, v3);
          }
          *(uint2 *)((uint16_t *)a.y + base) = pk;
        } else {
          const float v[4] = {v0, v1, v2, v3};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < a.N) store_from_f32(a.y, a.ydt, base + e, v[e]);
        }
      }
    }
  }
}

}  // namespace mtp
