// The draft chain around the head GEMM: RMSNorm, add + RMSNorm and the
// greedy token with its embedding row.
//
//   fused_rmsnorm       y = x * rstd * w,        rstd = 1 / sqrt(mean(x^2) + eps)
//   fused_add_rmsnorm   y = s * rstd * w,  s = x + r
//   argmax (+ gather)   token[m] = argmax_v logits[m, v]  (torch.argmax order),
//                       emb[m] = table[token[m]]
//
// The norms run one 256-thread workgroup per row (a row of the draft chain
// is a few KB; the row is read twice, the second time from cache); sums of
// squares and the scaled products in fp32, rounded once to the output dtype.
// The argmax spreads each row over S workgroups (segments of the vocabulary)
// so that a handful of rows still keeps many CUs reading; each workgroup publishes
// one 64-bit key (verify_tail.hpp) for its segment, and the last of a row's
// workgroups to arrive (a per-row ticket in the counter prefix) reduces them,
// writes the token and copies the embedding row.
#pragma once

#include "verify_tail.hpp"

namespace mtp {

// Sum over a 256-thread workgroup (every thread gets the total).
__device__ __forceinline__ float sum_256(float v, float *red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

template <bool ADD>
__global__ void __launch_bounds__(256)
rmsnorm_rows_kernel(const void *x, const void *r, int dt, const void *w, int wdt, void *y,
                    int N, float eps) {
  __shared__ float red[4];
  const int64_t row = (int64_t)blockIdx.x * N;
  float ss = 0.f;
  for (int i = threadIdx.x; i < N; i += 256) {
    float s = load_as_f32(x, dt, row + i);
    if constexpr (ADD) s += load_as_f32(r, dt, row + i);
    ss = __builtin_fmaf(s, s, ss);
  }
  ss = sum_256(ss, red);
  const float rstd = 1.0f / sqrtf(ss / (float)N + eps);
  for (int i = threadIdx.x; i < N; i += 256) {
    float s = load_as_f32(x, dt, row + i);
    if constexpr (ADD) s += load_as_f32(r, dt, row + i);
    const float g = w ? load_as_f32(w, wdt, i) : 1.f;
    store_from_f32(y, dt, row + i, s * rstd * g);
  }
}

// ---- 16-byte vector forms: rows that are whole 16-byte chunks, 16-byte
// aligned. Every load of a row (or segment) is issued before the arithmetic
// that uses it, so a row costs one memory round trip instead of one per
// element (the dtype is a template parameter, not a per-element switch);
// the norms keep the row in registers for their second pass.
template <int DT>
constexpr int vec_elems() { return DT == MTP_F32 ? 4 : 8; }
template <int DT>
__device__ __forceinline__ void unpack16(u32x4 v, float (&f)[vec_elems<DT>()]) {
  if constexpr (DT == MTP_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = __uint_as_float(v[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f32x2 t = unpack2<DT>(v[e]);
      f[2 * e] = t[0];
      f[2 * e + 1] = t[1];
    }
  }
}
template <int DT>
__device__ __forceinline__ u32x4 pack16(const float (&f)[vec_elems<DT>()]) {
  u32x4 v;
  if constexpr (DT == MTP_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = __float_as_uint(f[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = pack2<DT>(f[2 * e], f[2 * e + 1]);
  }
  return v;
}

// One 256-thread workgroup per row of N = 256 NV E or fewer elements (E per
// 16 bytes); W: a weight of the row's dtype; ADD: s = x + r in fp32. The
// same arithmetic as rmsnorm_rows_kernel (fp32 squares and products,
// (s * rstd) * w rounded once); the sum of squares is taken in another order.
template <int DT, bool W, bool ADD, int NV>
__global__ void __launch_bounds__(256)
rmsnorm_vec_kernel(const void *x, const void *r, const void *w, void *y, int N, float eps) {
  constexpr int E = vec_elems<DT>();
  __shared__ float red[4];
  const int nch = N / E;
  const int64_t row = (int64_t)blockIdx.x * nch;  // in 16-byte chunks
  u32x4 xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int q = threadIdx.x + 256 * c;
    if (q < nch) {
      xv[c] = ((const u32x4 *)x)[row + q];
      if constexpr (ADD) rv[c] = ((const u32x4 *)r)[row + q];
      if constexpr (W) wv[c] = ((const u32x4 *)w)[q];
    }
  }
  float sv[NV][E];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    if ((int)threadIdx.x + 256 * c >= nch) continue;
    unpack16<DT>(xv[c], sv[c]);
    if constexpr (ADD) {
      float t[E];
      unpack16<DT>(rv[c], t);
#pragma unroll
      for (int e = 0; e < E; ++e) sv[c][e] += t[e];
    }
#pragma unroll
    for (int e = 0; e < E; ++e) ss = __builtin_fmaf(sv[c][e], sv[c][e], ss);
  }
  ss = sum_256(ss, red);
  const float rstd = 1.0f / sqrtf(ss / (float)N + eps);
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int q = threadIdx.x + 256 * c;
    if (q >= nch) continue;
    float g[E], o[E];
    if constexpr (W) {
      unpack16<DT>(wv[c], g);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) g[e] = 1.f;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = sv[c][e] * rstd * g[e];
    ((u32x4 *)y)[row + q] = pack16<DT>(o);
  }
}

struct ArgmaxArgs {
  const void *logits;  // [M, V], row stride ld elements
  int dt;
  int64_t ld;
  int M, V;
  int S;                      // workgroups (segments) per row
  int seg;                    // vocabulary entries per segment
  unsigned long long *part;   // [M][S] segment keys (S > 1)
  unsigned *ticket;           // [M] arrival tickets, zero between launches (S > 1)
  int64_t *tokens;            // [M]
  const void *table;          // [Vt, H] embedding rows or null
  int tbytes;                 // bytes per table element (2 or 4)
  int H;
  void *emb;                  // [M, H] or null
  int emb16;                  // 1: table and emb rows whole 16-byte chunks, 16-byte aligned
};

__device__ __forceinline__ void copy_row(const ArgmaxArgs &a, int m, int64_t tok) {
  // every segment holds at least one column, so a key is never empty; the
  // clamp keeps the table read in bounds regardless
  if (!a.table || tok < 0 || tok >= a.V) return;
  if (a.tbytes == 2) {
    const uint16_t *src = (const uint16_t *)a.table + tok * a.H;
    uint16_t *dst = (uint16_t *)a.emb + (int64_t)m * a.H;
    for (int i = threadIdx.x; i < a.H; i += blockDim.x) dst[i] = src[i];
  } else {
    const uint32_t *src = (const uint32_t *)a.table + tok * a.H;
    uint32_t *dst = (uint32_t *)a.emb + (int64_t)m * a.H;
    for (int i = threadIdx.x; i < a.H; i += blockDim.x) dst[i] = src[i];
  }
}

// The embedding row of token tok, 16 bytes per thread per chunk (rows of
// whole chunks, 16-byte aligned).
__device__ __forceinline__ void copy_row16(const ArgmaxArgs &a, int m, int64_t tok) {
  if (!a.table || tok < 0 || tok >= a.V) return;
  const int nch = a.H * a.tbytes / 16;
  const u32x4 *src = (const u32x4 *)((const unsigned char *)a.table + tok * a.H * a.tbytes);
  u32x4 *dst = (u32x4 *)((unsigned char *)a.emb + (int64_t)m * a.H * a.tbytes);
  for (int i = threadIdx.x; i < nch; i += blockDim.x) dst[i] = src[i];
}

__device__ __forceinline__ unsigned long long wave_key_max(unsigned long long k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)k, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(k >> 32), off, 64);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    k = o > k ? o : k;
  }
  return k;
}

// DT < 0: any dtype, one element per load (a.dt); DT = F32 / BF16 / F16:
// the 16-byte form (rows of ld a whole number of chunks, 16-byte aligned,
// segments of a whole number of chunks), U chunk loads in flight per thread;
// the last partial chunk of a row (V not a multiple of E) is read one
// element at a time. Both forms reduce the same keys (the order of the
// comparisons inside a workgroup does not change the maximum key).
template <int DT>
__global__ void __launch_bounds__(256) argmax_rows_kernel(const ArgmaxArgs a) {
  __shared__ unsigned long long s_key[4];
  __shared__ int s_last;
  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  const int m = blockIdx.y, sg = blockIdx.x;
  const int64_t v0 = (int64_t)sg * a.seg;
  const int64_t v1 = v0 + a.seg < a.V ? v0 + a.seg : a.V;
  const int64_t row = (int64_t)m * a.ld;
  float bv = -__builtin_inff();
  int bn = 0x7fffffff;
  if constexpr (DT < 0) {
    for (int64_t v = v0 + th; v < v1; v += 256) {
      const float x = load_as_f32(a.logits, a.dt, row + v);
      if (argmax_better(x, (int)v, bv, bn)) {
        bv = x;
        bn = (int)v;
      }
    }
  } else {
    constexpr int E = vec_elems<DT>(), U = 8;
    const int nfull = (int)((v1 - v0) / E);
    const u32x4 *src = (const u32x4 *)a.logits + (row + v0) / E;
    for (int q0 = th; q0 < nfull; q0 += 256 * U) {
      u32x4 cv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + 256 * u;
        if (q < nfull) cv[u] = src[q];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = q0 + 256 * u;
        if (q >= nfull) break;
        float f[E];
        unpack16<DT>(cv[u], f);
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const int v = (int)(v0 + (int64_t)E * q + e);
          if (argmax_better(f[e], v, bv, bn)) {
            bv = f[e];
            bn = v;
          }
        }
      }
    }
    const int64_t vt = v0 + (int64_t)E * nfull + th;  // the partial chunk
    if (vt < v1) {
      const float x = load_as_f32(a.logits, DT, row + vt);
      if (argmax_better(x, (int)vt, bv, bn)) {
        bv = x;
        bn = (int)vt;
      }
    }
  }
  unsigned long long k = wave_key_max(bn == 0x7fffffff ? 0ull : argmax_key(bv, bn));
  if (lane == 0) s_key[wave] = k;
  __syncthreads();
  k = s_key[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) k = s_key[w] > k ? s_key[w] : k;
  if (a.S == 1) {
    const int64_t tok = argmax_key_index(k);
    if (th == 0) a.tokens[m] = tok;
    if (a.emb16) copy_row16(a, m, tok);
    else copy_row(a, m, tok);
    return;
  }
  if (th == 0) {
    __hip_atomic_store(a.part + (int64_t)m * a.S + sg, k, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    wait_stores();
    s_last = ticket_add(a.ticket + m) == (unsigned)(a.S - 1);
  }
  __syncthreads();
  if (!s_last) return;
  unsigned long long best = 0ull;
  for (int i = th; i < a.S; i += 256) {
    const unsigned long long p =
        __hip_atomic_load(a.part + (int64_t)m * a.S + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    best = p > best ? p : best;
  }
  best = wave_key_max(best);
  __syncthreads();
  if (lane == 0) s_key[wave] = best;
  __syncthreads();
  best = s_key[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) best = s_key[w] > best ? s_key[w] : best;
  const int64_t tok = argmax_key_index(best);
  if (th == 0) {
    a.tokens[m] = tok;
    ticket_reset(a.ticket + m);
  }
  if (a.emb16) copy_row16(a, m, tok);
  else copy_row(a, m, tok);
}

}  // namespace mtp
