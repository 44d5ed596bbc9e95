// Generic verify: the lm_head pass of fused_verify / fused_multi_verify for
// what the streaming kernels do not take — any K, any element alignment,
// hidden and weight of different float dtypes (the reference upcasts both
// to fp32, mtp_fused_verify.py:163, 180-182), and an optional bias of any
// float dtype.
//
//   top[m] = argmax_n (fp32(x[m]) . fp32(W[n]) + fp32(bias[n]))
//
// One thread per vocabulary column (256 per workgroup, grid-strided over
// the columns); the k loop goes in chunks of 32 whose hidden values for all
// rows are staged in LDS as fp32, so every thread's weight row is read once
// and every hidden value once per workgroup and chunk. fp32 FMA on the VALU
// (exact products of the upcast operands, fp32 accumulation). Each thread
// keeps a running (max, index) per row; the workgroup folds them with wave
// shuffles and LDS into one 64-bit key per row (verify_tail.hpp), merged
// across workgroups by atomic max; the last workgroup runs the acceptance.
#pragma once

#include "verify_tail.hpp"

namespace mtp {

struct VgenArgs {
  const void *x;     // hidden rows of this launch [M, K], row stride K
  int xdt;
  const void *w;     // [N, K]
  int wdt;
  const void *bias;  // [N] or null
  int bdt;
  int M, N, K;       // M <= 64
  unsigned long long *keys;  // [64], zero between launches
  unsigned *ticket;          // zero between launches
  VerifyOut out;
};

constexpr int kVgenThreads = 256;
constexpr int kVgenKC = 32;  // k per LDS chunk

template <int MR>
__global__ void __launch_bounds__(kVgenThreads)
verify_generic_kernel(const VgenArgs a) {
  __shared__ float xs[MR][kVgenKC + 1];
  __shared__ unsigned long long s_key[kVgenThreads / kWave][MR];
  __shared__ int s_flag;
  __shared__ int s_top[64];
  __shared__ int s_draft[64];
  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  const int M = a.M, N = a.N, K = a.K;

  float best_v[MR];
  int best_n[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    best_v[r] = -__builtin_inff();
    best_n[r] = 0x7fffffff;
  }
  for (int64_t c0 = (int64_t)blockIdx.x * kVgenThreads; c0 < N;
       c0 += (int64_t)gridDim.x * kVgenThreads) {
    const int64_t col = c0 + th;
    const bool live = col < N;
    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.f;
    for (int k0 = 0; k0 < K; k0 += kVgenKC) {
      __syncthreads();
      for (int i = th; i < MR * kVgenKC; i += kVgenThreads) {
        const int r = i / kVgenKC, kk = i % kVgenKC;
        xs[r][kk] = (r < M && k0 + kk < K) ? load_as_f32(a.x, a.xdt, (int64_t)r * K + k0 + kk)
                                            : 0.f;
      }
      __syncthreads();
      if (live) {
        const int kn = K - k0 < kVgenKC ? K - k0 : kVgenKC;
        for (int kk = 0; kk < kn; ++kk) {
          const float wv = load_as_f32(a.w, a.wdt, col * K + k0 + kk);
#pragma unroll
          for (int r = 0; r < MR; ++r) acc[r] = __builtin_fmaf(xs[r][kk], wv, acc[r]);
        }
      }
    }
    if (live) {
      const float bv = a.bias ? load_as_f32(a.bias, a.bdt, col) : 0.f;
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        const float v = acc[r] + bv;
        if (r < M && argmax_better(v, (int)col, best_v[r], best_n[r])) {
          best_v[r] = v;
          best_n[r] = (int)col;
        }
      }
    }
  }
  // per row: the wave's maximum key by shuffles, then the waves' in LDS
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    unsigned long long k = best_n[r] == 0x7fffffff ? 0ull : argmax_key(best_v[r], best_n[r]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint32_t lo = __shfl_xor((uint32_t)k, off, 64);
      const uint32_t hi = __shfl_xor((uint32_t)(k >> 32), off, 64);
      const unsigned long long o = ((unsigned long long)hi << 32) | lo;
      k = o > k ? o : k;
    }
    if (lane == 0) s_key[wave][r] = k;
  }
  __syncthreads();
  if (th < M) {
    unsigned long long k = s_key[0][th];
#pragma unroll
    for (int w = 1; w < kVgenThreads / kWave; ++w) k = s_key[w][th] > k ? s_key[w][th] : k;
    key_max(a.keys, th, k);
  }
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = ticket_add(a.ticket) == (unsigned)(gridDim.x - 1);
  __syncthreads();
  if (!s_flag) return;
  verify_finish(a.keys, M, a.out, s_top, s_draft);
  if (th == 0) ticket_reset(a.ticket);
}

typedef void (*VgenKernel)(VgenArgs);
// Kernel for up to `rows` rows (<= 64), or null.
VgenKernel vgen_pick(int rows);

}  // namespace mtp
