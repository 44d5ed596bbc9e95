// Cross-workgroup argmax keys and the acceptance chain shared by the verify
// kernels (skv.hpp, vgen.hpp).
//
// Each workgroup folds its columns into one (value, index) maximum per row
// and publishes it as a 64-bit key whose unsigned order is the argmax order
// of torch.argmax (NaN is the maximum, the lowest index wins ties): the high
// word is the order-preserving image of the float bits, the low word the
// complement of the index. An atomic max per row merges the workgroups; the
// last workgroup to arrive decodes the keys, re-zeroes them and runs the
// acceptance of fused_verify / fused_multi_verify (mtp_fused_verify.py:
// 159-166, 184-195).
#pragma once

#include "mtp_common.hpp"

namespace mtp {

// (value, column) -> key; unsigned key order == torch.argmax preference.
// Never 0 for a real column (0 marks "no column seen").
__device__ __forceinline__ unsigned long long argmax_key(float v, int n) {
  uint32_t b = __float_as_uint(v);
  if (v != v) b = 0x7fc00000u;  // every NaN alike: above +inf
  else if (v == 0.f) b = 0u;    // -0 == +0
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - (uint32_t)n);
}
__device__ __forceinline__ int argmax_key_index(unsigned long long k) {
  return (int)(0xffffffffu - (uint32_t)k);
}
__device__ __forceinline__ void key_max(unsigned long long *keys, int m, unsigned long long k) {
  if (k != 0ull) __hip_atomic_fetch_max(keys + m, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Outputs of one verify launch, already offset to the launch's rows (single
// token) or batch elements (chain).
struct VerifyOut {
  const int32_t *draft;  // [M] (single) or [M / S_seq, D] (chain)
  int8_t *accept;        // [M] or [M / S_seq, D]
  int32_t *accepted_n;   // [M / S_seq] (chain)
  int32_t *corrected;    // [M / S_seq] (chain)
  int32_t *top;          // [M] or null
  int S_seq, D;
  int multi;             // 1: chain acceptance, 0: single-token verify
  int textbook;          // chain convention: 0 the reference's, 1 textbook
};

// The acceptance chain of one batch element from its S = D + 1 argmax
// tokens tp[0..D] and drafts dr[0..D-1]; accept is prefix-masked (0 after
// the first rejection).
//   reference (mtp_fused_verify.py:136-154, 184-195): draft d is checked
//     against tp[d + 1] (s = 0 is the anchor); corrected = tp[0];
//   textbook speculative decoding: draft d is checked against tp[d];
//     corrected = tp[accepted_n] (the replacement token, or the bonus token
//     after D accepted drafts).
__device__ __forceinline__ void chain_accept(const int *tp, const int32_t *dr, int D,
                                             int textbook, int8_t *accept, int32_t *accepted_n,
                                             int32_t *corrected) {
  int n = 0;
  for (int d = 0; d < D; ++d) {
    const bool ok = (tp[d + 1 - textbook] == dr[d]) && (n == d);
    accept[d] = (int8_t)ok;
    if (ok) n = d + 1;
  }
  *accepted_n = n;
  *corrected = tp[textbook ? n : 0];
}

// Run by every thread of the last workgroup to arrive (after the acquire):
// decode and re-zero the M row keys, write top and the acceptance outputs.
// s_top / s_draft are LDS arrays of at least 64 ints.
__device__ __forceinline__ void verify_finish(unsigned long long *keys, int M, const VerifyOut &o,
                                              int *s_top, int *s_draft) {
  const int th = threadIdx.x, nth = blockDim.x;
  // the drafts (fewer than the rows) go to LDS with the same round trip as
  // the row keys; read in the acceptance chain, they would be re-read from
  // memory after every accept store (byte stores may alias them)
  const int nd = o.multi ? M / o.S_seq * o.D : M;
  for (int i = th; i < nd; i += nth)
    if (o.draft) s_draft[i] = o.draft[i];
  for (int m = th; m < M; m += nth) {
    const unsigned long long k =
        __hip_atomic_load(keys + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_top[m] = argmax_key_index(k);
    __hip_atomic_store(keys + m, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (o.top)
    for (int m = th; m < M; m += nth) o.top[m] = s_top[m];
  if (!o.multi) {
    for (int m = th; m < M; m += nth) o.accept[m] = (int8_t)(s_top[m] == s_draft[m]);
  } else {
    const int Sq = o.S_seq, Dd = o.D;
    for (int bl = th; bl < M / Sq; bl += nth)
      chain_accept(s_top + bl * Sq, s_draft + bl * Dd, Dd, o.textbook,
                   o.accept + (int64_t)bl * Dd, o.accepted_n + bl, o.corrected + bl);
  }
}

}  // namespace mtp
