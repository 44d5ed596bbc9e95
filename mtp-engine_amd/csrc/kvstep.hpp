// The KV step after verify: the paged-KV write of new tokens, the rollback /
// commit of the engine's verify consumer on device, and the batch prefix
// match of the radix cache.
//
//   paged_kv_write   pages[table[b, p], b, h, p % page_size, :] = new[b, t, h, :],
//                    p = start (+ t), start from the host or a device scalar
//   verify_commit    a_n = min_b accepted_n[b]; reject = any accept == 0;
//                    width = reject ? a_n + 1 : D; tokens[b] = reject ?
//                    draft[b, :a_n] ++ corrected[b] : draft[b]; kv length =
//                    checkpoint + width; optionally the tokens are appended
//                    to an id buffer at a device-held length
//   prefix_match     out[r] = first column where ids[r] differs from ids[0]
//                    (L when none)
//
// All three are small, latency-bound launches: they keep the per-step
// metadata on the device, so the decode loop reads no scalar back to the
// host between steps.
#pragma once

#include "mtp_common.hpp"

namespace mtp {

struct KvWriteArgs {
  const void *k_new, *v_new;  // [B, T, H, D] by element strides (batch, token, head), d contiguous
  int src_dt;
  int64_t s_sb, s_st, s_sh;
  void *k_pages, *v_pages;    // [P, B, H, page_size, D]
  int dst_dt;
  int64_t p_sp, p_sb, p_sh;
  const int32_t *table;       // [B, ld_tab] physical page of each logical position
  int64_t ld_tab;
  const int64_t *start_dev;   // device start position(s) or null
  int start_per_row;          // 1: start_dev[b], 0: start_dev[0]
  int64_t start_host;         // start when start_dev is null
  int B, T, H, D, page_size, npages;
};

// One wave per (b, t, h) row of D elements; 4 rows per workgroup. Positions
// outside the table and pages outside [0, npages) are skipped.
__global__ void __launch_bounds__(256) paged_kv_write_kernel(const KvWriteArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t rid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)a.B * a.T * a.H;
  if (rid >= nrows) return;
  const int h = (int)(rid % a.H);
  const int t = (int)((rid / a.H) % a.T);
  const int b = (int)(rid / ((int64_t)a.H * a.T));
  const int64_t start = a.start_dev ? a.start_dev[a.start_per_row ? b : 0] : a.start_host;
  const int64_t pos = start + t;
  if (pos < 0 || pos >= a.ld_tab) return;
  const int pid = a.table[(int64_t)b * a.ld_tab + pos];
  if (pid < 0 || pid >= a.npages) return;
  const int64_t src = (int64_t)b * a.s_sb + (int64_t)t * a.s_st + (int64_t)h * a.s_sh;
  const int64_t dst = (int64_t)pid * a.p_sp + (int64_t)b * a.p_sb + (int64_t)h * a.p_sh +
                      (int64_t)(pos % a.page_size) * a.D;
  const int eb = dtype_bytes(a.dst_dt);
  if (a.src_dt == a.dst_dt && eb == 2) {
    for (int d = lane; d < a.D; d += 64) {
      ((uint16_t *)a.k_pages)[dst + d] = ((const uint16_t *)a.k_new)[src + d];
      ((uint16_t *)a.v_pages)[dst + d] = ((const uint16_t *)a.v_new)[src + d];
    }
  } else if (a.src_dt == a.dst_dt && eb == 4) {
    for (int d = lane; d < a.D; d += 64) {
      ((uint32_t *)a.k_pages)[dst + d] = ((const uint32_t *)a.k_new)[src + d];
      ((uint32_t *)a.v_pages)[dst + d] = ((const uint32_t *)a.v_new)[src + d];
    }
  } else {
    for (int d = lane; d < a.D; d += 64) {
      store_from_f32(a.k_pages, a.dst_dt, dst + d, load_as_f32(a.k_new, a.src_dt, src + d));
      store_from_f32(a.v_pages, a.dst_dt, dst + d, load_as_f32(a.v_new, a.src_dt, src + d));
    }
  }
}

struct CommitArgs {
  const int8_t *accept;       // [B, D]
  const int32_t *accepted_n;  // [B]
  const int32_t *corrected;   // [B]
  const void *draft;          // [B, D] int32 or int64
  int draft_i64;
  int B, D;
  const int64_t *checkpoint;  // device: KV length before the draft was appended
  int64_t *kv_len;            // device out: checkpoint + width (may alias checkpoint)
  int64_t *tokens;            // [B, D + 1] out: this step's tokens, -1 past the width
  int32_t *width;             // device out: tokens per row this step
  int64_t *ids;               // [B, ld_ids] id buffer (contiguous rows) or null
  int64_t ld_ids;             // its row length: the capacity
  int64_t *ids_len;           // device: valid columns of ids (advanced by width)
};

__device__ __forceinline__ int64_t draft_at(const CommitArgs &a, int64_t i) {
  return a.draft_i64 ? ((const int64_t *)a.draft)[i] : (int64_t)((const int32_t *)a.draft)[i];
}

// One workgroup of 256 threads.
__global__ void __launch_bounds__(256) verify_commit_kernel(const CommitArgs a) {
  __shared__ int s_min[4], s_rej[4];
  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  int mn = 0x7fffffff, rej = 0;
  for (int b = th; b < a.B; b += 256) mn = min(mn, a.accepted_n[b]);
  for (int64_t i = th; i < (int64_t)a.B * a.D; i += 256) rej |= a.accept[i] == 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mn = min(mn, __shfl_xor(mn, off, 64));
    rej |= __shfl_xor(rej, off, 64);
  }
  if (lane == 0) {
    s_min[wave] = mn;
    s_rej[wave] = rej;
  }
  __syncthreads();
  // accepted_n of a consistent verify lies in [0, D]; clamped so that no
  // input can move a read or write outside the draft and token rows
  const int a_n = max(0, min(a.D, min(min(s_min[0], s_min[1]), min(s_min[2], s_min[3]))));
  const bool reject = (s_rej[0] | s_rej[1] | s_rej[2] | s_rej[3]) != 0;
  const int w = reject ? a_n + 1 : a.D;
  const int64_t base = a.ids ? max((int64_t)0, a.ids_len[0]) : 0;
  const int64_t ck = a.checkpoint[0];
  const int W1 = a.D + 1;
  for (int64_t i = th; i < (int64_t)a.B * W1; i += 256) {
    const int b = (int)(i / W1), j = (int)(i % W1);
    int64_t tok = -1;
    if (j < w) {
      tok = (reject && j == a_n) || j >= a.D ? (int64_t)a.corrected[b]
                                             : draft_at(a, (int64_t)b * a.D + j);
    }
    a.tokens[i] = tok;
    if (a.ids && j < w && base + j < a.ld_ids) a.ids[(int64_t)b * a.ld_ids + base + j] = tok;
  }
  __syncthreads();  // every read of the scalars happens before they are written
  if (th == 0) {
    a.kv_len[0] = ck + w;
    a.width[0] = w;
    // ids_len advances by the tokens that fit and never passes ld_ids: a
    // full buffer drops the rest, which the caller sees as an advance
    // shorter than width
    if (a.ids) a.ids_len[0] = base + min((int64_t)w, max((int64_t)0, a.ld_ids - base));
  }
}

// One wave per row; out[r] = first column c < L with ids[r, c] != ids[0, c], or L.
__global__ void __launch_bounds__(256)
prefix_match_kernel(const int64_t *ids, int64_t ld, int R, int L, int32_t *out) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  int first = L;
  for (int c0 = 0; c0 < L; c0 += 64) {
    const int c = c0 + lane;
    const bool diff = c < L && ids[(int64_t)r * ld + c] != ids[c];
    const unsigned long long m = __ballot(diff);
    if (m) {
      first = c0 + __builtin_ctzll(m);
      break;
    }
  }
  if (lane == 0) out[r] = first;
}

}  // namespace mtp
