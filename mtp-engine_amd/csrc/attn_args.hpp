// Launch arguments of the attention kernels (attn.hpp), shared with the
// host code that plans them.
#pragma once

#include <stdint.h>

namespace mtp {

constexpr int kAttnMaxChunks = 64;     // key chunks per (b, h)
constexpr int kAttnBlock = 64;         // keys per block (two wave halves of 32)
constexpr int kAttnRing = 2;           // key blocks in flight per workgroup
constexpr int kAttnTableWindow = 1024; // context keys whose pages sit in LDS at once
constexpr float kAttnRescale = 8.f;    // max gain (natural log) before O is rescaled
constexpr int kAttnMergeQ = 4;         // queries per chunk-merge workgroup

struct AttnArgs {
  const void *q;               // element strides: batch, query, head (d stride 1)
  int64_t q_sb, q_sn, q_sh;
  const void *kp, *vp;         // pages [P, B, H, page_size, D] or null (Lc == 0)
  const int32_t *table;        // [B, ld_tab] physical page of each context key
  int64_t ld_tab;
  int Lc, page_size, npages;
  int64_t p_sp, p_sb, p_sh;    // page element strides: page, batch, head
  const void *kd, *vd;         // dense keys or null (Lt == 0)
  int Lt;
  int64_t d_sb, d_sh, d_st;    // dense element strides: batch, head, key
  const void *mask;            // null, [Lt] or [NQ, Lt]
  int mask_dt, mask_2d;
  void *out;                   // element strides: batch, query, head
  int64_t o_sb, o_sn, o_sh;
  int B, NQ, H;
  float scale;
  int kv_fp8;                  // 1: K / V are fp8 e4m3 (fallback kernel only), 0: q's dtype
  const float *kscale, *vscale;  // per-head K / V scales [H] (fp8 KV) or null
  int nchunks, chunk_blocks;   // blocks of kAttnBlock keys (context, then dense) per chunk
  float *part;                 // [B*H][nchunks][16*ceil(NQ/16)][D]
  float *ml;                   // [B*H][nchunks][16*ceil(NQ/16)][2]
};

typedef void (*AttnKernel)(AttnArgs);
// Defined in attn.hip: the MFMA kernel and the chunk merge for (compute
// type, head dim) or null, and the fallback kernel.
AttnKernel attn_pick(int ct, int d);
AttnKernel attn_merge_pick(int ct, int d);
// The 32-query-tile kernel for 33 .. 64 queries at head dim 128 (attn2.hpp)
// and its dynamic LDS bytes.
AttnKernel attn2_pick(int ct);
int attn2_lds_bytes();
void (*attn_generic())(AttnArgs, int, int);
// Fallback for 256 < D <= kAttnWideMaxD (one workgroup per query), or null.
constexpr int kAttnWideMaxD = 8192;
void (*attn_generic_wide(int d))(AttnArgs, int, int);

}  // namespace mtp
