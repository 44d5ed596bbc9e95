// Host-side view of the persistent verify GEMM (skv.hpp): arguments and
// instantiation accessor.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace mtp {

constexpr int kSkvBN = 256;      // columns per tile

struct SkvArgs {
  const void *x;        // hidden rows of this chunk: [M, K] compute type, row stride K
  const void *w;        // [N, K] compute type
  const void *bias;     // [N] bias_dt (F32 / BF16 / F16) or null
  int bias_dt;
  int M, N, K;          // M <= 64
  int ntiles, nst;      // column tiles, stages (128 bytes of a W row) per tile
  int tw;               // columns per tile (a multiple of 8, at most kSkvBN)
  unsigned long long *keys;  // [64] packed (value, index) maxima, zero between launches
  unsigned *ticket;          // arrival ticket, zero between launches
  // outputs (already offset to this chunk's rows / batch elements)
  const int32_t *draft;  // [M] (single) or [M / S_seq, D] (multi)
  int8_t *accept;
  int32_t *accepted_n;
  int32_t *corrected;
  int32_t *top;  // [M] or null
  int S_seq, D;
  int multi;     // 1: chain acceptance, 0: single-token verify
  int textbook;  // chain convention (chain_accept): 0 the reference's, 1 textbook
};

typedef void (*SkvKernel)(SkvArgs);
// Kernel for compute type ct and mt row tiles: BF16 / F16 with 1-2 tiles of
// 32 rows, F32 with 1-4 tiles of 16 rows; null otherwise.
// mt: 32-row (16-bit) or 16-row (fp32) x tiles; r8 (fp32, mt 1..3): 8 rows
// after them.
SkvKernel skv_pick(int ct, int mt, bool r8);

}  // namespace mtp
