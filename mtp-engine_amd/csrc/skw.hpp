// Wave-specialised skinny GEMM for gfx950: the RMSNorm -> linear product of
// sk.hpp (at most 64 rows of 16-bit x, fp8-e4m3 or 16-bit W, tw <= 64
// output columns per workgroup over all of K, on a 64-wide MFMA tile whose
// rows past tw read zeros; the host picks tw to put one workgroup on every
// CU), after sk.hpp's prep
// launch (xg = x * gamma rounded to the type of x, written as MFMA B-operand
// blocks, and each row's sums of squares per K-slice):
//
//   y[m, n] = (rs[m] (xg[m, :] . W[n, :]) * wscale[n] + bias[n]), times scale
//   rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) (norm) or 1.
//
// Workgroup = 8 waves, two per SIMD, and one LDS ring of RW stages (a stage
// is 128 bytes of every W row and the xg blocks of the same k):
//  * waves 0-3 (compute) copy W into the ring with buffer loads that write
//    LDS directly (each wave 2 x 1 KB = 16 rows of a stage, RW - 1 stages
//    ahead) and run the MFMAs of their k-steps of a stage from LDS (A from
//    W, fp8 upcast exactly in registers; B from the xg blocks);
//  * waves 4-7 (x) copy the stage's xg blocks (1 KB each, contiguous) into
//    the same ring slot the same way.
// Each wave's loads complete in order (one vmcnt counter per wave), and a
// wave waits only for its own stream: W from HBM on the compute waves, xg
// from L2 on the x waves. Issued from the same waves, a wait for the L2
// stream would also wait for the HBM loads issued before it (the two-
// launch form, sk.hpp, interleaves them on every wave). One barrier per
// stage: in stage s the compute waves read slot s % RW while the copies of
// stage s + RW - 1 go to the slot stage s - 1 used.
//
// Layouts: W row r's 16-byte chunk c at position c ^ sk_swz(r) of its 128
// bytes in a slot (the copy of rows 8 c' .. 8 c' + 7 is one 1 KB
// instruction whose lane l fetches chunk (l % 8) ^ sk_swz(row)); the xg
// blocks as the prep writes them (block (32-row tile t, k-step j) = 1 KB,
// lane 32 g + row % 32 of lane group g). The k-slot order within a stage is
// sk_chunk_slot's, the same for W and xg. Stages start at 7 tile mod
// (stages), which spreads the HBM requests of workgroups in step over the
// channels.
#pragma once

#include "sk.hpp"
#include "skw_args.hpp"

namespace mtp {

constexpr int kSkwRW = 4;  // ring stages (4 measured faster than 5 and 6)

template <int CT, int WT, int MT>
__global__ void __launch_bounds__(512, 1)
skw_kernel(const SkwArgs a) {
  constexpr bool FP8 = WT == MTP_FP8E4M3;
  constexpr int UK = FP8 ? 128 : 64;      // k per stage
  constexpr int KS = UK / 16;             // MFMA k-steps per stage
  constexpr int KPW = KS / 4;             // k-steps per compute wave per stage
  constexpr int RW = kSkwRW;
  constexpr int WSB = kSkBN * kSkUB;      // W bytes of a stage (8 KB)
  constexpr int XSB = MT * KS * 1024;     // xg bytes of a stage
  constexpr int SLOT = WSB + XSB;
  constexpr int NWD = WSB / 1024 / 4;     // W copies per compute wave per stage
  constexpr int NXD = XSB / 1024 / 4;     // xg copies per x wave per stage
  constexpr int RING = RW * SLOT;
  constexpr int RED = 4 * 2 * MT * 64 * 64;  // end: the compute waves' partial tiles
  constexpr int PSSOFF = RING > RED ? RING : RED;         // prep row sums [16][64]
  constexpr int RSOFF = PSSOFF + kSkPrepMaxSlices * 256;  // row scales [64]
  static_assert((RW - 2) * NWD < 64 && (RW - 2) * NXD < 64, "vmcnt is 6 bits");
  // One LDS object: with several, the compiler tracks the LDS copies per
  // object and makes each LDS read of the ring wait for every copy in flight
  // (vmcnt 0), which serialises the ring.
  __shared__ __attribute__((aligned(1024))) unsigned char lds[RSOFF + 256];
  float *s_pss = (float *)(lds + PSSOFF);
  float *s_rs = (float *)(lds + RSOFF);

  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  const int N = a.N, K = a.K, nst = a.nst;
  // tw <= 64 output columns per workgroup; the MFMA tile stays 64 wide
  // (rows past the workgroup's columns read zeros and are not stored)
  const int tw = a.tw;
  const int tile = (int)blockIdx.x, n0 = tile * tw;
  const int nend = min(N, n0 + tw);
  const int rot = (7 * tile) % nst;
  auto k_stage = [&](int s) {
    const int r = s + rot;
    return r < nst ? r : r - nst;
  };

  // compute wave w's partial sums; in the end phase it owns output tile
  // (u, t) = (w % 2, w / 2) when t < MT
  const int ag = lane >> 5;
  const int ou = wave & 1, ot = (wave >> 1) & 1;
  const bool owner = wave < 4 && ot < MT;
  f32x16 acc[2][MT];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[u][t][e] = 0.f;
  float cws[16], cbi[16];

  if (wave < 4) {
    load_col_factors<4>(a.wscale, a.bias, a.bias_dt, N, n0 + 32 * ou + 4 * ag, 8, cws, cbi);
    const uint32_t ldw = (uint32_t)K * (FP8 ? 1u : 2u);
    const int nrows = nend - n0;  // rows past the workgroup's columns read zeros
    const __amdgpu_buffer_rsrc_t wrs =
        make_rsrc((const unsigned char *)a.w + (int64_t)n0 * ldw, (uint32_t)nrows * ldw);
    const __amdgpu_buffer_rsrc_t nrs = make_rsrc(a.w, 0u);
    uint32_t wvo[NWD];
#pragma unroll
    for (int v = 0; v < NWD; ++v) {
      const int row = 8 * (wave + 4 * v) + (lane >> 3);
      wvo[v] = (uint32_t)row * ldw + 16u * (uint32_t)((lane & 7) ^ sk_swz(row));
    }
    // Copies of stage s into ring slot `slot`. Stages past the last copy
    // through a descriptor of zero bytes (zeros into a slot that is never
    // computed on), so a stage always counts NWD instructions.
    auto issue = [&](int s, int slot) __attribute__((always_inline)) {
      const bool live = s < nst;
      const int soff = live ? k_stage(s) * kSkUB : 0;
#pragma unroll
      for (int v = 0; v < NWD; ++v)
        sk_lds_copy16<2>(live ? wrs : nrs, lds + slot * SLOT + (wave + 4 * v) * 1024, wvo[v],
                         soff);
    };
    auto compute = [&](int slot) __attribute__((always_inline)) {
      const unsigned char *wb = lds + slot * SLOT;
      const unsigned char *xb = wb + WSB;
      // fp8: the wave's two k-steps share one 16-byte chunk of each A row
      // (bytes 0-7: k-step 2 w, 8-15: 2 w + 1)
      u32x4 w8[2];
      if constexpr (FP8) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int row = 32 * u + (lane & 31);
          const int c = 2 * wave + ag;
          w8[u] = *(const u32x4 *)(wb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
        }
      }
#pragma unroll
      for (int jj = 0; jj < KPW; ++jj) {
        const int j = wave * KPW + jj;
        u32x4 bv[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) bv[t] = *(const u32x4 *)(xb + (t * KS + j) * 1024 + lane * 16);
        u32x4 av[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          if constexpr (FP8) {
            av[u][0] = fp8x2_to_ct<CT, false>(w8[u][2 * jj]);
            av[u][1] = fp8x2_to_ct<CT, true>(w8[u][2 * jj]);
            av[u][2] = fp8x2_to_ct<CT, false>(w8[u][2 * jj + 1]);
            av[u][3] = fp8x2_to_ct<CT, true>(w8[u][2 * jj + 1]);
          } else {
            const int row = 32 * u + (lane & 31);
            const int c = 2 * j + ag;
            av[u] = *(const u32x4 *)(wb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
          }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int u = 0; u < 2; ++u) acc[u][t] = mfma32<CT>(av[u], bv[t], acc[u][t]);
      }
    };
    for (int s = 0; s < RW - 1; ++s) issue(s, s);
    // stage 0 landed (stages 1 .. RW - 2 may be in flight)
    wait_vmcnt_barrier<(RW - 2) * NWD>();
    int slot = 0, fslot = RW - 1;  // slot of stage s; slot the copies of s + RW - 1 go to
    for (int s = 0; s < nst; ++s) {
      issue(s + RW - 1, fslot);
      compute(slot);
      slot = slot + 1 == RW ? 0 : slot + 1;
      fslot = fslot + 1 == RW ? 0 : fslot + 1;
      wait_vmcnt_barrier<(RW - 2) * NWD>();  // stage s + 1 landed, slot s free
    }
  } else {
    const int xw = wave - 4;
    // the prep's row sums, one 256-byte slice per copy (x wave w: slices
    // w, w + 4, ...), landed with this wave's first xg copies
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.pss, (uint32_t)a.nsl * 256u);
#pragma unroll
    for (int i = 0; i < kSkPrepMaxSlices / 4; ++i) {
      const int sl = xw + 4 * i;
      sk_lds_copy4(srs, (unsigned char *)(s_pss + 64 * sl),
                   sl < a.nsl ? (uint32_t)(sl * 64 + lane) * 4u : kOOB);
    }
    // xg copy i of a stage: block c = xw NXD + i = (tile t, k-step j)
    const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.xf, (uint32_t)(MT * nst * KS) * 1024u);
    const __amdgpu_buffer_rsrc_t nrs = make_rsrc(a.xf, 0u);
    auto issue = [&](int s, int slot) __attribute__((always_inline)) {
      const bool live = s < nst;
      const int sr = live ? k_stage(s) : 0;
#pragma unroll
      for (int i = 0; i < NXD; ++i) {
        const int c = xw * NXD + i, t = c / KS, j = c % KS;
        sk_lds_copy16<0>(live ? xrs : nrs, lds + slot * SLOT + WSB + c * 1024,
                         (uint32_t)(((t * nst + sr) * KS + j) * 1024 + lane * 16), 0);
      }
    };
    for (int s = 0; s < RW - 1; ++s) issue(s, s);
    wait_vmcnt_barrier<(RW - 2) * NXD>();
    int fslot = RW - 1;
    for (int s = 0; s < nst; ++s) {
      issue(s + RW - 1, fslot);
      fslot = fslot + 1 == RW ? 0 : fslot + 1;
      wait_vmcnt_barrier<(RW - 2) * NXD>();
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // copies past the last stage
  __syncthreads();

  // ---- end phase: the compute waves' partial tiles meet in LDS
  // ([wave][u][t][quad][lane] of f32x4: 16 lanes touch 256 contiguous
  // bytes); x-wave threads take the row scales from the prep's slices, in
  // slice order
  f32x4 *red = (f32x4 *)lds;
  if (wave < 4) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          red[(((wave * 2 + u) * MT + t) * 4 + g4) * 64 + lane] =
              f32x4{acc[u][t][4 * g4], acc[u][t][4 * g4 + 1], acc[u][t][4 * g4 + 2],
                    acc[u][t][4 * g4 + 3]};
  } else if (th - 256 < 32 * MT) {
    const int r = th - 256;
    float ss = 0.f;
    for (int sl = 0; sl < a.nsl; ++sl) ss += s_pss[64 * sl + r];
    s_rs[r] = a.norm ? 1.0f / sqrtf(ss / (float)K + a.eps) : 1.0f;
  }
  __syncthreads();
  if (!owner) return;
  f32x16 v;
#pragma unroll
  for (int e = 0; e < 16; ++e) v[e] = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 p = red[(((q * 2 + ou) * MT + ot) * 4 + g4) * 64 + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[4 * g4 + e] += p[e];
    }
  // lane's outputs: v[e] = D[n][m], m = 32 ot + lane % 32,
  // n = n0 + 32 ou + 8 (e / 4) + 4 (lane / 32) + e % 4
  const int m = 32 * ot + (lane & 31);
  if (m >= a.M) return;
  v *= s_rs[m];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int n = n0 + 32 * ou + 8 * g + 4 * ag;
    if (n >= nend) continue;
    float o[4];
#pragma unroll
    for (int jx = 0; jx < 4; ++jx)
      o[jx] = (a.bias ? v[4 * g + jx] * cws[4 * g + jx] + cbi[4 * g + jx]
                      : v[4 * g + jx] * cws[4 * g + jx]) * a.scale;
    const int64_t yb = (int64_t)m * N + n;
    if (n + 3 < nend && (N & 3) == 0) {
      uint2 pk;
      pk.x = pack2<CT>(o[0], o[1]);
      pk.y = pack2<CT>(o[2], o[3]);
      *(uint2 *)((uint16_t *)a.y + yb) = pk;
    } else {
      for (int jx = 0; jx < 4; ++jx)
        if (n + jx < nend) store_from_f32(a.y, CT, yb + jx, o[jx]);
    }
  }
}

}  // namespace mtp
