// x-resident skinny RMSNorm -> linear for gfx950: at most 64 rows of 16-bit
// x (bf16 / f16), W of fp8-e4m3 or the same 16-bit type, one launch.
//
//   y[m, n] = (rs[m] * sum_k xg[m, k] W[n, k]) * wscale[n] + bias[n], times scale
//   xg[m, k] = x[m, k] * gamma[k] rounded to the type of x,
//   rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) (norm) or 1
//
// What bounds this shape is HBM (W is read once) and, right behind it, the
// x bytes every workgroup needs for its columns: read through L2 once per
// step they cost as much as W. Here a workgroup copies its rows' x for its
// K-range into LDS once, at the start (at most 128 KB: all of K for <= 16
// rows, half of it for <= 32, a quarter for <= 64; the planner splits K
// that way and narrows the column tile so the grid still covers the CUs),
// and after that streams only W.
//
// Workgroup = 4 waves (one per SIMD) and a tile of 64 TA columns, of which
// the first tw are the workgroup's (the host narrows the tile by at most a
// quarter to put one workgroup on every CU; rows past tw read zeros); wave w
// owns A tiles (16 columns each) w TA .. w TA + TA - 1 against all rows,
// over every k of the split, so the waves never wait for each other in the
// main loop. A step is 128 bytes of every W row (128 k for fp8, 64 for
// 16-bit W):
//   * W comes HBM -> registers with 8-rows x 128-byte non-temporal loads
//     (the fastest pattern for this row layout; the MFMA operand layout's
//     16-rows x 64-byte loads stream 1.5x slower), NS - 1 steps ahead;
//   * per A tile, its 16 rows go to the wave's own 2 KB of LDS (16-byte
//     chunk c of row r at c ^ ((r / 2) % 8): both the stores and the
//     operand reads are bank-conflict free) and come back as the A operands
//     of v_mfma_f32_16x16x32; LDS executes a wave's accesses in order, so
//     the slot is reused without a barrier; fp8 is upcast exactly in
//     registers;
//   * the B operands (x) are read from the resident blocks.
// k-slot order: in a step, lane group g = lane / 16 of an operand covers
// k 8 KS g .. 8 KS g + 8 KS - 1, 8 of them per MFMA sub-step s (KS = 4 for
// fp8, 2 for 16-bit W): the A rows' chunks 2 g, 2 g + 1 (fp8: bytes 0-7 of
// a chunk in sub-step 2 i, 8-15 in 2 i + 1), the x blocks in the same order.
// Steps of a split start at 7 b mod (steps), b the workgroup: workgroups in
// step with each other then read different offsets of their rows, which
// spreads the requests over the HBM channels.
// End: the sums of squares of a row meet in LDS in a fixed order; one
// split applies the epilogue directly, otherwise every workgroup of a tile
// publishes its fp32 tile and sums of squares (coherent stores, arrival
// ticket; see the hand-off notes in mtp_common.hpp) and the last to arrive
// adds them up in split order.
#pragma once

#include "sk.hpp"
#include "skp_args.hpp"

namespace mtp {

__device__ __forceinline__ int skp_swz(int r) { return (r >> 1) & 7; }
// Position of 16-byte chunk c of row m (0..15) in an x block is
// c ^ skp_xswz(m): the B-operand reads of the 16 rows of one chunk then hit
// 16 distinct bank groups (KS 4: 256-byte rows, KS 2: 128-byte rows, two
// rows per 256 bytes).
template <int KS>
__device__ __forceinline__ int skp_xswz(int m) {
  if constexpr (KS == 4) return m & 15;
  else return (m >> 1) & 7;
}

template <int CT, int WT, int MT, int TA, bool GAM, bool H8>
__global__ void __launch_bounds__(64 * kSkpWaves, 1)
skp_kernel(const SkpArgs a) {
  constexpr bool FP8 = WT == MTP_FP8E4M3;
  constexpr int KS = FP8 ? 4 : 2;       // 32-k MFMA sub-steps per step
  constexpr int UK = 32 * KS;           // k per step
  constexpr int NWL = 2 * TA;           // W loads (8 rows x 128 B) per wave per step
  // register ring depth in steps (even: the pipeline alternates two
  // register sets by step parity); NS - 2 steps of W are in flight ahead of
  // the staged step: 48-64 KB per CU (one A tile: 8 steps measured faster
  // than 12: fp8 8 x 4096 x 4096 8.7 against 9.4 us, bf16 16 x 4096 x 4096
  // 10.7 against 11.1; 6 ties 8, 4 loses)
  constexpr int NS = TA == 1 ? 8 : TA == 2 ? 6 : 4;
  static_assert(NS % 2 == 0, "step parity selects the register set");
  constexpr int RB = 2 * UK;            // x bytes of a row per step
  constexpr int RPI = 1024 / RB;        // rows per 1 KB copy instruction
  constexpr int LPR = RB / 16;          // lanes per row in a copy
  // parts of 1 KB kept per x block: all KS, or (H8: at most 8 rows, one
  // 16-row tile) only the ones holding rows 0 .. 7; the B operands of rows
  // 8 .. 15 then read rows 0 .. 7 again (their outputs are never stored)
  constexpr int XP = H8 ? 8 / RPI : KS;
  constexpr int XB = XP * 1024;         // bytes of one x block
  static_assert(!H8 || MT == 1, "compact blocks hold one tile");
  constexpr int NSTMAX = kSkpXMaxBytes / (MT * XB);  // steps per split at most
  // x copy instructions of a wave: its steps (all for KS 4, every other one
  // for KS 2) times the tiles
  constexpr int NCJ = (NSTMAX + kSkpWaves / XP - 1) / (kSkpWaves / XP);
  static_assert((NS - 1) * NWL + NCJ * MT + kSkpGammaLoads < 64, "vmcnt is 6 bits");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  __shared__ float s_ss[kSkpWaves][64];
  __shared__ float s_rs[64];
  __shared__ int s_flag;

  const int th = threadIdx.x, lane = th & 63;
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
  const int N = a.N, K = a.K;
  const int b = blockIdx.x;
  int tile, sp;
  split_tile_of(b, a.G, a.S, a.xg != 0, tile, sp);
  // tw <= 64 TA output columns; the tile's rows past them read zeros and are
  // not stored
  const int n0 = tile * a.tw;
  const int nend = min(N, n0 + a.tw);
  const int st0 = sp * a.kb_per;
  const int nst = min(a.nkb, st0 + a.kb_per) - st0;  // steps of this split (>= 1)
  const int rot = (7 * b) % nst;
  auto rotated = [&](int q) __attribute__((always_inline)) {
    return q + rot < nst ? q + rot : q + rot - nst;
  };
  unsigned char *const lx = lds;  // x block (step qa, tile t, sub-step s): 1 KB
  unsigned char *const lw = lds + (size_t)MT * XB * a.kb_per + wave * 2048;
  unsigned char *const lg = lds + (size_t)MT * XB * a.kb_per + kSkpStaging;  // gamma

  // epilogue factors of the lane's columns n0 + 16 (w TA + i) + 4 (lane / 16) + e
  float cws[4 * TA], cbi[4 * TA];
  load_col_factors<TA>(a.wscale, a.bias, a.bias_dt, N, n0 + 16 * TA * wave + 4 * (lane >> 4), 16,
                       cws, cbi);

  // ---- the split's gamma and x go HBM/L2 -> LDS by buffer loads with the
  // LDS bit (no registers), then the W ring's prologue, so one wait covers
  // the copies while W keeps streaming. x block (step qa, tile t) holds the
  // tile's 16 rows x RB bytes of the step, row m at m RB, its 16-byte chunk c
  // at position c ^ skp_xswz(m); one copy instruction fills 1 KB of it (part
  // h = 0 .. KS - 1): RPI whole rows, lane l the position l % LPR of row
  // RPI h + l / LPR, so each instruction reads RPI contiguous RB-byte row
  // segments. Wave w copies part h = w % KS of the blocks of its steps (all
  // steps for KS 4, every other one for KS 2), starting at the workgroup's
  // rotated step, which spreads the copies of the grid over the L2 channels.
  // Parts whose rows are all >= M are not copied: those rows of the block
  // keep stale LDS bytes, which reach only outputs of rows >= M (never
  // stored).
  const int kr = nst * UK;  // k of this split
  if constexpr (GAM) {
    const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.gamma + st0 * UK, (uint32_t)kr * 4u);
#pragma unroll
    for (int j = 0; j < kSkpGammaLoads; ++j) {
      // 1 KB piece c of the split's gamma; its offset goes in the range-checked
      // vector offset, so the floats past the split read 0
      const int c = wave + kSkpWaves * j;
      if (c * 256 < kr) sk_lds_copy16<0>(grs, lg + 1024 * c, 1024u * c + 16u * lane, 0);
    }
  }
  const uint32_t ldx = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)a.M * ldx);
  const int xh = wave % XP;                       // part of every block this wave copies
  const int xq0 = wave / XP, xqs = kSkpWaves / XP;  // its steps: xq0 + xqs j
  const int cm = RPI * xh + lane / LPR;           // copy: row within the tile
  const int cp = lane % LPR;                      // ... its chunk position
  const uint32_t xvo = (uint32_t)cm * ldx + 16u * (uint32_t)(cp ^ skp_xswz<KS>(cm));
#pragma unroll
  for (int j = 0; j < NCJ; ++j) {
    const int jq = xq0 + xqs * j;
    if (jq >= nst) break;
    const int qa = rotated(jq);
#pragma unroll
    for (int t = 0; t < MT; ++t)
      if (16 * t + RPI * xh < a.M)
        sk_lds_copy16<0>(xrs, lx + (qa * MT + t) * XB + xh * 1024,
                         xvo + (uint32_t)(16 * t) * ldx, (st0 + qa) * RB);
  }

  const uint32_t ldw = (uint32_t)K * (FP8 ? 1u : 2u);
  const int nrows = nend - n0;
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc((const unsigned char *)a.w + (int64_t)n0 * ldw, (uint32_t)nrows * ldw);
  // W load v = 2 i + h of a step: rows 16 (w TA + i) + 8 h + lane / 8 of the
  // tile, bytes 16 (lane % 8) .. + 15 of the step
  uint32_t wvo[NWL];
#pragma unroll
  for (int v = 0; v < NWL; ++v) {
    const int row = 16 * (TA * wave + (v >> 1)) + 8 * (v & 1) + (lane >> 3);
    wvo[v] = (uint32_t)row * ldw + (uint32_t)st0 * (uint32_t)kSkpStageBytes + 16u * (lane & 7);
  }
  u32x4 wr[NS][NWL];
  // loads of step position q into ring slot `slot`; positions past the
  // split use an out-of-range vector offset (zeros, no memory access)
  auto issue = [&](int q, auto slotc) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
    const bool live = q < nst;
    const uint32_t soff = live ? (uint32_t)rotated(q) * (uint32_t)kSkpStageBytes : 0u;
#pragma unroll
    for (int v = 0; v < NWL; ++v)
      wr[slot][v] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, live ? wvo[v] : kOOB, soff, 2));
  };
  static_for<0, NS - 1>([&](auto pc) { issue(decltype(pc)::value, pc); });

  // copies landed (every wave's: gamma is shared). In place, per step
  // position: the row squares of x (kept per wave in registers until the
  // end) and xg = x * gamma rounded to the type of x. Positions 0 .. NS - 1
  // are done here, wave w taking w, w + 4, ...; the positions of each later
  // group of NS are done during the previous group's main-loop steps (one
  // wave per step), and a barrier closes every group, so most of this work
  // overlaps the W stream.
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 1) * NWL) : "memory");
  __syncthreads();
  float ss[MT][XP];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int h = 0; h < XP; ++h) ss[t][h] = 0.f;
  // lane's chunk in part h: row RPI h + lane / LPR, position lane % LPR
  int pc[XP];
#pragma unroll
  for (int h = 0; h < XP; ++h) pc[h] = (lane % LPR) ^ skp_xswz<KS>(RPI * h + lane / LPR);
  // one step position's blocks, all parts: reads first, then the writes
  auto inplace = [&](int q) __attribute__((always_inline)) {
    const int qa = rotated(q);
    u32x4 v[MT][XP];
    f32x4 g[XP][2];
#pragma unroll
    for (int h = 0; h < XP; ++h) {
      if constexpr (GAM) {
        const unsigned char *gp = lg + 4 * (qa * UK + 8 * pc[h]);
        g[h][0] = *(const f32x4 *)gp;
        g[h][1] = *(const f32x4 *)(gp + 16);
      }
#pragma unroll
      for (int t = 0; t < MT; ++t)
        if (16 * t + RPI * h < a.M)
          v[t][h] = *(const u32x4 *)(lx + (qa * MT + t) * XB + h * 1024 + lane * 16);
    }
#pragma unroll
    for (int h = 0; h < XP; ++h)
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        if (16 * t + RPI * h >= a.M) continue;
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f32x2 f = unpack2<CT>(v[t][h][e]);
          ss[t][h] = __builtin_fmaf(f[0], f[0], ss[t][h]);
          ss[t][h] = __builtin_fmaf(f[1], f[1], ss[t][h]);
          if constexpr (GAM) {
            const f32x4 &gg = g[h][e >> 1];
            o[e] = pack2<CT>(f[0] * gg[2 * (e & 1)], f[1] * gg[2 * (e & 1) + 1]);
          }
        }
        if constexpr (GAM)
          *(u32x4 *)(lx + (qa * MT + t) * XB + h * 1024 + lane * 16) = o;
      }
  };
#pragma unroll
  for (int j = 0; j < NS / kSkpWaves + 1; ++j) {
    const int q = wave + kSkpWaves * j;
    if (q < NS && q < nst) inplace(q);
  }
  __syncthreads();  // positions 0 .. NS - 1 ready

  // ---- main loop
  f32x4 acc[TA][MT];
#pragma unroll
  for (int i = 0; i < TA; ++i)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // staging addresses: store of load h (row 8 h + lane / 8, chunk lane % 8);
  // operand read of row lane % 16, chunks 2 g and 2 g + 1
  const int sr0 = lane >> 3, sr1 = 8 + (lane >> 3);
  const uint32_t st_a0 = sr0 * 128 + 16 * ((lane & 7) ^ skp_swz(sr0));
  const uint32_t st_a1 = sr1 * 128 + 16 * ((lane & 7) ^ skp_swz(sr1));
  const int ar = lane & 15, agp = lane >> 4;
  const uint32_t rd_a0 = ar * 128 + 16 * ((2 * agp) ^ skp_swz(ar));
  const uint32_t rd_a1 = ar * 128 + 16 * ((2 * agp + 1) ^ skp_swz(ar));
  // B operand of sub-step s: row ar, chunk KS agp + s of the x block
  uint32_t xrd[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int xr = H8 ? (ar & 7) : ar;
    xrd[s] = xr * RB + 16 * ((KS * agp + s) ^ skp_xswz<KS>(xr));
  }

  // Software pipeline, one step deep: step q stages step q + 1's W through
  // LDS and reads back its A operands and x fragments into registers, then
  // runs step q's conversions and MFMAs from the registers staged one step
  // earlier, so the LDS round trip of a step overlaps the previous step's
  // math. Ring: positions q + 1 .. q + NS - 1 in flight during step q.
  u32x4 ac[TA][2], an[TA][2];  // raw A operands (two 16-byte chunks per tile)
  u32x4 xc[MT][KS], xn[MT][KS];
  auto stage = [&](auto slotc, int q, u32x4 (&ao)[TA][2], u32x4 (&xo)[MT][KS])
      __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
    const int qa = rotated(q < nst ? q : 0);
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int s = 0; s < KS; ++s)
        xo[t][s] = *(const u32x4 *)(lx + (qa * MT + t) * XB + xrd[s]);
#pragma unroll
    for (int i = 0; i < TA; ++i) {
      *(u32x4 *)(lw + st_a0) = wr[slot][2 * i];
      *(u32x4 *)(lw + st_a1) = wr[slot][2 * i + 1];
      ao[i][0] = *(const u32x4 *)(lw + rd_a0);
      ao[i][1] = *(const u32x4 *)(lw + rd_a1);
    }
  };
  auto math = [&](const u32x4 (&a_)[TA][2], const u32x4 (&x_)[MT][KS])
      __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TA; ++i) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        u32x4 av;
        if constexpr (FP8) {
          const u32x4 &c = a_[i][s >> 1];
          const int h = (s & 1) * 2;
          av[0] = fp8x2_to_ct<CT, false>(c[h]);
          av[1] = fp8x2_to_ct<CT, true>(c[h]);
          av[2] = fp8x2_to_ct<CT, false>(c[h + 1]);
          av[3] = fp8x2_to_ct<CT, true>(c[h + 1]);
        } else {
          av = a_[i][s];
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[i][t] = mfma16<CT>(av, x_[t][s], acc[i][t]);
      }
    }
  };
  // step 0's W arrived: stage it
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * NWL) : "memory");
  stage(std::integral_constant<int, 0>{}, 0, ac, xc);
  auto step = [&](auto rc, int q, bool full) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::value;  // q % NS
    __builtin_amdgcn_sched_barrier(0);
    issue(q + NS - 1, std::integral_constant<int, (r + NS - 1) % NS>{});
    __builtin_amdgcn_sched_barrier(0);
    // step q + 1's W (the oldest NWL loads of the ring) has arrived
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NS - 2) * NWL) : "memory");
    if (full) {
      // the next group's position q + NS, by one wave; the last step of the
      // group waits for all of them before staging the group's first position
      if (wave == r % kSkpWaves && q + NS < nst) inplace(q + NS);
      if constexpr (r == NS - 1) __syncthreads();
    }
    if constexpr (r % 2 == 0) {
      stage(std::integral_constant<int, (r + 1) % NS>{}, q + 1, an, xn);
      math(ac, xc);
    } else {
      stage(std::integral_constant<int, (r + 1) % NS>{}, q + 1, ac, xc);
      math(an, xn);
    }
  };
  int q = 0;
  for (; q + NS <= nst; q += NS)
    static_for<0, NS>([&](auto rc) { step(rc, q + decltype(rc)::value, true); });
  static_for<0, NS - 1>([&](auto rc) {
    if (q + decltype(rc)::value < nst) step(rc, q + decltype(rc)::value, false);
  });
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the last step

  // sums of squares: the LPR lanes of a row, then the 4 waves in order
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int h = 0; h < XP; ++h) {
      float r = ss[t][h];
#pragma unroll
      for (int o = 1; o < LPR; o *= 2) r += __shfl_xor(r, o, 64);
      if (lane % LPR == 0) s_ss[wave][16 * t + RPI * h + lane / LPR] = r;
    }
  if (H8 && lane < 8) s_ss[wave][8 + lane] = 0.f;  // rows 8 .. 15 (none)
  __syncthreads();
  float ssr = 0.f;  // thread th < 16 MT: row th of this split
  if (th < 16 * MT) ssr = (s_ss[0][th] + s_ss[1][th]) + (s_ss[2][th] + s_ss[3][th]);

  // lane's outputs: acc[i][t][e] = D[n][m], m = 16 t + lane % 16,
  // n = n0 + 16 (w TA + i) + 4 (lane / 16) + e
  auto set_rs = [&](float sum) __attribute__((always_inline)) {
    if (th < 16 * MT) s_rs[th] = a.norm ? 1.0f / sqrtf(sum / (float)K + a.eps) : 1.0f;
    __syncthreads();
  };
  auto finish = [&](const f32x4 (&r)[TA][MT]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 16 * t + (lane & 15);
      if (m >= a.M) continue;
      const float rs = s_rs[m];
#pragma unroll
      for (int i = 0; i < TA; ++i) {
        const int n = n0 + 16 * (TA * wave + i) + 4 * (lane >> 4);
        if (n >= nend) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = (a.bias ? r[i][t][e] * rs * cws[4 * i + e] + cbi[4 * i + e]
                         : r[i][t][e] * rs * cws[4 * i + e]) * a.scale;
        const int64_t yb = (int64_t)m * N + n;
        if (n + 3 < nend && (N & 3) == 0) {
          uint2 pk;
          pk.x = pack2<CT>(o[0], o[1]);
          pk.y = pack2<CT>(o[2], o[3]);
          *(uint2 *)((uint16_t *)a.y + yb) = pk;
        } else {
          for (int e = 0; e < 4; ++e)
            if (n + e < nend) store_from_f32(a.y, CT, yb + e, o[e]);
        }
      }
    }
  };

  if (a.S == 1) {
    set_rs(ssr);
    finish(acc);
    return;
  }

  // ---- split-K hand-off: partial [tile][split][wave][i][t][lane] of f32x4
  constexpr uint32_t WAVEB = (uint32_t)TA * MT * 64u * 16u;
  constexpr uint32_t TILEB = (uint32_t)kSkpWaves * WAVEB;
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.part, (uint32_t)(a.S * a.G) * TILEB);
  auto part_off = [&](int qs, int i, int t) __attribute__((always_inline)) {
    return (uint32_t)(tile * a.S + qs) * TILEB + (uint32_t)wave * WAVEB +
           ((uint32_t)(i * MT + t) * 64u + (uint32_t)lane) * 16u;
  };
#pragma unroll
  for (int i = 0; i < TA; ++i)
#pragma unroll
    for (int t = 0; t < MT; ++t)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][t]), prs,
                                             part_off(sp, i, t), 0, kSc1);
  float *pss = a.part_ss + (int64_t)tile * a.S * 64;
  if (th < 16 * MT) pub_f32(pss + sp * 64 + th, ssr);
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = (ticket_add(a.ticket + tile) == (unsigned)(a.S - 1));
  __syncthreads();
  if (!s_flag) return;
  // last to arrive: sums in split order (its own terms from registers); the
  // loads of QB other splits go out together, at most 32 f32x4 per lane (the
  // main loop's registers are free by now)
  constexpr int QB = TA * MT >= 16 ? 2 : TA * MT >= 8 ? 4 : 8;
  f32x4 tot[TA][MT];
#pragma unroll
  for (int i = 0; i < TA; ++i)
#pragma unroll
    for (int t = 0; t < MT; ++t) tot[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float sst = 0.f;
  bool own_in = false;
  for (int r0 = 0; r0 < a.S - 1; r0 += QB) {
    f32x4 pv[QB][TA][MT];
    float ps[QB];
#pragma unroll
    for (int qq = 0; qq < QB; ++qq) {
      const int r = r0 + qq;  // r-th other split
      const int qs = r + (r >= sp ? 1 : 0);
      const bool ld = r < a.S - 1;
#pragma unroll
      for (int i = 0; i < TA; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          pv[qq][i][t] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, ld ? part_off(qs, i, t) : kOOB,
                                                           0, kSc1));
      ps[qq] = (ld && th < 16 * MT) ? get_f32(pss + qs * 64 + th) : 0.f;
    }
#pragma unroll
    for (int qq = 0; qq < QB; ++qq) {
      const int r = r0 + qq;
      if (r >= a.S - 1) break;
      const int qs = r + (r >= sp ? 1 : 0);
      if (!own_in && sp < qs) {
#pragma unroll
        for (int i = 0; i < TA; ++i)
#pragma unroll
          for (int t = 0; t < MT; ++t) tot[i][t] += acc[i][t];
        sst += ssr;
        own_in = true;
      }
#pragma unroll
      for (int i = 0; i < TA; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) tot[i][t] += pv[qq][i][t];
      sst += ps[qq];
    }
  }
  if (!own_in) {
#pragma unroll
    for (int i = 0; i < TA; ++i)
#pragma unroll
      for (int t = 0; t < MT; ++t) tot[i][t] += acc[i][t];
    sst += ssr;
  }
  set_rs(sst);
  finish(tot);
  if (th == 0) ticket_reset(a.ticket + tile);
}

}  // namespace mtp
