// Single-launch skinny RMSNorm -> linear for gfx950: at most 64 rows of
// 16-bit x (bf16 / f16), W of fp8-e4m3 or the same 16-bit type.
//
//   y[m, n] = (rs[m] * sum_k xg[m, k] W[n, k]) * wscale[n] + bias[n], times scale
//   xg[m, k] = x[m, k] * gamma[k] rounded to the type of x,
//   rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) (norm) or 1
//
// The row scale rs is applied to the fp32 sums rather than to x, so the norm
// needs no pass over x before the GEMM: the workgroups that stream W also
// stage x, square-sum it on the way and apply rs in their epilogue. W is
// read from HBM once; the cost that matters besides it is the x traffic,
// which every workgroup reads for its columns: per W byte, 2 M / (32 NW)
// bytes for fp8 W (NW waves, 32 columns each), so the workgroups are made
// wide (256 columns at NW = 8) and the K range is split among workgroups
// (split-K) until the grid covers the CUs; the host then narrows the
// workgroup's columns (tw, by at most a quarter) to put one workgroup on
// every CU, the tile's rows past them reading zeros.
//
// Workgroup = NW waves, tile of 32 NW columns x all rows, a range of stages.
// A stage is 128 bytes of every W row of the tile (128 k for fp8, 64 k for
// 16-bit W) and the matching x. Per stage:
//   * W comes HBM -> registers with 8-rows x 128-byte non-temporal loads
//     NS - 1 stages ahead, then goes to a double-buffered LDS stage (16-byte
//     chunk c of row r at c ^ sk_swz(r)) one step before use;
//   * x comes from the caller's row-major rows with the same 8-rows x
//     128-byte loads; on its way to LDS each lane adds the squares of its
//     8 values to the row's sum and multiplies them by gamma (staged in LDS
//     for the split's k at the start), and stores them at their place in
//     the B-operand blocks of v_mfma_f32_32x32x16 (64 lanes x 16 bytes per
//     k-step and 32-row tile);
//   * wave w runs the KS k-steps x MT row tiles of its 32 columns (A from
//     the W stage: fp8 is upcast exactly in registers).
//   The stages of a split are taken starting at 7 b mod (stages), b the
//   workgroup: workgroups in step with each other then read different
//   128-byte offsets of their rows, which spreads the requests over the HBM
//   channels.
// k-slot order for fp8 (two k-steps per 32 k): lane group g = lane / 32 of
// the A operand reads chunk 2 p + g (k 32 p + 16 g .. + 15) and takes its
// first 8 bytes in k-step 2 p, the other 8 in k-step 2 p + 1; the x staging
// stores k 32 p + 16 g + 8 h .. + 7 into k-step 2 p + h, lane group g. For
// 16-bit W, k-step j, lane group g holds k 16 j + 8 g .. + 7.
// End: the sums of squares of a row meet in LDS in a fixed order. One split
// (S == 1) applies the epilogue directly; otherwise every workgroup of a
// tile publishes its fp32 tile and sums of squares (coherent stores,
// arrival ticket; see the hand-off notes in mtp_common.hpp) and the last
// to arrive adds them up in split order.
#pragma once

#include "sk.hpp"
#include "skl_args.hpp"

namespace mtp {


template <int CT, int WT, int MT, int NW, bool GAM>
__global__ void __launch_bounds__(64 * NW, 1)
skl_kernel(const SklArgs a) {
  constexpr bool FP8 = WT == MTP_FP8E4M3;
  constexpr int NT = 64 * NW;                 // threads
  constexpr int BN = 32 * NW;                 // columns per workgroup
  constexpr int UK = FP8 ? 128 : 64;          // k per stage
  constexpr int KS = UK / 16;                 // MFMA k-steps per stage
  constexpr int XCH = UK * 2 / 128;           // 128-byte pieces of an x row per stage
  constexpr int WST = BN * kSkUB;             // W bytes of one stage
  constexpr int XST = MT * KS * 1024;         // x bytes of one stage (B-operand blocks)
  constexpr int NS = 4;                       // register ring stages (loads run NS - 1 ahead)
  constexpr int NWC = WST / 1024 / NW;        // W loads per wave per stage
  constexpr int NXL = MT * 4 * XCH;           // x loads per stage (8 rows x 128 bytes each)
  constexpr int NXC = (NXL + NW - 1) / NW;    // x loads per wave per stage
  constexpr int NV = NWC + NXC;               // vector-memory instructions per wave per stage
  constexpr int NGL = GAM ? kSklGammaMax / (4 * NT) : 0;  // 16-byte gamma loads per thread
  static_assert(NWC == 4, "W loads per wave per stage");
  static_assert((NS - 1) * NV + NGL < 64, "vmcnt is 6 bits");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_w[2 * WST];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_x[2 * XST];
  __shared__ __attribute__((aligned(16))) float s_g[GAM ? kSklGammaMax : 4];
  __shared__ float s_ss[NXC * NW][8];
  __shared__ float s_rs[64];
  __shared__ int s_flag;

  const int th = threadIdx.x, lane = th & 63;
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
  const int ag = lane >> 5;
  const int N = a.N, K = a.K;
  const int b = blockIdx.x;
  int tile, sp;
  split_tile_of(b, a.G, a.S, a.xg != 0, tile, sp);
  // tw <= BN output columns; the tile's rows past them read zeros and are
  // not stored
  const int n0 = tile * a.tw;
  const int nend = min(N, n0 + a.tw);
  const int st0 = sp * a.kb_per;
  const int nst = min(a.nkb, st0 + a.kb_per) - st0;  // stages of this split (>= 1)
  const int rot = (7 * b) % nst;
  float cws[16], cbi[16];  // epilogue factors of the lane's 16 columns
  load_col_factors<4>(a.wscale, a.bias, a.bias_dt, N, n0 + 32 * wave + 4 * ag, 8, cws, cbi);
  // stage of the split taken at position st < nst
  auto rotated = [&](int st) __attribute__((always_inline)) {
    return st + rot < nst ? st + rot : st + rot - nst;
  };

  // W load c (c = wave + NW i): rows 8 c .. 8 c + 7 of the tile, lane l: row
  // 8 c + l / 8, 16-byte chunk (l % 8) ^ sk_swz(row) of the stage's 128 bytes
  const uint32_t ldw = (uint32_t)K * (FP8 ? 1u : 2u);
  const int nrows = nend - n0;
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc((const unsigned char *)a.w + (int64_t)n0 * ldw, (uint32_t)nrows * ldw);
  uint32_t wvo[NWC];
#pragma unroll
  for (int i = 0; i < NWC; ++i) {
    const int row = 8 * (wave + NW * i) + (lane >> 3);
    const int chunk = (lane & 7) ^ sk_swz(row);
    wvo[i] = (uint32_t)row * ldw + 16u * chunk;
  }
  // x load c (c = wave + NW i, c < NXL): rows 8 (c % 4 MT) + l / 8 (rows
  // past M read as zeros), 16-byte piece q = 8 (c / 4 MT) + l % 8 of the
  // row's UK k of the stage; its place in LDS is lane 32 g + row % 32 of the
  // B-operand block (row / 32, j) for (j, g) = sk_chunk_slot(q)
  const uint32_t ldx = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)a.M * ldx);
  uint32_t xvo[NXC];
  int xl[NXC], xq[NXC];
  bool xon[NXC];  // wave-uniform: load c carries x
#pragma unroll
  for (int i = 0; i < NXC; ++i) {
    const int c = wave + NW * i;
    xon[i] = c < NXL;
    xl[i] = 0;
    xq[i] = 0;
    xvo[i] = kOOB;
    if (xon[i]) {
      const int row = 8 * (c % (4 * MT)) + (lane >> 3);
      const int q = 8 * (c / (4 * MT)) + (lane & 7);
      int j, g;
      sk_chunk_slot<FP8>(q, j, g);
      xvo[i] = (uint32_t)row * ldx + 16u * (uint32_t)q;
      xl[i] = (((row >> 5) * KS + j) * 64 + ((32 * g + (row & 31)) ^ sk_xswz(j, g))) * 16;
      xq[i] = q;
    }
  }

  // gamma of the split's k (fp32) -> LDS; the loads go out before the ring
  // is primed, so waiting for them waits for nothing later
  u32x4 gr[NGL > 0 ? NGL : 1];
  if constexpr (GAM) {
    const __amdgpu_buffer_rsrc_t grs =
        make_rsrc(a.gamma + (int64_t)st0 * UK, (uint32_t)(nst * UK) * 4u);
#pragma unroll
    for (int i = 0; i < NGL; ++i) gr[i] = bload16(grs, (uint32_t)(th + NT * i) * 16u);
  }

  u32x4 wr[NS][NWC];  // W register ring
  u32x4 xr[NS][NXC];  // x register ring
  // Instruction v (0 <= v < NV) of the stage at position st into ring slot
  // `slot`. Positions past the split (the ring runs NS - 1 ahead) load with
  // an out-of-range vector offset: zeros, no memory access (the scalar
  // offset is not part of the descriptor's range check), into a slot that is
  // never computed on, so the count of instructions per stage is always NV.
  auto issue = [&](auto vc, int st, auto slotc) __attribute__((always_inline)) {
    constexpr int v = decltype(vc)::value, slot = decltype(slotc)::value;
    const bool live = st < nst;
    const int str = st0 + (live ? rotated(st) : 0);
    if constexpr (v < NWC) {
      wr[slot][v] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, live ? wvo[v] : kOOB, str * kSkUB, 2));
    } else {
      constexpr int i = v - NWC;
      xr[slot][i] = __builtin_bit_cast(
          u32x4,
          __builtin_amdgcn_raw_buffer_load_b128(xrs, live ? xvo[i] : kOOB, str * (UK * 2), 0));
    }
  };

  f32x16 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;
  float ss[NXC];
#pragma unroll
  for (int i = 0; i < NXC; ++i) ss[i] = 0.f;

  // ring slot -> LDS buffer `buf` for the stage at position st
  auto to_lds = [&](auto slotc, int buf, int st) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
#pragma unroll
    for (int v = 0; v < NWC; ++v)
      *(u32x4 *)(lds_w + buf * WST + (wave + NW * v) * 1024 + lane * 16) = wr[slot][v];
    const int kst = rotated(st) * UK;  // k of the stage inside the split
#pragma unroll
    for (int i = 0; i < NXC; ++i) {
      if (!xon[i]) continue;
      u32x4 v = xr[slot][i];
      f32x4 g0 = f32x4{1.f, 1.f, 1.f, 1.f}, g1 = g0;
      if constexpr (GAM) {
        g0 = *(const f32x4 *)&s_g[kst + 8 * xq[i]];
        g1 = *(const f32x4 *)&s_g[kst + 8 * xq[i] + 4];
      }
      const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f32x2 f = unpack2<CT>(v[e]);
        ss[i] += f[0] * f[0] + f[1] * f[1];
        if constexpr (GAM) v[e] = pack2<CT>(f[0] * g[2 * e], f[1] * g[2 * e + 1]);
      }
      *(u32x4 *)(lds_x + buf * XST + xl[i]) = v;
    }
  };
  // this wave's 32 columns against all rows, the KS k-steps of the stage in
  // buffer `buf`; the NV loads of the stage at position st_ spread over them
  auto compute = [&](int buf, int st_, auto nslotc) __attribute__((always_inline)) {
    const unsigned char *wb = lds_w + buf * WST;
    const unsigned char *xb = lds_x + buf * XST;
    const int row = 32 * wave + (lane & 31);
    u32x4 wq;
    static_for<0, KS>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      // the loads stay where they are placed: bunched at the end of the
      // stage they would reach HBM a step later
      __builtin_amdgcn_sched_barrier(0);
      static_for<j * NV / KS, (j + 1) * NV / KS>([&](auto vc) { issue(vc, st_, nslotc); });
      __builtin_amdgcn_sched_barrier(0);
      u32x4 av;
      if constexpr (FP8) {
        if constexpr ((j & 1) == 0) {
          const int c = j + ag;  // chunk 2 (j / 2) + g: k-steps j and j + 1
          wq = *(const u32x4 *)(wb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
        }
        constexpr int h = (j & 1) * 2;
        av[0] = fp8x2_to_ct<CT, false>(wq[h]);
        av[1] = fp8x2_to_ct<CT, true>(wq[h]);
        av[2] = fp8x2_to_ct<CT, false>(wq[h + 1]);
        av[3] = fp8x2_to_ct<CT, true>(wq[h + 1]);
      } else {
        const int c = 2 * j + ag;
        av = *(const u32x4 *)(wb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const u32x4 bv =
            *(const u32x4 *)(xb + (t * KS + j) * 1024 + ((lane ^ sk_xswz(j, ag)) << 4));
        acc[t] = mfma32<CT>(av, bv, acc[t]);
      }
    });
  };

  // Pipeline: stages s + 1 .. s + NS - 1 load while s computes; unrolled by
  // the ring length so the ring slots are registers.
  static_for<0, NS - 1>([&](auto pc) {
    static_for<0, NV>([&](auto vc) { issue(vc, decltype(pc)::value, pc); });
    __builtin_amdgcn_sched_barrier(0);
  });
  if constexpr (GAM) {
#pragma unroll
    for (int i = 0; i < NGL; ++i) *(u32x4 *)&s_g[4 * (th + NT * i)] = gr[i];
    lds_barrier();
  }
  to_lds(std::integral_constant<int, 0>{}, 0, 0);
  lds_barrier();
  auto step = [&](auto rc, int s) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::value;  // s % NS
    __builtin_amdgcn_sched_barrier(0);
    // stage s + 1 to the other LDS buffer (the barrier below publishes it;
    // buffer s & 1 is rewritten only after the next barrier)
    if (s + 1 < nst) to_lds(std::integral_constant<int, (r + 1) % NS>{}, (s + 1) & 1, s + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(s & 1, s + NS - 1, std::integral_constant<int, (r + NS - 1) % NS>{});
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  };
  int s = 0;
  for (; s + NS <= nst; s += NS)
    static_for<0, NS>([&](auto rc) { step(rc, s + decltype(rc)::value); });
  static_for<0, NS - 1>([&](auto rc) {
    if (s + decltype(rc)::value < nst) step(rc, s + decltype(rc)::value);
  });
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the last stage

  // ---- sums of squares of the split: 8 lanes per row and load, then the
  // XCH loads of a row, in a fixed order
#pragma unroll
  for (int i = 0; i < NXC; ++i) {
    float v = ss[i];
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    if (xon[i] && (lane & 7) == 0) s_ss[wave + NW * i][lane >> 3] = v;
  }
  __syncthreads();
  float ssr = 0.f;  // thread th < 32 MT: row th
  if (th < 32 * MT) {
#pragma unroll
    for (int hc = 0; hc < XCH; ++hc) ssr += s_ss[hc * 4 * MT + (th >> 3)][th & 7];
  }
  auto set_rs = [&](float sum) __attribute__((always_inline)) {
    if (th < 32 * MT) s_rs[th] = a.norm ? 1.0f / sqrtf(sum / (float)K + a.eps) : 1.0f;
    __syncthreads();
  };

  // lane's outputs: r[t][e] = D[n][m], m = 32 t + lane % 32,
  // n = n0 + 32 wave + 8 (e / 4) + 4 (lane / 32) + e % 4
  auto finish = [&](const f32x16 (&r)[MT]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = 32 * t + (lane & 31);
      if (m >= a.M) continue;
      const float rs = s_rs[m];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + 32 * wave + 8 * g + 4 * ag;
        if (n >= nend) continue;
        float o[4];
#pragma unroll
        for (int jx = 0; jx < 4; ++jx)
          o[jx] = (a.bias ? r[t][4 * g + jx] * rs * cws[4 * g + jx] + cbi[4 * g + jx]
                          : r[t][4 * g + jx] * rs * cws[4 * g + jx]) * a.scale;
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
  };

  if (a.S == 1) {
    set_rs(ssr);
    finish(acc);
    return;
  }

  // ---- split-K hand-off: partial [tile][split][wave][t][4 quads][lane] of
  // f32x4 (consecutive lanes write consecutive 16 bytes), coherent stores
  constexpr uint32_t TILEB = (uint32_t)BN * 32u * MT * 4u;
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.part, (uint32_t)(a.S * a.G) * TILEB);
  auto part_off = [&](int q, int t, int g4) __attribute__((always_inline)) {
    return (uint32_t)(tile * a.S + q) * TILEB +
           ((uint32_t)((wave * MT + t) * 4 + g4) * 64u + (uint32_t)lane) * 16u;
  };
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 p4 = f32x4{acc[t][4 * g4], acc[t][4 * g4 + 1], acc[t][4 * g4 + 2],
                             acc[t][4 * g4 + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, p4), prs,
                                             part_off(sp, t, g4), 0, kSc1);
    }
  float *pss = a.part_ss + (int64_t)tile * a.S * 64;
  if (th < 32 * MT) pub_f32(pss + sp * 64 + th, ssr);
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = (ticket_add(a.ticket + tile) == (unsigned)(a.S - 1));
  __syncthreads();
  if (!s_flag) return;
  // last to arrive: sums in split order (its own terms from registers); the
  // loads of up to QB other splits go out together (one round trip for up
  // to QB + 1 splits)
  constexpr int QB = 4;
  f32x16 tot[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int e = 0; e < 16; ++e) tot[t][e] = 0.f;
  float sst = 0.f;
  bool own_in = false;
  for (int r0 = 0; r0 < a.S - 1; r0 += QB) {
    f32x4 pv[QB][MT][4];
    float ps[QB];
#pragma unroll
    for (int qq = 0; qq < QB; ++qq) {
      const int r = r0 + qq;  // r-th other split
      const int q = r + (r >= sp ? 1 : 0);
      const bool ld = r < a.S - 1;
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          pv[qq][t][g4] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, ld ? part_off(q, t, g4) : kOOB, 0,
                                                           kSc1));
      ps[qq] = (ld && th < 32 * MT) ? get_f32(pss + q * 64 + th) : 0.f;
    }
#pragma unroll
    for (int qq = 0; qq < QB; ++qq) {
      const int r = r0 + qq;
      if (r >= a.S - 1) break;
      const int q = r + (r >= sp ? 1 : 0);
      if (!own_in && sp < q) {
#pragma unroll
        for (int t = 0; t < MT; ++t) tot[t] += acc[t];
        sst += ssr;
        own_in = true;
      }
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
          for (int e = 0; e < 4; ++e) tot[t][4 * g4 + e] += pv[qq][t][g4][e];
      sst += ps[qq];
    }
  }
  if (!own_in) {
#pragma unroll
    for (int t = 0; t < MT; ++t) tot[t] += acc[t];
    sst += ssr;
  }
  set_rs(sst);
  finish(tot);
  if (th == 0) ticket_reset(a.ticket + tile);
}

}  // namespace mtp
