// x-resident weight-streaming GEMM for gfx950 (the RMSNorm -> linear path).
//
// y[M, N] = (x[M, K] . gamma) . W[N, K]^T, then rstd / channel scale / bias /
// scale in the epilogue, at most 64 rows of x per row chunk.
//
// Each workgroup owns NG = WN * NW output columns and a K-range of kb_per
// K-blocks (split `sp` of S). Its prologue stages x * gamma for the whole
// K-range into LDS once (MFMA-fragment order, rounded to the MFMA input
// type) and sums x^2 per row; after one barrier every wave streams its own W
// rows over its own contiguous share of the K-blocks with no further
// barrier: W goes straight from HBM to VGPRs with 16-byte buffer loads (at
// most 8 per K-block, double-buffered), x comes from LDS with conflict-free
// ds_read_b128, and MFMA accumulates D[n][m] in fp32. The WK waves that share
// columns are summed through LDS in fixed order; then either the epilogue
// runs (S == 1) or fp32 partials are published and the last workgroup of the
// column group sums the S partials in split order (agent-scope atomic data
// accesses and a relaxed arrival ticket, see mtp_common.hpp).
//
// The x staging maps each wave's 64 lanes to 16 rows x 4 consecutive 16-byte
// chunks: global reads are 64-byte runs per row, LDS writes cover 64
// consecutive 16-byte slots (no bank conflicts), and each lane keeps the
// sums of squares of its rows in registers for a fixed-order reduction.
#pragma once

#include "wstream.hpp"

namespace mtp {

template <int CT, int WT, int MT, int NSUB, int WN, int WK, int WBL>
__global__ void __launch_bounds__(WN * WK * 64)
wsx_kernel(const WsArgs a) {
  using Sh = WsShape<CT, WT, WBL>;
  constexpr int NT = WN * WK * 64;
  constexpr int NWAVES = WN * WK;
  constexpr int MPAD = MT * 16;
  constexpr int NW = NSUB * 16;
  constexpr int NG = WN * NW;
  constexpr int KB = Sh::KB, NWL = Sh::NWL, E = Sh::E, CPR = Sh::CPR, CPG = Sh::CPG;
  constexpr int WE = 16 / Sh::kWBytes;
  constexpr int BLK_SLOTS = MT * CPG * 64;  // 16-byte LDS slots per K-block
  constexpr int QPR = CPR / 4;              // chunk quads per row per K-block
  static_assert(CPR % 4 == 0, "a K-block holds whole chunk quads");

  extern __shared__ __attribute__((aligned(16))) unsigned char xlds[];  // kb_per * BLK_SLOTS * 16 B
  __shared__ float s_sq[NWAVES][MPAD];
  __shared__ float sq_row[MPAD];
  __shared__ int s_flag;

  u32x4 *xs = (u32x4 *)xlds;
  const int th = threadIdx.x;
  const int lane = th & 63;
  const int wave = th >> 6;
  const int wn = wave % WN;
  const int wk = wave / WN;
  const int lg = lane >> 4;
  const int l16 = lane & 15;

  int bid = blockIdx.x;
  if (a.xcd_map) {
    const int per = (a.G * a.S) >> 3;
    bid = (bid & 7) * per + (bid >> 3);
  }
  const int grp = bid / a.S;
  const int sp = bid - grp * a.S;
  const int mchunk = blockIdx.y;
  const int m0 = mchunk * a.rows_per_chunk;
  const int Mloc = min(a.rows_per_chunk, a.M - m0);
  const int K = a.K, N = a.N;
  const int kbA = sp * a.kb_per;
  const int nkb_wg = min(a.nkb, kbA + a.kb_per) - kbA;  // K-blocks of this workgroup

  // ---- W descriptor and per-wave K share --------------------------------
  const uint32_t ldw = (uint32_t)K * Sh::kWBytes;
  const int grp_rows = min(NG, N - grp * NG);
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc((const unsigned char *)a.w + (int64_t)grp * NG * ldw, (uint32_t)grp_rows * ldw);
  uint32_t wrow[NSUB];
#pragma unroll
  for (int u = 0; u < NSUB; ++u) wrow[u] = (uint32_t)(wn * NW + u * 16 + l16) * ldw + lg * 16;
  const int per_wave = (nkb_wg + WK - 1) / WK;
  const int my_kb0 = wk * per_wave;                      // local K-block index
  const int my_nkb = max(0, min(per_wave, nkb_wg - my_kb0));

  auto load_w = [&](u32x4 (&wr)[NSUB][NWL], int lkb) {  // lkb: local K-block
    const int kb = kbA + lkb;
#pragma unroll
    for (int j = 0; j < NWL; ++j) {
      const bool ok = (lkb < my_kb0 + my_nkb) && (kb * KB + (4 * j + lg) * WE < K);
      const uint32_t koff = (uint32_t)kb * KB * Sh::kWBytes + j * 64;
#pragma unroll
      for (int u = 0; u < NSUB; ++u) wr[u][j] = bload16(wrs, ok ? wrow[u] + koff : kOOB);
    }
  };

  u32x4 wA[NSUB][NWL], wB[NSUB][NWL];

  // ---- prologue: stage x * gamma for the workgroup's K-range --------------
  // x lives in L2 and W streams from HBM: the first x loads are issued before
  // the first W prefetch so they do not queue behind it; everything after
  // that overlaps with the W stream.
  {
    const uint32_t ldx = (uint32_t)K * Sh::kCtBytes;
    const __amdgpu_buffer_rsrc_t xrs =
        make_rsrc((const unsigned char *)a.x + (int64_t)m0 * ldx, (uint32_t)Mloc * ldx);
    const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.gamma, a.gamma ? (uint32_t)K * 4u : 0u);
    float sq[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) sq[t] = 0.f;
    // A wave stages chunk quads (4 consecutive 16-byte chunks of the K-range)
    // for all MT row tiles, so one gamma chunk serves MT x chunks; the loads
    // of QB quads are all issued before any is consumed.
    constexpr int GL = E / 4;  // 16-byte gamma loads per chunk
    constexpr int QB = (MT + GL) * 4 <= 16 ? 4 : ((MT + GL) * 2 <= 16 ? 2 : 1);
    const int nquads = QPR * nkb_wg;
    u32x4 xr[QB][MT];
    u32x4 gr[QB][GL];
    auto issue_x = [&](int q0) {  // quads past nquads load zeros (out of range)
#pragma unroll
      for (int b = 0; b < QB; ++b) {
        const int q = q0 + b;
        const int k = (kbA + q / QPR) * KB + ((q % QPR) * 4 + lg) * E;
        const bool kok = q < nquads && k < K;
#pragma unroll
        for (int t = 0; t < MT; ++t)
          xr[b][t] = bload16(xrs, kok ? (uint32_t)(t * 16 + l16) * ldx + (uint32_t)k * Sh::kCtBytes
                                      : kOOB);
#pragma unroll
        for (int p = 0; p < GL; ++p) gr[b][p] = bload16(grs, kok ? (uint32_t)(k + 4 * p) * 4u : kOOB);
      }
    };
    auto process_x = [&](int q0) {
#pragma unroll
      for (int b = 0; b < QB; ++b) {
        const int q = q0 + b;
        if (q >= nquads) break;
        const int lkb = q / QPR;
        const int c = (q % QPR) * 4 + lg;  // chunk inside the K-block
        // slot of chunk c: lane group and MFMA step of the W chunk holding it
        const int koff = c * E;
        const int wc = koff / WE;
        const int g = wc & 3;
        const int j = (wc >> 2) * (WE / E) + (koff % WE) / E;
        float gv[E];
#pragma unroll
        for (int e = 0; e < E; ++e) gv[e] = a.gamma ? __uint_as_float(gr[b][e >> 2][e & 3]) : 1.f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float v[E];
          if constexpr (CT == MTP_F32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(xr[b][t][e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const f32x2 p2 = unpack2<CT>(xr[b][t][e]);
              v[2 * e] = p2[0];
              v[2 * e + 1] = p2[1];
            }
          }
          float s = 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) s += v[e] * v[e];
          sq[t] += s;
          u32x4 o;
          if constexpr (CT == MTP_F32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = __float_as_uint(v[e] * gv[e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              o[e] = pack2<CT>(v[2 * e] * gv[2 * e], v[2 * e + 1] * gv[2 * e + 1]);
          }
          xs[lkb * BLK_SLOTS + (t * CPG + j) * 64 + l16 + 16 * g] = o;
        }
      }
    };
    int q0 = wave * QB;
    issue_x(q0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(wA, my_kb0);
    __builtin_amdgcn_sched_barrier(0);
    process_x(q0);
    for (q0 += NWAVES * QB; q0 < nquads; q0 += NWAVES * QB) {
      issue_x(q0);
      process_x(q0);
    }
    // fixed-order row sums: lane groups of a wave, then waves
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float s = sq[t];
      s += __shfl_xor(s, 16, 64);
      s += __shfl_xor(s, 32, 64);
      if (lg == 0) s_sq[wave][t * 16 + l16] = s;
    }
  }
  __syncthreads();
  if (th < MPAD) {
    float s = 0.f;
    for (int w = 0; w < NWAVES; ++w) s += s_sq[w][th];
    sq_row[th] = s;
  }

  // ---- main loop: independent per wave ------------------------------------
  f32x4 acc[MT][NSUB];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NSUB; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const u32x4 (&wr)[NSUB][NWL], int lkb) {
    const u32x4 *src = xs + lkb * BLK_SLOTS;
    if constexpr (CT == MTP_F32) {
#pragma unroll
      for (int j = 0; j < CPG; ++j) {
        u32x4 xb[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) xb[t] = src[(t * CPG + j) * 64 + lane];
        float wv[NSUB][4];
#pragma unroll
        for (int u = 0; u < NSUB; ++u) {
          if constexpr (WT == MTP_F32) {
#pragma unroll
            for (int e = 0; e < 4; ++e) wv[u][e] = __uint_as_float(wr[u][j][e]);
          } else {
            const uint32_t d = wr[u][j >> 2][j & 3];
            const f32x2 lo = fp8x2_to_f32(d, false), hi = fp8x2_to_f32(d, true);
            wv[u][0] = lo[0]; wv[u][1] = lo[1]; wv[u][2] = hi[0]; wv[u][3] = hi[1];
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            const float bv = __uint_as_float(xb[t][e]);
#pragma unroll
            for (int u = 0; u < NSUB; ++u) acc[t][u] = mfma16_f32(wv[u][e], bv, acc[t][u]);
          }
      }
    } else {
#pragma unroll
      for (int s = 0; s < Sh::STEPS; ++s) {
        u32x4 av[NSUB];
#pragma unroll
        for (int u = 0; u < NSUB; ++u) {
          if constexpr (WT == CT) {
            av[u] = wr[u][s];
          } else {
            const u32x4 q = wr[u][s >> 1];
            const uint32_t d0 = (s & 1) ? q[2] : q[0];
            const uint32_t d1 = (s & 1) ? q[3] : q[1];
            av[u][0] = fp8x2_to_ct<CT, false>(d0);
            av[u][1] = fp8x2_to_ct<CT, true>(d0);
            av[u][2] = fp8x2_to_ct<CT, false>(d1);
            av[u][3] = fp8x2_to_ct<CT, true>(d1);
          }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const u32x4 bv = src[(t * CPG + s) * 64 + lane];
#pragma unroll
          for (int u = 0; u < NSUB; ++u) acc[t][u] = mfma16<CT>(av[u], bv, acc[t][u]);
        }
      }
    }
  };

  // Prefetches past the wave's share use out-of-range offsets (zeros, no
  // memory traffic); compute on such a block would only add zeros, and the
  // loop never runs it.
  int i = 0;
  for (; i + 1 < my_nkb; i += 2) {
    load_w(wB, my_kb0 + i + 1);
    compute(wA, my_kb0 + i);
    load_w(wA, my_kb0 + i + 2);
    compute(wB, my_kb0 + i + 1);
  }
  if (i < my_nkb) compute(wA, my_kb0 + i);

  // ---- reduction over the WK waves sharing columns, by all threads ----------
  // Every wave parks its accumulators in LDS; each thread then owns output
  // quads (row m, 4 columns) of the workgroup tile, consecutive threads take
  // consecutive rows (conflict-free LDS reads), and sums the WK copies in
  // fixed order.
  __syncthreads();  // x is dead from here on
  f32x4 *red = (f32x4 *)xlds;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NSUB; ++u) red[((wave * MT + t) * NSUB + u) * 64 + lane] = acc[t][u];
  __syncthreads();

  constexpr int Q = NG / 4;          // column quads per workgroup tile
  constexpr int ITEMS = MPAD * Q;    // output quads per workgroup tile
  auto tile_sum = [&](int item, int &m, int &nl) {
    m = item % MPAD;
    const int n4 = item / MPAD;
    nl = n4 * 4;                                    // column inside the tile
    const int wn_ = nl / NW, u = (nl % NW) >> 4, lgq = (nl & 15) >> 2;
    const int ln = (m & 15) + 16 * lgq, t = m >> 4;
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < WK; ++q) s += red[(((q * WN + wn_) * MT + t) * NSUB + u) * 64 + ln];
    return s;
  };

  auto finish = [&](int m, int n, f32x4 v, float sqsum) {
    const float rs = a.norm ? 1.0f / sqrtf(sqsum / (float)K + a.eps) : 1.0f;
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nn = min(n + j, N - 1);
      float t = v[j] * rs;
      if (a.wscale) t *= a.wscale[nn];
      if (a.bias) t += load_as_f32(a.bias, a.bias_dt, nn);
      o[j] = t * a.scale;
    }
    const int64_t base = (int64_t)(m0 + m) * N + n;
    if (n + 3 < N && (N & 3) == 0) {
      if constexpr (CT == MTP_F32) {
        *(f32x4 *)((float *)a.y + base) = f32x4{o[0], o[1], o[2], o[3]};
      } else {
        uint2 pk;
        pk.x = pack2<CT>(o[0], o[1]);
        pk.y = pack2<CT>(o[2], o[3]);
        *(uint2 *)((uint16_t *)a.y + base) = pk;
      }
    } else {
      for (int j = 0; j < 4; ++j)
        if (n + j < N) store_from_f32(a.y, CT, base + j, o[j]);
    }
  };

  if (a.S == 1) {
    for (int item = th; item < ITEMS; item += NT) {
      int m, nl;
      const f32x4 s = tile_sum(item, m, nl);
      const int n = grp * NG + nl;
      if (m < Mloc && n < N) finish(m, n, s, sq_row[m]);
    }
    return;
  }

  // Split-K: partials [chunk][split][group][quad][MPAD] of f32x4, so that
  // consecutive threads write / read consecutive 16 bytes; published and read
  // back with 16-byte coherent (sc1) buffer accesses.
  const uint32_t part_bytes = (uint32_t)(a.S * a.G) * ITEMS * 16u;
  const __amdgpu_buffer_rsrc_t prs =
      make_rsrc((const unsigned char *)a.part + (int64_t)mchunk * part_bytes, part_bytes);
  float *sqp = a.sqp + (int64_t)mchunk * a.G * a.S * MPAD;
  unsigned *ticket = a.ticket + (int64_t)mchunk * a.G;
  for (int item = th; item < ITEMS; item += NT) {
    int m, nl;
    const f32x4 s = tile_sum(item, m, nl);
    const uint32_t off = ((uint32_t)(sp * a.G + grp) * ITEMS + item) * 16u;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, s), prs, off, 0, kSc1);
  }
  if (th < MPAD) pub_f32(sqp + ((int64_t)grp * a.S + sp) * MPAD + th, sq_row[th]);
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = (ticket_add(ticket + grp) == (unsigned)(a.S - 1));
  __syncthreads();
  if (!s_flag) return;
  for (int item = th; item < ITEMS; item += NT) {
    const int m = item % MPAD;
    const int n = grp * NG + (item / MPAD) * 4;
    if (m >= Mloc || n >= N) continue;
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
    for (int q = 0; q < a.S; ++q) {
      const uint32_t off = ((uint32_t)(q * a.G + grp) * ITEMS + item) * 16u;
      s += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kSc1));
      ss += get_f32(sqp + ((int64_t)grp * a.S + q) * MPAD + m);
    }
    finish(m, n, s, ss);
  }
  if (th == 0) ticket_reset(ticket + grp);
}

}  // namespace mtp
