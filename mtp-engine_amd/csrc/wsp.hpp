// Pipelined weight-streaming GEMM for gfx950: the RMSNorm -> linear path.
//
// y[M, N] = (x[M, K] . gamma) . W[N, K]^T, then rstd / channel scale / bias /
// scale in the epilogue, at most 64 rows of x per row chunk.
//
// Unit of work: a "unit" is 64 bytes of every W row (64 fp8, 32 bf16/f16 or
// 16 fp32 values of k). One 16-byte buffer load per lane covers 16 W rows
// of a unit: lane (g = lane / 16, r = lane % 16) reads bytes [16g, 16g + 16)
// of the unit in row r, so the four lanes of a row read 64 contiguous bytes.
// Rows are whole units (K * sizeof(W) % 64 == 0, checked by the planner).
//
// Workgroup = WN x WK waves. It owns NG = WN * 16 * NSUB output columns and
// a range of units (split `sp` of S cross-workgroup K-splits); K-group wk
// walks a contiguous share of that range one unit per stage, all K-groups in
// lock-step with one barrier per stage.
//
// Per stage a wave issues NSUB W loads (HBM) and at most a few x loads (L2).
// Stage s: issue W(s + 2); wait for W(s) and x(s + 1); barrier; MFMAs of
// unit s (x from the LDS ring) interleaved with staging x(s + 1) into the
// ring; issue x(s + 3). W and x rotate through three register slots, so two
// stages of W are in flight while a unit is multiplied (reissuing only after
// the MFMAs halves the bytes in flight and costs a third of the bandwidth).
// The per-stage loads address through buffer descriptors
// whose base advances by one unit per stage on the scalar unit (and whose
// size is 0 past the K-group's range), so lanes keep fixed offsets and
// out-of-range rows or units read as zero without vector address math.
//
// x staging: the WN waves of a K-group share the unit's x blocks. A block
// is the B operand of one MFMA step for one 16-row tile: 64 lanes x 16 bytes
// laid out so that lane l's MFMA fragment sits at 16 * l (conflict-free
// ds_write_b128 / ds_read_b128). The staging lane accumulates the RMSNorm
// sums of squares as the diagonal of x . x^T with one MFMA per block (fp32 x:
// vector FMAs) and, with gamma (GAM), multiplies x by gamma in fp32 (gamma
// kept in LDS for the workgroup's K-range) and rounds to the MFMA input
// type; without gamma the fragment is copied as loaded. A three-slot LDS ring
// lets a wave write unit s + 1 while slower waves still read unit s.
//
// MFMA: D[n][m] += W[n, k] x[m, k] with A = W (16 rows of n) and B = x (16
// rows of m); bf16/f16 16x16x32 (fp8 W upcast exactly in registers) or fp32
// 16x16x4. Lane l of D holds row m = l % 16 and columns 4 (l / 16) + j.
//
// End: the WK K-groups are summed through LDS in fixed order by all threads;
// then the epilogue runs (S == 1) or fp32 partials are published and the
// last workgroup of the column group sums the S partials in split order
// (agent-scope atomic data accesses and a relaxed arrival ticket, see
// mtp_common.hpp). Row statistics are applied in the epilogue: rstd[m] *
// (x[m] . W[n]) equals (x[m] * rstd[m]) . W[n] up to fp32 rounding.
#pragma once

#include "wstream.hpp"

namespace mtp {

template <int CT, int WT>
struct WspShape {
  static constexpr int kWBytes = dtype_bytes(WT);
  static constexpr int kXBytes = dtype_bytes(CT);
  static constexpr int KU = 64 / kWBytes;  // k per unit
  static constexpr int WV = 16 / kWBytes;  // k per 16-byte W lane chunk
  static constexpr int XV = 16 / kXBytes;  // k per 16-byte x fragment
  static constexpr int H = WV / XV;        // x fragments per W lane chunk
};

constexpr int kWspRing = 3;  // LDS ring slots
constexpr int kWspGJ = 4;    // gamma 16-byte loads per thread (prologue)

// Dynamic LDS bytes of a wsp launch: the x ring plus (with gamma) gamma for
// the K-range and one padding unit, or the K-group reduction area, whichever
// is larger.
constexpr size_t wsp_lds_bytes(int mt, int h, int nsub, int wn, int wk, int64_t units_per_group,
                               int ku, bool gam) {
  const size_t ring = (size_t)kWspRing * wk * mt * h * 1024;
  const size_t gsz = gam ? ((size_t)wk * units_per_group + 1) * ku * 4 : 0;
  const size_t red = (size_t)wk * wn * mt * nsub * 1024;
  return ring + gsz > red ? ring + gsz : red;
}

template <int CT, int WT, int MT, int NSUB, int WN, int WK, bool GAM>
__global__ void __launch_bounds__(WN * WK * 64)
wsp_kernel(const WsArgs a) {
  using Sh = WspShape<CT, WT>;
  constexpr int NT = WN * WK * 64;
  constexpr int NWAVES = WN * WK;
  constexpr int MPAD = MT * 16;
  constexpr int NW = NSUB * 16;
  constexpr int NG = WN * NW;
  constexpr int KU = Sh::KU, WV = Sh::WV, XV = Sh::XV, H = Sh::H;
  constexpr int XB = MT * H;              // x blocks per unit and K-group
  constexpr int XW = (XB + WN - 1) / WN;  // x blocks staged per wave
  constexpr int SLOT = WK * XB * 64;      // 16-byte LDS slots per ring slot

  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ float s_sq[NWAVES][MPAD];
  __shared__ float sq_row[MPAD];
  __shared__ int s_flag;

  u32x4 *ring = (u32x4 *)lds;
  float *glds = (float *)(lds + (size_t)kWspRing * SLOT * 16);

  const int th = threadIdx.x;
  const int lane = th & 63;
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
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

  // Output quads: item = m + MPAD q holds columns 4 q .. 4 q + 3 of row m of
  // the tile; thread th stores items th + NT i. Their epilogue factors are
  // loaded in one batch before the stores (held through the main loop they
  // would cost registers the pipeline needs).
  constexpr int Q = NG / 4;                   // column quads per workgroup tile
  constexpr int ITEMS = MPAD * Q;             // output quads per workgroup tile
  constexpr int IPT = (ITEMS + NT - 1) / NT;  // output quads per thread
  float fws[IPT][4], fbi[IPT][4];
  auto load_factors = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < IPT; ++it)
      load_col_factors<1>(a.wscale, a.bias, a.bias_dt, N, grp * NG + ((th + it * NT) / MPAD) * 4,
                          0, fws[it], fbi[it]);
  };

  // Units: kb_per per split, nkb in total.
  const int u_wg0 = sp * a.kb_per;
  const int u_wg1 = min(a.nkb, u_wg0 + a.kb_per);
  const int upg = (u_wg1 - u_wg0 + WK - 1) / WK;  // stages
  const int u_kg0 = u_wg0 + wk * upg;
  const int u_kg1 = min(u_wg1, u_kg0 + upg);
  const int k_wg0 = u_wg0 * KU;
  const int k_lim = min(K, u_wg1 * KU);

  // ---- operand streams ---------------------------------------------------
  const uint32_t ldw = (uint32_t)K * Sh::kWBytes;
  const int grp_rows = min(NG, N - grp * NG);
  const unsigned char *wbase = (const unsigned char *)a.w + (int64_t)grp * NG * ldw;
  const uint32_t w_bytes = (uint32_t)grp_rows * ldw;
  uint32_t wvo[NSUB];
#pragma unroll
  for (int u = 0; u < NSUB; ++u) wvo[u] = (uint32_t)(wn * NW + u * 16 + l16) * ldw + lg * 16;

  const uint32_t ldx = (uint32_t)K * Sh::kXBytes;
  const unsigned char *xbase = (const unsigned char *)a.x + (int64_t)m0 * ldx;
  const uint32_t x_bytes = (uint32_t)Mloc * ldx;
  // This wave's x blocks: b = wn + WN * i -> tile t = b / H, fragment h = b % H.
  int xb_t[XW], xb_kof[XW];
  bool xb_ok[XW];
  uint32_t xvo[XW];
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    const int b = wn + WN * i;
    xb_ok[i] = b < XB;
    xb_t[i] = b / H;
    xb_kof[i] = lg * WV + (b % H) * XV;  // k offset inside the unit
    xvo[i] = xb_ok[i] ? (uint32_t)(xb_t[i] * 16 + l16) * ldx + (uint32_t)xb_kof[i] * Sh::kXBytes
                      : kOOB;
  }

  auto load_w = [&](u32x4 (&wr)[NSUB], int s) {
    const int unit = u_kg0 + s;
    const uint32_t adv = (uint32_t)unit * 64u;
    const __amdgpu_buffer_rsrc_t r = make_rsrc(wbase + adv, unit < u_kg1 ? w_bytes - adv : 0u);
#pragma unroll
    for (int u = 0; u < NSUB; ++u) wr[u] = bload16_nt(r, wvo[u]);
  };
  auto load_x = [&](u32x4 (&xr)[XW], int s) {
    const int unit = u_kg0 + s;
    const uint32_t adv = (uint32_t)unit * (KU * Sh::kXBytes);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(xbase + adv, unit < u_kg1 ? x_bytes - adv : 0u);
#pragma unroll
    for (int i = 0; i < XW; ++i) xr[i] = bload16(r, xvo[i]);
  };

  // Sums of squares: 16-bit x accumulates x . x^T per block with MFMA (the
  // diagonal is the row sum), fp32 x per lane with FMAs.
  f32x4 sqacc[XW];
  float sqv[XW];
#pragma unroll
  for (int i = 0; i < XW; ++i) {
    sqacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    sqv[i] = 0.f;
  }

  // x fragment -> (sum of squares, [* gamma, round]) -> ring slot of stage s.
  auto put_x = [&](const u32x4 (&xr)[XW], int s) {
    const int unit = u_kg0 + s;
    u32x4 *dst = ring + (s % kWspRing) * SLOT + wk * XB * 64 + lane;
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      if (!xb_ok[i]) continue;
      const int b = wn + WN * i;
      float v[XV];
      if constexpr (CT == MTP_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = __uint_as_float(xr[i][e]);
          sqv[i] += v[e] * v[e];
        }
      } else {
        sqacc[i] = mfma16<CT>(xr[i], xr[i], sqacc[i]);
      }
      u32x4 o = xr[i];
      if constexpr (GAM) {
        const float *gp = glds + (unit * KU - k_wg0) + xb_kof[i];
        float gv[XV];
#pragma unroll
        for (int e = 0; e < XV; e += 4) {
          const f32x4 g4 = *(const f32x4 *)(gp + e);
          gv[e] = g4[0]; gv[e + 1] = g4[1]; gv[e + 2] = g4[2]; gv[e + 3] = g4[3];
        }
        if constexpr (CT == MTP_F32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = __float_as_uint(v[e] * gv[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f32x2 p2 = unpack2<CT>(xr[i][e]);
            o[e] = pack2<CT>(p2[0] * gv[2 * e], p2[1] * gv[2 * e + 1]);
          }
        }
      }
      dst[b * 64] = o;
    }
  };

  f32x4 acc[MT][NSUB];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NSUB; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const u32x4 (&wr)[NSUB], int s) {
    const u32x4 *src = ring + (s % kWspRing) * SLOT + wk * XB * 64 + lane;
    if constexpr (CT == MTP_F32) {
      float wv[NSUB][WV];
#pragma unroll
      for (int u = 0; u < NSUB; ++u) {
        if constexpr (WT == MTP_F32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) wv[u][e] = __uint_as_float(wr[u][e]);
        } else {
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const f32x2 lo = fp8x2_to_f32(wr[u][d], false), hi = fp8x2_to_f32(wr[u][d], true);
            wv[u][4 * d] = lo[0]; wv[u][4 * d + 1] = lo[1];
            wv[u][4 * d + 2] = hi[0]; wv[u][4 * d + 3] = hi[1];
          }
        }
      }
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const u32x4 xb = src[(t * H + h) * 64];
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int u = 0; u < NSUB; ++u)
              acc[t][u] = mfma16_f32(wv[u][h * 4 + e], __uint_as_float(xb[e]), acc[t][u]);
        }
    } else {
      u32x4 av[NSUB][H];
#pragma unroll
      for (int u = 0; u < NSUB; ++u) {
        if constexpr (WT == CT) {
          av[u][0] = wr[u];
        } else {
#pragma unroll
          for (int h = 0; h < H; ++h) {
            const uint32_t d0 = wr[u][2 * h], d1 = wr[u][2 * h + 1];
            av[u][h][0] = fp8x2_to_ct<CT, false>(d0);
            av[u][h][1] = fp8x2_to_ct<CT, true>(d0);
            av[u][h][2] = fp8x2_to_ct<CT, false>(d1);
            av[u][h][3] = fp8x2_to_ct<CT, true>(d1);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const u32x4 bv = src[(t * H + h) * 64];
#pragma unroll
          for (int u = 0; u < NSUB; ++u) acc[t][u] = mfma16<CT>(av[u][h], bv, acc[t][u]);
        }
    }
  };

  // ---- prologue -------------------------------------------------------------
  // Loads retire in issue order and the wait counts at the loop head must
  // hold on entry and on the back edge alike, so every issue point is pinned
  // with a scheduling barrier: when stage s starts, the pending loads end
  // with W(s), x(s + 1), W(s + 1), x(s + 2).
  // Gamma covers the K-groups' units plus one padding unit (the last stage
  // stages a unit it never computes) and is 0 past the K-range, so padding
  // multiplies zeros by finite values.
  const int ng16 = GAM ? (WK * upg + 1) * KU / 4 : 0;  // 16-byte gamma chunks in LDS
  u32x4 gr[kWspGJ];
  if constexpr (GAM) {
    const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.gamma, (uint32_t)K * 4u);
#pragma unroll
    for (int j = 0; j < kWspGJ; ++j) {
      const int c = th + j * NT;
      const int k = k_wg0 + 4 * c;
      gr[j] = bload16(grs, (c < ng16 && k < k_lim) ? (uint32_t)k * 4u : kOOB);
    }
  }
  u32x4 x0[XW], x1[XW], x2[XW];
  u32x4 w0[NSUB], w1[NSUB], w2[NSUB];
  __builtin_amdgcn_sched_barrier(0);
  load_x(x0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_w(w0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_x(x1, 1);
  __builtin_amdgcn_sched_barrier(0);
  load_w(w1, 1);
  __builtin_amdgcn_sched_barrier(0);
  load_x(x2, 2);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (GAM) {
#pragma unroll
    for (int j = 0; j < kWspGJ; ++j) {
      const int c = th + j * NT;
      if (c < ng16) *(u32x4 *)(glds + 4 * c) = gr[j];
    }
    __syncthreads();
  }
  put_x(x0, 0);

  // ---- main loop ------------------------------------------------------------
  // Stage s: issue W(s + 2) first (W(s - 1)'s registers are free), so two
  // stages of W stay in flight while unit s is multiplied; barrier; MFMAs of
  // unit s with staging of x(s + 1); issue x(s + 3) into x(s)'s registers.
  // W and x rotate through three register slots: unrolled by three.
  auto stage = [&](int s_, u32x4 (&wc)[NSUB], u32x4 (&wn2)[NSUB], const u32x4 (&xp)[XW],
                   u32x4 (&xn)[XW]) {
    __builtin_amdgcn_sched_barrier(0);
    load_w(wn2, s_ + 2);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    compute(wc, s_);
    put_x(xp, s_ + 1);
    __builtin_amdgcn_sched_barrier(0);
    load_x(xn, s_ + 3);
    __builtin_amdgcn_sched_barrier(0);
  };
  int s = 0;
  for (; s + 3 <= upg; s += 3) {
    stage(s, w0, w2, x1, x0);
    stage(s + 1, w1, w0, x2, x1);
    stage(s + 2, w2, w1, x0, x2);
  }
  if (s < upg) stage(s, w0, w2, x1, x0);
  if (s + 1 < upg) stage(s + 1, w1, w0, x2, x1);

  // ---- row sums of squares: lane groups, then waves, in fixed order --------
  // The diagonal element (r, r) of a block's x . x^T sits in lane
  // 16 * (r / 4) + r, register r % 4.
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < XW; ++i) {
      float d;
      if constexpr (CT == MTP_F32) {
        d = sqv[i];
      } else {
        const int j = l16 & 3;
        const f32x4 q = sqacc[i];
        d = (l16 >> 2) != lg ? 0.f : (j == 0 ? q[0] : j == 1 ? q[1] : j == 2 ? q[2] : q[3]);
      }
      v += (xb_ok[i] && xb_t[i] == t) ? d : 0.f;
    }
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (lg == 0) s_sq[wave][t * 16 + l16] = v;
  }

  // ---- reduction over the WK K-groups, by all threads -----------------------
  __syncthreads();  // the ring is dead from here on
  if (th < MPAD) {
    float v = 0.f;
    for (int w = 0; w < NWAVES; ++w) v += s_sq[w][th];
    sq_row[th] = v;
  }
  f32x4 *red = (f32x4 *)lds;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NSUB; ++u) red[((wave * MT + t) * NSUB + u) * 64 + lane] = acc[t][u];
  __syncthreads();

  auto tile_sum = [&](int item, int &m, int &nl) {
    m = item % MPAD;
    nl = (item / MPAD) * 4;
    const int wn_ = nl / NW, u = (nl % NW) >> 4, lgq = (nl & 15) >> 2;
    const int ln = (m & 15) + 16 * lgq, t = m >> 4;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < WK; ++q) v += red[(((q * WN + wn_) * MT + t) * NSUB + u) * 64 + ln];
    return v;
  };

  // fw / fb: the factors of columns n .. n + 3
  auto finish = [&](int m, int n, f32x4 v, float sqsum, const float *fw, const float *fb) {
    const float rs = a.norm ? 1.0f / sqrtf(sqsum / (float)K + a.eps) : 1.0f;
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float t = v[j] * rs * fw[j];
      if (a.bias) t += fb[j];
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
    load_factors();
#pragma unroll
    for (int it = 0; it < IPT; ++it) {
      const int item = th + it * NT;
      if (item >= ITEMS) break;
      int m, nl;
      const f32x4 v = tile_sum(item, m, nl);
      const int n = grp * NG + nl;
      if (m < Mloc && n < N) finish(m, n, v, sq_row[m], fws[it], fbi[it]);
    }
    return;
  }

  // Split-K: partials [chunk][split][group][item] of f32x4 (consecutive
  // threads write / read consecutive 16 bytes) with 16-byte coherent (sc1)
  // buffer accesses; partial sums of squares beside them.
  const uint32_t part_bytes = (uint32_t)(a.S * a.G) * ITEMS * 16u;
  const __amdgpu_buffer_rsrc_t prs =
      make_rsrc((const unsigned char *)a.part + (int64_t)mchunk * part_bytes, part_bytes);
  float *sqp = a.sqp + (int64_t)mchunk * a.G * a.S * MPAD;
  unsigned *ticket = a.ticket + (int64_t)mchunk * a.G;
  for (int item = th; item < ITEMS; item += NT) {
    int m, nl;
    const f32x4 v = tile_sum(item, m, nl);
    const uint32_t off = ((uint32_t)(sp * a.G + grp) * ITEMS + item) * 16u;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), prs, off, 0, kSc1);
  }
  if (th < MPAD) pub_f32(sqp + ((int64_t)grp * a.S + sp) * MPAD + th, sq_row[th]);
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = (ticket_add(ticket + grp) == (unsigned)(a.S - 1));
  __syncthreads();
  if (!s_flag) return;
  // The last workgroup sums the splits in split order; loads go out four
  // splits at a time (past the last split: zeros) so their latencies
  // overlap, the first four before the row statistics are read.
  f32x4 t4[IPT][4];
  auto load_batch = [&](int q0) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < IPT; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int item = th + it * NT, q = q0 + j;
        const uint32_t off = (item < ITEMS && q < a.S)
                                 ? ((uint32_t)(q * a.G + grp) * ITEMS + item) * 16u
                                 : kOOB;
        t4[it][j] =
            __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kSc1));
      }
  };
  load_batch(0);
  if (th < MPAD) {
    float ss = 0.f;
    for (int q0 = 0; q0 < a.S; q0 += 4) {
      float s4[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int q = q0 + j < a.S ? q0 + j : q0;
        s4[j] = get_f32(sqp + ((int64_t)grp * a.S + q) * MPAD + th);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (q0 + j < a.S) ss += s4[j];
    }
    sq_row[th] = ss;
  }
  __syncthreads();
  load_factors();
  f32x4 v[IPT];
#pragma unroll
  for (int it = 0; it < IPT; ++it) v[it] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int q0 = 0;;) {
#pragma unroll
    for (int it = 0; it < IPT; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[it] += t4[it][j];
    q0 += 4;
    if (q0 >= a.S) break;
    load_batch(q0);
  }
#pragma unroll
  for (int it = 0; it < IPT; ++it) {
    const int item = th + it * NT;
    const int m = item % MPAD;
    const int n = grp * NG + (item / MPAD) * 4;
    if (item < ITEMS && m < Mloc && n < N) finish(m, n, v[it], sq_row[m], fws[it], fbi[it]);
  }
  if (th == 0) ticket_reset(ticket + grp);
}

}  // namespace mtp
