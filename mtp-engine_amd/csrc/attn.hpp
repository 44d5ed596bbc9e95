// Single-query-per-row softmax attention for gfx950: the tree / paged
// attention family and the multi-query tree-verify step built from them.
//
// One launch covers, for every (batch b, head h), a set of NQ <= 64 queries
// q[b, n, h, :] attending under one softmax to
//   * Lc context keys of a paged cache: key t is pages[table[b, t], b, h,
//     t % page_size, :] (pages [P, B, H, page_size, D]), and
//   * Lt dense keys k[b, h, t, :] (arbitrary element strides), masked by a
//     1-D mask [Lt] (shared by all queries) or a 2-D mask [NQ, Lt]
//     (value > 0.5 = attend; masked scores are -inf, so a query with every
//     key masked yields NaN like the reference's eager softmax).
//
// Keys go by blocks of 64: the context blocks (the last one possibly
// partial), then the dense blocks. Workgroup (b*H + h, chunk c) of 8 waves
// takes chunk_blocks consecutive blocks; wave w owns query tile w / 2
// (queries 16 (w / 2) .. + 15) and key half w % 2 (keys 32 (w % 2) .. + 31
// of every block), so each SIMD runs two independent softmax chains. Every
// wave loads. Per block:
//   * K and V rows come from HBM with 16-byte non-temporal loads into a
//     register ring R blocks deep (the page of every context key is looked
//     up in an LDS copy of the chunk's page-table window, so no load waits
//     on another), then go to a double-buffered LDS area: K rows as they
//     are, V transposed to [d][key] with keys t and t + 16 of a half side by
//     side in one dword and the 16-byte groups of a half-row swizzled by d;
//   * S^T[t][q] = K[t] . Q[q]     MFMA 16x16x32, A = K rows, B = Q^T (regs);
//   * online softmax per query (the accumulator lane of q holds 8 keys:
//     t = 4g + j and 16 + 4g + j, so the row max / sum are two VALU lane
//     swaps).
//     The running max only moves when a block's max exceeds it by more than
//     kAttnRescale, so O is rescaled rarely (probabilities stay <= e^8);
//   * O^T[d][q] += V^T[d][t] P^T[t][q]: the S^T accumulators, rounded to
//     the MFMA input type and paired (key t, key t + 16), are the B operand
//     as they are; A = the paired V^T row segment, one 16-byte LDS read.
// The two key halves are merged through LDS. With one chunk the workgroup
// writes the output; otherwise it writes (m, l, O) and attn_merge_kernel
// combines the chunks in chunk order.
#pragma once

#include "attn_args.hpp"
#include "wstream.hpp"

namespace mtp {

__device__ __forceinline__ bool mask_on(const void *m, int dt, int64_t i) {
  switch (dt) {
    case MTP_F32: return ((const float *)m)[i] > 0.5f;
    case MTP_BF16:
    case MTP_F16: return load_as_f32(m, dt, i) > 0.5f;
    default: return ((const uint8_t *)m)[i] > 0;  // U8 / bool
  }
}

template <int CT>
__device__ __forceinline__ void attn_store4(const AttnArgs &a, int b, int q, int h, int d, f32x4 v,
                                            float inv) {
  uint16_t *op = (uint16_t *)a.out + (int64_t)b * a.o_sb + (int64_t)q * a.o_sn +
                 (int64_t)h * a.o_sh + d;
  uint2 pk;
  pk.x = pack2<CT>(v[0] * inv, v[1] * inv);
  pk.y = pack2<CT>(v[2] * inv, v[3] * inv);
  *(uint2 *)op = pk;
}

template <int CT, int D>
__global__ void __launch_bounds__(512)
attn_kernel(const AttnArgs a) {
  constexpr int NT = 512;
  constexpr int KB = kAttnBlock;       // keys per block (two halves of 32)
  constexpr int DC = D / 8;            // 16-byte chunks per key row
  constexpr int NPC = 32 * DC;         // (half, key t, key t + 16, chunk) per block
  constexpr int PPT = (NPC + NT - 1) / NT;
  constexpr int R = kAttnRing;         // blocks in flight
  constexpr int KROW = D + 8;          // K row in LDS (elements)
  constexpr int VROW = KB + 8;         // V^T row in LDS (elements)
  constexpr int DS = D / 32;           // MFMA k-steps over d
  constexpr int DT = D / 16;           // O^T tiles
  constexpr int TW = kAttnTableWindow; // page-table window (keys)
  constexpr int WB = TW / KB;          // blocks per window
  static_assert(KB == 64, "two key halves of 32");
  static_assert(R >= 2 && R % 2 == 0 && R < WB, "ring depth: even (LDS buffer parity), below a window");
  static_assert(4 * DT * 64 * 16 <= 2 * (int)sizeof(uint16_t) * KB * KROW, "half merge fits the K buffers");
  __shared__ __attribute__((aligned(16))) uint16_t sk[2][KB * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t sv[2][D * VROW];
  __shared__ int64_t s_off[TW];        // byte offset of a context key's row in the pages, -1: none
  __shared__ int s_valid[2][KB];

  const int th = threadIdx.x;
  const int lane = th & 63;
  const int wave = th >> 6;
  const int lg = lane >> 4;
  const int l16 = lane & 15;
  const int qt = wave >> 1;            // query tile
  const int kh = wave & 1;             // key half
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int c = blockIdx.y;
  const int QP = ((a.NQ + 15) >> 4) * 16;  // query rows incl. padding
  const bool qwave = qt * 16 < a.NQ;

  const int nctx_all = (a.Lc + KB - 1) / KB;
  const int ntot = nctx_all + (a.Lt + KB - 1) / KB;
  const int cb0 = c * a.chunk_blocks;
  const int nb = max(0, min(ntot, cb0 + a.chunk_blocks) - cb0);

  const uint16_t *qbase = (const uint16_t *)a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const int qi = qt * 16 + l16;  // this lane's query in the accumulator layout
  u32x4 qf[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s)
    qf[s] = qi < a.NQ ? *(const u32x4 *)(qbase + (int64_t)qi * a.q_sn + s * 32 + 8 * lg)
                      : u32x4{0u, 0u, 0u, 0u};
  const int64_t page_bh = (int64_t)b * a.p_sb + (int64_t)h * a.p_sh;
  const int64_t dense_bh = (int64_t)b * a.d_sb + (int64_t)h * a.d_sh;

  // ---- page-table window: s_off[i] for the keys of blocks w0 .. w0 + WB - 1
  auto load_window = [&](int w0) {
#pragma unroll
    for (int i = th; i < TW; i += NT) {
      const int tok = (cb0 + w0) * KB + i;
      int64_t off = -1;
      if (tok < a.Lc) {
        const int page = a.table[(int64_t)b * a.ld_tab + tok];
        if (page >= 0 && page < a.npages)
          off = ((int64_t)page * a.p_sp + page_bh + (int64_t)(tok % a.page_size) * D) * 2;
      }
      s_off[i] = off;
    }
  };

  // ---- staging: global -> register ring -> LDS ------------------------------
  // Thread group p covers keys 32 kh_ + t and 32 kh_ + t + 16, 16-byte chunk dc.
  u32x4 rk[R][PPT][2], rv[R][PPT][2];
  int rok[R];
  auto group_of = [&](int p, int &khp, int &t, int &dc) {
    const int pc = (th + p * NT) % NPC;
    khp = pc / (16 * DC);
    const int rem = pc - khp * (16 * DC);
    t = rem / DC;
    dc = rem - t * DC;
  };
  auto fetch = [&](auto slot_c, int j) {
    constexpr int slot = decltype(slot_c)::value;
    // blocks past the chunk load nothing (their ring slot is never computed)
    if (j >= nb) return;
    const int gb = cb0 + j;
    const bool ctx = gb < nctx_all;
    const char *kb_ = ctx ? (const char *)a.kp : (const char *)a.kd;
    const char *vb_ = ctx ? (const char *)a.vp : (const char *)a.vd;
    int okm = 0;
#pragma unroll
    for (int p = 0; p < PPT; ++p) {
      int khp, t, dc;
      group_of(p, khp, t, dc);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int tk = 32 * khp + t + 16 * hf;  // key within the block
        int64_t off;
        bool ok;
        if (ctx) {
          off = s_off[(j % WB) * KB + tk];
          ok = off >= 0;
        } else {
          const int key = (gb - nctx_all) * KB + tk;
          ok = key < a.Lt;
          off = (dense_bh + (int64_t)key * a.d_st) * 2;
        }
        // a missing key loads nothing (zeros, masked by its valid bit)
        rk[slot][p][hf] = u32x4{0u, 0u, 0u, 0u};
        rv[slot][p][hf] = u32x4{0u, 0u, 0u, 0u};
        if (ok) {
          rk[slot][p][hf] = ld_nt16(kb_ + off + dc * 16);
          rv[slot][p][hf] = ld_nt16(vb_ + off + dc * 16);
        }
        okm |= (int)ok << (2 * p + hf);
      }
    }
    rok[slot] = okm;
  };
  auto put = [&](auto slot_c, auto buf_c) {
    constexpr int slot = decltype(slot_c)::value;
    constexpr int buf = decltype(buf_c)::value;
#pragma unroll
    for (int p = 0; p < PPT; ++p) {
      if (th + p * NT >= NPC) continue;
      int khp, t, dc;
      group_of(p, khp, t, dc);
      const int k0 = 32 * khp + t;
      *(u32x4 *)&sk[buf][k0 * KROW + dc * 8] = rk[slot][p][0];
      *(u32x4 *)&sk[buf][(k0 + 16) * KROW + dc * 8] = rk[slot][p][1];
      const u32x4 v0 = rv[slot][p][0], v1 = rv[slot][p][1];
      // rows d = 8 dc .. 8 dc + 7: 16-byte group (t >> 2) ^ ((d >> 4) & 3) of the half
      const int pos = 32 * khp + (4 * ((t >> 2) ^ ((dc >> 1) & 3)) + (t & 3)) * 2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = dc * 8 + 2 * e;
        *(uint32_t *)&sv[buf][d * VROW + pos] = __builtin_amdgcn_perm(v1[e], v0[e], 0x05040100u);
        *(uint32_t *)&sv[buf][(d + 1) * VROW + pos] =
            __builtin_amdgcn_perm(v1[e], v0[e], 0x07060302u);
      }
      if (dc == 0) {
        s_valid[buf][k0] = (rok[slot] >> (2 * p)) & 1;
        s_valid[buf][k0 + 16] = (rok[slot] >> (2 * p + 1)) & 1;
      }
    }
  };

  // ---- per-wave online softmax state --------------------------------------
  float m = -INFINITY, l = 0.f;
  f32x4 o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](auto buf_c, int j) {
    constexpr int buf = decltype(buf_c)::value;
    const int gb = cb0 + j;
    const bool dense = gb >= nctx_all;
    float s[8];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const u32x4 ka =
            *(const u32x4 *)&sk[buf][(32 * kh + tt * 16 + l16) * KROW + ds * 32 + 8 * lg];
        acc = mfma16<CT>(ka, qf[ds], acc);
      }
#pragma unroll
      for (int j2 = 0; j2 < 4; ++j2) s[tt * 4 + j2] = acc[j2] * a.scale;
    }
    // validity (key present) and mask (dense keys: the 8 mask values of the
    // lane are loaded together, one dtype switch around all of them)
    int mbits = 0xff;
    if (dense && a.mask) {
      int64_t mi[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key =
            min((gb - nctx_all) * KB + 32 * kh + (e >> 2) * 16 + 4 * lg + (e & 3), a.Lt - 1);
        mi[e] = a.mask_2d ? (int64_t)min(qi, a.NQ - 1) * a.Lt + key : key;
      }
      mbits = 0;
      switch (a.mask_dt) {
        case MTP_F32:
#pragma unroll
          for (int e = 0; e < 8; ++e) mbits |= (int)(((const float *)a.mask)[mi[e]] > 0.5f) << e;
          break;
        case MTP_BF16:
#pragma unroll
          for (int e = 0; e < 8; ++e)
            mbits |= (int)(load_as_f32(a.mask, MTP_BF16, mi[e]) > 0.5f) << e;
          break;
        case MTP_F16:
#pragma unroll
          for (int e = 0; e < 8; ++e)
            mbits |= (int)(load_as_f32(a.mask, MTP_F16, mi[e]) > 0.5f) << e;
          break;
        default:  // U8 / bool
#pragma unroll
          for (int e = 0; e < 8; ++e) mbits |= (int)(((const uint8_t *)a.mask)[mi[e]] > 0) << e;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 32 * kh + (e >> 2) * 16 + 4 * lg + (e & 3);
      if (s_valid[buf][t] == 0 || !((mbits >> e) & 1)) s[e] = -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, s[e]);
    mx = max_over_lane_groups(mx);
    // move the running max (and rescale O, l) only when some query of the
    // wave gained more than kAttnRescale over it
    if (__ballot(mx > m + kAttnRescale) != 0) {
      const float mn = fmaxf(m, mx);
      const float alpha = mn == -INFINITY ? 1.f : __expf(m - mn);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
      m = mn;
    }
    const bool none = m == -INFINITY;  // every key so far masked
    float p[8], ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = none ? 0.f : __expf(s[e] - m);
      ps += p[e];
    }
    l += sum_over_lane_groups(ps);
    // k-slot 8g + 2i + hf of this lane's group is key 4g + i + 16 hf
    u32x4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = pack2<CT>(p[i], p[4 + i]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = dt * 16 + l16;
      const u32x4 va =
          *(const u32x4 *)&sv[buf][d * VROW + 32 * kh + 8 * (lg ^ ((d >> 4) & 3))];
      o[dt] = mfma16<CT>(va, pb, o[dt]);
    }
  };

  // ---- block loop: blocks j + 1 .. j + R in flight while j is multiplied ----
  if (nb > 0) {
    if (cb0 < nctx_all) {
      load_window(0);
      __syncthreads();
    }
    static_for<0, R>([&](auto u) { fetch(u, decltype(u)::value); });
    put(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
    fetch(std::integral_constant<int, 0>{}, R);
    lds_barrier();
    for (int j0 = 0; j0 < nb; j0 += R) {
      static_for<0, R>([&](auto u) {
        constexpr int U = decltype(u)::value;
        const int j = j0 + U;
        if (j >= nb) return;  // uniform: past the chunk
        put(std::integral_constant<int, (U + 1) % R>{}, std::integral_constant<int, (U + 1) & 1>{});
        const int jn = j + 1 + R;
        if (jn % WB == 0 && jn < nb && cb0 + jn < nctx_all) {
          // next page-table window: every fetch of the old one is behind the
          // last barrier
          load_window(jn);
          __syncthreads();
        }
        fetch(std::integral_constant<int, (U + 1) % R>{}, jn);
        if (qwave) compute(std::integral_constant<int, U & 1>{}, j);
        lds_barrier();
      });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads of blocks past the chunk
  }

  // ---- key halves: half 1 hands (m, l, O) to half 0 through LDS -------------
  f32x4 *red_o = (f32x4 *)&sk[0][0];   // [dt][query tile][lane], over both K buffers
  float *red_ml = (float *)&sv[0][0];  // [query tile][lane][2]
  if (kh == 1 && qwave) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) red_o[(dt * 4 + qt) * 64 + lane] = o[dt];
    red_ml[(qt * 64 + lane) * 2] = m;
    red_ml[(qt * 64 + lane) * 2 + 1] = l;
  }
  lds_barrier();
  if (kh == 1 || !qwave) return;
  {
    const float m2 = red_ml[(qt * 64 + lane) * 2], l2 = red_ml[(qt * 64 + lane) * 2 + 1];
    const float mn = fmaxf(m, m2);
    if (mn != -INFINITY) {
      const float e1 = __expf(m - mn), e2 = __expf(m2 - mn);
      l = l * e1 + l2 * e2;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] = o[dt] * e1 + red_o[(dt * 4 + qt) * 64 + lane] * e2;
      m = mn;
    }
  }

  // ---- results: lane (g, r) holds O[q = 16 qt + r][d = 16 dt + 4 g + j] -------
  if (a.nchunks == 1) {
    if (qi < a.NQ) {
      const float inv = 1.f / l;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) attn_store4<CT>(a, b, qi, h, dt * 16 + 4 * lg, o[dt], inv);
    }
    return;
  }
  float *pp = a.part + (((int64_t)bh * a.nchunks + c) * QP + qi) * D;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) *(f32x4 *)(pp + dt * 16 + 4 * lg) = o[dt];
  if (lg == 0) {
    float *mlp = a.ml + (((int64_t)bh * a.nchunks + c) * QP + qi) * 2;
    mlp[0] = m;
    mlp[1] = l;
  }
}

// Chunk merge: workgroup (b*H + h, kAttnMergeQ queries), thread (query, 4
// columns): (M, L, O) <- (M, L, O) (+) (m_c, l_c, O_c) in chunk order, eight
// chunks of loads in flight; out = O / L (every chunk masked: L = 0 and the
// output NaN, as the reference's softmax of an all -inf row). Small
// workgroups spread the partial reads over every CU.
template <int CT, int D>
__global__ void __launch_bounds__(D / 4 * kAttnMergeQ)
attn_merge_kernel(const AttnArgs a) {
  constexpr int C4 = D / 4;
  constexpr int F = 8;
  const int th = threadIdx.x;
  const int qr = th / C4, d4 = th - (th / C4) * C4;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int q = blockIdx.y * kAttnMergeQ + qr;
  if (q >= a.NQ) return;
  const int QP = ((a.NQ + 15) >> 4) * 16;
  const float *pb = a.part + ((int64_t)bh * a.nchunks * QP + q) * D + d4 * 4;
  const float *mlb = a.ml + ((int64_t)bh * a.nchunks * QP + q) * 2;
  float M = -INFINITY, L = 0.f;
  f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < a.nchunks; c0 += F) {
    f32x4 po[F];
    f32x2 pml[F];
    static_for<0, F>([&](auto f) {
      constexpr int FI = decltype(f)::value;
      const int cc = min(c0 + FI, a.nchunks - 1);
      pml[FI] = *(const f32x2 *)(mlb + (int64_t)cc * QP * 2);
      po[FI] = *(const f32x4 *)(pb + (int64_t)cc * QP * D);
    });
    static_for<0, F>([&](auto f) {
      constexpr int FI = decltype(f)::value;
      if (c0 + FI < a.nchunks) {
        const float Mn = fmaxf(M, pml[FI][0]);
        if (Mn != -INFINITY) {
          const float ea = __expf(M - Mn), eb = __expf(pml[FI][0] - Mn);
          L = L * ea + pml[FI][1] * eb;
          O = O * ea + po[FI] * eb;
          M = Mn;
        }
      }
    });
  }
  attn_store4<CT>(a, b, q, h, d4 * 4, O, 1.f / L);
}

// Fallback for shapes the MFMA kernel does not take (fp32 q / k / v, head
// dims other than 64 / 128, more than 64 queries): one wave per (b, query,
// h), keys in order, lanes split d. Same semantics and key sources.
__device__ __forceinline__ float load_kv_f32(const void *p, int dt, int64_t i) {
  if (dt == MTP_FP8E4M3) return __builtin_amdgcn_cvt_f32_fp8((uint32_t)((const uint8_t *)p)[i], 0);
  return load_as_f32(p, dt, i);
}

__global__ void __launch_bounds__(64) attn_generic_kernel(const AttnArgs a, int D, int ct) {
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int qi = blockIdx.y;
  const int64_t qoff = (int64_t)b * a.q_sb + (int64_t)qi * a.q_sn + (int64_t)h * a.q_sh;
  float qv[4], ov[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    qv[i] = d < D ? load_as_f32(a.q, ct, qoff + d) : 0.f;
    ov[i] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int total = a.Lc + a.Lt;
  // K / V in q's dtype, or fp8 with per-head scales (scores and values are
  // scaled in fp32 after the dot products)
  const int kdt = a.kv_fp8 ? MTP_FP8E4M3 : ct;
  const float ks = a.kscale ? a.kscale[h] : 1.f, vs = a.vscale ? a.vscale[h] : 1.f;
  for (int t = 0; t < total; ++t) {
    int64_t off;
    const void *kb, *vb;
    bool ok = true;
    if (t < a.Lc) {
      const int page = a.table[(int64_t)b * a.ld_tab + t];
      ok = page >= 0 && page < a.npages;
      off = (int64_t)(ok ? page : 0) * a.p_sp + (int64_t)b * a.p_sb + (int64_t)h * a.p_sh +
            (int64_t)(t % a.page_size) * D;
      kb = a.kp;
      vb = a.vp;
    } else {
      const int key = t - a.Lc;
      off = (int64_t)b * a.d_sb + (int64_t)h * a.d_sh + (int64_t)key * a.d_st;
      kb = a.kd;
      vb = a.vd;
      if (a.mask) ok = mask_on(a.mask, a.mask_dt, a.mask_2d ? (int64_t)qi * a.Lt + key : key);
    }
    float sp = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      if (d < D) sp += qv[i] * load_kv_f32(kb, kdt, off + d);
    }
#pragma unroll
    for (int w = 32; w > 0; w >>= 1) sp += __shfl_xor(sp, w, 64);
    const float s = ok ? sp * ks * a.scale : -INFINITY;
    const float mn = fmaxf(m, s);
    const bool none = mn == -INFINITY;
    const float alpha = none ? 1.f : __expf(m - mn);
    const float p = none ? 0.f : __expf(s - mn);
    l = l * alpha + p;
    m = mn;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      ov[i] = ov[i] * alpha + (d < D ? p * (load_kv_f32(vb, kdt, off + d) * vs) : 0.f);
    }
  }
  const int64_t ooff = (int64_t)b * a.o_sb + (int64_t)qi * a.o_sn + (int64_t)h * a.o_sh;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < D) store_from_f32(a.out, ct, ooff + d, ov[i] / l);
  }
}

// Fallback for head dims above 256 (the tree monolith's single-head shape,
// D = the hidden size): one 256-thread workgroup per (b, query, head); each
// thread owns q and the output accumulator at d = t, t + 256, ...; the dot
// product of every key is reduced over the workgroup (wave shuffles, then a
// double-buffered LDS slot per wave, one barrier per key).
template <int NV>
__global__ void __launch_bounds__(256) attn_generic_wide_kernel(const AttnArgs a, int D, int ct) {
  __shared__ float red[2][4];
  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int qi = blockIdx.y;
  const int64_t qoff = (int64_t)b * a.q_sb + (int64_t)qi * a.q_sn + (int64_t)h * a.q_sh;
  float qv[NV], ov[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = th + 256 * i;
    qv[i] = d < D ? load_as_f32(a.q, ct, qoff + d) : 0.f;
    ov[i] = 0.f;
  }
  const int kdt = a.kv_fp8 ? MTP_FP8E4M3 : ct;
  const float ks = a.kscale ? a.kscale[h] : 1.f, vs = a.vscale ? a.vscale[h] : 1.f;
  float m = -INFINITY, l = 0.f;
  const int total = a.Lc + a.Lt;
  for (int t = 0; t < total; ++t) {
    int64_t off;
    const void *kb, *vb;
    bool ok = true;
    if (t < a.Lc) {
      const int page = a.table[(int64_t)b * a.ld_tab + t];
      ok = page >= 0 && page < a.npages;
      off = (int64_t)(ok ? page : 0) * a.p_sp + (int64_t)b * a.p_sb + (int64_t)h * a.p_sh +
            (int64_t)(t % a.page_size) * D;
      kb = a.kp;
      vb = a.vp;
    } else {
      const int key = t - a.Lc;
      off = (int64_t)b * a.d_sb + (int64_t)h * a.d_sh + (int64_t)key * a.d_st;
      kb = a.kd;
      vb = a.vd;
      if (a.mask) ok = mask_on(a.mask, a.mask_dt, a.mask_2d ? (int64_t)qi * a.Lt + key : key);
    }
    float sp = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = th + 256 * i;
      if (d < D) sp += qv[i] * load_kv_f32(kb, kdt, off + d);
    }
#pragma unroll
    for (int w = 32; w > 0; w >>= 1) sp += __shfl_xor(sp, w, 64);
    if (lane == 0) red[t & 1][wave] = sp;
    __syncthreads();
    sp = (red[t & 1][0] + red[t & 1][1]) + (red[t & 1][2] + red[t & 1][3]);
    const float s = ok ? sp * ks * a.scale : -INFINITY;
    const float mn = fmaxf(m, s);
    const bool none = mn == -INFINITY;
    const float alpha = none ? 1.f : __expf(m - mn);
    const float p = none ? 0.f : __expf(s - mn);
    l = l * alpha + p;
    m = mn;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = th + 256 * i;
      ov[i] = ov[i] * alpha + (d < D ? p * (load_kv_f32(vb, kdt, off + d) * vs) : 0.f);
    }
  }
  const int64_t ooff = (int64_t)b * a.o_sb + (int64_t)qi * a.o_sn + (int64_t)h * a.o_sh;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = th + 256 * i;
    if (d < D) store_from_f32(a.out, ct, ooff + d, ov[i] / l);
  }
}

}  // namespace mtp
