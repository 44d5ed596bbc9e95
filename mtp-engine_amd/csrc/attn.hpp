// Single-query-per-row softmax attention for gfx950: the tree / paged
// attention family and the multi-query tree-verify step built from them.
//
// One launch covers, for every (batch b, head h), a set of NQ queries
// q[b, n, h, :] attending under one softmax to
//   * Lc context keys of a paged cache: key t is pages[table[b, t], b, h,
//     t % page_size, :] (pages [P, B, H, page_size, D]), and
//   * Lt dense keys k[b, h, t, :] (arbitrary element strides), masked by a
//     1-D mask [Lt] (shared by all queries) or a 2-D mask [NQ, Lt]
//     (value > 0.5 = attend; masked scores are -inf, so a query with every
//     key masked yields NaN like the reference's eager softmax).
//
// Workgroup (b*H + h, chunk c): QT waves, wave w owns queries 16w..16w+15.
// Keys go by blocks of 32: the workgroup stages K (natural layout) and V
// (transposed, [d][t]) of the next block into a double-buffered LDS area
// while the current block is multiplied. Per wave and block:
//   S^T[t][q] = K[t] . Q[q]       MFMA 16x16x32, A = K rows, B = Q^T (regs)
//   online softmax per query (the accumulator lane of q holds 8 keys:
//   t = 4g + j and 16 + 4g + j, so the row max / sum are two xor-shuffles)
//   O^T[d][q] += V^T[d][t] P^T[t][q]   the S^T accumulators, rounded to the
//   MFMA input type, are the B operand as they are (k-slots of lane group g
//   are keys {4g..4g+3, 16+4g..16+4g+3}); A = V^T from LDS.
// Context chunks are split over blockIdx.y; the dense keys ride with the
// last chunk. With more than one chunk every workgroup publishes (m, l, O)
// and the last to arrive for (b, h) merges them in chunk order.
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

template <int CT, int D, int QT>
__global__ void __launch_bounds__(QT * 64)
attn_kernel(const AttnArgs a) {
  constexpr int NT = QT * 64;
  constexpr int QP = QT * 16;
  constexpr int KB = 32;               // keys per block
  constexpr int DC = D / 8;            // 16-byte chunks per key row
  constexpr int KROW = D + 8;          // K row in LDS (elements)
  constexpr int VROW = KB + 8;         // V^T row in LDS (elements)
  constexpr int NCH = KB * DC;         // 16-byte chunks of K (or V) per block
  constexpr int CPT = (NCH + NT - 1) / NT;
  constexpr int DS = D / 32;           // MFMA k-steps over d
  constexpr int DT = D / 16;           // O^T tiles
  __shared__ __attribute__((aligned(16))) uint16_t sk[2][KB * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t sv[2][D * VROW];
  __shared__ int s_valid[2][KB];
  __shared__ int s_flag;
  __shared__ float s_wt[QP][kAttnMaxChunks];

  const int th = threadIdx.x;
  const int lane = th & 63;
  const int wave = th >> 6;
  const int lg = lane >> 4;
  const int l16 = lane & 15;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int c = blockIdx.y;

  const int nctx_all = (a.Lc + KB - 1) / KB;
  const int cb0 = c * a.chunk_blocks;
  const int nctx = max(0, min(nctx_all, cb0 + a.chunk_blocks) - cb0);
  const int ndense = (c == a.nchunks - 1) ? (a.Lt + KB - 1) / KB : 0;
  const int nb = nctx + ndense;

  const uint16_t *qbase = (const uint16_t *)a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh;
  const int qi = wave * 16 + l16;  // this lane's query in the accumulator layout
  u32x4 qf[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s)
    qf[s] = qi < a.NQ ? *(const u32x4 *)(qbase + (int64_t)qi * a.q_sn + s * 32 + 8 * lg)
                      : u32x4{0u, 0u, 0u, 0u};

  // ---- staging of one block (registers <- global) ----------------------
  u32x4 rk[CPT], rv[CPT];
  bool rval[CPT];
  auto fetch = [&](int blk) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int cid = th + i * NT;
      const int t = cid / DC, dc = cid - (cid / DC) * DC;
      bool ok = cid < NCH;
      const uint16_t *kptr = nullptr, *vptr = nullptr;
      if (blk < nctx) {
        const int tok = (cb0 + blk) * KB + t;
        ok = ok && tok < a.Lc;
        const int page = ok ? a.table[(int64_t)b * a.ld_tab + tok] : 0;
        ok = ok && page >= 0 && page < a.npages;
        const int64_t off = (int64_t)page * a.p_sp + (int64_t)b * a.p_sb + (int64_t)h * a.p_sh +
                            (int64_t)(tok % a.page_size) * D + dc * 8;
        kptr = (const uint16_t *)a.kp + off;
        vptr = (const uint16_t *)a.vp + off;
      } else {
        const int key = (blk - nctx) * KB + t;
        ok = ok && key < a.Lt;
        const int64_t off =
            (int64_t)b * a.d_sb + (int64_t)h * a.d_sh + (int64_t)key * a.d_st + dc * 8;
        kptr = (const uint16_t *)a.kd + off;
        vptr = (const uint16_t *)a.vd + off;
      }
      rval[i] = ok;
      rk[i] = ok ? *(const u32x4 *)kptr : u32x4{0u, 0u, 0u, 0u};
      rv[i] = ok ? *(const u32x4 *)vptr : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto put = [&](int buf) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int cid = th + i * NT;
      if (cid >= NCH) continue;
      const int t = cid / DC, dc = cid - (cid / DC) * DC;
      *(u32x4 *)&sk[buf][t * KROW + dc * 8] = rk[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sv[buf][(dc * 8 + 2 * e) * VROW + t] = (uint16_t)(rv[i][e] & 0xffffu);
        sv[buf][(dc * 8 + 2 * e + 1) * VROW + t] = (uint16_t)(rv[i][e] >> 16);
      }
      if (dc == 0) s_valid[buf][t] = rval[i];
    }
  };

  // ---- per-wave online softmax state --------------------------------------
  float m = -INFINITY, l = 0.f;
  f32x4 o[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf, int blk) {
    float s[8];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const u32x4 ka = *(const u32x4 *)&sk[buf][(tt * 16 + l16) * KROW + ds * 32 + 8 * lg];
        acc = mfma16<CT>(ka, qf[ds], acc);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) s[tt * 4 + j] = acc[j] * a.scale;
    }
    // validity (key present) and mask (dense keys)
    const bool dense = blk >= nctx;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = (e >> 2) * 16 + 4 * lg + (e & 3);
      bool ok = s_valid[buf][t] != 0;
      if (ok && dense && a.mask) {
        const int key = (blk - nctx) * KB + t;
        const int64_t mi = a.mask_2d ? (int64_t)min(qi, a.NQ - 1) * a.Lt + key : key;
        ok = mask_on(a.mask, a.mask_dt, mi);
      }
      if (!ok) s[e] = -INFINITY;
    }
    float mx = s[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, s[e]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    const bool none = mn == -INFINITY;  // every key so far masked
    const float alpha = none ? 1.f : __expf(m - mn);
    float p[8], ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p[e] = none ? 0.f : __expf(s[e] - mn);
      ps += p[e];
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mn;
    u32x4 pb;
    pb[0] = pack2<CT>(p[0], p[1]);
    pb[1] = pack2<CT>(p[2], p[3]);
    pb[2] = pack2<CT>(p[4], p[5]);
    pb[3] = pack2<CT>(p[6], p[7]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      o[dt] *= alpha;
      const uint16_t *vr = &sv[buf][(dt * 16 + l16) * VROW + 4 * lg];
      const uint2 lo = *(const uint2 *)vr;
      const uint2 hi = *(const uint2 *)(vr + 16);
      const u32x4 va = u32x4{lo.x, lo.y, hi.x, hi.y};
      o[dt] = mfma16<CT>(va, pb, o[dt]);
    }
  };

  // ---- block loop: fetch j + 1 while j is multiplied ------------------------
  if (nb > 0) fetch(0);
  for (int j = 0; j < nb; ++j) {
    put(j & 1);
    if (j + 1 < nb) fetch(j + 1);
    __syncthreads();
    compute(j & 1, j);
  }

  // ---- results -------------------------------------------------------------
  // Lane (g, r) holds O[q = 16 * wave + r][d = 16 * dt + 4 * g + j].
  auto store_out = [&](int q, int d, f32x4 v, float inv) {
    uint16_t *op = (uint16_t *)a.out + (int64_t)b * a.o_sb + (int64_t)q * a.o_sn +
                   (int64_t)h * a.o_sh + d;
    uint2 pk;
    pk.x = pack2<CT>(v[0] * inv, v[1] * inv);
    pk.y = pack2<CT>(v[2] * inv, v[3] * inv);
    *(uint2 *)op = pk;
  };
  if (a.nchunks == 1) {
    if (qi < a.NQ) {
      const float inv = 1.f / l;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) store_out(qi, dt * 16 + 4 * lg, o[dt], inv);
    }
    return;
  }
  const int64_t pbase = ((int64_t)bh * a.nchunks + c) * QP;
  const uint32_t part_bytes = (uint32_t)a.nchunks * QP * D * 4u;
  const __amdgpu_buffer_rsrc_t prs =
      make_rsrc(a.part + (int64_t)bh * a.nchunks * QP * D, part_bytes);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const uint32_t off = (uint32_t)((c * QP + qi) * D + dt * 16 + 4 * lg) * 4u;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[dt]), prs, off, 0, kSc1);
  }
  if (lg == 0) {
    pub_f32(a.ml + (pbase + qi) * 2, m);
    pub_f32(a.ml + (pbase + qi) * 2 + 1, l);
  }
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = ticket_add(a.ticket + bh) == (unsigned)(a.nchunks - 1);
  __syncthreads();
  if (!s_flag) return;
  // Merge the chunks in chunk order: out = sum_c e^(m_c - M) O_c / sum_c e^(m_c - M) l_c
  // (every chunk masked: M = -inf and the weights are NaN, as the reference's
  // softmax of an all -inf row). Per-query weights first, then the outputs.
  const float *mlb = a.ml + (int64_t)bh * a.nchunks * QP * 2;
  if (th < QP) {
    float M = -INFINITY;
    for (int cc = 0; cc < a.nchunks; ++cc) M = fmaxf(M, get_f32(mlb + ((int64_t)cc * QP + th) * 2));
    float L = 0.f;
    for (int cc = 0; cc < a.nchunks; ++cc) {
      const float w = __expf(get_f32(mlb + ((int64_t)cc * QP + th) * 2) - M);
      L += w * get_f32(mlb + ((int64_t)cc * QP + th) * 2 + 1);
      s_wt[th][cc] = w;
    }
    const float inv = 1.f / L;
    for (int cc = 0; cc < a.nchunks; ++cc) s_wt[th][cc] *= inv;
  }
  __syncthreads();
  for (int item = th; item < QP * DC * 2; item += NT) {
    const int q = item / (DC * 2);
    const int d = (item - q * DC * 2) * 4;
    if (q >= a.NQ) continue;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int cc = 0; cc < a.nchunks; ++cc) {
      const uint32_t off = (uint32_t)((cc * QP + q) * D + d) * 4u;
      acc += s_wt[q][cc] *
             __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, kSc1));
    }
    store_out(q, d, acc, 1.f);
  }
  if (th == 0) ticket_reset(a.ticket + bh);
}

// Fallback for shapes the MFMA kernel does not take (fp32 q / k / v, head
// dims other than 64 / 128, more than 64 queries): one wave per (b, query,
// h), keys in order, lanes split d. Same semantics and key sources.
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
      if (d < D) sp += qv[i] * load_as_f32(kb, ct, off + d);
    }
#pragma unroll
    for (int w = 32; w > 0; w >>= 1) sp += __shfl_xor(sp, w, 64);
    const float s = ok ? sp * a.scale : -INFINITY;
    const float mn = fmaxf(m, s);
    const bool none = mn == -INFINITY;
    const float alpha = none ? 1.f : __expf(m - mn);
    const float p = none ? 0.f : __expf(s - mn);
    l = l * alpha + p;
    m = mn;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      ov[i] = ov[i] * alpha + (d < D ? p * load_as_f32(vb, ct, off + d) : 0.f);
    }
  }
  const int64_t ooff = (int64_t)b * a.o_sb + (int64_t)qi * a.o_sn + (int64_t)h * a.o_sh;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < D) store_from_f32(a.out, ct, ooff + d, ov[i] / l);
  }
}

}  // namespace mtp
