// Wide-tile attention for gfx950: 33 .. 64 queries per (batch, head), head
// dim 128, 16-bit q / K / V. Same semantics, key sources, chunking and
// partial format as attn_kernel (attn.hpp); a different decomposition that
// moves a third as many LDS bytes per key and no K / V bytes through VGPRs.
//
// Workgroup (b*H + h, chunk c) of 8 waves takes the chunk's 64-key blocks
// two at a time (a step of 128 keys). Wave w owns query group qg = w & 1
// (queries 32 qg .. + 31) and key group kg = w >> 1 (keys 32 kg .. + 31 of
// every step), so every K row and V row is read from LDS by two waves
// (16-query tiles need four).
//   * K and V rows go HBM -> LDS by non-temporal buffer loads with the LDS
//     bit (no registers, no VALU): one instruction fills 1 KB = 4 rows of 256 B,
//     lane i the 16-byte position i % 16 of row i / 16, which holds the
//     row's chunk (i % 16) ^ swz(row). Two step buffers (64 KB each): step
//     s + 1 lands while step s is multiplied. Keys that are missing (past
//     the chunk, no page, past Lt) use an out-of-range offset and read 0.
//   * S^T[t][q] = K[t] . Q[q]    v_mfma_f32_32x32x16: A = K rows (one
//     16-byte LDS read per lane and k-step), B = Q^T (registers, loaded
//     once). Lane l then holds 16 keys t = 8 (v / 4) + 4 (l / 32) + v % 4 of
//     query l % 32: the row max / sum are one lane swap (l ^ 32).
//   * O^T[d][q] += V^T[d][t] P^T[t][q]: B = the S^T accumulators as they
//     are (k-step s2 holds keys 16 s2 + 8 (u / 4) + 4 (l / 32) + u % 4 in
//     slot 8 (l / 32) + u), A = V^T in the same key order, read from the
//     row-major V rows with ds_read_b64_tr_b16: in each 16-lane group, lane
//     j reads 4 d of row key0 + j / 4 and receives 4 keys of d = j.
//   * online softmax per query and key group (the running max moves only
//     when a step's max exceeds it by more than kAttnRescale); at the end
//     the four key groups of a query group merge through LDS, each wave
//     merging one 32-d tile in a fixed order.
// swz(r) = 4 (r % 4) + (r / 4) % 4 keeps both read patterns (16
// consecutive rows of one chunk; 4 consecutive rows x 4 consecutive
// chunks) on distinct banks.
#pragma once

#include "attn.hpp"

namespace mtp {

typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int kAttn2Steps = 2;                         // step buffers
constexpr int kAttn2Buf = 2 * 128 * 256;               // K + V bytes of a step (D 128)
constexpr int kAttn2Lds = kAttn2Steps * kAttn2Buf + kAttnTableWindow * 4 + kAttn2Steps * 128;

template <int CT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (CT == MTP_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ int attn2_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// K / V rows are read once per launch: non-temporal copies (tree-verify
// attention + linear 33.5-34.5 -> 32.8-33.6 us per step on one box).
__device__ __forceinline__ void attn2_dma16(__amdgpu_buffer_rsrc_t r, unsigned char *lds,
                                            uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, 0, 0, 2);
#else
  (void)r; (void)lds; (void)voff;
#endif
}

__device__ __forceinline__ uint64_t attn2_tr16(const unsigned char *p) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint64_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                          (__attribute__((address_space(3))) s16x4 *)p));
#else
  (void)p;
  return 0;
#endif
}

template <int CT>
__global__ void __launch_bounds__(512, 1) attn2_kernel(const AttnArgs a) {
  constexpr int D = 128;
  constexpr int RB = 2 * D;             // bytes of a key row
  constexpr int SK = 128;               // keys per step
  constexpr int KBY = SK * RB;          // K bytes of a step
  constexpr int KB = kAttnBlock;        // 64-key blocks (chunking unit)
  constexpr int TW = kAttnTableWindow;  // context keys of the page window
  constexpr int WB = TW / KB;           // blocks per window
  constexpr uint32_t kNoKey = 0xffffffffu;
  static_assert(KB == 64 && WB % 2 == 0, "steps pair whole blocks inside a window");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
  uint32_t *const s_off = (uint32_t *)(lds + kAttn2Steps * kAttn2Buf);  // [TW]
  uint8_t *const s_valid = (uint8_t *)(s_off + TW);                     // [steps][SK]

  const int th = threadIdx.x, lane = th & 63;
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
  const int qg = wave & 1, kg = wave >> 1;
  const int hi = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int c = blockIdx.y;
  const int nctx = (a.Lc + KB - 1) / KB;
  const int ntot = nctx + (a.Lt + KB - 1) / KB;
  const int cb0 = c * a.chunk_blocks;
  const int nb = max(0, min(ntot, cb0 + a.chunk_blocks) - cb0);  // blocks of the chunk
  const int nsteps = (nb + 1) >> 1;
  const int QP = ((a.NQ + 15) >> 4) * 16;

  // ---- Q^T operand of the query group: lane l holds q = 32 qg + l % 32,
  // d = 16 ks + 8 (l / 32) .. + 7
  const int qi = 32 * qg + l32;
  const uint16_t *qrow =
      (const uint16_t *)a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)qi * a.q_sn;
  u32x4 qf[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    qf[ks] = qi < a.NQ ? *(const u32x4 *)(qrow + 16 * ks + 8 * hi) : u32x4{0u, 0u, 0u, 0u};

  // ---- key sources: pages (byte offsets from the window) and dense rows
  const __amdgpu_buffer_rsrc_t kprs = make_rsrc(a.kp, (uint32_t)((int64_t)a.npages * a.p_sp * 2));
  const __amdgpu_buffer_rsrc_t vprs = make_rsrc(a.vp, (uint32_t)((int64_t)a.npages * a.p_sp * 2));
  const int64_t dense_bh = (int64_t)b * a.d_sb + (int64_t)h * a.d_sh;
  const uint32_t dbytes = a.Lt > 0 ? (uint32_t)(((int64_t)(a.Lt - 1) * a.d_st + D) * 2) : 0u;
  const __amdgpu_buffer_rsrc_t kdrs =
      make_rsrc(a.kd ? (const uint16_t *)a.kd + dense_bh : nullptr, dbytes);
  const __amdgpu_buffer_rsrc_t vdrs =
      make_rsrc(a.vd ? (const uint16_t *)a.vd + dense_bh : nullptr, dbytes);
  const int64_t page_bh = (int64_t)b * a.p_sb + (int64_t)h * a.p_sh;

  // page-table window: s_off[i] for the keys of blocks w0 .. w0 + WB - 1
  auto load_window = [&](int w0) {
#pragma unroll
    for (int i = th; i < TW; i += 512) {
      const int tok = (cb0 + w0) * KB + i;
      uint32_t off = kNoKey;
      if (tok < a.Lc) {
        const int page = a.table[(int64_t)b * a.ld_tab + tok];
        if (page >= 0 && page < a.npages)
          off = (uint32_t)(((int64_t)page * a.p_sp + page_bh + (int64_t)(tok % a.page_size) * D) * 2);
      }
      s_off[i] = off;
    }
  };

  // ---- step s (blocks 2 s, 2 s + 1 of the chunk) into buffer `buf`: four K
  // and four V copy instructions per wave, rows 4 n .. 4 n + 3 with
  // n = wave + 8 u (u = 0 .. 3); every wave issues all eight
  const int drow = lane >> 4, dpos = lane & 15;
  auto issue = [&](int s, int buf) {
    unsigned char *kb = lds + buf * kAttn2Buf;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int n = wave + 8 * u;
      const int r = 4 * n + drow;            // key row of the step
      const int jb = 2 * s + (n >> 4);       // block of the chunk (uniform per instruction)
      const int gb = cb0 + jb;
      const bool ctx = gb < nctx;
      const uint32_t cho = 16u * (uint32_t)(dpos ^ attn2_swz(r));
      uint32_t voff = kOOB;
      if (jb < nb) {
        if (ctx) {
          const uint32_t o = s_off[(jb % WB) * KB + (r & 63)];
          if (o != kNoKey) voff = o + cho;
        } else {
          const int key = (gb - nctx) * KB + (r & 63);
          if (key < a.Lt) voff = (uint32_t)((int64_t)key * a.d_st * 2) + cho;
        }
      }
      if (dpos == 0) s_valid[buf * SK + r] = voff != kOOB;
      if (ctx) {
        attn2_dma16(kprs, kb + n * 1024, voff);
        attn2_dma16(vprs, kb + KBY + n * 1024, voff);
      } else {
        attn2_dma16(kdrs, kb + n * 1024, voff);
        attn2_dma16(vdrs, kb + KBY + n * 1024, voff);
      }
    }
  };

  // ---- per-wave online softmax state: lane l, query 32 qg + l % 32
  float m = -INFINITY, lsum = 0.f;
  f32x16 o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[dt][v] = 0.f;

  auto compute = [&](int s, int buf) {
    const unsigned char *kb = lds + buf * kAttn2Buf;
    const unsigned char *vb = kb + KBY;
    const int jb = 2 * s + (kg >> 1);  // the wave's 32 keys sit in this block
    if (jb >= nb) return;              // wave-uniform: past the chunk
    const int gb = cb0 + jb;
    // S^T: A = K rows 32 kg + l % 32, chunk 2 ks + l / 32
    const int kr = 32 * kg + l32;
    const unsigned char *krow = kb + kr * RB;
    const int ksw = attn2_swz(kr);
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.f;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const u32x4 ka = *(const u32x4 *)(krow + 16 * ((2 * ks + hi) ^ ksw));
      acc = mfma32<CT>(ka, qf[ks], acc);
    }
    // key of slot v: 32 kg + 8 (v / 4) + 4 hi + v % 4 (4 runs of 4)
    uint32_t vbits[4];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      vbits[r4] = *(const uint32_t *)(s_valid + buf * SK + 32 * kg + 8 * r4 + 4 * hi);
    int mbits = 0xffff;
    if (gb >= nctx && a.mask) {
      // mask element of slot v: row min(q, NQ - 1) (2-D) and key
      // min(kbase + 8 (v / 4) + v % 4, Lt - 1)
      const int kbase = (gb - nctx) * KB + ((32 * kg) & 63) + 4 * hi;
      const int64_t qrow_m = a.mask_2d ? (int64_t)min(qi, a.NQ - 1) * a.Lt : 0;
      const int kmax = a.Lt - 1;
      mbits = 0;
      switch (a.mask_dt) {
        case MTP_F32: {
          const float *mp = (const float *)a.mask + qrow_m;
#pragma unroll
          for (int v = 0; v < 16; ++v)
            mbits |= (int)(mp[min(kbase + 8 * (v >> 2) + (v & 3), kmax)] > 0.5f) << v;
          break;
        }
        case MTP_BF16:
        case MTP_F16: {
          const uint16_t *mp = (const uint16_t *)a.mask + qrow_m;
          const int dt_ = a.mask_dt;
#pragma unroll
          for (int v = 0; v < 16; ++v)
            mbits |= (int)(load_as_f32(mp, dt_, min(kbase + 8 * (v >> 2) + (v & 3), kmax)) > 0.5f)
                     << v;
          break;
        }
        default: {  // U8 / bool
          const uint8_t *mp = (const uint8_t *)a.mask + qrow_m;
#pragma unroll
          for (int v = 0; v < 16; ++v)
            mbits |= (int)(mp[min(kbase + 8 * (v >> 2) + (v & 3), kmax)] > 0) << v;
        }
      }
    }
    // scores in place of the accumulator
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const bool ok = ((vbits[v >> 2] >> (8 * (v & 3))) & 0xffu) != 0 && ((mbits >> v) & 1);
      acc[v] = ok ? acc[v] * a.scale : -INFINITY;
    }
    float mx = acc[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mx = fmaxf(mx, acc[v]);
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                       false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    if (__ballot(mx > m + kAttnRescale) != 0) {
      const float mn = fmaxf(m, mx);
      const float alpha = mn == -INFINITY ? 1.f : __expf(m - mn);
      lsum *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) o[dt] *= alpha;
      m = mn;
    }
    const bool none = m == -INFINITY;  // every key so far masked
    float ps = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      acc[v] = none ? 0.f : __expf(acc[v] - m);
      ps += acc[v];
    }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps),
                                                       false, false);
      lsum += __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    u32x4 pb[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i) pb[s2][i] = pack2<CT>(acc[8 * s2 + 2 * i], acc[8 * s2 + 2 * i + 1]);
    // V^T tiles by transpose reads: 16-lane group G = l / 16 reads rows
    // key0 + j / 4 (key0 = 32 kg + 16 s2 + 4 (G / 2), + 8 for slots 4 .. 7),
    // elements 32 dt + 16 (G % 2) + 4 (j % 4) .. + 3
    const int G = lane >> 4, j = lane & 15;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int ra = 32 * kg + 16 * s2 + 4 * (G >> 1) + (j >> 2), rb = ra + 8;
      const unsigned char *pa = vb + ra * RB + 8 * (j & 1);
      const unsigned char *pbp = vb + rb * RB + 8 * (j & 1);
      const int swa = attn2_swz(ra), swb = attn2_swz(rb);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        const int ch = 4 * dt + 2 * (G & 1) + ((j & 3) >> 1);
        const uint64_t lo = attn2_tr16(pa + 16 * (ch ^ swa));
        const uint64_t hi8 = attn2_tr16(pbp + 16 * (ch ^ swb));
        u32x4 va;
        va[0] = (uint32_t)lo;
        va[1] = (uint32_t)(lo >> 32);
        va[2] = (uint32_t)hi8;
        va[3] = (uint32_t)(hi8 >> 32);
        o[dt] = mfma32<CT>(va, pb[s2], o[dt]);
      }
    }
  };

  // ---- step loop: step s + 1 lands while step s is multiplied
  if (nsteps > 0) {
    if (cb0 < nctx) {
      load_window(0);
      __syncthreads();
    }
    // Q in registers before the copies go out (its wait then counts no copy)
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) asm volatile("" ::"v"(qf[ks]));
    // One step in flight: step s + 1 goes out once step s has landed, into
    // the buffer step s - 1 was multiplied from (every wave is past that).
    // Two steps in flight per workgroup (128 KB) measured slower: step 0
    // then lands only when most of the grid's 2 x 14 MB has been served.
    issue(0, 0);
    for (int s = 0; s < nsteps; ++s) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (s + 1 < nsteps) {
        if (((2 * (s + 1)) % WB) == 0 && cb0 + 2 * (s + 1) < nctx) {
          load_window(2 * (s + 1));
          __syncthreads();
        }
        issue(s + 1, (s + 1) & 1);
      }
      compute(s, s & 1);
    }
  }
  __syncthreads();  // step buffers free for the key-group merge

  // ---- key groups of a query group merge through LDS: wave (qg, kg)
  // publishes (m, l) and its O^T tiles dt != kg, then merges tile dt = kg
  // over kg' = 0 .. 3 in order
  float *const red_o = (float *)lds;                                 // [qg][dt][kg'][v][lane]
  float *const red_ml = (float *)(lds + 2 * (D / 32) * 4 * 16 * 64 * 4);  // [qg][kg][lane][2]
  red_ml[((qg * 4 + kg) * 64 + lane) * 2] = m;
  red_ml[((qg * 4 + kg) * 64 + lane) * 2 + 1] = lsum;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    if (dt == kg) continue;
#pragma unroll
    for (int v = 0; v < 16; ++v)
      red_o[(((qg * (D / 32) + dt) * 4 + kg) * 16 + v) * 64 + lane] = o[dt][v];
  }
  __syncthreads();
  float mk[4], lk[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    mk[k] = red_ml[((qg * 4 + k) * 64 + lane) * 2];
    lk[k] = red_ml[((qg * 4 + k) * 64 + lane) * 2 + 1];
  }
  const float M = fmaxf(fmaxf(mk[0], mk[1]), fmaxf(mk[2], mk[3]));
  float L = 0.f;
  f32x16 O;
#pragma unroll
  for (int v = 0; v < 16; ++v) O[v] = 0.f;
  const int dt = kg;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float e = M == -INFINITY ? 0.f : __expf(mk[k] - M);
    L += lk[k] * e;
    if (k == kg) {
      // own tile from registers (static index: a runtime one would spill o)
#pragma unroll
      for (int d2 = 0; d2 < D / 32; ++d2)
        if (d2 == kg) {
#pragma unroll
          for (int v = 0; v < 16; ++v) O[v] += o[d2][v] * e;
        }
    } else {
#pragma unroll
      for (int v = 0; v < 16; ++v)
        O[v] += red_o[(((qg * (D / 32) + dt) * 4 + k) * 16 + v) * 64 + lane] * e;
    }
  }
  if (qi >= a.NQ) return;
  // lane holds O^T[d][q]: d = 32 dt + 8 (v / 4) + 4 hi + v % 4, q = qi
  if (a.nchunks == 1) {
    const float inv = 1.f / L;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      f32x4 t4 = f32x4{O[4 * r4], O[4 * r4 + 1], O[4 * r4 + 2], O[4 * r4 + 3]};
      attn_store4<CT>(a, b, qi, h, 32 * dt + 8 * r4 + 4 * hi, t4, inv);
    }
    return;
  }
  float *pp = a.part + (((int64_t)bh * a.nchunks + c) * QP + qi) * D + 32 * dt + 4 * hi;
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4)
    *(f32x4 *)(pp + 8 * r4) = f32x4{O[4 * r4], O[4 * r4 + 1], O[4 * r4 + 2], O[4 * r4 + 3]};
  if (kg == 0 && hi == 0) {
    float *mlp = a.ml + (((int64_t)bh * a.nchunks + c) * QP + qi) * 2;
    mlp[0] = M;
    mlp[1] = L;
  }
}

}  // namespace mtp
