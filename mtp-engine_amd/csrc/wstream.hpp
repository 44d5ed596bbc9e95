// Skinny-M weight-streaming GEMM for gfx950: the engine of the RMSNorm ->
// linear family and of the verify lm_head pass.
//
// Problem: y[M, N] = epilogue( x[M, K] . W[N, K]^T ) with at most 64 rows of
// x per row chunk (tree-node counts / verify rows) and large N, K. W
// dominates the traffic and is read exactly once; the work is HBM-bound.
//
// Work decomposition
//   workgroup  = WN x WK waves; it owns NG = WN * NW output columns
//                (NW = 16 * NSUB per wave) and a contiguous K-range (split
//                `sp` of S cross-workgroup K-splits).
//   wave (wn, wk) streams W rows [n0 + wn*NW, +NW) over the K-blocks
//                kb = kbA + r*WK + wk of its workgroup's range, straight from
//                HBM into VGPRs with 16-byte buffer loads and one K-block of
//                look-ahead (double-buffered registers). Buffer descriptors
//                bound every stream, so rows past N or M read as zero with no
//                branch; K-tail chunks get an out-of-range offset.
//   x            the waves of wk-group wk stage the x K-block their group
//                consumes into LDS: fp32 upcast, sum of squares for the
//                RMSNorm statistic, optional gamma multiply, rounding to the
//                MFMA input type, written in MFMA-fragment order so every
//                B-operand read is one conflict-free ds_read_b128.
//                Double-buffered across rounds, one barrier per round; the
//                next round's x loads are issued before its W loads, so the
//                wait for x leaves the W prefetch in flight (vmcnt retires in
//                issue order).
//   MFMA         D[n][m] += W[n, k] x[m, k]: A = W (16 rows of n), B = x
//                (16 columns of m), 16x16x32 bf16/f16 or 16x16x4 f32.
//                Inside a K-block, load j of lane group g reads 16-byte chunk
//                4j + g of the row's K-block segment, so the four lanes of a
//                row read 64 contiguous bytes per instruction; x is staged
//                with the same permutation of k.
//   reduction    waves wk > 0 hand their accumulators to wk == 0 through
//                LDS (fixed order); then either the epilogue runs directly
//                (S == 1), or fp32 partials are published to the workspace and
//                the last workgroup of the column group (relaxed arrival
//                ticket, agent-scope atomic data accesses: see mtp_common.hpp)
//                sums the S partials in split order, runs the epilogue and
//                re-arms the ticket for the next launch.
// Row statistics are applied in the epilogue: rstd[m] * (x[m] . W[n]) equals
// (x[m] * rstd[m]) . W[n] up to fp32 rounding, so MFMA inputs stay exact.
#pragma once

#include "mtp_common.hpp"
#include "verify_tail.hpp"

namespace mtp {

enum { EPI_LINEAR = 0, EPI_ARGMAX = 1 };

struct WsArgs {
  // operands
  const void *x;        // [M, K] CT
  const void *w;        // [N, K] WT
  const float *wscale;  // [N] or null (per output channel)
  const float *gamma;   // [K] fp32 or null
  const void *bias;     // [N] bias_dt or null
  void *y;              // [M, N] CT (EPI_LINEAR)
  int bias_dt;
  int M, N, K;
  float eps, scale;
  int norm;
  // decomposition
  int rows_per_chunk;  // rows of x per blockIdx.y chunk (<= MT * 16)
  int S;               // K-splits
  int G;               // column groups = ceil(N / NG)
  int kb_per;          // K-blocks per split
  int nkb;             // total K-blocks = ceil(K / KB)
  int xcd_map;         // 1: blockIdx -> (group, split) keeps a group's splits on one XCD
  // workspace (per row chunk; the kernel adds the chunk offset)
  float *part;       // [chunks][S][MPAD][G*NG]          split-K partials
  float *sqp;        // [chunks][G][S][MPAD]             partial sums of squares
  unsigned *ticket;  // [chunks][G] (EPI_LINEAR) / [chunks] (EPI_ARGMAX)
  float *amax_val;   // [chunks][G][MPAD]                (EPI_ARGMAX)
  int *amax_idx;     // [chunks][G][MPAD]                (EPI_ARGMAX)
  // verify (EPI_ARGMAX)
  const int32_t *draft;  // [B, D] (multi) or [M] (single)
  int8_t *accept;
  int32_t *accepted_n;
  int32_t *corrected;
  int32_t *top;  // [rows] or null
  int S_seq, D;  // multi-verify: hidden rows per batch element, drafts
  int multi;     // 1: chain acceptance, 0: single-token verify
  int textbook;  // chain convention (chain_accept): 0 the reference's, 1 textbook
};

template <int CT, int WT, int WBL>
struct WsShape {
  static constexpr int kCtBytes = dtype_bytes(CT);
  static constexpr int kWBytes = dtype_bytes(WT);
  static constexpr int LG = WBL / kWBytes;  // k per lane group per K-block
  static constexpr int KB = 4 * LG;         // k per K-block
  static constexpr int NWL = WBL / 16;      // 16-byte W loads per lane per subtile
  static constexpr int E = 16 / kCtBytes;   // x elements per 16-byte chunk
  static constexpr int CPR = KB / E;        // x chunks per row per K-block
  static constexpr int CPG = LG / E;        // x chunks per lane group
  static constexpr int STEPS = (CT == MTP_F32) ? LG : LG / 8;
};

// Buffer descriptor over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Streaming (non-temporal) variant for data read once: weights.
__device__ __forceinline__ u32x4 bload16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
constexpr uint32_t kOOB = 0x80000000u;  // an offset past any descriptor's range

// Epilogue factors of the 4 G output columns n0 + gs (i / 4) + i % 4
// (i < 4 G): wscale[n] (1 without wscale) and bias[n] as fp32 (0 without
// bias), through buffer descriptors (columns >= N read 0). The dtype choice
// sits outside the loads so they go out in one batch: issued at the start
// of a kernel their latency hides behind its main loop, and even at the end
// they cost one round trip instead of one per element (a load placed
// between output stores that might alias it waits for its own).
template <int G>
__device__ __forceinline__ void load_col_factors(const float *wscale, const void *bias,
                                                 int bias_dt, int N, int n0, int gs,
                                                 float (&ws)[4 * G], float (&bi)[4 * G]) {
  uint32_t off[4 * G];
#pragma unroll
  for (int i = 0; i < 4 * G; ++i) {
    off[i] = (uint32_t)(n0 + gs * (i >> 2) + (i & 3));
    ws[i] = 1.0f;
    bi[i] = 0.f;
  }
  if (wscale) {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(wscale, (uint32_t)N * 4u);
#pragma unroll
    for (int i = 0; i < 4 * G; ++i)
      ws[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off[i] * 4u, 0, 0));
  }
  if (bias) {
    if (bias_dt == MTP_F32) {
      const __amdgpu_buffer_rsrc_t r = make_rsrc(bias, (uint32_t)N * 4u);
#pragma unroll
      for (int i = 0; i < 4 * G; ++i)
        bi[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off[i] * 4u, 0, 0));
    } else {
      const __amdgpu_buffer_rsrc_t r = make_rsrc(bias, (uint32_t)N * 2u);
      uint32_t h[4 * G];
#pragma unroll
      for (int i = 0; i < 4 * G; ++i) h[i] = __builtin_amdgcn_raw_buffer_load_b16(r, off[i] * 2u, 0, 0);
      const bool bf = bias_dt == MTP_BF16;
#pragma unroll
      for (int i = 0; i < 4 * G; ++i) bi[i] = bf ? bf16_bits_to_f32(h[i]) : f16_bits_to_f32(h[i]);
    }
  }
}
// Cache-policy operand of the buffer intrinsics selecting sc1: the same
// agent-coherent access the compiler emits for agent-scope atomic loads and
// stores, here 16 bytes wide (see the hand-off notes in mtp_common.hpp).
constexpr int kSc1 = 16;

template <int CT, int WT, int MT, int NSUB, int WN, int WK, int WBL, int EPI>
__global__ void __launch_bounds__(WN * WK * 64)
wstream_kernel(const WsArgs a) {
  using Sh = WsShape<CT, WT, WBL>;
  constexpr int NT = WN * WK * 64;
  constexpr int TW = WN * 64;  // staging threads per wk-group
  constexpr int MPAD = MT * 16;
  constexpr int NW = NSUB * 16;
  constexpr int NG = WN * NW;
  constexpr int KB = Sh::KB, NWL = Sh::NWL, E = Sh::E;
  constexpr int CPR = Sh::CPR, CPG = Sh::CPG;
  constexpr int BLK_SLOTS = MT * CPG * 64;  // 16-byte LDS slots per K-block
  constexpr int ROUND_SLOTS = WK * BLK_SLOTS;
  constexpr int PPB = MPAD * CPR;            // x chunks per K-block
  constexpr int XIT = (PPB + TW - 1) / TW;   // chunks per staging thread
  constexpr int QR = TW / CPR;               // rows covered per staging iteration
  constexpr int WE = 16 / Sh::kWBytes;       // W elements per 16-byte chunk
  static_assert(CPR <= 64 && 64 % CPR == 0, "row chunks must tile a wave");

  constexpr int XBUF_BYTES = 2 * ROUND_SLOTS * 16;
  constexpr int RED_BYTES = (WK > 1) ? (WK - 1) * WN * 64 * MT * NSUB * 16 : 16;
  constexpr int POOL_BYTES = XBUF_BYTES > RED_BYTES ? XBUF_BYTES : RED_BYTES;
  __shared__ __attribute__((aligned(16))) unsigned char pool[POOL_BYTES];
  __shared__ float sq_red[WK * XIT * QR];
  __shared__ float sq_row[MPAD];
  __shared__ int s_flag;
  __shared__ float s_bval[WN][MPAD];
  __shared__ int s_bidx[WN][MPAD];
  __shared__ int s_top[MPAD];

  u32x4 *xbuf = (u32x4 *)pool;

  const int th = threadIdx.x;
  const int lane = th & 63;
  const int wave = th >> 6;
  const int wn = wave % WN;
  const int wk = wave / WN;
  const int lg = lane >> 4;
  const int l16 = lane & 15;

  // ---- block -> (column group, split), XCD-aware -------------------------
  int bid = blockIdx.x;
  if (a.xcd_map) {
    const int per = (a.G * a.S) >> 3;  // host guarantees divisibility
    bid = (bid & 7) * per + (bid >> 3);
  }
  const int grp = bid / a.S;
  const int sp = bid - grp * a.S;
  const int mchunk = blockIdx.y;
  const int m0 = mchunk * a.rows_per_chunk;
  const int Mloc = min(a.rows_per_chunk, a.M - m0);
  const int K = a.K, N = a.N;

  const int kbA = sp * a.kb_per;
  const int kbB = min(a.nkb, kbA + a.kb_per);
  const int nrounds = (kbB - kbA + WK - 1) / WK;
  const int n_wave0 = grp * NG + wn * NW;

  // ---- W streaming: one descriptor over this group's rows ------------------
  const uint32_t ldw = (uint32_t)K * Sh::kWBytes;
  const int grp_rows = min(NG, N - grp * NG);
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc((const unsigned char *)a.w + (int64_t)grp * NG * ldw, (uint32_t)grp_rows * ldw);
  uint32_t wrow[NSUB];
#pragma unroll
  for (int u = 0; u < NSUB; ++u) wrow[u] = (uint32_t)(wn * NW + u * 16 + l16) * ldw + lg * 16;

  auto load_w = [&](u32x4 (&wr)[NSUB][NWL], int kb) {
#pragma unroll
    for (int j = 0; j < NWL; ++j) {
      const bool ok = (kb < kbB) && (kb * KB + (4 * j + lg) * WE < K);
      const uint32_t koff = (uint32_t)kb * KB * Sh::kWBytes + j * 64;
#pragma unroll
      for (int u = 0; u < NSUB; ++u) wr[u][j] = bload16_nt(wrs, ok ? wrow[u] + koff : kOOB);
    }
  };

  // ---- x staging: thread -> (wk-group, chunk column), rows q0 + i*QR ------
  const uint32_t ldx = (uint32_t)K * Sh::kCtBytes;
  const __amdgpu_buffer_rsrc_t xrs =
      make_rsrc((const unsigned char *)a.x + (int64_t)m0 * ldx, (uint32_t)Mloc * ldx);
  const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.gamma, a.gamma ? (uint32_t)K * 4u : 0u);
  const int s_wk = th / TW;
  const int tw = th % TW;
  const int my_c = tw % CPR;
  const int q0 = tw / CPR;
  const int my_k_off = my_c * E;
  // the W chunk holding this x chunk, its lane group and the MFMA slot
  const int my_wc = my_k_off / WE;
  const int my_g = my_wc & 3;
  const int my_j = (my_wc >> 2) * (WE / E) + (my_k_off % WE) / E;
  u32x4 xr[XIT];
  u32x4 gr[E / 4];
  float sq[XIT];
#pragma unroll
  for (int i = 0; i < XIT; ++i) sq[i] = 0.f;

  auto load_x = [&](int r) {
    const int kb = kbA + r * WK + s_wk;
    const int k = kb * KB + my_k_off;
    const bool kok = kb < kbB && k < K;
#pragma unroll
    for (int i = 0; i < XIT; ++i) {
      const int m = q0 + i * QR;
      xr[i] = bload16(xrs, (kok && m < MPAD) ? (uint32_t)m * ldx + (uint32_t)k * Sh::kCtBytes : kOOB);
    }
    // without gamma the descriptor is empty and these loads return zeros
#pragma unroll
    for (int q = 0; q < E / 4; ++q) gr[q] = bload16(grs, kok ? (uint32_t)(k + 4 * q) * 4u : kOOB);
  };

  auto store_x = [&](int buf) {
    u32x4 *dst = xbuf + buf * ROUND_SLOTS + s_wk * BLK_SLOTS;
    float gv[E];
#pragma unroll
    for (int e = 0; e < E; ++e) gv[e] = a.gamma ? __uint_as_float(gr[e >> 2][e & 3]) : 1.f;
#pragma unroll
    for (int i = 0; i < XIT; ++i) {
      const int m = q0 + i * QR;
      if (m >= MPAD) continue;
      float v[E];
      if constexpr (CT == MTP_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(xr[i][e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f32x2 t = unpack2<CT>(xr[i][e]);
          v[2 * e] = t[0];
          v[2 * e + 1] = t[1];
        }
      }
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) s += v[e] * v[e];
      sq[i] += s;
      u32x4 o;
      if constexpr (CT == MTP_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __float_as_uint(v[e] * gv[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = pack2<CT>(v[2 * e] * gv[2 * e], v[2 * e + 1] * gv[2 * e + 1]);
      }
      dst[((m >> 4) * CPG + my_j) * 64 + (m & 15) + 16 * my_g] = o;
    }
  };

  // ---- MFMA over one K-block ----------------------------------------------
  f32x4 acc[MT][NSUB];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int u = 0; u < NSUB; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const u32x4 (&wr)[NSUB][NWL], int buf) {
    const u32x4 *src = xbuf + buf * ROUND_SLOTS + wk * BLK_SLOTS;
    if constexpr (CT == MTP_F32) {
      // 16x16x4 f32: one k per lane per step; x slot j holds steps 4j .. 4j+3.
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
          } else {  // fp8: the 4 values of dword (j & 3) of load (j >> 2)
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
          } else {  // fp8 -> CT, 8 values per step
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

  // ---- main loop ------------------------------------------------------------
  // Rounds alternate between register buffers wA / wB and LDS buffers 0 / 1.
  // Prefetches are issued unconditionally: past the last round they use
  // out-of-range offsets and return zeros without touching memory, and the
  // straight-line issue lets the compiler count outstanding loads exactly.
  u32x4 wA[NSUB][NWL], wB[NSUB][NWL];
  if (nrounds > 0) {
    load_x(0);
    __builtin_amdgcn_sched_barrier(0);
    load_w(wA, kbA + wk);
    __builtin_amdgcn_sched_barrier(0);
    store_x(0);
  }
  __syncthreads();
  int r = 0;
  for (; r + 1 < nrounds; r += 2) {
    load_x(r + 1);
    __builtin_amdgcn_sched_barrier(0);
    load_w(wB, kbA + (r + 1) * WK + wk);
    __builtin_amdgcn_sched_barrier(0);
    compute(wA, 0);
    store_x(1);
    __syncthreads();
    load_x(r + 2);
    __builtin_amdgcn_sched_barrier(0);
    load_w(wA, kbA + (r + 2) * WK + wk);
    __builtin_amdgcn_sched_barrier(0);
    compute(wB, 1);
    store_x(0);
    __syncthreads();
  }
  if (r < nrounds) {  // odd round count: the last round sits in wA / buffer 0
    compute(wA, 0);
    __syncthreads();
  }

// ---- row statistics over this K-range -----------------------------------------
#pragma unroll
  for (int i = 0; i < XIT; ++i) {
    float s = sq[i];
#pragma unroll
    for (int off = 1; off < CPR; off <<= 1) s += __shfl_xor(s, off, 64);
    if (my_c == 0) sq_red[(s_wk * XIT + i) * QR + q0] = s;
  }
  __syncthreads();
  if (th < MPAD) {
    float s = 0.f;
    for (int q = 0; q < WK; ++q) s += sq_red[(q * XIT + th / QR) * QR + th % QR];
    sq_row[th] = s;
  }

  // ---- cross-wave K reduction (fixed order) -------------------------------------
  if constexpr (WK > 1) {
    f32x4 *red = (f32x4 *)pool;  // x buffers are dead: all waves passed the last barrier
    if (wk > 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
          red[(((wk - 1) * WN + wn) * (MT * NSUB) + t * NSUB + u) * 64 + lane] = acc[t][u];
    }
    __syncthreads();
    if (wk == 0) {
      for (int q = 1; q < WK; ++q)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int u = 0; u < NSUB; ++u)
            acc[t][u] += red[(((q - 1) * WN + wn) * (MT * NSUB) + t * NSUB + u) * 64 + lane];
    }
  }
  __syncthreads();

  const int Npad = a.G * NG;
  // epilogue factors of the lane's columns n_wave0 + 16 u + 4 (lane / 16) + j,
  // in one batch (held through the main loop they would cost registers)
  float cws[4 * NSUB], cbi[4 * NSUB];
  load_col_factors<NSUB>(EPI == EPI_LINEAR ? a.wscale : nullptr, a.bias, a.bias_dt, a.N,
                         n_wave0 + 4 * lg, 16, cws, cbi);

  if constexpr (EPI == EPI_LINEAR) {
    // v = columns n .. n+3 of local row m; sqsum = the row's sum of squares.
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
      if (wk == 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int m = t * 16 + l16;
          if (m >= Mloc) continue;
          const float sqs = sq_row[m];
#pragma unroll
          for (int u = 0; u < NSUB; ++u) {
            const int n = n_wave0 + u * 16 + 4 * lg;
            if (n < N) finish(m, n, acc[t][u], sqs, cws + 4 * u, cbi + 4 * u);
          }
        }
      }
      return;
    }

    // split-K: publish partials; the last workgroup of the group reduces.
    float *part = a.part + (int64_t)mchunk * a.S * MPAD * Npad;
    float *sqp = a.sqp + (int64_t)mchunk * a.G * a.S * MPAD;
    unsigned *ticket = a.ticket + (int64_t)mchunk * a.G;
    if (wk == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int m = t * 16 + l16;
#pragma unroll
        for (int u = 0; u < NSUB; ++u) {
          const int n = n_wave0 + u * 16 + 4 * lg;
          float *dst = part + ((int64_t)sp * MPAD + m) * Npad + n;
#pragma unroll
          for (int j = 0; j < 4; ++j) pub_f32(dst + j, acc[t][u][j]);
        }
      }
    }
    if (th < MPAD) pub_f32(sqp + ((int64_t)grp * a.S + sp) * MPAD + th, sq_row[th]);
    wait_stores();
    __syncthreads();
    if (th == 0) s_flag = (ticket_add(ticket + grp) == (unsigned)(a.S - 1));
    __syncthreads();
    if (!s_flag) return;
    constexpr int Q = NG / 4;
    for (int item = th; item < MPAD * Q; item += NT) {
      const int m = item / Q;
      const int n = grp * NG + 4 * (item - m * Q);
      if (m >= Mloc || n >= N) continue;
      float fw[4], fb[4];
      load_col_factors<1>(a.wscale, a.bias, a.bias_dt, N, n, 0, fw, fb);
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
      float ss = 0.f;
      for (int q = 0; q < a.S; ++q) {
        const float *src = part + ((int64_t)q * MPAD + m) * Npad + n;
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] += get_f32(src + j);
        ss += get_f32(sqp + ((int64_t)grp * a.S + q) * MPAD + m);
      }
      finish(m, n, s, ss, fw, fb);
    }
    if (th == 0) ticket_reset(ticket + grp);
  } else {
    // ---- EPI_ARGMAX (S == 1): per-row (max, lowest index) over the group ----
    if (wk == 0) {
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        float bv = -__builtin_inff();
        int bi = 0x7fffffff;
#pragma unroll
        for (int u = 0; u < NSUB; ++u) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int n = n_wave0 + u * 16 + 4 * lg + j;
            if (n < N) {
              float v = acc[t][u][j];
              if (a.bias) v += cbi[4 * u + j];
              if (argmax_better(v, n, bv, bi)) {
                bv = v;
                bi = n;
              }
            }
          }
        }
#pragma unroll
        for (int off = 16; off < 64; off <<= 1) {
          const float ov = __shfl_xor(bv, off, 64);
          const int oi = __shfl_xor(bi, off, 64);
          if (argmax_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (lg == 0) {
          s_bval[wn][t * 16 + l16] = bv;
          s_bidx[wn][t * 16 + l16] = bi;
        }
      }
    }
    __syncthreads();
    float *pv = a.amax_val + (int64_t)mchunk * a.G * MPAD;
    int *pi = a.amax_idx + (int64_t)mchunk * a.G * MPAD;
    if (th < MPAD) {
      float bv = s_bval[0][th];
      int bi = s_bidx[0][th];
      for (int q = 1; q < WN; ++q)
        if (argmax_better(s_bval[q][th], s_bidx[q][th], bv, bi)) {
          bv = s_bval[q][th];
          bi = s_bidx[q][th];
        }
      pub_f32(pv + (int64_t)grp * MPAD + th, bv);
      pub_i32(pi + (int64_t)grp * MPAD + th, bi);
    }
    wait_stores();
    __syncthreads();
    unsigned *ticket = a.ticket + mchunk;
    if (th == 0) s_flag = (ticket_add(ticket) == (unsigned)(a.G - 1));
    __syncthreads();
    if (!s_flag) return;
    // Final argmax over all groups: wave w handles rows w, w + waves, ...
    for (int m = wave; m < Mloc; m += WN * WK) {
      float bv = -__builtin_inff();
      int bi = 0x7fffffff;
      for (int gq = lane; gq < a.G; gq += 64) {
        const float v = get_f32(pv + (int64_t)gq * MPAD + m);
        const int ix = get_i32(pi + (int64_t)gq * MPAD + m);
        if (argmax_better(v, ix, bv, bi)) {
          bv = v;
          bi = ix;
        }
      }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (argmax_better(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (lane == 0) s_top[m] = bi;
    }
    __syncthreads();
    if (a.top)
      for (int m = th; m < Mloc; m += NT) a.top[m0 + m] = s_top[m];
    if (!a.multi) {
      for (int m = th; m < Mloc; m += NT) a.accept[m0 + m] = (int8_t)(s_top[m] == a.draft[m0 + m]);
    } else {
      const int Sq = a.S_seq, Dd = a.D;
      const int b0 = m0 / Sq;
      for (int bl = th; bl < Mloc / Sq; bl += NT) {
        const int b = b0 + bl;
        chain_accept(s_top + bl * Sq, a.draft + (int64_t)b * Dd, Dd, a.textbook,
                     a.accept + (int64_t)b * Dd, a.accepted_n + b, a.corrected + b);
      }
    }
    if (th == 0) ticket_reset(ticket);
  }
}

}  // namespace mtp
