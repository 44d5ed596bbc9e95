// Skinny weight-streaming GEMM for gfx950: the RMSNorm -> linear path at
// M <= 64 rows of x with 16-bit x (bf16 / f16) and fp8-e4m3 or 16-bit W.
//
//   y[m, n] = (rs[m] (xg[m, :] . W[n, :]) * wscale[n] + bias[n]), times scale
//   xg[m, k] = x[m, k] * gamma[k] rounded to the type of x,
//   rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) (norm) or 1 (applied to the fp32 sums)
//
// Two launches (one without gamma: the raw-x form below):
//  1. sk_prep8_kernel, blocks of 8 rows x one K-slice (rows padded to whole
//     32-row tiles, padding rows zero): xg = x * gamma rounded to the MFMA
//     input type (the type of x), written as the B operands of
//     v_mfma_f32_32x32x16 (for each 32-row tile, stage and k-step, one 1 KB
//     block of 64 lanes x 16 bytes), and each row's sum of squares per
//     slice; the GEMM sums the slices and applies rs to its fp32 sums.
//     Doing this once per launch instead of once per column group keeps the
//     GEMM free of per-element vector work on x.
//  2. sk_kernel: bound by reading W once from HBM. A "stage" is 128 bytes
//     of every W row (128 fp8 or 64 16-bit values of k). Workgroup = 4 waves
//     and a tile of 64 output columns x all (<= 64) rows of x; the waves
//     split the k-steps of each stage (fp8: wave w takes k-steps 2w, 2w + 1;
//     16-bit W: k-step w), so every operand is read by exactly one wave, and
//     their partial sums meet in LDS at the end. Per stage the workgroup
//     copies W (64 rows x 128 bytes: one instruction covers 8 rows x 128
//     contiguous bytes, the pattern that streams HBM fastest among the ones
//     an MFMA row layout allows) into registers, and each wave loads its own
//     xn blocks (1 KB contiguous per MFMA operand) into registers. Both
//     register rings run NS - 1 stages ahead (NS = 6: 40 KB of W per CU;
//     register loads keep more bytes in flight per CU than buffer loads into
//     LDS, and a deeper ring measured slower); the loads of a stage
//     are spread over the wave's MFMAs. One stage before it is used, a stage
//     of W goes from registers to LDS (double-buffered), where each wave
//     reads the A operands of its k-steps. One barrier per stage.
//     W sits in LDS row-major with 16-byte chunk c of row r at position
//     c ^ sk_swz(r) (the A-operand reads of 16 consecutive rows then hit
//     distinct bank groups); for fp8 the A operand is upcast exactly in
//     registers.
//     k-slot order: within 32 k of a stage (two k-steps for fp8), lane group
//     g = lane / 32 holds k 16 g .. 16 g + 15, the first 8 in k-step 2p, the
//     other 8 in k-step 2p + 1 (16-bit W: k-step j, lane group g holds
//     k 16 j + 8 g .. + 7); the prep writes xg in the same order.
//  The stages of a split are taken starting at 7 tile mod (stages): tiles in
//  step with each other then read different 128-byte offsets of their rows,
//  which spreads the requests over the HBM channels (the same offset of every
//  row at once concentrates them on few channels).
//  End: S == 1 applies the epilogue directly; otherwise the workgroups of a
//  tile hand fp32 partial sums to the last one to arrive (coherent stores,
//  arrival ticket; see the hand-off notes in mtp_common.hpp), which sums them
//  in split order.
#pragma once

#include <type_traits>

#include "sk_args.hpp"
#include "wstream.hpp"

namespace mtp {

typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;

template <int CT>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (CT == MTP_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// LDS position of 16-byte chunk c of W row r inside the row's 128 bytes is
// c ^ sk_swz(r): the A-operand reads of 16 consecutive rows (rows r and r + 8
// are 1 KB apart, the same banks) then hit 16 distinct bank groups.
__device__ __forceinline__ int sk_swz(int r) { return (r >> 1) & 7; }
// Kernels that stage raw x rows into B-operand blocks (1 KB per k-step j and
// 32-row tile, lane L = 32 g + row % 32 holding 8 k of lane group g) put
// lane L at slot L ^ sk_xswz(j, g): the stores of one 8-rows x 128-byte load
// (two rows x 8 chunks per 16 lanes, every chunk a different (j % 4, g))
// then hit 16 distinct bank groups, and the B reads stay a permutation
// within each 16-lane group.
__device__ __forceinline__ int sk_xswz(int j, int g) { return 4 * (j & 3) + 2 * g; }

// (k-step, lane group) of 16-byte chunk q (8 k) of a stage.
template <bool FP8>
__device__ __forceinline__ void sk_chunk_slot(int q, int &j, int &g) {
  if constexpr (FP8) {
    j = 2 * (q >> 2) + (q & 1);
    g = (q >> 1) & 1;
  } else {
    j = q >> 1;
    g = q & 1;
  }
}

// 16 bytes per lane from a buffer straight into LDS (lane i writes bytes
// 16 i .. 16 i + 15 after `lds`). The body exists only in the device pass:
// the host pass cannot form the LDS address-space pointer, and an invalid
// expression there would silently drop the host stubs of the kernels.
template <int AUX>
__device__ __forceinline__ void sk_lds_copy16(__amdgpu_buffer_rsrc_t r, unsigned char *lds,
                                              uint32_t voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                           voff, soff, 0, AUX);
#else
  (void)r; (void)lds; (void)voff; (void)soff;
#endif
}

// 4 bytes per lane into LDS (lane i writes bytes 4 i .. 4 i + 3 after `lds`).
__device__ __forceinline__ void sk_lds_copy4(__amdgpu_buffer_rsrc_t r, unsigned char *lds,
                                             uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 4,
                                           voff, 0, 0, 0);
#else
  (void)r; (void)lds; (void)voff;
#endif
}

// ---------------------------------------------------------------------------
// 1. prep
// Prep of 8 rows x one K-slice of 256 CH k per block (block (g, s): rows
// 8 g .. 8 g + 7, chunks 32 CH s ..): xg = x * gamma rounded to the MFMA
// type into the xn blocks, and each row's sum of squares over the slice
// into ss[s][64]; the GEMM applies rs to its fp32 sums. Lane 8 c + r of a
// wave holds row r of chunk c, so a load instruction reads 8 rows x 128
// contiguous bytes and the 8 lanes of a chunk store one whole 128-byte line
// of an xn block; gamma comes in the same round trip as x.
template <int CT, bool FP8, bool GAM, int CH>
__global__ void __launch_bounds__(256)
sk_prep8_kernel(const SkPrepArgs a, float *pss) {
  constexpr int UK = FP8 ? 128 : 64, KS = UK / 16, QPS = UK / 8;
  __shared__ float red[4][8];
  const int th = threadIdx.x, r = th & 7, wave = th >> 6;
  const int m = 8 * (int)blockIdx.x + r;
  const int K = a.K, nst = K / UK, nq = K / 8;
  const int qb = (int)blockIdx.y * 32 * CH + (th >> 3);
  const u32x4 *xr = (const u32x4 *)((const uint16_t *)a.x + (int64_t)min(m, a.M - 1) * K);
  u32x4 xv[CH];
  f32x4 g0[CH], g1[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int q = qb + 32 * i;
    xv[i] = q < nq && m < a.M ? xr[q] : u32x4{0u, 0u, 0u, 0u};
    g0[i] = g1[i] = f32x4{1.f, 1.f, 1.f, 1.f};
    if constexpr (GAM) {
      if (q < nq) {
        g0[i] = ((const f32x4 *)a.gamma)[2 * q];
        g1[i] = ((const f32x4 *)a.gamma)[2 * q + 1];
      }
    }
  }
  float ss = 0.f;
  u32x4 *xf = (u32x4 *)a.xf;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int q = qb + 32 * i;
    const float g[8] = {g0[i][0], g0[i][1], g0[i][2], g0[i][3],
                        g1[i][0], g1[i][1], g1[i][2], g1[i][3]};
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f32x2 f = unpack2<CT>(xv[i][e]);
      ss += f[0] * f[0] + f[1] * f[1];
      o[e] = pack2<CT>(f[0] * g[2 * e], f[1] * g[2 * e + 1]);
    }
    if (q < nq) {
      const int st = q / QPS, qq = q - st * QPS;
      int j, gg;
      sk_chunk_slot<FP8>(qq, j, gg);
      xf[(((int64_t)(m >> 5) * nst + st) * KS + j) * 64 + 32 * gg + (m & 31)] = o;
    }
  }
  // row r: lanes r, r + 8, ... of each wave, then the four waves in order
  ss += __shfl_xor(ss, 8, 64);
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  if ((th & 63) < 8) red[wave][r] = ss;
  __syncthreads();
  if (th < 8)
    pss[blockIdx.y * 64 + 8 * blockIdx.x + th] =
        ((red[0][th] + red[1][th]) + red[2][th]) + red[3][th];
}

// ---------------------------------------------------------------------------
// 2. GEMM. XR (raw x, no gamma): the caller's row-major x rows come in with
// the W loads' pattern (8 rows x 128 contiguous bytes per instruction) and
// go to LDS B-operand blocks beside W one stage before use (lane 32 g + m
// of block (tile, k-step j) at slot (32 g + m) ^ sk_xswz(j, g)); the sums of
// squares of the rows are taken on the way to LDS (v_dot2 of each 16-byte
// piece with itself, fp32 sums; every row's pieces arrive in one wave, so a
// row's sum needs only the 8 lanes that hold it), and rs multiplies the
// fp32 sums in the epilogue: no prep launch.
template <int CT>
__device__ __forceinline__ float sk_sumsq2(uint32_t v, float acc) {
  if constexpr (CT == MTP_BF16) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, v),
                                           __builtin_bit_cast(bf16x2_t, v), acc, false);
  } else {
    typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, v), __builtin_bit_cast(f16x2_t, v),
                                  acc, false);
  }
}

template <int CT, int WT, int MT, bool XR>
__global__ void __launch_bounds__(256, 1)
sk_kernel(const SkArgs a) {
  constexpr bool FP8 = WT == MTP_FP8E4M3;
  constexpr int UK = FP8 ? 128 : 64;         // k per stage
  constexpr int KS = UK / 16;                // MFMA k-steps per stage
  constexpr int KPW = KS / 4;                // k-steps per wave per stage
  constexpr int STAGE = kSkBN * kSkUB;       // W bytes of one LDS buffer (8 KB)
  // register ring stages (loads run NS - 1 ahead; even: LDS buffer = slot
  // parity). 6 measured faster than 8 on every shape tried (fp8 64 x 14336
  // x 4096 23.1 against 23.9 us; bf16 64 x 4096 x 4096 without gamma 13.4
  // against 14.1); 4 only ties it at fp8 with gamma and 64 rows and loses
  // elsewhere (bf16 64 x 4096 x 4096 14.6, fp8 32 x 14336 x 4096 20.5)
  constexpr int NS = 6;
  constexpr int NWC = STAGE / 1024 / 4;      // W loads per wave per stage (2)
  constexpr int NXL = MT * KPW;              // xn loads per wave per stage
  constexpr int NV = NWC + NXL;              // vector-memory instructions per wave per stage
  constexpr int RED = 4 * 2 * MT * 64 * 64;  // end-phase partial tiles of the four waves
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * STAGE > RED ? 2 * STAGE : RED];
  static_assert((NS - 1) * NV < 64, "vmcnt is 6 bits");
  __shared__ int s_flag;
  constexpr int XST = MT * KS * 1024;      // XR: x B-operand bytes of one stage
  __shared__ __attribute__((aligned(1024))) unsigned char ldsx[XR ? 2 * XST : 16];
  __shared__ float s_sq[XR ? 64 : 1];     // XR: row sums of squares (this k-range)
  __shared__ float s_rs[64];              // row scales
  __shared__ float s_pss[XR ? 1 : kSkPrepMaxSlices * 64];  // prep form: the prep's row sums

  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  const int N = a.N, K = a.K;

  // blockIdx -> (column tile, split): the splits of a tile on one XCD
  // (bf16 64 x 4096 x 4096, 4 splits: 14.5 -> 14.2 us; fp8 24 x 4096 x
  // 4096: 11.5 -> 11.1 us)
  int tile, sp;
  split_tile_of((int)blockIdx.x, a.G, a.S, true, tile, sp);
  const int n0 = tile * kSkBN;
  // end-phase owner of this wave (see below) and its column factors
  const int ou = wave & 1, ot = wave >> 1;
  const bool owner = ot < MT;
  float cws[16], cbi[16];
  load_col_factors<4>(a.wscale, a.bias, a.bias_dt, N, n0 + 32 * ou + 4 * (lane >> 5), 8, cws, cbi);
  const int st0 = sp * a.kb_per;
  const int nst = min(a.nkb, st0 + a.kb_per) - st0;  // stages of this split (>= 1)

  // W load c (c = wave + 4 i): rows 8 c .. 8 c + 7, lane l: row 8 c + l / 8;
  // the LDS write of a load is 64 lanes x 16 bytes contiguous, so the
  // swizzle (chunk c' of the row at position c' ^ sk_swz(row)) is in the chunk
  // a lane fetches
  const uint32_t ldw = (uint32_t)K * (FP8 ? 1u : 2u);
  const int nrows = min(kSkBN, N - n0);
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc((const unsigned char *)a.w + (int64_t)n0 * ldw, (uint32_t)nrows * ldw);
  uint32_t wvo[NWC];
#pragma unroll
  for (int i = 0; i < NWC; ++i) {
    const int row = 8 * (wave + 4 * i) + (lane >> 3);
    const int chunk = (lane & 7) ^ sk_swz(row);
    wvo[i] = (uint32_t)row * ldw + (uint32_t)st0 * kSkUB + 16u * chunk;
  }
  // xn load i = t * KPW + jj of the wave: tile t, k-step wave * KPW + jj
  const int nst_all = a.nkb;
  const __amdgpu_buffer_rsrc_t xrs =
      XR ? make_rsrc(a.x, (uint32_t)a.M * (uint32_t)K * 2u)
         : make_rsrc(a.xf, (uint32_t)(MT * nst_all * KS) * 1024u);
  uint32_t xvo[NXL];
  int xl[XR ? NXL : 1];  // XR: LDS byte offset of load i's 16 bytes in a stage
#pragma unroll
  for (int i = 0; i < NXL; ++i) {
    if constexpr (XR) {
      // load c = wave + 4 i: rows 8 (c mod 4 MT) + lane / 8 (rows >= M fall
      // past the descriptor: zeros), 16-byte piece q = 8 (c / 4 MT) + lane % 8
      // of the row's UK k of the stage
      const int c = wave + 4 * i;
      const int row = 8 * (c % (4 * MT)) + (lane >> 3);
      const int q = 8 * (c / (4 * MT)) + (lane & 7);
      int j, g;
      sk_chunk_slot<FP8>(q, j, g);
      xvo[i] = (uint32_t)((row * K + st0 * UK) * 2 + 16 * q);
      xl[i] = (((row >> 5) * KS + j) * 64 + ((32 * g + (row & 31)) ^ sk_xswz(j, g))) * 16;
    } else {
      const int t = i / KPW, j = wave * KPW + i % KPW;
      xvo[i] = (uint32_t)(((t * nst_all + st0) * KS + j) * 1024 + lane * 16);
    }
  }
  u32x4 xr[NS][NXL];   // xn register ring
  u32x4 wr[NS][NWC];   // W register ring
  // The split's stages are taken starting at 7 tile mod nst: workgroups in
  // step with each other then read different 128-byte offsets of their W
  // rows, which spreads the requests over the HBM channels.
  const int rot = (7 * tile) % nst;

  // Instruction v (0 <= v < NV) of stage st into ring slot `slot`. Stages
  // past the split load with an out-of-range vector offset: zeros, no memory
  // access (the scalar offset is not part of the descriptor's range check),
  // into a slot that is never computed on, so the count of instructions per
  // stage is always NV.
  auto issue = [&](auto vc, int st, auto slotc) __attribute__((always_inline)) {
    constexpr int v = decltype(vc)::value, slot = decltype(slotc)::value;
    const bool live = st < nst;
    const int str = live ? (st + rot < nst ? st + rot : st + rot - nst) : 0;
    if constexpr (v < NWC) {
      wr[slot][v] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, live ? wvo[v] : kOOB, str * kSkUB, 2));
    } else {
      constexpr int i = v - NWC;
      xr[slot][i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, live ? xvo[i] : kOOB,
                                                       XR ? str * UK * 2 : str * KS * 1024, 0));
    }
  };

  f32x16 acc[2][MT];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[u][t][e] = 0.f;
  // XR: the lane's sums of squares of rows 8 (w + 4 t) + lane / 8 (t < MT:
  // x load i covers rows 8 ((w + 4 i) mod 4 MT) + lane / 8, so t = i mod MT)
  float ssl[XR ? MT : 1];
#pragma unroll
  for (int t = 0; t < (XR ? MT : 1); ++t) ssl[t] = 0.f;

  // This wave's k-steps of a stage (A from W rows 32 u + lane % 32, B from
  // the xn blocks), with the copies of stage `nst_` spread over them.
  const int ag = lane >> 5;
  // W of ring slot `slot` to LDS buffer b
  auto w_to_lds = [&](auto slotc, int b) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
#pragma unroll
    for (int v = 0; v < NWC; ++v)
      *(u32x4 *)(lds + b * STAGE + (wave + 4 * v) * 1024 + lane * 16) = wr[slot][v];
    if constexpr (XR) {
#pragma unroll
      for (int i = 0; i < NXL; ++i) {
        *(u32x4 *)(ldsx + b * XST + xl[i]) = xr[slot][i];
#pragma unroll
        for (int e = 0; e < 4; ++e) ssl[i % MT] = sk_sumsq2<CT>(xr[slot][i][e], ssl[i % MT]);
      }
    }
  };
  auto compute = [&](auto slotc, int nst_, auto nslotc) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
    const unsigned char *base = lds + (slot & 1) * STAGE;
    static_for<0, KPW>([&](auto jc) {
      constexpr int jj = decltype(jc)::value;
      static_for<jj * NV / KPW, (jj + 1) * NV / KPW>([&](auto vc) { issue(vc, nst_, nslotc); });
      const int j = wave * KPW + jj;  // k-step of the stage
      u32x4 av[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int row = 32 * u + (lane & 31);
        if constexpr (FP8) {
          // chunk 2 (j / 2) + g holds k-steps j (bytes 0..7) and j + 1 (8..15)
          const int c = 2 * (j >> 1) + ag;
          const u32x4 w = *(const u32x4 *)(base + row * kSkUB + ((c ^ sk_swz(row)) << 4));
          const int h = (j & 1) * 2;
          av[u][0] = fp8x2_to_ct<CT, false>(w[h]);
          av[u][1] = fp8x2_to_ct<CT, true>(w[h]);
          av[u][2] = fp8x2_to_ct<CT, false>(w[h + 1]);
          av[u][3] = fp8x2_to_ct<CT, true>(w[h + 1]);
        } else {
          const int c = 2 * j + ag;
          av[u] = *(const u32x4 *)(base + row * kSkUB + ((c ^ sk_swz(row)) << 4));
        }
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const u32x4 bv =
            XR ? *(const u32x4 *)(ldsx + (slot & 1) * XST + (t * KS + j) * 1024 +
                                  ((lane ^ sk_xswz(j, ag)) << 4))
               : xr[slot][t * KPW + jj];
#pragma unroll
        for (int u = 0; u < 2; ++u) acc[u][t] = mfma32<CT>(av[u], bv, acc[u][t]);
      }
    });
  };

  // Pipeline: stages s + 1 .. s + NS - 1 are loading while s computes; the
  // loop is unrolled by the ring length so the ring slots are compile-time
  // registers (moving registers between slots would wait for the loads just
  // issued). Scheduling barriers keep each phase in place: work on a slot
  // hoisted ahead of its phase would wait for loads issued just before, and
  // the prologue keeps the loop's load order (the wait counts at the loop
  // head are the minimum over both ways in).
  if constexpr (!XR) {
    // the prep's per-slice row sums, 64 floats per copy (wave w: slices w,
    // w + 4, ...), into LDS; read after the main loop's barriers
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.pss, (uint32_t)a.nsl * 256u);
#pragma unroll
    for (int i = 0; i < kSkPrepMaxSlices / 4; ++i) {
      const int s = wave + 4 * i;
      sk_lds_copy4(srs, (unsigned char *)(s_pss + 64 * s), s < a.nsl ? (uint32_t)(s * 64 + lane) * 4u : kOOB);
    }
  }
  static_for<0, NS - 1>([&](auto pc) {
    static_for<0, NV>([&](auto vc) { issue(vc, decltype(pc)::value, pc); });
    __builtin_amdgcn_sched_barrier(0);
  });
  w_to_lds(std::integral_constant<int, 0>{}, 0);
  lds_barrier();
  auto step = [&](auto rc, int s) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::value;  // s % NS
    __builtin_amdgcn_sched_barrier(0);
    // W of stage s + 1 to the other LDS buffer (the barrier below publishes
    // it; buffer s & 1 is rewritten only after the next barrier)
    if (s + 1 < nst) w_to_lds(std::integral_constant<int, (r + 1) % NS>{}, (s + 1) & 1);
    __builtin_amdgcn_sched_barrier(0);
    // MFMAs of stage s; ring slot r - 1 (stage s - 1, done) refills with
    // stage s + NS - 1
    compute(rc, s + NS - 1, std::integral_constant<int, (r + NS - 1) % NS>{});
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
  __syncthreads();
  if constexpr (XR) {
    // the 8 lanes of each row (lane / 8), then one store per row
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float v = ssl[t];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      if ((lane & 7) == 0) s_sq[8 * (wave + 4 * t) + (lane >> 3)] = v;
    }
  }

  // ---- the four waves' partial tiles meet in LDS: wave w sums output tile
  // (u, t) = (w % 2, w / 2) (waves past the MT tiles only contribute)
  // [wave][u][t][quad][lane] of f32x4: a 16-lane group touches 256
  // contiguous bytes (64 bytes per lane would put 4 lanes on each bank)
  f32x4 *red = (f32x4 *)lds;
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        red[(((wave * 2 + u) * MT + t) * 4 + g4) * 64 + lane] =
            f32x4{acc[u][t][4 * g4], acc[u][t][4 * g4 + 1], acc[u][t][4 * g4 + 2],
                  acc[u][t][4 * g4 + 3]};
  __syncthreads();
  f32x16 v;
#pragma unroll
  for (int e = 0; e < 16; ++e) v[e] = 0.f;
  if (owner) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const f32x4 p = red[(((q * 2 + ou) * MT + ot) * 4 + g4) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * g4 + e] += p[e];
      }
  }

  // lane's outputs: v[e] = D[n][m], m = 32 ot + lane % 32,
  // n = n0 + 32 ou + 8 (e / 4) + 4 (lane / 32) + e % 4
  auto finish = [&](const f32x16 &r0) {
    const int m = 32 * ot + (lane & 31);
    if (m >= a.M) return;
    f32x16 r = r0;
    r *= s_rs[m];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0 + 32 * ou + 8 * g + 4 * ag;
      float o[4];
#pragma unroll
      for (int jx = 0; jx < 4; ++jx)
        o[jx] = (a.bias ? r[4 * g + jx] * cws[4 * g + jx] + cbi[4 * g + jx]
                        : r[4 * g + jx] * cws[4 * g + jx]) * a.scale;
      const int64_t yb = (int64_t)m * N + n;
      if (n + 3 < N && (N & 3) == 0) {
        uint2 pk;
        pk.x = pack2<CT>(o[0], o[1]);
        pk.y = pack2<CT>(o[2], o[3]);
        *(uint2 *)((uint16_t *)a.y + yb) = pk;
      } else {
        for (int jx = 0; jx < 4; ++jx)
          if (n + jx < N) store_from_f32(a.y, CT, yb + jx, o[jx]);
      }
    }
  };

  // XR: this workgroup's sums of squares of row th (its k-range)
  float ssw = 0.f;
  if constexpr (XR) {
    if (th < 32 * MT) ssw = s_sq[th];
  }
  auto set_rs = [&](float ss) {
    if (th < 32 * MT) s_rs[th] = a.norm ? 1.0f / sqrtf(ss / (float)K + a.eps) : 1.0f;
  };
  if constexpr (!XR) {
    // the prep's slices in order (its copies landed before the main loop's
    // first wait)
    float ss = 0.f;
    if (th < 32 * MT)
      for (int s = 0; s < a.nsl; ++s) ss += s_pss[64 * s + th];
    set_rs(ss);
    __syncthreads();
  }
  if (a.S == 1) {
    if constexpr (XR) {
      set_rs(ssw);
      __syncthreads();
    }
    if (owner) finish(v);
    return;
  }

  // Split-K hand-off: partial [tile][split][owner wave][4 quads][lane] of
  // f32x4 (consecutive lanes write consecutive 16 bytes), coherent stores.
  constexpr uint32_t TILEB = (uint32_t)2 * MT * 4u * 64u * 16u;
  const uint32_t part_bytes = (uint32_t)(a.S * a.G) * TILEB;
  const __amdgpu_buffer_rsrc_t prs = make_rsrc(a.part, part_bytes);
  auto part_off = [&](int q, int g4) {
    return (uint32_t)(tile * a.S + q) * TILEB +
           ((uint32_t)(wave * 4 + g4) * 64u + (uint32_t)lane) * 16u;
  };
  if (owner) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 p4 = f32x4{v[4 * g4], v[4 * g4 + 1], v[4 * g4 + 2], v[4 * g4 + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, p4), prs,
                                             part_off(sp, g4), 0, kSc1);
    }
  }
  // XR: the split's sums of squares, [tile][split][64 rows]
  const __amdgpu_buffer_rsrc_t qrs =
      make_rsrc(a.part_ss, XR ? (uint32_t)(a.S * a.G) * 256u : 0u);
  if constexpr (XR) {
    if (th < 32 * MT)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, ssw), qrs,
                                            ((uint32_t)(tile * a.S + sp) * 64u + th) * 4u, 0, kSc1);
  }
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = (ticket_add(a.ticket + tile) == (unsigned)(a.S - 1));
  __syncthreads();
  if (!s_flag) return;
  if constexpr (XR) {
    // every split's sums of row th in split order (own term from registers)
    float ss = 0.f;
    if (th < 32 * MT) {
      // four splits' loads together per round trip
      for (int q0 = 0; q0 < a.S; q0 += 4) {
        float pv[4];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int q = q0 + qq;
          const bool ld = q < a.S && q != sp;
          pv[qq] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(
                         qrs, ld ? ((uint32_t)(tile * a.S + q) * 64u + th) * 4u : kOOB, 0, kSc1));
        }
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int q = q0 + qq;
          if (q < a.S) ss += q == sp ? ssw : pv[qq];
        }
      }
    }
    set_rs(ss);
    __syncthreads();
  }
  if (owner) {
    // sums in split order (its own term from registers); the loads of QB
    // splits go out together, one round trip for up to QB splits
    constexpr int QB = 4;
    f32x16 tot;
#pragma unroll
    for (int e = 0; e < 16; ++e) tot[e] = 0.f;
    for (int q0 = 0; q0 < a.S; q0 += QB) {
      f32x4 pv[QB][4];
#pragma unroll
      for (int qq = 0; qq < QB; ++qq) {
        const int q = q0 + qq;
        const bool ld = q < a.S && q != sp;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          pv[qq][g4] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(prs, ld ? part_off(q, g4) : kOOB, 0,
                                                           kSc1));
      }
#pragma unroll
      for (int qq = 0; qq < QB; ++qq) {
        const int q = q0 + qq;
        if (q >= a.S) break;
        if (q == sp) {
          tot += v;
          continue;
        }
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
#pragma unroll
          for (int e = 0; e < 4; ++e) tot[4 * g4 + e] += pv[qq][g4][e];
      }
    }
    finish(tot);
  }
  if (th == 0) ticket_reset(a.ticket + tile);
}

}  // namespace mtp
