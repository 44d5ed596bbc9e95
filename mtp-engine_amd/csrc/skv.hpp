// Persistent weight-streaming verify for gfx950: the lm_head pass of
// fused_verify / fused_multi_verify, hidden rows and weights of one dtype
// (bf16, f16 or fp32), optional bias of any float dtype.
//
//   top[m] = argmax_n (x[m] . W[n] + bias[n])   (torch.argmax: NaN is the
//                                                maximum, the lowest index
//                                                wins ties)
//
// One launch of one workgroup per CU streams W once.
// Workgroup b takes the tw-column tiles b, b + grid, b + 2 grid, ... (tw
// <= kSkvBN: the host narrows the 256-column MFMA tile so that the tiles
// make whole rounds of one workgroup per CU; columns past tw read zeros
// and never enter the argmax)
// back to back; the stages (128 bytes of every W row of a tile: 64 k of
// 16-bit W, 32 k of fp32 W) of all its tiles form one sequence, so the
// register rings run across tile boundaries without draining; each tile's
// stages start at 7 b mod nst. W is addressed through one buffer descriptor
// per tile (a tile is 256 rows), so W may be any size. 8 waves; wave w owns
// columns 32 w .. + 31 of every tile against all (<= 64) rows, over every k,
// so a tile ends with no reduction between waves. Per stage:
//   * W (256 rows x 128 bytes) comes HBM -> registers with 8-rows x 128-byte
//     non-temporal loads NS - 1 stages ahead, then goes to a double-buffered
//     LDS stage (16-byte chunk c of row r at c ^ sk_swz(r)) one step before use;
//   * x comes from the caller's row-major hidden rows with the same
//     8-rows x 128-byte loads (one per wave per stage at most); its requests
//     are a fifth of the stage's, so they take little of the memory pipeline
//     the W stream needs;
//   * 16-bit: each wave runs 4 k-steps x MT 32-row tiles of
//     v_mfma_f32_32x32x16 (x stored as B-operand blocks);
//     fp32 (TF32 never used): x stored row-major like W; lane group g of a
//     wave reads 16-byte chunk 4 j + g (j = 0, 1) of 16 rows, and the four
//     fp32 values of the chunk feed four v_mfma_f32_16x16x4_f32, for 2 W
//     tiles x MT 16-row x tiles (each MFMA sums k = 4 (4 j + g) + i over the
//     lane groups g, i fixed; A and B use the same k of every slot).
//     R8: 8 more rows after the MT 16-row tiles (40 rows = 2 tiles + 8) on
//     v_mfma_f32_4x4x1_16b_f32, whose 16 blocks are 4 rows x 4 columns x
//     one k each: A = the 8 rows (lanes 4 b + r: row 4 rg + r, the k of
//     lane group b / 4), B = the same W registers the 16-row tiles use, so
//     block b sums one k in four of the step and the four k-groups meet by
//     two lane shuffles at the end of a tile. Same MFMA rate as the 16-row
//     tiles on 8 rows instead of 16 padded ones.
// At the end of a tile each lane adds the bias to its columns and folds
// them into a running (max, index) per row. At the end the waves' maxima
// meet in LDS and one lane per row publishes (value, index) as a 64-bit key
// whose unsigned order is the argmax order (order-preserving float bits,
// then the complement of the index) with an atomic max; the last workgroup
// to arrive decodes the keys, runs the acceptance and re-zeroes the keys and
// its ticket for the next launch.
#pragma once

#include "sk.hpp"
#include "skv_args.hpp"
#include "verify_tail.hpp"

namespace mtp {

// Bias element n (past the end: 0) as fp32; dt is F32, BF16 or F16.
__device__ __forceinline__ float skv_bias_at(__amdgpu_buffer_rsrc_t r, int dt, int n) {
  if (dt == MTP_F32)
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, 4u * (uint32_t)n, 0, 0));
  const uint32_t h = __builtin_amdgcn_raw_buffer_load_b16(r, 2u * (uint32_t)n, 0, 0);
  return dt == MTP_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

// CT: compute type (BF16, F16, F32); MT: x row tiles (32 rows for 16-bit,
// 16 rows for fp32); R8 (fp32): 8 rows after them.
template <int CT, int MT, bool R8>
__global__ void __launch_bounds__(512, 1)
skv_kernel(const SkvArgs a) {
  constexpr bool F32 = CT == MTP_F32;
  constexpr int BN = kSkvBN;                 // columns per tile
  constexpr int TR = F32 ? 16 : 32;          // rows per x tile
  constexpr int KS = F32 ? 2 : 4;            // compute steps per stage
  constexpr int WST = BN * kSkUB;            // W bytes of one stage (32 KB)
  constexpr int XR = MT * TR + (R8 ? 8 : 0);  // x rows
  constexpr int XST = XR * kSkUB;            // x bytes of one stage
  constexpr int NS = 4;                      // register ring stages (loads run NS - 1 ahead)
  constexpr int NWC = WST / 1024 / 8;        // W loads per wave per stage (4)
  constexpr int NXC = (XST / 1024 + 7) / 8;  // x loads per wave per stage (<= 1)
  constexpr int NV = NWC + NXC;
  constexpr int NQ = F32 ? 8 : 16;           // columns per lane per tile
  static_assert(NXC == 1, "one x block per wave and stage at most");
  static_assert((NS - 1) * NV < 64, "vmcnt is 6 bits");
  static_assert(XR <= 64, "at most 64 rows");
  static_assert(!R8 || F32, "the 8-row remainder is an fp32 form");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_w[2 * WST];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_x[2 * XST];
  __shared__ unsigned long long s_key[8][64];
  __shared__ int s_flag;
  __shared__ int s_top[64];
  __shared__ int s_draft[64];

  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  const int N = a.N, nst = a.nst;
  const int b = blockIdx.x, grid = gridDim.x;
  const int ntl = (a.ntiles - b + grid - 1) / grid;  // this workgroup's tiles (>= 1)
  const int total = ntl * nst;                       // its stages
  // Stage order inside a tile starts at 7 b mod nst: workgroups in step
  // with each other then read different 128-byte offsets of their rows,
  // which spreads the requests over the HBM channels (the same offset of
  // every row at once concentrates them; measured 1.3x slower).
  const int rot = (7 * b) % nst;

  const uint32_t ldw = (uint32_t)a.K * (uint32_t)dtype_bytes(CT);
  // W of tile t: rows t * tw .. t * tw + tw - 1 (rows past them, or past N,
  // read zeros)
  const int tw = a.tw;
  auto w_rsrc = [&](int tile) __attribute__((always_inline)) {
    const int rows = min(tw, N - tile * tw);
    return make_rsrc((const unsigned char *)a.w + (size_t)tile * tw * ldw, (uint32_t)rows * ldw);
  };
  // W load c (c = wave + 8 i): rows 8 c .. 8 c + 7 of the tile, lane l: row
  // 8 c + l / 8, 16-byte chunk (l % 8) ^ sk_swz(row) of the stage's 128 bytes
  uint32_t wvo[NWC];
#pragma unroll
  for (int i = 0; i < NWC; ++i) {
    const int row = 8 * (wave + 8 * i) + (lane >> 3);
    const int chunk = (lane & 7) ^ sk_swz(row);
    wvo[i] = (uint32_t)row * ldw + 16u * chunk;
  }
  // x load of wave w (w < XST / 1024): rows 8 w .. 8 w + 7 (rows past M read
  // as zeros), lane l: row 8 w + l / 8, 16-byte chunk c = l % 8 of the
  // stage. 16-bit: k 8 c .. + 7, lane 32 (c % 2) + row % 32 of B-operand
  // block (row / 32, c / 2); fp32: row-major like W.
  const bool xloader = wave < XST / 1024;
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)a.M * ldw);
  const int xrow = 8 * wave + (lane >> 3), xc = lane & 7;
  const uint32_t xvo = (uint32_t)xrow * ldw + 16u * (uint32_t)xc;
  const int xlds =
      F32 ? xrow * kSkUB + ((xc ^ sk_swz(xrow)) << 4)
          : ((xrow >> 5) * KS + (xc >> 1)) * 1024 +
                ((32 * (xc & 1) + (xrow & 31)) ^ sk_xswz(xc >> 1, xc & 1)) * 16;
  u32x4 wr[NS][NWC];  // W register ring
  u32x4 xr[NS];       // x register ring

  // The stage being issued, as (tile iteration, stage in tile); stages past
  // the last re-read the last one into a slot that is never computed on.
  int is_i = 0, is_st = 0;
  auto issue = [&](auto vc, auto slotc) __attribute__((always_inline)) {
    constexpr int v = decltype(vc)::value, slot = decltype(slotc)::value;
    const int str = is_st + rot < nst ? is_st + rot : is_st + rot - nst;
    if constexpr (v < NWC) {
      const uint32_t off = wvo[v] + (uint32_t)str * (uint32_t)kSkUB;
      wr[slot][v] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc(b + is_i * grid), off, 0, 2));
    } else {
      const uint32_t off = xvo + (uint32_t)str * (uint32_t)kSkUB;
      xr[slot] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0));
    }
  };
  auto advance = [&]() __attribute__((always_inline)) {
    if (is_i * nst + is_st + 1 < total) {
      if (++is_st == nst) {
        is_st = 0;
        ++is_i;
      }
    }
  };

  // 16-bit: acc[t] of x tile t (32 rows) x the wave's 32 columns;
  // fp32: acc4[u][t] of W tile u (16 columns) x x tile t (16 rows)
  f32x16 acc[F32 ? 1 : MT];
  f32x4 acc4[2][F32 ? MT : 1];
  // R8: accR[u][rg] of W tile u x rows MT * 16 + 4 rg .. + 3, per k-group
  f32x4 accR[2][2];
  auto zero_acc = [&]() __attribute__((always_inline)) {
    if constexpr (R8) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int rg = 0; rg < 2; ++rg)
#pragma unroll
          for (int e = 0; e < 4; ++e) accR[u][rg][e] = 0.f;
    }
    if constexpr (F32) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc4[u][t][e] = 0.f;
    } else {
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;
    }
  };
  zero_acc();

  const int ag = lane >> 5, g4 = lane >> 4;
  auto to_lds = [&](auto slotc, int buf) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
#pragma unroll
    for (int v = 0; v < NWC; ++v)
      *(u32x4 *)(lds_w + buf * WST + (wave + 8 * v) * 1024 + lane * 16) = wr[slot][v];
    if (xloader) *(u32x4 *)(lds_x + buf * XST + xlds) = xr[slot];
  };
  // this wave's 32 columns against all rows, compute steps J0 .. J1 - 1 of
  // the stage in buffer `buf`; the NV loads of the stage NS - 1 ahead spread
  // over the KS steps
  auto compute = [&](int buf, auto nslotc, auto j0c, auto j1c) __attribute__((always_inline)) {
    const unsigned char *wb = lds_w + buf * WST;
    const unsigned char *xb = lds_x + buf * XST;
    static_for<decltype(j0c)::value, decltype(j1c)::value>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      static_for<j * NV / KS, (j + 1) * NV / KS>([&](auto vc) { issue(vc, nslotc); });
      if constexpr (F32) {
        const int c = 4 * j + g4;
        u32x4 av[2], bv[MT];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int row = 32 * wave + 16 * u + (lane & 15);
          av[u] = *(const u32x4 *)(wb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int row = 16 * t + (lane & 15);
          bv[t] = *(const u32x4 *)(xb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
        }
        u32x4 bx[2];
        if constexpr (R8) {
#pragma unroll
          for (int rg = 0; rg < 2; ++rg) {
            const int row = 16 * MT + 4 * rg + (lane & 3);
            bx[rg] = *(const u32x4 *)(xb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int t = 0; t < MT; ++t)
              acc4[u][t] = mfma16_f32(__uint_as_float(av[u][i]), __uint_as_float(bv[t][i]),
                                      acc4[u][t]);
          if constexpr (R8) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
              for (int rg = 0; rg < 2; ++rg)
                accR[u][rg] = mfma4_f32(__uint_as_float(bx[rg][i]), __uint_as_float(av[u][i]),
                                        accR[u][rg]);
          }
        }
      } else {
        const int row = 32 * wave + (lane & 31);
        const int c = 2 * j + ag;
        const u32x4 av = *(const u32x4 *)(wb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const u32x4 bv =
              *(const u32x4 *)(xb + (t * KS + j) * 1024 + ((lane ^ sk_xswz(j, ag)) << 4));
          acc[t] = mfma32<CT>(av, bv, acc[t]);
        }
      }
    });
  };

  // Column (within a tile) of this lane's value q (q < NQ), the same for
  // every row it holds. 16-bit: 32 wave + 8 (q / 4) + 4 (l / 32) + q % 4
  // (rows 32 t + l % 32); fp32: 32 wave + 16 (q / 4) + 4 (l / 16) + q % 4
  // (rows 16 t + l % 16).
  auto col_of = [&](int q) __attribute__((always_inline)) {
    return F32 ? 32 * wave + 16 * (q >> 2) + 4 * g4 + (q & 3)
               : 32 * wave + 8 * (q >> 2) + 4 * ag + (q & 3);
  };
  // The bias of the lane's columns of the tile being computed, loaded when
  // the tile starts (one element per load: any N, any alignment)
  const bool has_bias = a.bias != nullptr;
  const __amdgpu_buffer_rsrc_t brs =
      make_rsrc(a.bias, has_bias ? (uint32_t)N * (uint32_t)dtype_bytes(a.bias_dt) : 0u);
  float bias_v[NQ];
  // R8: the lane's remainder columns are 32 wave + 16 u + lane % 16
  float bias_r[2];
  auto load_bias = [&](int tile) __attribute__((always_inline)) {
    if (has_bias) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) bias_v[q] = skv_bias_at(brs, a.bias_dt, tile * tw + col_of(q));
      if constexpr (R8) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
          bias_r[u] = skv_bias_at(brs, a.bias_dt, tile * tw + 32 * wave + 16 * u + (lane & 15));
      }
    } else {
#pragma unroll
      for (int q = 0; q < NQ; ++q) bias_v[q] = 0.f;
      bias_r[0] = bias_r[1] = 0.f;
    }
  };

  // Running per-row maximum of x tile t over this lane's columns.
  float best_v[MT];
  int best_n[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    best_v[t] = -__builtin_inff();
    best_n[t] = 0x7fffffff;
  }
  // R8: row MT * 16 + 4 rg + r over the lane's remainder columns
  float bestr_v[2][4];
  int bestr_n[2][4];
#pragma unroll
  for (int rg = 0; rg < 2; ++rg)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bestr_v[rg][r] = -__builtin_inff();
      bestr_n[rg][r] = 0x7fffffff;
    }
  auto end_tile = [&](int tile) __attribute__((always_inline)) {
    if constexpr (R8) {
      // the four k-groups of a block (lanes l, l ^ 16, l ^ 32, l ^ 48) sum
      // in the same order on every lane; register r of lane l is then row
      // MT * 16 + 4 rg + r, column 32 wave + 16 u + l % 16
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) {
          f32x4 v = accR[u][rg];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += __shfl_xor(v[e], 16, 64);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] += __shfl_xor(v[e], 32, 64);
          const int cn = 32 * wave + 16 * u + (lane & 15), n = tile * tw + cn;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = v[r] + bias_r[u];
            if (cn < tw && n < N && argmax_better(x, n, bestr_v[rg][r], bestr_n[rg][r])) {
              bestr_v[rg][r] = x;
              bestr_n[rg][r] = n;
            }
          }
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int n = tile * tw + col_of(q);
        const float v = (F32 ? acc4[q >> 2][t][q & 3] : acc[t][q]) + bias_v[q];
        if (col_of(q) < tw && n < N && argmax_better(v, n, best_v[t], best_n[t])) {
          best_v[t] = v;
          best_n[t] = n;
        }
      }
    zero_acc();
  };

  // Pipeline: stages s + 1 .. s + NS - 1 load while s computes; unrolled by
  // the ring length so the ring slots are registers.
  static_for<0, NS - 1>([&](auto pc) {
    static_for<0, NV>([&](auto vc) { issue(vc, pc); });
    advance();
    __builtin_amdgcn_sched_barrier(0);
  });
  to_lds(std::integral_constant<int, 0>{}, 0);
  lds_barrier();
  // 16-bit: stage s + 1 goes to LDS first, then the stage's MFMAs. fp32
  // (MFMA-bound): the first compute step's MFMAs are issued before the
  // wait for stage s + 1's loads and its LDS stores, so the MFMA pipe has
  // queued work while the wave waits on memory.
  auto step = [&](auto rc, int s) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::value;  // s % NS
    using nslot = std::integral_constant<int, (r + NS - 1) % NS>;
    constexpr int JS = F32 ? 1 : 0;  // compute steps before the LDS stores
    __builtin_amdgcn_sched_barrier(0);
    compute(s & 1, nslot{}, std::integral_constant<int, 0>{}, std::integral_constant<int, JS>{});
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < total) to_lds(std::integral_constant<int, (r + 1) % NS>{}, (s + 1) & 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(s & 1, nslot{}, std::integral_constant<int, JS>{}, std::integral_constant<int, KS>{});
    advance();
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  };
  // nst is a multiple of NS (the host checks it), so ring slot s % NS of
  // stage s is the same compile-time slot in every tile
  for (int i = 0; i < ntl; ++i) {
    load_bias(b + i * grid);
    for (int s0 = 0; s0 < nst; s0 += NS) {
      const int s = i * nst + s0;
      static_for<0, NS>([&](auto rc) { step(rc, s + decltype(rc)::value); });
    }
    end_tile(b + i * grid);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the last stage

  // ---- publish: the lanes holding other columns of the same rows (l ^ 32;
  // fp32 also l ^ 16) merge; then the 8 waves' maxima of a row meet in LDS;
  // one atomic max per row ----------------------------------------------------
#pragma unroll
  for (int t = 0; t < MT; ++t) {
#pragma unroll
    for (int sh = F32 ? 16 : 32; sh <= 32; sh *= 2) {
      const float ov = __shfl_xor(best_v[t], sh, 64);
      const int on = __shfl_xor(best_n[t], sh, 64);
      if (argmax_better(ov, on, best_v[t], best_n[t])) {
        best_v[t] = ov;
        best_n[t] = on;
      }
    }
    if (lane < TR)
      s_key[wave][TR * t + lane] =
          best_n[t] == 0x7fffffff ? 0ull : argmax_key(best_v[t], best_n[t]);
  }
  if constexpr (R8) {
    // the 16 column lanes of each remainder row (the other lane groups hold
    // the same values)
#pragma unroll
    for (int rg = 0; rg < 2; ++rg)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int sh = 1; sh < 16; sh *= 2) {
          const float ov = __shfl_xor(bestr_v[rg][r], sh, 64);
          const int on = __shfl_xor(bestr_n[rg][r], sh, 64);
          if (argmax_better(ov, on, bestr_v[rg][r], bestr_n[rg][r])) {
            bestr_v[rg][r] = ov;
            bestr_n[rg][r] = on;
          }
        }
        if (lane == 0)
          s_key[wave][16 * MT + 4 * rg + r] =
              bestr_n[rg][r] == 0x7fffffff ? 0ull : argmax_key(bestr_v[rg][r], bestr_n[rg][r]);
      }
  }
  __syncthreads();
  if (th < a.M) {
    unsigned long long k = s_key[0][th];
#pragma unroll
    for (int w = 1; w < 8; ++w) k = s_key[w][th] > k ? s_key[w][th] : k;
    key_max(a.keys, th, k);
  }
  wait_stores();
  __syncthreads();
  if (th == 0) s_flag = ticket_add(a.ticket) == (unsigned)(grid - 1);
  __syncthreads();
  if (!s_flag) return;
  VerifyOut o;
  o.draft = a.draft;
  o.accept = a.accept;
  o.accepted_n = a.accepted_n;
  o.corrected = a.corrected;
  o.top = a.top;
  o.S_seq = a.S_seq;
  o.D = a.D;
  o.multi = a.multi;
  o.textbook = a.textbook;
  verify_finish(a.keys, a.M, o, s_top, s_draft);
  if (th == 0) ticket_reset(a.ticket);
}

}  // namespace mtp
