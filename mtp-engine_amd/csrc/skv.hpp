// Persistent weight-streaming verify for gfx950: the lm_head pass of
// fused_verify / fused_multi_verify with 16-bit hidden rows and weights and
// no bias.
//
//   top[m] = argmax_n (x[m] . W[n])   (torch.argmax: NaN is the maximum,
//                                      the lowest index wins ties)
//
// One launch of one workgroup per CU streams W once.
// Workgroup b takes the kSkvBN-column tiles b, b + grid, b + 2 grid, ...
// back to back; the stages (64 k = 128 bytes of every W row of a tile) of
// all its tiles form one sequence, so the register rings run across tile
// boundaries without draining; each tile's stages start at 7 b mod nst. 8 waves; wave w owns columns 32 w .. + 31 of
// every tile against all (<= 64) rows, over every k, so a tile ends with
// no reduction between waves. Per stage:
//   * W (256 rows x 128 bytes) comes HBM -> registers with 8-rows x 128-byte
//     non-temporal loads NS - 1 stages ahead, then goes to a double-buffered
//     LDS stage (16-byte chunk c of row r at c ^ sk_swz(r)) one step before use;
//   * x comes from the caller's row-major hidden rows with the same
//     8-rows x 128-byte loads (one per wave per stage), each lane storing
//     its 16 bytes into LDS at their place in the B-operand blocks of the
//     stage; its requests are a fifth of the stage's, so they take little
//     of the memory pipeline the W stream needs;
//   * each wave runs 4 k-steps x MT row tiles of v_mfma_f32_32x32x16.
// At the end of a tile each lane folds its 16 columns of each of its rows
// into a running (max, index). At the end the waves' maxima meet in LDS and
// one lane per row publishes (value, index) as a 64-bit key whose unsigned
// order is the argmax order (order-preserving float bits, then the
// complement of the index) with an atomic max; the last workgroup to
// arrive decodes the keys, runs the acceptance and re-zeroes the keys and
// its ticket for the next launch.
#pragma once

#include "sk.hpp"
#include "skv_args.hpp"
#include "verify_tail.hpp"

namespace mtp {

template <int CT, int MT>
__global__ void __launch_bounds__(512, 1)
skv_kernel(const SkvArgs a) {
  constexpr int BN = kSkvBN;                 // columns per tile
  constexpr int KS = 4;                      // MFMA k-steps per stage
  constexpr int WST = BN * kSkUB;            // W bytes of one stage (32 KB)
  constexpr int XST = MT * KS * 1024;        // x bytes of one stage
  constexpr int NS = 4;                      // register ring stages (loads run NS - 1 ahead)
  constexpr int NWC = WST / 1024 / 8;        // W loads per wave per stage (4)
  constexpr int NXC = (XST / 1024 + 7) / 8;  // x loads per wave per stage (<= 1)
  constexpr int NV = NWC + NXC;
  static_assert(NXC == 1, "one x block per wave and stage at most");
  static_assert((NS - 1) * NV < 64, "vmcnt is 6 bits");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_w[2 * WST];
  __shared__ __attribute__((aligned(1024))) unsigned char lds_x[2 * XST];
  __shared__ unsigned long long s_key[8][64];
  __shared__ int s_flag;
  __shared__ int s_top[64];
  __shared__ int s_draft[64];

  const int th = threadIdx.x, lane = th & 63, wave = th >> 6;
  const int N = a.N, K = a.K, nst = a.nst;
  const int b = blockIdx.x, grid = gridDim.x;
  const int ntl = (a.ntiles - b + grid - 1) / grid;  // this workgroup's tiles (>= 1)
  const int total = ntl * nst;                       // its stages
  // Stage order inside a tile starts at 7 b mod nst: workgroups in step
  // with each other then read different 128-byte offsets of their rows,
  // which spreads the requests over the HBM channels (the same offset of
  // every row at once concentrates them; measured 1.3x slower).
  const int rot = (7 * b) % nst;

  const uint32_t ldw = (uint32_t)K * 2u;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.w, (uint32_t)N * ldw);
  // W load c (c = wave + 8 i): rows 8 c .. 8 c + 7 of the tile, lane l: row
  // 8 c + l / 8, 16-byte chunk (l % 8) ^ sk_swz(row) of the stage's 128 bytes
  uint32_t wvo[NWC];
#pragma unroll
  for (int i = 0; i < NWC; ++i) {
    const int row = 8 * (wave + 8 * i) + (lane >> 3);
    const int chunk = (lane & 7) ^ sk_swz(row);
    wvo[i] = (uint32_t)row * ldw + 16u * chunk;
  }
  // x load of wave w (w < 4 MT): rows 8 w .. 8 w + 7 (rows past M read as
  // zeros), lane l: row 8 w + l / 8, k 8 (l % 8) .. + 7 of the stage, which
  // is lane 32 (c % 2) + row % 32 of B-operand block (row / 32, c / 2), c = l % 8
  const bool xloader = wave < 4 * MT;
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)a.M * ldw);
  const int xrow = 8 * wave + (lane >> 3), xc = lane & 7;
  const uint32_t xvo = (uint32_t)xrow * ldw + 16u * (uint32_t)xc;
  const int xlds = ((xrow >> 5) * KS + (xc >> 1)) * 1024 +
                   ((32 * (xc & 1) + (xrow & 31)) ^ sk_xswz(xc >> 1, xc & 1)) * 16;
  u32x4 wr[NS][NWC];  // W register ring
  u32x4 xr[NS];       // x register ring

  // The stage being issued, as (tile iteration, stage in tile); stages past
  // the last re-read the last one into a slot that is never computed on.
  int is_i = 0, is_st = 0;
  auto issue = [&](auto vc, auto slotc) __attribute__((always_inline)) {
    constexpr int v = decltype(vc)::value, slot = decltype(slotc)::value;
    if constexpr (v < NWC) {
      const int str = is_st + rot < nst ? is_st + rot : is_st + rot - nst;
      const uint32_t off = wvo[v] + (uint32_t)(b + is_i * grid) * (uint32_t)BN * ldw +
                           (uint32_t)str * (uint32_t)kSkUB;
      wr[slot][v] = __builtin_bit_cast(u32x4,
                                       __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2));
    } else {
      const int str = is_st + rot < nst ? is_st + rot : is_st + rot - nst;
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

  f32x16 acc[MT];
  auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[t][e] = 0.f;
  };
  zero_acc();

  const int ag = lane >> 5;
  auto to_lds = [&](auto slotc, int buf) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
#pragma unroll
    for (int v = 0; v < NWC; ++v)
      *(u32x4 *)(lds_w + buf * WST + (wave + 8 * v) * 1024 + lane * 16) = wr[slot][v];
    if (xloader) *(u32x4 *)(lds_x + buf * XST + xlds) = xr[slot];
  };
  // this wave's 32 columns against all rows, the 4 k-steps of the stage in
  // buffer `buf`; the NV loads of the stage NS - 1 ahead spread over them
  auto compute = [&](int buf, auto nslotc) __attribute__((always_inline)) {
    const unsigned char *wb = lds_w + buf * WST;
    const unsigned char *xb = lds_x + buf * XST;
    const int row = 32 * wave + (lane & 31);
    static_for<0, KS>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      static_for<j * NV / KS, (j + 1) * NV / KS>([&](auto vc) { issue(vc, nslotc); });
      const int c = 2 * j + ag;
      const u32x4 av = *(const u32x4 *)(wb + row * kSkUB + ((c ^ sk_swz(row)) << 4));
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const u32x4 bv =
            *(const u32x4 *)(xb + (t * KS + j) * 1024 + ((lane ^ sk_xswz(j, ag)) << 4));
        acc[t] = mfma32<CT>(av, bv, acc[t]);
      }
    });
    advance();
  };

  // Running per-row maximum: lane l covers rows 32 t + l % 32 (t < MT) over
  // the columns 32 wave + 8 (e / 4) + 4 (l / 32) + e % 4 of every tile.
  float best_v[MT];
  int best_n[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    best_v[t] = -__builtin_inff();
    best_n[t] = 0x7fffffff;
  }
  auto end_tile = [&](int tile) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int n = tile * BN + 32 * wave + 8 * (e >> 2) + 4 * ag + (e & 3);
        const float v = acc[t][e];
        if (n < N && argmax_better(v, n, best_v[t], best_n[t])) {
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
  auto step = [&](auto rc, int s) __attribute__((always_inline)) {
    constexpr int r = decltype(rc)::value;  // s % NS
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < total) to_lds(std::integral_constant<int, (r + 1) % NS>{}, (s + 1) & 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(s & 1, std::integral_constant<int, (r + NS - 1) % NS>{});
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
  };
  // nst is a multiple of NS (the host checks it), so ring slot s % NS of
  // stage s is the same compile-time slot in every tile
  for (int i = 0; i < ntl; ++i) {
    for (int s0 = 0; s0 < nst; s0 += NS) {
      const int s = i * nst + s0;
      static_for<0, NS>([&](auto rc) { step(rc, s + decltype(rc)::value); });
    }
    end_tile(b + i * grid);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // loads past the last stage

  // ---- publish: lanes l and l + 32 hold other columns of the same rows; then
  // the 8 waves' maxima of a row meet in LDS; one atomic max per row --------
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const float ov = __shfl_xor(best_v[t], 32, 64);
    const int on = __shfl_xor(best_n[t], 32, 64);
    if (argmax_better(ov, on, best_v[t], best_n[t])) {
      best_v[t] = ov;
      best_n[t] = on;
    }
    if (lane < 32)
      s_key[wave][32 * t + lane] = best_n[t] == 0x7fffffff ? 0ull : argmax_key(best_v[t], best_n[t]);
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
  verify_finish(a.keys, a.M, o, s_top, s_draft);
  if (th == 0) ticket_reset(a.ticket);
}

}  // namespace mtp
