// Small fp32 RMSNorm -> linear for gfx950 (TF32 off), one launch of
// 16-column workgroups: sf32_kernel for at most 16 rows of fp32 x and
// K <= 1024 (one round trip of loads), sf32s_kernel (below) for larger K or
// 17 .. 32 rows (each wave's K-range streamed through LDS).
//
//   y[m, n] = (rs[m] * sum_k (x[m, k] gamma[k]) W[n, k] + bias[n]) * scale,
//   rs[m] = 1 / sqrt(mean_k x[m, k]^2 + eps) (norm) or 1
//
// The shape (the fp32 RMSNorm+linear configuration: x [16, 1024],
// W [4096, 1024]) moves 16.8 MB and is bound by launch latency and the
// first round trip, not by sustained bandwidth. So every workgroup takes
// only 16 columns (N / 16 workgroups: 256 for N = 4096, every CU), and
// every load of the launch goes out at once: wave w of the NW covers
// k = KPW w .. KPW w + KPW - 1 (KPW = 1024 / NW) of the 16 W rows and the
// 16 x rows. The loads go straight to a wave-private LDS area (buffer loads
// with the LDS bit, no VGPRs), each instruction 4 rows x 256 contiguous
// bytes: k-block b (64 k) of rows 4 q .. 4 q + 3 for instruction 4 b + q,
// all of x first, then W. This pattern streams faster than loading each
// lane's MFMA operand slot directly (16 rows x 64 bytes per instruction):
// 6.35 against 7.45 us per call at the shape above. In LDS, 16-byte chunk c
// of row r (of a k-block) sits at slot c ^ r, so the operand reads below
// (16 rows, one chunk) hit 16 different bank groups. As soon as a k-block
// of W has landed its 16 MFMAs run: lane l = 16 g + r reads, for
// each 16-k chunk j, W[n0 + r] and x[r] at k = KPW w + 16 j + 4 g .. + 3,
// its slot of 4 consecutive v_mfma_f32_16x16x4_f32 (A = W rows, B = x
// rows, k-slot g). x * gamma is formed in fp32 registers and the squares
// of x are summed on the way; the waves' 16x16 sums and row squares meet in
// LDS in a fixed order.
#pragma once

#include "mtp_common.hpp"
#include "sf32_args.hpp"
#include "wstream.hpp"

namespace mtp {

// 16 bytes per lane from a buffer straight into LDS (lane i writes bytes
// 16 i .. 16 i + 15 after `lds`); device pass only (the host pass cannot
// form the LDS address-space pointer).
__device__ __forceinline__ void sf32_dma16(__amdgpu_buffer_rsrc_t r, unsigned char *lds,
                                           uint32_t voff, int aux) {
#if defined(__HIP_DEVICE_COMPILE__)
  if (aux)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                             voff, 0, 0, 2);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16,
                                             voff, 0, 0, 0);
#else
  (void)r; (void)lds; (void)voff; (void)aux;
#endif
}

template <bool GAM, int NW>
__global__ void __launch_bounds__(64 * NW, 1) sf32_kernel(const Sf32Args a) {
  constexpr int KPW = kSf32MaxK / NW;  // k per wave
  constexpr int CPW = KPW / 16;        // 16-k chunks (4 MFMA k-slots x 4) per wave
  constexpr int KB = KPW / 64;         // 64-k blocks per wave (4 load instructions each)
  static_assert(KPW % 64 == 0 && 2 * CPW < 64, "k-blocks of 64; vmcnt is 6 bits");
  // One LDS object (with several, the compiler waits for every LDS copy in
  // flight before each LDS read): per wave W then x, each [KB][16 rows][16
  // chunks of 16 bytes]; then the waves' sums, row squares and gamma.
  constexpr int LD = NW * 2 * KB * 4096;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[LD + NW * (64 * 16 + 16 * 4 + 64 * 16)];
  f32x4(*const s_acc)[64] = (f32x4(*)[64])(lds + LD);
  float(*const s_ss)[16] = (float(*)[16])(lds + LD + NW * 64 * 16);
  f32x4(*const s_g)[64] = (f32x4(*)[64])(lds + LD + NW * (64 * 16 + 16 * 4));
  const int th = threadIdx.x, lane = th & 63;
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int n0 = blockIdx.x * 16;
  const int K = a.K;
  // rows past M / N and k past K read 0 through the descriptors' range
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(a.w + (int64_t)n0 * K, (uint32_t)(min(16, a.N - n0) * K) * 4u);
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)(a.M * K) * 4u);
  const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.gamma, GAM ? (uint32_t)K * 4u : 0u);
  // Issued before the W / x copies, so the copies' waits below count only
  // each other: gamma of the wave's KPW k (lane L < KPW / 4: k KPW w + 4 L
  // .. + 3) and the raw bias of the lane's output columns n0 + 4 g + e.
  f32x4 gl = f32x4{1.f, 1.f, 1.f, 1.f};
  if constexpr (GAM)
    gl = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                   grs, lane < KPW / 4 ? (uint32_t)(KPW * wave + 4 * lane) * 4u : kOOB, 0, 0));
  uint32_t braw[4] = {0u, 0u, 0u, 0u};
  if (a.bias) {
    const uint32_t nb = (uint32_t)(n0 + 4 * g);
    if (a.bias_dt == MTP_F32) {
      const __amdgpu_buffer_rsrc_t brs = make_rsrc(a.bias, (uint32_t)a.N * 4u);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        braw[e] = __builtin_amdgcn_raw_buffer_load_b32(brs, (nb + e) * 4u, 0, 0);
    } else {
      const __amdgpu_buffer_rsrc_t brs = make_rsrc(a.bias, (uint32_t)a.N * 2u);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        braw[e] = __builtin_amdgcn_raw_buffer_load_b16(brs, (nb + e) * 2u, 0, 0);
    }
  }
  // Copy instruction i = 4 b + q: rows rr = 4 q + lane / 16, k-block b;
  // lane slot s = lane % 16 takes chunk s ^ rr of its row (k = KPW w +
  // 64 b + 4 (s ^ rr)); chunks at or past K (K % 16 == 0) use an
  // out-of-range offset and land as zeros. All of x (L2-resident after the
  // first workgroups) goes first, then W from HBM: 6.35 against 6.72 us per
  // call with the two interleaved per k-block.
  unsigned char *const lw = lds + 2 * KB * 4096 * wave;
  unsigned char *const lx = lw + KB * 4096;
  uint32_t ro[4 * KB];
#pragma unroll
  for (int i = 0; i < 4 * KB; ++i) {
    const int rr = 4 * (i & 3) + (lane >> 4);
    const int k = KPW * wave + 64 * (i >> 2) + 4 * ((lane & 15) ^ rr);
    ro[i] = k < K ? (uint32_t)(rr * K + k) * 4u : kOOB;
    sf32_dma16(xrs, lx + 1024 * i, ro[i], 0);
  }
#pragma unroll
  for (int i = 0; i < 4 * KB; ++i) sf32_dma16(wrs, lw + 1024 * i, ro[i], 1);
  f32x4 gv[CPW];
  if constexpr (GAM) {
    s_g[wave][lane] = gl;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < CPW; ++i) gv[i] = s_g[wave][4 * i + g];
  }

  // four independent accumulators (one per e), so consecutive MFMAs do not
  // wait for each other's results; summed in a fixed order below
  float ss = 0.f;
  f32x4 ac[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) ac[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  static_for<0, KB>([&](auto bc) {
    constexpr int b = decltype(bc)::value;
    // k-block b's 4 W copies (and every earlier copy, x included) have
    // landed in LDS
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * (KB - 1 - b)) : "memory");
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 4 * b + jj;
      const int off = 4096 * b + 256 * r + 16 * ((4 * jj + g) ^ r);
      const f32x4 wv = *(const f32x4 *)(lw + off);
      const f32x4 xv = *(const f32x4 *)(lx + off);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xe = xv[e];
        ss = __builtin_fmaf(xe, xe, ss);
        const float bx = GAM ? xe * gv[j][e] : xe;
        ac[e] = mfma16_f32(wv[e], bx, ac[e]);
      }
    }
  });
  const f32x4 acc = ((ac[0] + ac[1]) + ac[2]) + ac[3];
  // row squares: the 4 lane groups of row r, then the waves in order
  ss += __shfl_xor(ss, 16, 64);
  ss += __shfl_xor(ss, 32, 64);
  if (g == 0) s_ss[wave][r] = ss;
  s_acc[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  // lane holds D[n = 4 g + e][m = r]; the waves' sums in wave order
  f32x4 t = s_acc[0][lane];
  float sq = s_ss[0][r];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    t += s_acc[w][lane];
    sq += s_ss[w][r];
  }
  const float rs = a.norm ? 1.0f / sqrtf(sq / (float)K + a.eps) : 1.0f;
  const int m = r;
  if (m >= a.M) return;
  const int n = n0 + 4 * g;
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float bi = !a.bias                  ? 0.f
                     : a.bias_dt == MTP_F32   ? __builtin_bit_cast(float, braw[e])
                     : a.bias_dt == MTP_BF16 ? bf16_bits_to_f32(braw[e])
                                              : f16_bits_to_f32(braw[e]);
    o[e] = (a.bias ? t[e] * rs + bi : t[e] * rs) * a.scale;
  }
  float *yr = a.y + (int64_t)m * a.N;
  if (n + 3 < a.N && (a.N & 3) == 0) {
    *(f32x4 *)(yr + n) = f32x4{o[0], o[1], o[2], o[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < a.N) yr[n + e] = o[e];
  }
}

// 4 bytes per lane from a buffer straight into LDS (lane i writes bytes
// 4 i .. 4 i + 3 after `lds`); device pass only.
__device__ __forceinline__ void sf32_dma4(__amdgpu_buffer_rsrc_t r, unsigned char *lds,
                                          uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 4,
                                           voff, 0, 0, 0);
#else
  (void)r; (void)lds; (void)voff;
#endif
}

// Streaming form for K > kSf32MaxK or 17 .. 32 rows (the same 16-column
// workgroups, the same sums; MT = 1 or 2 tiles of 16 x rows): wave w owns
// k = KW w .. KW w + KW - 1 (KW = K / NW rounded up to 64) and streams it in
// blocks of 64 k through a ring of kSf32Ring blocks in its own LDS area
// (with one block per wave, the other waves of its SIMD keep the memory
// busy while it waits). A block's copies: gamma (4 bytes per lane, 64 k),
// then the MT x tiles, then W, each 4 rows x 256 contiguous bytes per
// instruction with the chunk c of row r at slot c ^ r, as above. Block b is
// waited for with a fixed count (the kSf32Ring - 1 younger blocks in
// flight), its 16 MT MFMAs run (one W fragment feeds every tile), and its
// slot is refilled with block b + kSf32Ring; refills past the wave's range
// use out-of-range offsets (zeros, no memory access) so the count stays
// fixed. Wave t < MT finishes row tile t.
template <bool GAM, int NW, int MT>
__global__ void __launch_bounds__(64 * NW, 1) sf32s_kernel(const Sf32Args a) {
  constexpr int RD = kSf32Ring;
  constexpr int WB = 4096;                       // one 64-k block of 16 rows
  constexpr int GO = (1 + MT) * WB;                // gamma's offset in a slot
  constexpr int SLOT = GO + (GAM ? 256 : 0);        // W, MT x tiles, gamma
  constexpr int C = 4 + 4 * MT + (GAM ? 1 : 0);     // copy instructions per block
  static_assert((RD - 1) * C < 64, "vmcnt is 6 bits");
  constexpr int LD = NW * RD * SLOT;
  // one LDS object (see sf32_kernel): the rings, then the waves' sums
  __shared__ __attribute__((aligned(1024))) unsigned char lds[LD + NW * MT * (64 * 16 + 16 * 4)];
  f32x4(*const s_acc)[MT][64] = (f32x4(*)[MT][64])(lds + LD);
  float(*const s_ss)[MT][16] = (float(*)[MT][16])(lds + LD + NW * MT * 64 * 16);
  const int th = threadIdx.x, lane = th & 63;
  const int wave = __builtin_amdgcn_readfirstlane(th >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int n0 = blockIdx.x * 16;
  const int K = a.K;
  const int KW = (K + 64 * NW - 1) / (64 * NW) * 64;  // k per wave
  const int nb = KW / 64;                             // blocks per wave
  const int kw0 = KW * wave;
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(a.w + (int64_t)n0 * K, (uint32_t)(min(16, a.N - n0) * K) * 4u);
  const __amdgpu_buffer_rsrc_t xrs = make_rsrc(a.x, (uint32_t)(a.M * K) * 4u);
  const __amdgpu_buffer_rsrc_t grs = make_rsrc(a.gamma, GAM ? (uint32_t)K * 4u : 0u);
  // raw bias of the lane's output columns n0 + 4 g + e, before the ring
  uint32_t braw[4] = {0u, 0u, 0u, 0u};
  if (a.bias) {
    const uint32_t nbias = (uint32_t)(n0 + 4 * g);
    if (a.bias_dt == MTP_F32) {
      const __amdgpu_buffer_rsrc_t brs = make_rsrc(a.bias, (uint32_t)a.N * 4u);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        braw[e] = __builtin_amdgcn_raw_buffer_load_b32(brs, (nbias + e) * 4u, 0, 0);
    } else {
      const __amdgpu_buffer_rsrc_t brs = make_rsrc(a.bias, (uint32_t)a.N * 2u);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        braw[e] = __builtin_amdgcn_raw_buffer_load_b16(brs, (nbias + e) * 2u, 0, 0);
    }
  }
  unsigned char *const ring = lds + wave * RD * SLOT;
  // copy q of a block: row rr = 4 q + lane / 16, chunk (lane % 16) ^ rr
  int rq[4], kq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    rq[q] = 4 * q + (lane >> 4);
    kq[q] = 4 * ((lane & 15) ^ rq[q]);
  }
  auto issue = [&](int blk, auto slotc) __attribute__((always_inline)) {
    constexpr int slot = decltype(slotc)::value;
    unsigned char *const sb = ring + slot * SLOT;
    const int kb = kw0 + 64 * blk;
    const bool live = blk < nb;
    if constexpr (GAM)
      sf32_dma4(grs, sb + GO, live && kb + lane < K ? (uint32_t)(kb + lane) * 4u : kOOB);
    uint32_t off[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int k = kb + kq[q];
      off[q] = live && k < K ? (uint32_t)(rq[q] * K + k) * 4u : kOOB;
    }
    // x tile t: rows 16 t + rr (rows past M read 0 through the range)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        sf32_dma16(xrs, sb + (1 + t) * WB + 1024 * q,
                   off[q] == kOOB ? kOOB : off[q] + (uint32_t)(64 * t * K), 0);
#pragma unroll
    for (int q = 0; q < 4; ++q) sf32_dma16(wrs, sb + 1024 * q, off[q], 1);
  };
  static_for<0, RD>([&](auto sc) { issue(decltype(sc)::value, sc); });

  float ss[MT];
  f32x4 ac[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    ss[t] = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ac[t][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int b0 = 0; b0 < nb; b0 += RD) {
    static_for<0, RD>([&](auto sc) {
      constexpr int slot = decltype(sc)::value;
      const int blk = b0 + slot;
      if (blk < nb) {
        // block blk's copies have landed (the RD - 1 younger blocks may not)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((RD - 1) * C) : "memory");
        const unsigned char *const sb = ring + slot * SLOT;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int off = 256 * r + 16 * ((4 * jj + g) ^ r);
          const f32x4 wv = *(const f32x4 *)(sb + off);
          f32x4 xv[MT];
#pragma unroll
          for (int t = 0; t < MT; ++t) xv[t] = *(const f32x4 *)(sb + (1 + t) * WB + off);
          f32x4 gv = f32x4{1.f, 1.f, 1.f, 1.f};
          if constexpr (GAM) gv = *(const f32x4 *)(sb + GO + 64 * jj + 16 * g);
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float xe = xv[t][e];
              ss[t] = __builtin_fmaf(xe, xe, ss[t]);
              const float bx = GAM ? xe * gv[e] : xe;
              ac[t][e] = mfma16_f32(wv[e], bx, ac[t][e]);
            }
        }
        // the slot's reads are done before its refill is issued
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(blk + RD, sc);
      }
    });
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // refills past the end
#pragma unroll
  for (int tt = 0; tt < MT; ++tt) {
    float v = ss[tt];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (g == 0) s_ss[wave][tt][r] = v;
    s_acc[wave][tt][lane] = ((ac[tt][0] + ac[tt][1]) + ac[tt][2]) + ac[tt][3];
  }
  __syncthreads();
  // wave tt < MT finishes row tile tt, the waves' sums in wave order
  if (wave >= MT) return;
  const int tt = wave;
  f32x4 t = s_acc[0][tt][lane];
  float sq = s_ss[0][tt][r];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    t += s_acc[w][tt][lane];
    sq += s_ss[w][tt][r];
  }
  const float rs = a.norm ? 1.0f / sqrtf(sq / (float)K + a.eps) : 1.0f;
  const int m = 16 * tt + r;
  if (m >= a.M) return;
  const int n = n0 + 4 * g;
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float bi = !a.bias                  ? 0.f
                     : a.bias_dt == MTP_F32   ? __builtin_bit_cast(float, braw[e])
                     : a.bias_dt == MTP_BF16 ? bf16_bits_to_f32(braw[e])
                                              : f16_bits_to_f32(braw[e]);
    o[e] = (a.bias ? t[e] * rs + bi : t[e] * rs) * a.scale;
  }
  float *yr = a.y + (int64_t)m * a.N;
  if (n + 3 < a.N && (a.N & 3) == 0) {
    *(f32x4 *)(yr + n) = f32x4{o[0], o[1], o[2], o[3]};
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n + e < a.N) yr[n + e] = o[e];
  }
}

}  // namespace mtp
