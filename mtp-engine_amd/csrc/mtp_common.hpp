// Shared device helpers for the gfx950 kernels: vector types, dtype
// conversions, MFMA wrappers and the argmax ordering torch uses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/mtp_hip.h"

namespace mtp {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kWave = 64;

__host__ __device__ constexpr int dtype_bytes(int dt) {
  return dt == MTP_F32 ? 4
       : dt == MTP_BF16 ? 2
       : dt == MTP_F16 ? 2
       : dt == MTP_FP8E4M3 ? 1
       : dt == MTP_U8 ? 1
       : dt == MTP_I8 ? 1
       : dt == MTP_I32 ? 4
       : dt == MTP_I64 ? 8 : 0;
}

// ---- scalar conversions ---------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h;
  uint16_t b = (uint16_t)bits16;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// Load element i of a tensor of dtype dt (F32/BF16/F16) as fp32.
__device__ __forceinline__ float load_as_f32(const void *p, int dt, int64_t i) {
  if (dt == MTP_F32) return ((const float *)p)[i];
  uint32_t b = ((const uint16_t *)p)[i];
  return dt == MTP_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Round fp32 to the storage dtype (round-to-nearest-even, as torch's .to()).
__device__ __forceinline__ void store_from_f32(void *p, int dt, int64_t i, float v) {
  if (dt == MTP_F32) {
    ((float *)p)[i] = v;
  } else if (dt == MTP_BF16) {
    __bf16 h = (__bf16)v;
    ((__bf16 *)p)[i] = h;
  } else {
    _Float16 h = (_Float16)v;
    ((_Float16 *)p)[i] = h;
  }
}

// Pack two fp32 into two 16-bit floats of type CT (BF16 or F16), RNE.
template <int CT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (CT == MTP_BF16) {
    bf16x2 r;
    r[0] = (__bf16)a;
    r[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, r);
  } else {
    f16x2 r;
    r[0] = (_Float16)a;
    r[1] = (_Float16)b;
    return __builtin_bit_cast(uint32_t, r);
  }
}

// Unpack a dword holding two 16-bit floats of type DT into fp32.
template <int DT>
__device__ __forceinline__ f32x2 unpack2(uint32_t w) {
  f32x2 r;
  if constexpr (DT == MTP_BF16) {
    r[0] = __uint_as_float(w << 16);
    r[1] = __uint_as_float(w & 0xffff0000u);
  } else {
    r[0] = f16_bits_to_f32(w & 0xffffu);
    r[1] = f16_bits_to_f32(w >> 16);
  }
  return r;
}

// Two fp8 e4m3fn values (the 16-bit half `hi` of w) -> two 16-bit floats of
// type CT, exact (every e4m3fn value is representable in bf16 and f16).
template <int CT, bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_ct(uint32_t w) {
  if constexpr (CT == MTP_BF16) {
    return __builtin_bit_cast(uint32_t,
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  } else {
    return __builtin_bit_cast(uint32_t,
                              __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
}

__device__ __forceinline__ f32x2 fp8x2_to_f32(uint32_t w, bool hi) {
  return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true)
            : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
}

// ---- MFMA ------------------------------------------------------------------
// 16x16 output tile, fp32 accumulate. Operand lane layout (wave64):
//   A (16 x Kstep): lane l holds row (l % 16), k-slots 8*(l/16) .. +7
//   B (Kstep x 16): lane l holds col (l % 16), k-slots 8*(l/16) .. +7
//   D (16 x 16):    lane l holds col (l % 16), rows 4*(l/16) .. +3
// (for the f32 variant, Kstep = 4 and each lane holds one k-slot, l / 16).

template <int CT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (CT == MTP_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
}

__device__ __forceinline__ f32x4 mfma16_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
// 16 independent 4 x 4 x 1 fp32 products: block b = lane / 4 takes A from
// lanes 4 b .. 4 b + 3 and B from the same lanes; register r of lane l
// accumulates A[lane 4 b + r] * B[lane l] (layout checked on the device).
__device__ __forceinline__ f32x4 mfma4_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
}

// ---- compile-time loops and split waits -------------------------------------
// f(integral_constant<int, I>) for I = LO .. HI - 1, each a compile-time
// index (register arrays indexed by it stay in registers).
template <int LO, int HI, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (LO < HI) {
    f(std::integral_constant<int, LO>{});
    static_for<LO + 1, HI>(f);
  }
}

// Wait until at most N vector-memory loads of this wave are outstanding and
// its LDS accesses have completed, then meet the workgroup at a barrier.
// Unlike __syncthreads() this does not drain every load: later loads stay in
// flight. The memory clobber keeps the compiler from moving memory accesses
// across it.
template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
// LDS accesses completed, then the workgroup barrier; vector-memory loads
// stay in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---- cross-lane reductions without LDS ----------------------------------------
// v_permlane16_swap(x, x) gives lane l the pair (x[l], x[l ^ 16]) and
// v_permlane32_swap(x, x) the pair (x[l], x[l ^ 32]) (in lane order), so
// two of them reduce over the lanes l, l ^ 16, l ^ 32, l ^ 48 on the VALU.
__device__ __forceinline__ float max_over_lane_groups(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float sum_over_lane_groups(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// ---- argmax ordering (torch.argmax) ---------------------------------------
// NaN is the maximum; among equal values (or among NaNs) the lower index wins.
__device__ __forceinline__ bool argmax_better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

// ---- memory ---------------------------------------------------------------
__device__ __forceinline__ u32x4 ld_nt16(const void *p) {
  return __builtin_nontemporal_load((const u32x4 *)p);
}
__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }

// ---- cross-workgroup hand-off ----------------------------------------------
// Data handed between workgroups of one launch (split-K partials, argmax
// keys, block maxima) is only ever accessed through agent-scope atomics or
// sc1 buffer accesses, which gfx950 performs at the device coherence point,
// past the per-XCD L2s: the producer publishes, waits until its stores have
// completed (s_waitcnt vmcnt(0): acknowledged by the coherence point), meets
// its workgroup at a barrier, then one thread bumps the arrival ticket with
// an agent-scope RMW; the workgroup that sees the final count issues its
// coherent loads only after that (control dependency and barrier), so they
// cannot be served from a copy older than the producers' completed stores.
// The ordering rests on these hardware rules rather than on a release /
// acquire pair: on gfx950 an agent-scope acquire is an L2 invalidate
// (buffer_inv sc1) of the whole XCD, under every other workgroup there, and
// measured 6-7 us per launch on the split-K kernels (fp8 M = 8 linear
// 18.0 -> 24.8 us, fp32 M = 16 9.9 -> 13.7 us); the release alone (an L2
// write-back per arriving workgroup) adds about 1 us and orders nothing
// without the acquire.
__device__ __forceinline__ void pub_f32(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pub_i32(int *p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float get_f32(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int get_i32(const int *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Every thread: wait for its own stores/atomics to complete.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }
// Split-K grid of G column tiles x S splits: (tile, split) of block b. With
// xg and G % 8 == 0 the S splits of a tile are blocks of one XCD (blocks
// are dealt to the 8 XCDs as b mod 8), so a tile's hand-off and arrival
// ticket stay on one XCD; otherwise the splits of a tile are consecutive
// blocks. Any bijection gives the same result.
__device__ __forceinline__ void split_tile_of(int b, int G, int S, bool xg, int &tile, int &sp) {
  if (xg && S > 1 && (G & 7) == 0) {
    const int r = b >> 3, t8 = r / S;
    tile = 8 * t8 + (b & 7);
    sp = r - t8 * S;
  } else {
    tile = b / S;
    sp = b - tile * S;
  }
}
// Arrival count at the coherence point (returns the previous value).
__device__ __forceinline__ unsigned ticket_add(unsigned *t) {
  return __hip_atomic_fetch_add(t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ticket_reset(unsigned *t) {
  __hip_atomic_store(t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace mtp
