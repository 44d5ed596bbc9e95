// Arguments and instantiation accessors of the grouped INT4 GEMM (int4g.hpp),
// shared by its instantiation unit and the host planner.
#pragma once

#include <stdint.h>

namespace mtp {

struct I4Args {
  const void *xn;         // fp16 x, fragment-major, rows padded to gm * MT * 32
  const float *omul;      // [M] output multiplier of each row
  const uint8_t *packed;  // [N, K / 2]
  const void *scales;     // fp16 [ng, ldst], transposed and column-normalised by the prep kernel
  const float *cmul;      // [ldst] power of two undoing each column's scale normalisation
  int ldst;               // row stride of the transposed scales (>= columns of y covered)
  void *y;                // [M, N] in ydt
  int ydt;
  int yvec;               // N % 4 == 0 and y 8-byte aligned (16-bit ydt)
  int M, N, K, group, ng;
  int glog;               // log2(group) when group is a power of two, else -1
  int nibble;             // MTP_NIBBLE_OFFSET8 / MTP_NIBBLE_TWOS
  int gn, gm;             // column groups of 128 NA and row groups of 32 MT
};

typedef void (*I4Kernel)(I4Args);
typedef void (*I4PrepKernel)(const void *, int64_t, int64_t, const void *, float, int, void *,
                             float *, int64_t, const void *, int, int64_t, int64_t, int64_t,
                             uint16_t *, float *);
// Wave layouts of the GEMM: 4 waves on 4 row groups; 8 waves on 4 row
// groups x 2 k-halves. (4 waves on 2 row groups x 2 k-halves with NA 4, 256
// accumulators per wave, halves the x reads per MFMA but spills and runs
// one wave per SIMD: M 256 K 8192 N 28672 138 us against 127 us.)
constexpr int kI4Rows4 = 0, kI4Rows4KHalves = 1;
// Weight rows of a workgroup: NA 32-row subtiles per wave on each of 4 row
// groups.
inline int int4_bn(int na) { return 128 * na; }
// GEMM kernel for MT 32-row x tiles and NA subtiles per row group ((1, 1),
// (2, 1), (4, 2)) in a wave layout for offset-8 or (twos) two's-complement
// nibbles, or null.
I4Kernel int4_gemm_pick(int mt, int na, int layout, bool twos);
// Prep kernel for x dtype xdt and gamma dtype gdt (-1: no gamma), or null.
I4PrepKernel int4_prep(int xdt, int gdt);

}  // namespace mtp
