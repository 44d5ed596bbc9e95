// Instantiations of the grouped INT4 GEMM (int4g.hpp).
#include "int4g.hpp"

namespace mtp {

template <bool TWOS>
static I4Kernel int4_gemm_pick_t(int mt, int na, int layout) {
  if (layout == kI4Rows4) {
    if (mt == 1 && na == 1) return int4_gemm_kernel<1, 1, 4, false, TWOS>;
    if (mt == 2 && na == 1) return int4_gemm_kernel<2, 1, 4, false, TWOS>;
    if (mt == 4 && na == 2) return int4_gemm_kernel<4, 2, 4, false, TWOS>;
  } else if (layout == kI4Rows4KHalves) {
    if (mt == 1 && na == 1) return int4_gemm_kernel<1, 1, 8, true, TWOS>;
    if (mt == 2 && na == 1) return int4_gemm_kernel<2, 1, 8, true, TWOS>;
    if (mt == 4 && na == 2) return int4_gemm_kernel<4, 2, 8, true, TWOS>;
  }
  return nullptr;
}

I4Kernel int4_gemm_pick(int mt, int na, int layout, bool twos) {
  return twos ? int4_gemm_pick_t<true>(mt, na, layout) : int4_gemm_pick_t<false>(mt, na, layout);
}

template <int XDT>
I4PrepKernel int4_prep_x(int gdt) {
  switch (gdt) {
    case -1: return int4_prep_kernel<XDT, -1>;
    case MTP_F32: return int4_prep_kernel<XDT, MTP_F32>;
    case MTP_BF16: return int4_prep_kernel<XDT, MTP_BF16>;
    case MTP_F16: return int4_prep_kernel<XDT, MTP_F16>;
  }
  return nullptr;
}

I4PrepKernel int4_prep(int xdt, int gdt) {
  switch (xdt) {
    case MTP_F32: return int4_prep_x<MTP_F32>(gdt);
    case MTP_BF16: return int4_prep_x<MTP_BF16>(gdt);
    case MTP_F16: return int4_prep_x<MTP_F16>(gdt);
  }
  return nullptr;
}

}  // namespace mtp
