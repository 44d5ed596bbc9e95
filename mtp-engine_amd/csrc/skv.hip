// Instantiations of the persistent verify GEMM (skv.hpp).
#include "skv.hpp"

namespace mtp {

SkvKernel skv_pick(int ct, int mt, bool r8) {
  if (ct == MTP_BF16 && !r8) {
    if (mt == 1) return skv_kernel<MTP_BF16, 1, false>;
    if (mt == 2) return skv_kernel<MTP_BF16, 2, false>;
  } else if (ct == MTP_F16 && !r8) {
    if (mt == 1) return skv_kernel<MTP_F16, 1, false>;
    if (mt == 2) return skv_kernel<MTP_F16, 2, false>;
  } else if (ct == MTP_F32 && !r8) {
    if (mt == 1) return skv_kernel<MTP_F32, 1, false>;
    if (mt == 2) return skv_kernel<MTP_F32, 2, false>;
    if (mt == 3) return skv_kernel<MTP_F32, 3, false>;
    if (mt == 4) return skv_kernel<MTP_F32, 4, false>;
  } else if (ct == MTP_F32) {
    if (mt == 1) return skv_kernel<MTP_F32, 1, true>;
    if (mt == 2) return skv_kernel<MTP_F32, 2, true>;
    if (mt == 3) return skv_kernel<MTP_F32, 3, true>;
  }
  return nullptr;
}

}  // namespace mtp
