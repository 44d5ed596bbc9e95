// Instantiations of the persistent verify GEMM (skv.hpp).
#include "skv.hpp"

namespace mtp {

SkvKernel skv_pick(int ct, int mt) {
  if (ct == MTP_BF16) {
    if (mt == 1) return skv_kernel<MTP_BF16, 1>;
    if (mt == 2) return skv_kernel<MTP_BF16, 2>;
  } else if (ct == MTP_F16) {
    if (mt == 1) return skv_kernel<MTP_F16, 1>;
    if (mt == 2) return skv_kernel<MTP_F16, 2>;
  } else if (ct == MTP_F32) {
    if (mt == 1) return skv_kernel<MTP_F32, 1>;
    if (mt == 2) return skv_kernel<MTP_F32, 2>;
    if (mt == 3) return skv_kernel<MTP_F32, 3>;
    if (mt == 4) return skv_kernel<MTP_F32, 4>;
  }
  return nullptr;
}

}  // namespace mtp
