// Instantiations of the wave-specialised skinny GEMM (skw.hpp).
#include "skw.hpp"

namespace mtp {

template <int CT, int WT>
SkwKernel skw_pick_w(int mt) {
  if (mt == 1) return skw_kernel<CT, WT, 1>;
  if (mt == 2) return skw_kernel<CT, WT, 2>;
  return nullptr;
}

SkwKernel skw_pick(int ct, int wt, int mt) {
  if (ct == MTP_BF16) {
    if (wt == MTP_FP8E4M3) return skw_pick_w<MTP_BF16, MTP_FP8E4M3>(mt);
    if (wt == MTP_BF16) return skw_pick_w<MTP_BF16, MTP_BF16>(mt);
  } else if (ct == MTP_F16) {
    if (wt == MTP_FP8E4M3) return skw_pick_w<MTP_F16, MTP_FP8E4M3>(mt);
    if (wt == MTP_F16) return skw_pick_w<MTP_F16, MTP_F16>(mt);
  }
  return nullptr;
}

}  // namespace mtp
