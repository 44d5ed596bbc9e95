// Instantiations of the x-resident skinny RMSNorm -> linear kernel (skp.hpp)
// for bf16 x.
#include "skp.hpp"

namespace mtp {


template <int WT, int MT, int TA>
static SkpKernel skp_pick_g(bool gam) {
  return gam ? skp_kernel<MTP_BF16, WT, MT, TA, true> : skp_kernel<MTP_BF16, WT, MT, TA, false>;
}

template <int WT, int MT>
static SkpKernel skp_pick_ta(int ta, bool gam) {
  if (ta == 1) return skp_pick_g<WT, MT, 1>(gam);
  if (ta == 2) return skp_pick_g<WT, MT, 2>(gam);
  if (ta == 4) return skp_pick_g<WT, MT, 4>(gam);
  return nullptr;
}

template <int WT>
static SkpKernel skp_pick_mt(int mt, int ta, bool gam) {
  if (mt == 1) return skp_pick_ta<WT, 1>(ta, gam);
  if (mt == 2) return skp_pick_ta<WT, 2>(ta, gam);
  if (mt == 3) return skp_pick_ta<WT, 3>(ta, gam);
  if (mt == 4) return skp_pick_ta<WT, 4>(ta, gam);
  return nullptr;
}

SkpKernel skp_pick_bf16(int wt, int mt, int ta, bool gam) {
  if (wt == MTP_FP8E4M3) return skp_pick_mt<MTP_FP8E4M3>(mt, ta, gam);
  if (wt == MTP_BF16) return skp_pick_mt<MTP_BF16>(mt, ta, gam);
  return nullptr;
}

}  // namespace mtp
