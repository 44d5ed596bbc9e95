// Instantiations of the x-resident skinny RMSNorm -> linear kernel (skp.hpp)
// for bf16 x.
#include "skp.hpp"

namespace mtp {


template <int WT, int MT, int TA, bool H8>
static SkpKernel skp_pick_g(bool gam) {
  return gam ? skp_kernel<MTP_BF16, WT, MT, TA, true, H8> : skp_kernel<MTP_BF16, WT, MT, TA, false, H8>;
}

template <int WT, int MT, bool H8>
static SkpKernel skp_pick_ta(int ta, bool gam) {
  if (ta == 1) return skp_pick_g<WT, MT, 1, H8>(gam);
  if (ta == 2) return skp_pick_g<WT, MT, 2, H8>(gam);
  if (ta == 4) return skp_pick_g<WT, MT, 4, H8>(gam);
  return nullptr;
}

template <int WT>
static SkpKernel skp_pick_mt(int mt, int ta, bool gam, bool h8) {
  if (h8) return mt == 1 ? skp_pick_ta<WT, 1, true>(ta, gam) : nullptr;
  if (mt == 1) return skp_pick_ta<WT, 1, false>(ta, gam);
  if (mt == 2) return skp_pick_ta<WT, 2, false>(ta, gam);
  if (mt == 3) return skp_pick_ta<WT, 3, false>(ta, gam);
  if (mt == 4) return skp_pick_ta<WT, 4, false>(ta, gam);
  return nullptr;
}

SkpKernel skp_pick_bf16(int wt, int mt, int ta, bool gam, bool h8) {
  if (wt == MTP_FP8E4M3) return skp_pick_mt<MTP_FP8E4M3>(mt, ta, gam, h8);
  if (wt == MTP_BF16) return skp_pick_mt<MTP_BF16>(mt, ta, gam, h8);
  return nullptr;
}

}  // namespace mtp
