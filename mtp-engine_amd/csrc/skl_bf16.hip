// Instantiations of the single-launch skinny RMSNorm -> linear (skl.hpp)
// for bf16 x.
#include "skl.hpp"

namespace mtp {

template <int WT, int MT, int NW>
static SklKernel skl_pick_g(bool gam) {
  return gam ? skl_kernel<MTP_BF16, WT, MT, NW, true> : skl_kernel<MTP_BF16, WT, MT, NW, false>;
}

template <int WT>
static SklKernel skl_pick_w(int mt, int nw, bool gam) {
  if (mt == 1 && nw == 4) return skl_pick_g<WT, 1, 4>(gam);
  if (mt == 1 && nw == 8) return skl_pick_g<WT, 1, 8>(gam);
  if (mt == 2 && nw == 4) return skl_pick_g<WT, 2, 4>(gam);
  if (mt == 2 && nw == 8) return skl_pick_g<WT, 2, 8>(gam);
  return nullptr;
}

SklKernel skl_pick_bf16(int wt, int mt, int nw, bool gam) {
  if (wt == MTP_FP8E4M3) return skl_pick_w<MTP_FP8E4M3>(mt, nw, gam);
  if (wt == MTP_BF16) return skl_pick_w<MTP_BF16>(mt, nw, gam);
  return nullptr;
}

SklKernel skl_pick(int ct, int wt, int mt, int nw, bool gam) {
  if (ct == MTP_BF16) return skl_pick_bf16(wt, mt, nw, gam);
  if (ct == MTP_F16) return skl_pick_f16(wt, mt, nw, gam);
  return nullptr;
}

}  // namespace mtp
