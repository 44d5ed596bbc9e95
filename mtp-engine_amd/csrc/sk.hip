// Instantiations of the skinny weight-streaming GEMM (sk.hpp).
#include "sk.hpp"

namespace mtp {

template <int CT, int WT>
SkKernel sk_pick_w(int mt, bool xr) {
  if (mt == 1) return xr ? sk_kernel<CT, WT, 1, true> : sk_kernel<CT, WT, 1, false>;
  if (mt == 2) return xr ? sk_kernel<CT, WT, 2, true> : sk_kernel<CT, WT, 2, false>;
  return nullptr;
}

SkKernel sk_pick(int ct, int wt, int mt, bool xr) {
  if (ct == MTP_BF16) {
    if (wt == MTP_FP8E4M3) return sk_pick_w<MTP_BF16, MTP_FP8E4M3>(mt, xr);
    if (wt == MTP_BF16) return sk_pick_w<MTP_BF16, MTP_BF16>(mt, xr);
  } else if (ct == MTP_F16) {
    if (wt == MTP_FP8E4M3) return sk_pick_w<MTP_F16, MTP_FP8E4M3>(mt, xr);
    if (wt == MTP_F16) return sk_pick_w<MTP_F16, MTP_F16>(mt, xr);
  }
  return nullptr;
}

template <int CT>
SkPrepKernel sk_prep_ct(bool fp8, bool gam) {
  if (fp8) return gam ? sk_prep_kernel<CT, true, true> : sk_prep_kernel<CT, true, false>;
  return gam ? sk_prep_kernel<CT, false, true> : sk_prep_kernel<CT, false, false>;
}

SkPrepKernel sk_prep_pick(int ct, int wt, bool gam) {
  if (ct == MTP_BF16) return sk_prep_ct<MTP_BF16>(wt == MTP_FP8E4M3, gam);
  if (ct == MTP_F16) return sk_prep_ct<MTP_F16>(wt == MTP_FP8E4M3, gam);
  return nullptr;
}

}  // namespace mtp
