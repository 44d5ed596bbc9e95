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

template <int CT, bool FP8, bool GAM>
SkPrep8Kernel sk_prep8_c(int ch) {
  if (ch == 1) return sk_prep8_kernel<CT, FP8, GAM, 1>;
  if (ch == 2) return sk_prep8_kernel<CT, FP8, GAM, 2>;
  if (ch == 4) return sk_prep8_kernel<CT, FP8, GAM, 4>;
  return nullptr;
}

template <int CT>
SkPrep8Kernel sk_prep8_ct(bool fp8, bool gam, int ch) {
  if (fp8) return gam ? sk_prep8_c<CT, true, true>(ch) : sk_prep8_c<CT, true, false>(ch);
  return gam ? sk_prep8_c<CT, false, true>(ch) : sk_prep8_c<CT, false, false>(ch);
}

SkPrep8Kernel sk_prep8_pick(int ct, int wt, bool gam, int ch) {
  if (ct == MTP_BF16) return sk_prep8_ct<MTP_BF16>(wt == MTP_FP8E4M3, gam, ch);
  if (ct == MTP_F16) return sk_prep8_ct<MTP_F16>(wt == MTP_FP8E4M3, gam, ch);
  return nullptr;
}

}  // namespace mtp
