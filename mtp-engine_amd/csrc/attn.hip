// Instantiations of the attention kernels (attn.hpp).
#include "attn.hpp"

namespace mtp {

template <int CT, int D>
AttnKernel attn_pick_qt(int qt) {
  switch (qt) {
    case 1: return attn_kernel<CT, D, 1>;
    case 2: return attn_kernel<CT, D, 2>;
    case 3: return attn_kernel<CT, D, 3>;
    case 4: return attn_kernel<CT, D, 4>;
  }
  return nullptr;
}

// The MFMA kernel for (compute type, head dim, query tiles), or null.
AttnKernel attn_pick(int ct, int d, int qt) {
  if (ct == MTP_BF16) {
    if (d == 64) return attn_pick_qt<MTP_BF16, 64>(qt);
    if (d == 128) return attn_pick_qt<MTP_BF16, 128>(qt);
  } else if (ct == MTP_F16) {
    if (d == 64) return attn_pick_qt<MTP_F16, 64>(qt);
    if (d == 128) return attn_pick_qt<MTP_F16, 128>(qt);
  }
  return nullptr;
}

void (*attn_generic())(AttnArgs, int, int) { return attn_generic_kernel; }

}  // namespace mtp
