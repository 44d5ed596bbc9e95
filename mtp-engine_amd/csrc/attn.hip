// Instantiations of the attention kernels (attn.hpp).
#include "attn.hpp"

namespace mtp {

// The MFMA kernel for (compute type, head dim), or null.
AttnKernel attn_pick(int ct, int d) {
  if (ct == MTP_BF16) {
    if (d == 64) return attn_kernel<MTP_BF16, 64>;
    if (d == 128) return attn_kernel<MTP_BF16, 128>;
  } else if (ct == MTP_F16) {
    if (d == 64) return attn_kernel<MTP_F16, 64>;
    if (d == 128) return attn_kernel<MTP_F16, 128>;
  }
  return nullptr;
}

// The chunk merge for (compute type, head dim), or null.
AttnKernel attn_merge_pick(int ct, int d) {
  if (ct == MTP_BF16) {
    if (d == 64) return attn_merge_kernel<MTP_BF16, 64>;
    if (d == 128) return attn_merge_kernel<MTP_BF16, 128>;
  } else if (ct == MTP_F16) {
    if (d == 64) return attn_merge_kernel<MTP_F16, 64>;
    if (d == 128) return attn_merge_kernel<MTP_F16, 128>;
  }
  return nullptr;
}

void (*attn_generic())(AttnArgs, int, int) { return attn_generic_kernel; }

}  // namespace mtp
