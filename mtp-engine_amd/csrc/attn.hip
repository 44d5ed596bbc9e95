// Instantiations of the attention kernels (attn.hpp).
#include "attn.hpp"
#include "attn2.hpp"

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

// The 32-query-tile kernel (head dim 128) for a compute type, or null.
AttnKernel attn2_pick(int ct) {
  if (ct == MTP_BF16) return attn2_kernel<MTP_BF16>;
  if (ct == MTP_F16) return attn2_kernel<MTP_F16>;
  return nullptr;
}
int attn2_lds_bytes() { return kAttn2Lds; }

void (*attn_generic())(AttnArgs, int, int) { return attn_generic_kernel; }

void (*attn_generic_wide(int d))(AttnArgs, int, int) {
  if (d <= 512) return attn_generic_wide_kernel<2>;
  if (d <= 1024) return attn_generic_wide_kernel<4>;
  if (d <= 2048) return attn_generic_wide_kernel<8>;
  if (d <= 4096) return attn_generic_wide_kernel<16>;
  if (d <= kAttnWideMaxD) return attn_generic_wide_kernel<32>;
  return nullptr;
}

}  // namespace mtp
