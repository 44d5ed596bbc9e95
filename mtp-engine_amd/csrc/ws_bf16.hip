// Instantiations of the weight-streaming kernel at compute type BF16.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel ws_pick_bf16(int wt, int mt, int v, int epi) {
  if (epi == EPI_LINEAR) {
    if (wt == MTP_BF16) return ws_pick<MTP_BF16, MTP_BF16, EPI_LINEAR>(mt, v);
    if (wt == MTP_FP8E4M3) return ws_pick<MTP_BF16, MTP_FP8E4M3, EPI_LINEAR>(mt, v);
  } else {
    if (wt == MTP_BF16) return ws_pick<MTP_BF16, MTP_BF16, EPI_ARGMAX>(mt, v);
  }
  return nullptr;
}

}  // namespace mtp

namespace mtp {

WsKernel wsx_pick_bf16(int wt, int mt, int v) {
  if (wt == MTP_BF16) return wsx_pick<MTP_BF16, MTP_BF16>(mt, v);
  if (wt == MTP_FP8E4M3) return wsx_pick<MTP_BF16, MTP_FP8E4M3>(mt, v);
  return nullptr;
}

}  // namespace mtp
