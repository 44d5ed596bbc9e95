// Instantiations of the verify (argmax) weight-streaming kernel at compute
// type BF16.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel ws_pick_bf16(int wt, int mt, int v, int epi) {
  if (epi == EPI_ARGMAX && wt == MTP_BF16) return ws_pick<MTP_BF16, MTP_BF16, EPI_ARGMAX>(mt, v);
  return nullptr;
}

}  // namespace mtp
