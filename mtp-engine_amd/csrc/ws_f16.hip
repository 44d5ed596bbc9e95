// Instantiations of the verify (argmax) weight-streaming kernel at compute
// type F16.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel ws_pick_f16(int wt, int mt, int v, int epi) {
  if (epi == EPI_ARGMAX && wt == MTP_F16) return ws_pick<MTP_F16, MTP_F16, EPI_ARGMAX>(mt, v);
  return nullptr;
}

}  // namespace mtp
