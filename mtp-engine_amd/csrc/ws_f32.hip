// Instantiations of the verify (argmax) weight-streaming kernel at compute
// type F32.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel ws_pick_f32(int wt, int mt, int v, int epi) {
  if (epi == EPI_ARGMAX && wt == MTP_F32) return ws_pick<MTP_F32, MTP_F32, EPI_ARGMAX>(mt, v);
  return nullptr;
}

}  // namespace mtp
