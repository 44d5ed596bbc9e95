// Instantiations of the pipelined linear kernel: x F32, weights F32.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel wsp_pick_f32_f32(int mt, int v, bool gam) {
  return gam ? wsp_pick<MTP_F32, MTP_F32, true>(mt, v) : wsp_pick<MTP_F32, MTP_F32, false>(mt, v);
}

}  // namespace mtp
