// Instantiations of the pipelined linear kernel: x F16, weights F16.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel wsp_pick_f16_f16(int mt, int v, bool gam) {
  return gam ? wsp_pick<MTP_F16, MTP_F16, true>(mt, v) : wsp_pick<MTP_F16, MTP_F16, false>(mt, v);
}

}  // namespace mtp
