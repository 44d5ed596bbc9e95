// Instantiations of the pipelined linear kernel: x F16, weights FP8E4M3.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel wsp_pick_f16_fp8(int mt, int v, bool gam) {
  return gam ? wsp_pick<MTP_F16, MTP_FP8E4M3, true>(mt, v) : wsp_pick<MTP_F16, MTP_FP8E4M3, false>(mt, v);
}

}  // namespace mtp
