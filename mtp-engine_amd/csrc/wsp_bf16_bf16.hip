// Instantiations of the pipelined linear kernel: x BF16, weights BF16.
#include "ws_dispatch.hpp"

namespace mtp {

WsKernel wsp_pick_bf16_bf16(int mt, int v, bool gam) {
  return gam ? wsp_pick<MTP_BF16, MTP_BF16, true>(mt, v) : wsp_pick<MTP_BF16, MTP_BF16, false>(mt, v);
}

}  // namespace mtp
