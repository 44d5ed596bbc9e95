// Instantiations of the generic verify kernel (vgen.hpp).
#include "vgen.hpp"

namespace mtp {

VgenKernel vgen_pick(int rows) {
  if (rows <= 8) return verify_generic_kernel<8>;
  if (rows <= 16) return verify_generic_kernel<16>;
  if (rows <= 32) return verify_generic_kernel<32>;
  if (rows <= 64) return verify_generic_kernel<64>;
  return nullptr;
}

}  // namespace mtp
