// Instantiations and launch of the small fp32 RMSNorm -> linear kernel
// (sf32.hpp).
#include "abi_util.hpp"
#include "sf32.hpp"

namespace mtp {

int launch_sf32(const Sf32Args &a, hipStream_t st) {
  if (a.M < 1 || a.M > 32 || a.K < 16 || a.K > kSf32StreamMaxK || a.K % 16 != 0 || a.N < 1)
    return MTP_ERR_SHAPE;
  const unsigned blocks = (unsigned)((a.N + 15) / 16);
  if (a.M > 16 || a.K > kSf32MaxK) {
    // streaming form, one or two 16-row tiles
    const dim3 grid(blocks), block(64 * kSf32sWaves);
    if (a.M > 16) {
      if (a.gamma)
        hipLaunchKernelGGL((sf32s_kernel<true, kSf32sWaves, 2>), grid, block, 0, st, a);
      else
        hipLaunchKernelGGL((sf32s_kernel<false, kSf32sWaves, 2>), grid, block, 0, st, a);
    } else {
      if (a.gamma)
        hipLaunchKernelGGL((sf32s_kernel<true, kSf32sWaves, 1>), grid, block, 0, st, a);
      else
        hipLaunchKernelGGL((sf32s_kernel<false, kSf32sWaves, 1>), grid, block, 0, st, a);
    }
    return launch_status();
  }
  if (a.gamma)
    hipLaunchKernelGGL((sf32_kernel<true, kSf32Waves>), dim3(blocks), dim3(64 * kSf32Waves), 0, st, a);
  else
    hipLaunchKernelGGL((sf32_kernel<false, kSf32Waves>), dim3(blocks), dim3(64 * kSf32Waves), 0, st, a);
  return launch_status();
}

}  // namespace mtp
