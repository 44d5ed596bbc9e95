// Instantiations and launch of the small fp32 RMSNorm -> linear kernel
// (sf32.hpp).
#include "abi_util.hpp"
#include "sf32.hpp"

namespace mtp {

int launch_sf32(const Sf32Args &a, hipStream_t st) {
  if (a.M < 1 || a.M > 32 || a.K < 16 || a.K > kSf32StreamMaxK || a.K % 16 != 0 || a.N < 1)
    return MTP_ERR_SHAPE;
  const unsigned blocks = (unsigned)((a.N + 15) / 16);
  // The one-round-trip kernel (one 139 KB workgroup per CU) only while its
  // workgroups fit the CUs at once and K > 512; otherwise the streaming form
  // (76 KB, two per CU) measured faster, us per call (one round trip /
  // streaming): 16 x 4096 x 1024 6.25 / 6.76, 16 x 8192 x 1024 11.3 / 10.8,
  // 16 x 14336 x 1024 19.3 / 17.0, 8 x 32000 x 1024 36.1 / 28.8, 4 x 4096 x
  // 512 5.28 / 4.78.
  const bool one_trip = a.M <= 16 && a.K <= kSf32MaxK && a.K > 512 &&
                        (int)blocks <= device_cus();
  if (!one_trip) {
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
