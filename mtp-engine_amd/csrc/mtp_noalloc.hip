// Allocation-free multi-verify: mtp_fused_multi_verify with its workspace in
// a static device array of the library instead of caller memory, for callers
// that cannot allocate (code under graph capture, tight serving loops).
//
// The array `scratch` holds kNoallocScratchBytes per device (each GPU the
// library runs on keeps its own copy until the process ends). Its device
// address is looked up once per device, with that device current, by
// hipGetSymbolAddress (mtp_noalloc_init, or else the first call on that
// device); host code uses only that address, never the array's name. Every
// call clears the counter prefix (tickets and row keys) with a kernel before
// the verify launches, so the previous call's contents do not matter; two
// calls that overlap on one GPU share the array and race. A call needs the
// counter prefix on the persistent and generic verify kernels, and the
// column-group kernel's per-tile maxima besides on that route.
#include <hip/hip_runtime.h>

#include <mutex>

#include "abi_util.hpp"

using namespace mtp;

namespace {

constexpr size_t kNoallocScratchBytes = (size_t)1 << 20;  // 1 MiB per device
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
void *g_scratch_ptr[kMaxDevices];
int g_scratch_status[kMaxDevices];
std::once_flag g_scratch_once[kMaxDevices];

__global__ void __launch_bounds__(256) clear_words_kernel(uint32_t *p, int n4) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n4; i += gridDim.x * 256) p[i] = 0u;
}

// The current device's copy of `scratch` (looked up on the first call made
// with that device current).
int scratch_of_current_device(void **out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    note_hip_error(e);
    return MTP_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) return MTP_ERR_ARG;
  std::call_once(g_scratch_once[dev], [dev] {
    void *p = nullptr;
    const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (r != hipSuccess || !p) {
      note_hip_error(r);
      g_scratch_status[dev] = MTP_ERR_LAUNCH;
      return;
    }
    g_scratch_ptr[dev] = p;
    g_scratch_status[dev] = MTP_OK;
  });
  if (g_scratch_status[dev] != MTP_OK) return g_scratch_status[dev];
  *out = g_scratch_ptr[dev];
  return MTP_OK;
}

}  // namespace

extern "C" {

size_t mtp_noalloc_scratch_bytes(void) { return kNoallocScratchBytes; }

int mtp_noalloc_init(void) {
  void *ws = nullptr;
  return scratch_of_current_device(&ws);
}

int mtp_fused_multi_verify_noalloc(const void *hidden, int h_dtype, int64_t B, int64_t S,
                                   int64_t K, const void *weight, int w_dtype, int64_t V,
                                   const void *bias, int bias_dtype, const int32_t *draft,
                                   int64_t D, int8_t *accept, int32_t *accepted_n,
                                   int32_t *corrected, int32_t *top_out, void *stream) {
  // the argument checks of mtp_fused_multi_verify, before any launch
  if (!is_float_dt(h_dtype) || !is_float_dt(w_dtype)) return MTP_ERR_DTYPE;
  if (bias && !is_float_dt(bias_dtype)) return MTP_ERR_DTYPE;
  if (B < 0 || S < 1 || D < 0 || S != D + 1 || K <= 0 || V <= 0 || S > 64 ||
      B * S > INT32_MAX || K > INT32_MAX || V > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (B == 0) return MTP_OK;
  if (!hidden || !weight || !accepted_n || !corrected || (D > 0 && (!draft || !accept)))
    return MTP_ERR_NULL;
  const int route = mtp_verify_route(hidden, h_dtype, B * S, S, K, weight, w_dtype, V, bias);
  if (route < 0) return route;
  const size_t need = route == MTP_VERIFY_ROUTE_COLUMN_GROUP
                          ? mtp_verify_workspace_bytes(h_dtype, B * S, S, V, K)
                          : kCounterBytes;
  if (need > kNoallocScratchBytes) return MTP_ERR_WORKSPACE;
  void *ws = nullptr;
  int s = scratch_of_current_device(&ws);
  if (s != MTP_OK) return s;
  hipLaunchKernelGGL(clear_words_kernel, dim3(16), dim3(256), 0, (hipStream_t)stream,
                     (uint32_t *)ws, (int)(kCounterBytes / 4));
  s = launch_status();
  if (s != MTP_OK) return s;
  return mtp_fused_multi_verify(hidden, h_dtype, B, S, K, weight, w_dtype, V, bias, bias_dtype,
                                draft, D, accept, accepted_n, corrected, top_out, ws,
                                kNoallocScratchBytes, stream);
}

}  // extern "C"
