// Tile variants of the weight-streaming kernels and their dispatch. The
// instantiations live in one translation unit per compute type (verify:
// ws_bf16.hip, ws_f16.hip, ws_f32.hip) or per dtype pair (linear:
// wsp_<ct>_<wt>.hip) so they compile in parallel.
//
// A wave keeps at most NSUB * WBL / 16 <= 8 sixteen-byte W loads per K-block
// in flight (double-buffered: <= 16 outstanding): on gfx950 waves with more
// outstanding vector loads than that lose half their HBM throughput, so the
// bytes in flight per CU come from more waves instead.
#pragma once

#include "wsp.hpp"
#include "wstream.hpp"

namespace mtp {

struct WsVariant {
  int nsub, wn, wk, wbl;
};

typedef void (*WsKernel)(WsArgs);

// Variant table shared by all dtype pairs (index 0 = default before the
// per-shape choice in the planner); see ws_effective for dtype coercions.
constexpr WsVariant kWsVar[] = {
    {2, 8, 1, 64},   // 0: 512 threads, 256 columns
    {2, 4, 2, 64},   // 1: 512 threads, 128 columns, 2-way K split in the workgroup
    {2, 8, 2, 64},   // 2: 1024 threads, 256 columns
    {2, 4, 4, 32},   // 3: 1024 threads, 128 columns, 4-way K split
    {4, 4, 2, 32},   // 4: 512 threads, 256 columns
    {2, 16, 1, 64},  // 5: 1024 threads, 512 columns
    {4, 4, 1, 64},   // 6: 256 threads, 256 columns (16 loads per K-block)
    {2, 4, 1, 64},   // 7: 256 threads, 128 columns
};
constexpr int kWsNumVar = 8;

// Effective shape at a dtype pair: fp8 weights with a K-split inside the
// workgroup use 32-byte lane runs, and fp32 activations with fp8 weights
// use 32-byte runs without a K split, so the x LDS stays <= 64 KB.
constexpr WsVariant ws_effective(int ct, int wt, WsVariant v) {
  if (ct == MTP_F32 && wt == MTP_FP8E4M3) return WsVariant{v.nsub, v.wn * v.wk, 1, 32};
  if (wt == MTP_FP8E4M3 && v.wk > 1) return WsVariant{v.nsub, v.wn, v.wk, 32};
  return v;
}

inline int ws_num_variants(int) { return kWsNumVar; }
inline WsVariant ws_variant(int ct, int wt, int v) { return ws_effective(ct, wt, kWsVar[v]); }

template <int CT, int WT, int MT, int EPI, int I>
WsKernel ws_inst() {
  constexpr WsVariant v = ws_effective(CT, WT, kWsVar[I]);
  return wstream_kernel<CT, WT, MT, v.nsub, v.wn, v.wk, v.wbl, EPI>;
}

template <int CT, int WT, int MT, int EPI>
WsKernel ws_pick_mt(int v) {
  switch (v) {
    case 0: return ws_inst<CT, WT, MT, EPI, 0>();
    case 1: return ws_inst<CT, WT, MT, EPI, 1>();
    case 2: return ws_inst<CT, WT, MT, EPI, 2>();
    case 3: return ws_inst<CT, WT, MT, EPI, 3>();
    case 4: return ws_inst<CT, WT, MT, EPI, 4>();
    case 5: return ws_inst<CT, WT, MT, EPI, 5>();
    case 6: return ws_inst<CT, WT, MT, EPI, 6>();
    case 7: return ws_inst<CT, WT, MT, EPI, 7>();
  }
  return nullptr;
}

template <int CT, int WT, int EPI>
WsKernel ws_pick(int mt, int v) {
  switch (mt) {
    case 1: return ws_pick_mt<CT, WT, 1, EPI>(v);
    case 2: return ws_pick_mt<CT, WT, 2, EPI>(v);
    case 3: return ws_pick_mt<CT, WT, 3, EPI>(v);
    case 4: return ws_pick_mt<CT, WT, 4, EPI>(v);
  }
  return nullptr;
}

// ---- pipelined linear kernel (wsp.hpp) -------------------------------------
// {nsub, wn, wk}: a wave covers 16 * nsub columns, wn waves share one x ring
// per K-group, wk K-groups per workgroup.
struct WspVariant {
  int nsub, wn, wk;
};
constexpr WspVariant kWspVar[] = {
    {2, 2, 8},  // 0: 1024 threads, 64 columns
    {2, 4, 4},  // 1: 1024 threads, 128 columns
    {2, 8, 2},  // 2: 1024 threads, 256 columns
    {2, 4, 2},  // 3: 512 threads, 128 columns
    {2, 2, 4},  // 4: 512 threads, 64 columns
    {4, 2, 4},  // 5: 512 threads, 128 columns, 64 columns per wave
    {1, 4, 4},  // 6: 1024 threads, 64 columns, 16 columns per wave
    {4, 4, 2},  // 7: 512 threads, 256 columns, 64 columns per wave
};
constexpr int kWspNumVar = 8;

template <int CT, int WT, int MT, int I, bool GAM>
WsKernel wsp_inst() {
  constexpr WspVariant v = kWspVar[I];
  return wsp_kernel<CT, WT, MT, v.nsub, v.wn, v.wk, GAM>;
}

template <int CT, int WT, bool GAM>
WsKernel wsp_pick(int mt, int v) {
#define MTP_WSP_CASES(MT)                          \
  switch (v) {                                     \
    case 0: return wsp_inst<CT, WT, MT, 0, GAM>(); \
    case 1: return wsp_inst<CT, WT, MT, 1, GAM>(); \
    case 2: return wsp_inst<CT, WT, MT, 2, GAM>(); \
    case 3: return wsp_inst<CT, WT, MT, 3, GAM>(); \
    case 4: return wsp_inst<CT, WT, MT, 4, GAM>(); \
    case 5: return wsp_inst<CT, WT, MT, 5, GAM>(); \
    case 6: return wsp_inst<CT, WT, MT, 6, GAM>(); \
    case 7: return wsp_inst<CT, WT, MT, 7, GAM>(); \
  }                                                \
  return nullptr;
  switch (mt) {
    case 1: { MTP_WSP_CASES(1) }
    case 2: { MTP_WSP_CASES(2) }
    case 3: { MTP_WSP_CASES(3) }
    case 4: { MTP_WSP_CASES(4) }
  }
#undef MTP_WSP_CASES
  return nullptr;
}

// Defined in ws_<ct>.hip: the verify (argmax) kernel at that compute type for
// (M tiles, variant), or null if not instantiated.
WsKernel ws_pick_bf16(int wt, int mt, int v, int epi);
WsKernel ws_pick_f16(int wt, int mt, int v, int epi);
WsKernel ws_pick_f32(int wt, int mt, int v, int epi);
// Defined in wsp_<ct>_<wt>.hip: the linear kernel for (M tiles, variant,
// gamma present).
WsKernel wsp_pick_bf16_bf16(int mt, int v, bool gam);
WsKernel wsp_pick_bf16_fp8(int mt, int v, bool gam);
WsKernel wsp_pick_f16_f16(int mt, int v, bool gam);
WsKernel wsp_pick_f16_fp8(int mt, int v, bool gam);
WsKernel wsp_pick_f32_f32(int mt, int v, bool gam);
WsKernel wsp_pick_f32_fp8(int mt, int v, bool gam);

inline WsKernel wsp_pick_kernel(int ct, int wt, int mt, int v, bool gam) {
  const bool f8 = wt == MTP_FP8E4M3;
  if (!f8 && wt != ct) return nullptr;
  switch (ct) {
    case MTP_BF16: return f8 ? wsp_pick_bf16_fp8(mt, v, gam) : wsp_pick_bf16_bf16(mt, v, gam);
    case MTP_F16: return f8 ? wsp_pick_f16_fp8(mt, v, gam) : wsp_pick_f16_f16(mt, v, gam);
    case MTP_F32: return f8 ? wsp_pick_f32_fp8(mt, v, gam) : wsp_pick_f32_f32(mt, v, gam);
  }
  return nullptr;
}

inline WsKernel ws_pick_kernel(int ct, int wt, int mt, int v, int epi) {
  switch (ct) {
    case MTP_BF16: return ws_pick_bf16(wt, mt, v, epi);
    case MTP_F16: return ws_pick_f16(wt, mt, v, epi);
    case MTP_F32: return ws_pick_f32(wt, mt, v, epi);
  }
  return nullptr;
}

}  // namespace mtp
