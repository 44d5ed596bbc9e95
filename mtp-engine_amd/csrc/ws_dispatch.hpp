// Tile variants of the weight-streaming kernel and their dispatch. The
// instantiations live in one translation unit per compute type
// (ws_bf16.hip, ws_f16.hip, ws_f32.hip) so they compile in parallel.
//
// A wave keeps at most NSUB * WBL / 16 <= 8 sixteen-byte W loads per K-block
// in flight (double-buffered: <= 16 outstanding): on gfx950 waves with more
// outstanding vector loads than that lose half their HBM throughput, so the
// bytes in flight per CU come from more waves instead.
#pragma once

#include "wstream.hpp"
#include "wsx.hpp"

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

// ---- x-resident linear kernel (wsx.hpp) -----------------------------------
constexpr WsVariant kWsxVar[] = {
    {2, 2, 8, 64},  // 0: 1024 threads, 64 columns, 8-way K split in the workgroup
    {2, 4, 4, 64},  // 1: 1024 threads, 128 columns
    {2, 4, 2, 64},  // 2: 512 threads, 128 columns
    {2, 2, 4, 64},  // 3: 512 threads, 64 columns
};
constexpr int kWsxNumVar = 4;

// fp32 activations with fp8 weights use 32-byte lane runs (K-block of 128).
constexpr WsVariant wsx_effective(int ct, int wt, WsVariant v) {
  if (ct == MTP_F32 && wt == MTP_FP8E4M3) return WsVariant{v.nsub, v.wn, v.wk, 32};
  return v;
}
inline WsVariant wsx_variant(int ct, int wt, int v) { return wsx_effective(ct, wt, kWsxVar[v]); }

template <int CT, int WT, int MT, int I>
WsKernel wsx_inst() {
  constexpr WsVariant v = wsx_effective(CT, WT, kWsxVar[I]);
  return wsx_kernel<CT, WT, MT, v.nsub, v.wn, v.wk, v.wbl>;
}

template <int CT, int WT>
WsKernel wsx_pick(int mt, int v) {
#define MTP_WSX_CASES(MT)                   \
  switch (v) {                              \
    case 0: return wsx_inst<CT, WT, MT, 0>(); \
    case 1: return wsx_inst<CT, WT, MT, 1>(); \
    case 2: return wsx_inst<CT, WT, MT, 2>(); \
    case 3: return wsx_inst<CT, WT, MT, 3>(); \
  }                                         \
  return nullptr;
  switch (mt) {
    case 1: { MTP_WSX_CASES(1) }
    case 2: { MTP_WSX_CASES(2) }
    case 3: { MTP_WSX_CASES(3) }
    case 4: { MTP_WSX_CASES(4) }
  }
#undef MTP_WSX_CASES
  return nullptr;
}

// Defined in ws_<ct>.hip: the kernel for (weight type, M tiles, variant,
// epilogue) at that compute type, or null if not instantiated.
WsKernel ws_pick_bf16(int wt, int mt, int v, int epi);
WsKernel ws_pick_f16(int wt, int mt, int v, int epi);
WsKernel ws_pick_f32(int wt, int mt, int v, int epi);
WsKernel wsx_pick_bf16(int wt, int mt, int v);
WsKernel wsx_pick_f16(int wt, int mt, int v);
WsKernel wsx_pick_f32(int wt, int mt, int v);

inline WsKernel wsx_pick_kernel(int ct, int wt, int mt, int v) {
  switch (ct) {
    case MTP_BF16: return wsx_pick_bf16(wt, mt, v);
    case MTP_F16: return wsx_pick_f16(wt, mt, v);
    case MTP_F32: return wsx_pick_f32(wt, mt, v);
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
