// Tile variants of the weight-streaming kernel and their dispatch. The
// instantiations live in one translation unit per compute type
// (ws_bf16.hip, ws_f16.hip, ws_f32.hip) so they compile in parallel.
#pragma once

#include "wstream.hpp"

namespace mtp {

struct WsVariant {
  int nsub, wn, wk, wbl;
};

typedef void (*WsKernel)(WsArgs);

// Variant tables: index 0 is the default of the dtype pair, the others are
// sweep options selectable at run time.
constexpr WsVariant kWsVar16[] = {{4, 4, 1, 64}, {2, 4, 2, 32}, {2, 4, 1, 64}, {4, 2, 2, 32}};
constexpr int kWsNumVar16 = 4;
constexpr WsVariant kWsVar32[] = {{4, 4, 1, 64}, {2, 4, 1, 64}};
constexpr WsVariant kWsVar32Fp8[] = {{4, 4, 1, 32}, {2, 4, 1, 32}};
constexpr int kWsNumVar32 = 2;

inline int ws_num_variants(int ct) { return ct == MTP_F32 ? kWsNumVar32 : kWsNumVar16; }
inline WsVariant ws_variant(int ct, int wt, int v) {
  if (ct == MTP_F32) return wt == MTP_FP8E4M3 ? kWsVar32Fp8[v] : kWsVar32[v];
  return kWsVar16[v];
}

template <int CT, int WT, int MT, int EPI>
WsKernel ws_pick_mt(int v) {
  if constexpr (CT == MTP_F32) {
    constexpr int WB = (WT == MTP_FP8E4M3) ? 32 : 64;
    switch (v) {
      case 0: return wstream_kernel<CT, WT, MT, 4, 4, 1, WB, EPI>;
      case 1: return wstream_kernel<CT, WT, MT, 2, 4, 1, WB, EPI>;
    }
  } else {
    switch (v) {
      case 0: return wstream_kernel<CT, WT, MT, 4, 4, 1, 64, EPI>;
      case 1: return wstream_kernel<CT, WT, MT, 2, 4, 2, 32, EPI>;
      case 2: return wstream_kernel<CT, WT, MT, 2, 4, 1, 64, EPI>;
      case 3: return wstream_kernel<CT, WT, MT, 4, 2, 2, 32, EPI>;
    }
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

// Defined in ws_<ct>.hip: the kernel for (weight type, M tiles, variant,
// epilogue) at that compute type, or null if not instantiated.
WsKernel ws_pick_bf16(int wt, int mt, int v, int epi);
WsKernel ws_pick_f16(int wt, int mt, int v, int epi);
WsKernel ws_pick_f32(int wt, int mt, int v, int epi);

inline WsKernel ws_pick_kernel(int ct, int wt, int mt, int v, int epi) {
  switch (ct) {
    case MTP_BF16: return ws_pick_bf16(wt, mt, v, epi);
    case MTP_F16: return ws_pick_f16(wt, mt, v, epi);
    case MTP_F32: return ws_pick_f32(wt, mt, v, epi);
  }
  return nullptr;
}

}  // namespace mtp
