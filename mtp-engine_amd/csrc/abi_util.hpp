// Host-side helpers shared by the C-ABI translation units: launch status,
// the last HIP error string, pointer and dtype predicates.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "../../include/mtp_hip.h"

namespace mtp {

// Text of the last HIP error a failed launch saw on this thread (defined in
// mtp_hip.hip).
extern thread_local char g_last_hip_error[256];

inline void note_hip_error(hipError_t e) {
  std::strncpy(g_last_hip_error, hipGetErrorString(e), sizeof(g_last_hip_error) - 1);
}

// MTP_OK, or MTP_ERR_LAUNCH when the runtime rejected the last launch.
inline int launch_status() {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return MTP_OK;
  note_hip_error(e);
  return MTP_ERR_LAUNCH;
}

// Workspace layout shared by every entry point: the counter prefix (zero
// between launches) comes first. Its last 512 bytes hold the verify
// kernels' 64 row keys; arrival tickets use the 4-byte slots before them.
constexpr size_t kCounterBytes = MTP_WORKSPACE_COUNTER_BYTES;
constexpr size_t kSkvKeysBytes = 64 * 8;
constexpr size_t kSkvKeysOff = kCounterBytes - kSkvKeysBytes;
constexpr int64_t kCounterSlots = (int64_t)(kSkvKeysOff / 4);

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Launch-planning overrides (tile variants, split counts, route switches).
// The MTP_* environment variables seed them once per process; after that
// only mtp_set_tuning() changes them. -1 = not set (the planner decides).
enum TuneKey {
  kTuneSkl,              // MTP_SKL: 1 force the single-launch skinny kernel, 0 off
  kTuneSkSplits,         // MTP_SK_SPLITS: K-splits of the two-launch skinny kernel
  kTuneWsVariant,        // MTP_WS_TUNE="variant,splits": row-chunk kernel variant
  kTuneWsSplits,         //   ... and its K-splits
  kTuneSklWaves,         // MTP_SKL_WAVES: 4 or 8
  kTuneSklSplits,        // MTP_SKL_SPLITS
  kTuneAttnChunkBlocks,  // MTP_ATTN_CHUNK_BLOCKS: key blocks per attention chunk
  kTuneInt4Waves,        // MTP_INT4_WAVES: 4 or 8
  kTuneVerifyWstream,    // MTP_VERIFY_WSTREAM: 1 = column-group verify kernel
  kTuneSkp,              // MTP_SKP: x-resident skinny kernel, 1 force where it applies, 0 off
  kTuneSkpSplits,        // MTP_SKP_SPLITS: its K-splits (at least the LDS-bound count)
  kTuneSkpTa,            // MTP_SKP_TA: its A tiles per wave, 1, 2 or 4
  kTuneSf32,             // MTP_SF32: small fp32 kernel, 0 off (default on where it applies)
  kTuneSkpH8,            // MTP_SKP_H8: compact x blocks of the x-resident kernel (<= 8 rows), 0 off
  kTuneAttn32,           // MTP_ATTN32: 32-query-tile attention (33 .. 64 queries, D 128), 0 off
  kTuneSkXraw,           // MTP_SK_XRAW: 0 keeps sk's prep launch without gamma (default: raw x)
  kTuneSkw,              // MTP_SKW: wave-specialised skinny kernel, 1 force where it applies, 0 off
  kTuneSkwTw,            // MTP_SKW_TW: its output columns per workgroup (8 .. 64, multiple of 8)
  kTuneSkpTw,            // MTP_SKP_TW: x-resident kernel's columns per workgroup (multiple of 8)
  kTuneSklTw,            // MTP_SKL_TW: single-launch kernel's columns per workgroup (multiple of 8)
  kTuneSkvR8,            // MTP_SKV_R8: fp32 verify, 8 rows after whole 16-row tiles on the 4x4 MFMA (0: off)
  kTuneSkvTw,            // MTP_SKV_TW: streaming verify's columns per tile (8 .. 256, multiple of 8)
  kTuneCount
};
int tune(TuneKey k);
// Compute units of the current device (queried once per device; 256, the
// MI355X count, when no device answers).
int device_cus();

inline bool is_float_dt(int dt) { return dt == MTP_F32 || dt == MTP_BF16 || dt == MTP_F16; }
inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace mtp
