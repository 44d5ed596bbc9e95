// C ABI of the gfx950 verify/draft hot path: argument validation, launch
// planning and kernel dispatch. Declarations and the reference interface
// each entry point replaces are in include/mtp_hip.h.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>

#include "abi_util.hpp"
#include "attn_args.hpp"
#include "generic.hpp"
#include "int4g_args.hpp"
#include "quant.hpp"
#include "sf32_args.hpp"
#include "sk_args.hpp"
#include "skl_args.hpp"
#include "skp_args.hpp"
#include "skv_args.hpp"
#include "skw_args.hpp"
#include "vgen.hpp"
#include "ws_dispatch.hpp"

namespace mtp {
thread_local char g_last_hip_error[256] = "";

namespace {
std::atomic<int> g_tune[kTuneCount];
std::once_flag g_tune_once;
const char *const kTuneNames[kTuneCount] = {
    "skl", "sk_splits", "ws_variant", "ws_splits", "skl_waves", "skl_splits",
    "attn_chunk_blocks", "int4_waves", "verify_wstream", "skp", "skp_splits", "skp_ta", "sf32", "skp_h8", "attn32", "sk_xraw",
    "skw", "skw_tw", "skp_tw", "skl_tw", "skv_r8", "skv_tw"};

int env_int(const char *name, int dflt) {
  const char *e = std::getenv(name);
  return (e && *e) ? std::atoi(e) : dflt;
}

void tune_init() {
  for (auto &t : g_tune) t.store(-1, std::memory_order_relaxed);
  if (const char *e = std::getenv("MTP_SKL")) {
    if (*e) g_tune[kTuneSkl].store(*e == '0' ? 0 : 1, std::memory_order_relaxed);
  }
  g_tune[kTuneSkSplits].store(env_int("MTP_SK_SPLITS", -1), std::memory_order_relaxed);
  if (const char *e = std::getenv("MTP_WS_TUNE")) {
    int v = -1, sp = -1;
    if (*e && std::sscanf(e, "%d,%d", &v, &sp) >= 1) {
      g_tune[kTuneWsVariant].store(v, std::memory_order_relaxed);
      g_tune[kTuneWsSplits].store(sp, std::memory_order_relaxed);
    }
  }
  g_tune[kTuneSklWaves].store(env_int("MTP_SKL_WAVES", -1), std::memory_order_relaxed);
  g_tune[kTuneSklSplits].store(env_int("MTP_SKL_SPLITS", -1), std::memory_order_relaxed);
  g_tune[kTuneAttnChunkBlocks].store(env_int("MTP_ATTN_CHUNK_BLOCKS", -1),
                                     std::memory_order_relaxed);
  g_tune[kTuneInt4Waves].store(env_int("MTP_INT4_WAVES", -1), std::memory_order_relaxed);
  if (const char *e = std::getenv("MTP_VERIFY_WSTREAM"))
    if (*e) g_tune[kTuneVerifyWstream].store(1, std::memory_order_relaxed);
  g_tune[kTuneSkp].store(env_int("MTP_SKP", -1), std::memory_order_relaxed);
  g_tune[kTuneSkpSplits].store(env_int("MTP_SKP_SPLITS", -1), std::memory_order_relaxed);
  g_tune[kTuneSkpTa].store(env_int("MTP_SKP_TA", -1), std::memory_order_relaxed);
  g_tune[kTuneSf32].store(env_int("MTP_SF32", -1), std::memory_order_relaxed);
  g_tune[kTuneSkpH8].store(env_int("MTP_SKP_H8", -1), std::memory_order_relaxed);
  g_tune[kTuneAttn32].store(env_int("MTP_ATTN32", -1), std::memory_order_relaxed);
  g_tune[kTuneSkXraw].store(env_int("MTP_SK_XRAW", -1), std::memory_order_relaxed);
  g_tune[kTuneSkw].store(env_int("MTP_SKW", -1), std::memory_order_relaxed);
  g_tune[kTuneSkwTw].store(env_int("MTP_SKW_TW", -1), std::memory_order_relaxed);
  g_tune[kTuneSkpTw].store(env_int("MTP_SKP_TW", -1), std::memory_order_relaxed);
  g_tune[kTuneSklTw].store(env_int("MTP_SKL_TW", -1), std::memory_order_relaxed);
  g_tune[kTuneSkvR8].store(env_int("MTP_SKV_R8", -1), std::memory_order_relaxed);
  g_tune[kTuneSkvTw].store(env_int("MTP_SKV_TW", -1), std::memory_order_relaxed);
}
}  // namespace

int tune(TuneKey k) {
  std::call_once(g_tune_once, tune_init);
  return g_tune[k].load(std::memory_order_relaxed);
}

int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        c <= 0)
      c = 256;
    cache[dev].store(c, std::memory_order_relaxed);
    v = c;
  }
  return v;
}
}  // namespace mtp

using namespace mtp;

namespace {

// Row-chunk kernel overrides for sweeps (variant, splits; -1 = the plan's).
void tune_override(int &variant, int &splits) {
  const int v = tune(kTuneWsVariant), sp = tune(kTuneWsSplits);
  if (v >= 0) variant = v;
  if (sp > 0) splits = sp;
}

typedef WsVariant Variant;
int num_variants(int ct) { return ws_num_variants(ct); }
Variant get_variant(int ct, int wt, int v) { return ws_variant(ct, wt, v); }
WsKernel pick_kernel(int ct, int wt, int mt, int v, int epi) {
  return ws_pick_kernel(ct, wt, mt, v, epi);
}

bool fast_pair(int ct, int wt) {
  if (!is_float_dt(ct)) return false;
  return wt == ct || wt == MTP_FP8E4M3;
}

// 2 workgroups per CU
int target_blocks() { return 2 * device_cus(); }

struct Plan {
  bool generic = true;
  int ct = 0, wt = 0, mt = 0, variant = 0;
  Variant var{};
  int NG = 0, KB = 0, G = 0, S = 1, kb_per = 0, nkb = 0;
  int rows_per_chunk = 64, chunks = 0, xcd_map = 0;
  size_t part_off = 0, sqp_off = 0, ticket_off = 0, aval_off = 0, aidx_off = 0, total = 0;
};


// Launch plan for the weight-streaming kernel. `rows_per_chunk` rows of x go
// to each blockIdx.y chunk. epi == EPI_ARGMAX forces S == 1.
Plan make_plan(int ct, int wt, int64_t M, int64_t N, int64_t K, int epi, int rows_per_chunk) {
  Plan p;
  p.ct = ct;
  p.wt = wt;
  const int cb = dtype_bytes(ct), wb = dtype_bytes(wt);
  if (!fast_pair(ct, wt) || M <= 0 || N <= 0 || K <= 0) return p;
  if (K % (16 / cb) != 0 || K % (16 / wb) != 0) return p;
  if (epi == EPI_ARGMAX && wt != ct) return p;
  // buffer descriptors span one column group of W and one row chunk of x;
  // both must stay below the out-of-range offset 2^31
  if ((int64_t)256 * K * wb >= (int64_t)1 << 31 || (int64_t)64 * K * cb >= (int64_t)1 << 31)
    return p;
  p.rows_per_chunk = rows_per_chunk;
  p.chunks = (int)((M + rows_per_chunk - 1) / rows_per_chunk);
  const int rows = (int)(M < rows_per_chunk ? M : rows_per_chunk);
  p.mt = (rows + 15) / 16;
  // verify: 512 columns per workgroup of 16 waves streamed the lm_head fastest
  int variant = epi == EPI_ARGMAX ? 5 : 0, splits = -1;
  tune_override(variant, splits);
  if (variant >= num_variants(ct)) variant = 0;
  p.variant = variant;
  p.var = get_variant(ct, wt, variant);
  const int LG = p.var.wbl / wb;
  p.KB = 4 * LG;
  p.NG = p.var.wn * p.var.nsub * 16;
  p.G = (int)((N + p.NG - 1) / p.NG);
  p.nkb = (int)((K + p.KB - 1) / p.KB);
  int S = 1;
  if (epi == EPI_LINEAR) {
    const int rounds = (p.nkb + p.var.wk - 1) / p.var.wk;
    S = splits > 0 ? splits : (target_blocks() + p.G * p.chunks / 2) / (p.G * p.chunks);
    if (S < 1) S = 1;
    if (S > rounds) S = rounds;
    // split-K needs one counter per (chunk, group) in the counter prefix
    if ((int64_t)p.chunks * p.G > kCounterSlots) S = 1;
  } else if (p.chunks > kCounterSlots) {
    return Plan{};
  }
  // K-blocks per split, rounded to whole rounds of WK blocks; drop empty splits.
  int rounds_per = ((p.nkb + p.var.wk - 1) / p.var.wk + S - 1) / S;
  p.kb_per = rounds_per * p.var.wk;
  p.S = (p.nkb + p.kb_per - 1) / p.kb_per;
  const int total = p.G * p.S;
  p.xcd_map = (total % 8 == 0 && (total / 8) % p.S == 0) ? 1 : 0;
  const int MPAD = p.mt * 16;
  const int64_t Npad = (int64_t)p.G * p.NG;
  // Layout: [counter prefix | partials]. Counters always start at offset 0
  // and every launch leaves the ones it used at zero, so one workspace can
  // serve any sequence of calls with different shapes and kernels.
  size_t off = kCounterBytes;
  p.ticket_off = 0;
  if (epi == EPI_LINEAR) {
    if (p.S > 1) {
      p.part_off = off;
      off += align_up((size_t)p.chunks * p.S * MPAD * Npad * 4, 256);
      p.sqp_off = off;
      off += align_up((size_t)p.chunks * p.G * p.S * MPAD * 4, 256);
    } else {
      off = 0;  // no workspace at all
    }
  } else {
    p.aval_off = off;
    off += align_up((size_t)p.chunks * p.G * MPAD * 4, 256);
    p.aidx_off = off;
    off += align_up((size_t)p.chunks * p.G * MPAD * 4, 256);
  }
  p.total = off;
  p.generic = false;
  return p;
}

int launch_ws(const Plan &p, WsArgs &a, int epi, void *ws, hipStream_t st) {
  WsKernel k = pick_kernel(p.ct, p.wt, p.mt, p.variant, epi);
  if (!k) return MTP_ERR_DTYPE;
  unsigned char *w8 = (unsigned char *)ws;
  a.rows_per_chunk = p.rows_per_chunk;
  a.S = p.S;
  a.G = p.G;
  a.kb_per = p.kb_per;
  a.nkb = p.nkb;
  a.xcd_map = p.xcd_map;
  if (epi == EPI_LINEAR) {
    if (p.S > 1) {
      a.part = (float *)(w8 + p.part_off);
      a.sqp = (float *)(w8 + p.sqp_off);
      a.ticket = (unsigned *)(w8 + p.ticket_off);
    }
  } else {
    a.amax_val = (float *)(w8 + p.aval_off);
    a.amax_idx = (int *)(w8 + p.aidx_off);
    a.ticket = (unsigned *)(w8 + p.ticket_off);
  }
  const int threads = p.var.wn * p.var.wk * 64;
  dim3 grid((unsigned)(p.G * p.S), (unsigned)p.chunks, 1);
  hipLaunchKernelGGL(k, grid, dim3(threads), 0, st, a);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Pipelined linear kernel: plan and launch.
constexpr size_t kLdsMax = 150 * 1024;  // dynamic LDS limit we allow
// aim for most of the CUs busy (200 of 256)
int wsp_min_blocks() { return device_cus() * 200 / 256; }

struct PlanX {
  bool ok = false;
  int ct = 0, wt = 0, mt = 0, variant = 0;
  bool gam = false;
  WspVariant var{};
  int NG = 0, G = 0, S = 1, kb_per = 0, nkb = 0;
  int chunks = 0, xcd_map = 0;
  size_t lds = 0, part_off = 0, sqp_off = 0, total = 0;
};

// Default tile variant per row count: up to 32 rows (<= 4 x blocks of a
// unit) 64 columns per workgroup without K-splits on large N; 64 rows split
// 128 columns over two K-halves so x loads stay <= W loads per wave.
// fp32 x with a short K (at most 64 units of 64 bytes): the 8-way K split
// inside the workgroup of variant 0 caps the grid's K-splits at two, so the
// 4-way variant 4 takes it (x [16, 1024], W [4096, 1024], TF32 off: 9.9 us
// with four K-splits against 12.9 us).
int wsp_default_variant(int rows, int ct, int64_t nkb) {
  if (rows <= 32 && ct == MTP_F32 && nkb <= 64) return 4;
  return rows <= 32 ? 0 : 1;
}

// A kernel that would keep registers in scratch memory is not used: its
// launches cost orders of magnitude more than the register-resident
// variants. Queried once per (dtypes, tiles, variant, gamma).
bool wsp_usable(int ct, int wt, int mt, int v, bool gam) {
  // 0: not queried yet, 1: usable, 2: not usable (static storage starts at 0)
  static std::atomic<signed char> cache[3][2][4][kWspNumVar][2];
  const int ci = ct == MTP_BF16 ? 0 : ct == MTP_F16 ? 1 : 2;
  std::atomic<signed char> &c = cache[ci][wt == MTP_FP8E4M3][mt - 1][v][gam];
  signed char s = c.load(std::memory_order_relaxed);
  if (s == 0) {
    WsKernel k = wsp_pick_kernel(ct, wt, mt, v, gam);
    hipFuncAttributes fa{};
    // without a device the attributes are unknown; the launch reports errors
    const bool ok =
        k && (hipFuncGetAttributes(&fa, (const void *)k) != hipSuccess || fa.localSizeBytes == 0);
    s = ok ? 1 : 2;
    c.store(s, std::memory_order_relaxed);
  }
  return s == 1;
}

PlanX make_plan_x(int ct, int wt, int64_t M, int64_t N, int64_t K, bool gam) {
  PlanX p;
  p.ct = ct;
  p.wt = wt;
  p.gam = gam;
  const int cb = dtype_bytes(ct), wb = dtype_bytes(wt);
  if (!fast_pair(ct, wt) || M <= 0 || N <= 0 || K <= 0) return p;
  // whole 64-byte units per W row (and so whole 16-byte x fragments)
  if ((K * wb) % 64 != 0) return p;
  // buffer descriptors span one column group of W and one row chunk of x;
  // both stay below the out-of-range offset 2^31
  if ((int64_t)256 * K * wb >= (int64_t)1 << 31 || (int64_t)64 * K * cb >= (int64_t)1 << 31)
    return p;
  p.chunks = (int)((M + 63) / 64);
  const int rows = (int)(M < 64 ? M : 64);
  p.mt = (rows + 15) / 16;
  int variant = wsp_default_variant(rows, ct, (K * wb + 63) / 64), splits = -1;
  tune_override(variant, splits);
  if (variant >= kWspNumVar) variant = 0;
  if (!wsp_usable(ct, wt, p.mt, variant, gam)) variant = 1;
  if (!wsp_usable(ct, wt, p.mt, variant, gam)) return p;
  p.variant = variant;
  p.var = kWspVar[variant];
  const int KU = 64 / wb;                 // k per unit (64 bytes of a W row)
  const int H = (16 / wb) / (16 / cb);    // x fragments per W lane chunk
  p.NG = p.var.wn * p.var.nsub * 16;
  p.G = (int)((N + p.NG - 1) / p.NG);
  p.nkb = (int)((K + KU - 1) / KU);
  int S = 1;
  if (splits > 0) {
    S = splits;
  } else {
    // more K-splits while the grid is short of CUs and every K-group keeps
    // >= 4 stages
    while ((int64_t)p.G * S * p.chunks < wsp_min_blocks() && p.nkb / (S + 1) >= 4 * p.var.wk) ++S;
  }
  if (S > p.nkb) S = p.nkb;
  if (S > 1 && (int64_t)p.chunks * p.G > kCounterSlots) return p;
  p.kb_per = (p.nkb + S - 1) / S;
  p.S = (p.nkb + p.kb_per - 1) / p.kb_per;
  const int total = p.G * p.S;
  p.xcd_map = (total % 8 == 0 && (total / 8) % p.S == 0) ? 1 : 0;
  const int64_t upg = (p.kb_per + p.var.wk - 1) / p.var.wk;
  const int nt = p.var.wn * p.var.wk * 64;
  // gamma of the K-range (plus one padding unit) is staged by kWspGJ 16-byte
  // loads per thread
  if (gam && (p.var.wk * upg + 1) * KU / 4 > (int64_t)kWspGJ * nt) return p;
  p.lds = wsp_lds_bytes(p.mt, H, p.var.nsub, p.var.wn, p.var.wk, upg, KU, gam);
  if (p.lds > kLdsMax) return p;
  const int MPAD = p.mt * 16;
  const int64_t Npad = (int64_t)p.G * p.NG;
  // split-K partials of one row chunk sit behind one buffer descriptor
  if (p.S > 1 && (int64_t)p.S * MPAD * Npad * 4 >= (int64_t)1 << 31) return p;
  size_t off = 0;
  if (p.S > 1) {
    off = kCounterBytes;
    p.part_off = off;
    off += align_up((size_t)p.chunks * p.S * MPAD * Npad * 4, 256);
    p.sqp_off = off;
    off += align_up((size_t)p.chunks * p.G * p.S * MPAD * 4, 256);
  }
  p.total = off;
  p.ok = true;
  return p;
}

int launch_wsp(const PlanX &p, WsArgs &a, void *ws, hipStream_t st) {
  WsKernel k = wsp_pick_kernel(p.ct, p.wt, p.mt, p.variant, p.gam);
  if (!k) return MTP_ERR_DTYPE;
  unsigned char *w8 = (unsigned char *)ws;
  a.rows_per_chunk = 64;
  a.S = p.S;
  a.G = p.G;
  a.kb_per = p.kb_per;
  a.nkb = p.nkb;
  a.xcd_map = p.xcd_map;
  if (p.S > 1) {
    a.part = (float *)(w8 + p.part_off);
    a.sqp = (float *)(w8 + p.sqp_off);
    a.ticket = (unsigned *)w8;
  }
  const hipError_t e = hipFuncSetAttribute((const void *)k,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds);
  if (e != hipSuccess) {
    note_hip_error(e);
    return MTP_ERR_LAUNCH;
  }
  const int threads = p.var.wn * p.var.wk * 64;
  dim3 grid((unsigned)(p.G * p.S), (unsigned)p.chunks, 1);
  hipLaunchKernelGGL(k, grid, dim3(threads), p.lds, st, a);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Skinny weight-streaming plan (sk.hpp): at most 64 rows of 16-bit x, W of
// fp8 or the same 16-bit type, whole 128-byte stages per W row.
struct PlanSk {
  bool ok = false;
  int ct = 0, wt = 0, mt = 0;
  bool gam = false, xr = false, skw = false;
  int G = 0, S = 1, kb_per = 0, nkb = 0;
  int tw = kSkBN;       // output columns per workgroup (the wave-specialised GEMM may take fewer)
  int ch = 1, nsl = 0;  // prep form: 256 ch k per prep slice, slices
  size_t xf_off = 0, pss_off = 0, part_off = 0, ss_off = 0, total = 0;
};

// aim for most of the CUs busy (200 of 256)
int sk_min_blocks() { return device_cus() * 200 / 256; }
// Columns per workgroup for a kernel whose natural tile is `full` columns
// (S K-splits each): the multiple of 8 that puts at most one workgroup on
// every CU, when that narrows the tile by at most a quarter (the grid
// already covers most of the CUs; narrower tiles would multiply the x
// bytes per output column), else `full`.
int fill_width(int64_t N, int S, int full) {
  const int64_t cus = device_cus();
  const int64_t per = (N * S + cus - 1) / cus;
  const int64_t w = (per + 7) / 8 * 8;
  return (w < full && 4 * w >= 3 * (int64_t)full) ? (int)w : full;
}
// Columns per workgroup (a multiple of 8, at most `full`) that split N S
// columns into whole rounds of one workgroup per CU: the fewest rounds R
// whose width ceil(N S / (CUs R)) fits, so the grid ends within 8 columns
// per workgroup of a whole round (a partial last round of a few workgroups
// costs about as much as a full one).
int round_width(int64_t N, int S, int full) {
  const int64_t cus = device_cus();
  for (int64_t R = 1;; ++R) {
    const int64_t w = ((N * S + cus * R - 1) / (cus * R) + 7) / 8 * 8;
    if (w <= full) return (int)w;
  }
}
constexpr int kSkMinStages = 4;    // stages per split at least

// Tile: 64 columns x all rows of x (<= 64); K-splits only while the grid is
// short of CUs. Without gamma the GEMM reads the raw x rows and applies rs
// to its fp32 sums (no prep launch; tuning key sk_xraw 0 keeps the prep).
// Workspace: counters, the xn blocks (prep form), split-K partials (and the
// splits' sums of squares in the raw form).
PlanSk make_plan_sk(int ct, int wt, int64_t M, int64_t N, int64_t K, bool gam,
                    bool skw = false) {
  PlanSk p;
  p.ct = ct;
  p.wt = wt;
  p.gam = gam;
  p.skw = skw;
  if (ct != MTP_BF16 && ct != MTP_F16) return p;
  if (wt != MTP_FP8E4M3 && wt != ct) return p;
  // 17 .. 64 rows: the row-chunk kernel (wsp) is faster below that
  // (fp8 K 4096 N 14336: 8 rows 19.3 us wsp / 20.8 sk, 32 rows 25.5 / 21.2)
  const int force = tune(kTuneSkSplits);
  const bool forced = force > 0;
  if (M <= 0 || M > 64 || N <= 0 || K <= 0 || (M <= 16 && !forced)) return p;
  if (tune(kTuneWsVariant) >= 0 || tune(kTuneWsSplits) > 0) return p;  // sweeps of wsp
  const int wb = dtype_bytes(wt);
  if ((K * wb) % kSkUB != 0 || K > kSkMaxK) return p;
  // buffer descriptors: the workgroup's W rows, all xn blocks
  if ((int64_t)kSkBN * K * wb >= (int64_t)1 << 31 || (int64_t)sk_xf_bytes(M, K) >= (int64_t)1 << 31)
    return p;
  p.mt = M <= 32 ? 1 : 2;
  // raw x whenever there is no gamma (bf16 64 x 4096 x 4096: 14.5 us
  // against 16.3 with the prep; bf16 32 x 4096 x 4096: 12.0 against 14.5;
  // fp8 64 x 14336 x 4096: 25.1 either way)
  p.xr = !gam && tune(kTuneSkXraw) != 0 && !skw;
  if (skw) {
    // the wave-specialised GEMM spreads the columns over every CU when the
    // 64-column grid leaves a few idle (its MFMA tile stays 64 wide). fp8
    // 64 x 14336 x 4096: 56 columns, 256 workgroups, 21.15 us against 21.64
    // with 64 columns (224 workgroups); bf16 28.0 against 30.2. Tuning key
    // skw_tw sets the width.
    const int t = tune(kTuneSkwTw);
    if (t > 0) {
      if (t > kSkBN || t % 8 != 0) return p;
      p.tw = t;
    } else {
      p.tw = fill_width(N, 1, kSkBN);
    }
  }
  p.G = (int)((N + p.tw - 1) / p.tw);
  p.nkb = (int)(K * wb / kSkUB);
  int S = 1;
  if (skw) {
    S = 1;  // the wave-specialised GEMM has no K-splits
  } else if (forced) {
    S = force;
  } else {
    while ((int64_t)p.G * S < sk_min_blocks() && p.nkb / (S + 1) >= kSkMinStages) ++S;
  }
  if (S > p.nkb) S = p.nkb;
  p.kb_per = (p.nkb + S - 1) / S;
  p.S = (p.nkb + p.kb_per - 1) / p.kb_per;
  if ((int64_t)p.G * p.S > INT32_MAX) return p;
  if (p.S > 1 && p.G > kCounterSlots) return p;
  size_t off = kCounterBytes;
  if (!p.xr) {
    p.xf_off = off;
    off += align_up(sk_xf_bytes(M, K), 256);
    // prep slices: 256 ch k each, at most kSkPrepMaxSlices of them
    const int64_t nq = K / 8;
    p.ch = 1;
    while (p.ch < 4 && (nq + 32 * p.ch - 1) / (32 * p.ch) > kSkPrepMaxSlices) p.ch *= 2;
    p.nsl = (int)((nq + 32 * p.ch - 1) / (32 * p.ch));
    if (p.nsl > kSkPrepMaxSlices) return p;
    p.pss_off = off;
    off += align_up((size_t)kSkPrepMaxSlices * 64 * sizeof(float), 256);
  }
  if (p.S > 1) {
    const size_t part = (size_t)p.S * p.G * sk_tile_bytes(p.mt);
    if (part >= ((size_t)1 << 31)) return p;
    p.part_off = off;
    off += align_up(part, 256);
    if (p.xr) {
      p.ss_off = off;
      off += align_up((size_t)p.S * p.G * 64 * sizeof(float), 256);
    }
  }
  p.total = off;
  p.ok = (skw ? skw_pick(ct, wt, p.mt) != nullptr : sk_pick(ct, wt, p.mt, p.xr) != nullptr) &&
         (p.xr || sk_prep8_pick(ct, wt, gam, p.ch) != nullptr);
  return p;
}

int launch_sk(const PlanSk &p, const void *x, const float *gamma, float eps, int norm,
              SkArgs &a, void *ws, hipStream_t st) {
  SkKernel k = sk_pick(p.ct, p.wt, p.mt, p.xr);
  if (!k && !p.skw) return MTP_ERR_DTYPE;
  unsigned char *w8 = (unsigned char *)ws;
  if (p.xr) {
    a.x = x;
    a.norm = norm;
    a.eps = eps;
    if (p.S > 1) a.part_ss = (float *)(w8 + p.ss_off);
  } else {
    SkPrep8Kernel pk = sk_prep8_pick(p.ct, p.wt, p.gam, p.ch);
    if (!pk) return MTP_ERR_DTYPE;
    SkPrepArgs pa;
    pa.x = x;
    pa.gamma = gamma;
    pa.xf = w8 + p.xf_off;
    pa.M = a.M;
    pa.K = a.K;
    pa.norm = norm;
    pa.eps = eps;
    float *pss = (float *)(w8 + p.pss_off);
    hipLaunchKernelGGL(pk, dim3((unsigned)(4 * p.mt), (unsigned)p.nsl), dim3(256), 0, st, pa, pss);
    int s = launch_status();
    if (s != MTP_OK) return s;
    a.xf = pa.xf;
    a.pss = pss;
    a.nsl = p.nsl;
    a.norm = norm;
    a.eps = eps;
  }
  if (p.skw) {
    SkwKernel kw = skw_pick(p.ct, p.wt, p.mt);
    if (!kw) return MTP_ERR_DTYPE;
    SkwArgs wa{};
    wa.xf = a.xf;
    wa.pss = a.pss;
    wa.nsl = a.nsl;
    wa.norm = a.norm;
    wa.eps = a.eps;
    wa.w = a.w;
    wa.wscale = a.wscale;
    wa.bias = a.bias;
    wa.bias_dt = a.bias_dt;
    wa.y = a.y;
    wa.M = a.M;
    wa.N = a.N;
    wa.K = a.K;
    wa.scale = a.scale;
    wa.nst = p.nkb;
    wa.tw = p.tw;
    hipLaunchKernelGGL(kw, dim3((unsigned)p.G), dim3(512), 0, st, wa);
    return launch_status();
  }
  a.G = p.G;
  a.S = p.S;
  a.kb_per = p.kb_per;
  a.nkb = p.nkb;
  if (p.S > 1) {
    a.part = (float *)(w8 + p.part_off);
    a.ticket = (unsigned *)w8;
  }
  hipLaunchKernelGGL(k, dim3((unsigned)(p.G * p.S)), dim3(256), 0, st, a);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Single-launch skinny plan (skl.hpp): at most 64 rows of 16-bit x, W of fp8
// or the same 16-bit type, whole 128-byte stages per W row, the norm folded
// into the GEMM. Tiles of 32 nw columns; K-splits until the grid covers the
// CUs once. Workspace: counters, split-K partial tiles and sums of squares.
struct PlanSkl {
  bool ok = false;
  int ct = 0, wt = 0, mt = 0, nw = 8;
  bool gam = false;
  int G = 0, S = 1, kb_per = 0, nkb = 0;
  int tw = 256;  // output columns per workgroup (<= 32 nw)
  size_t part_off = 0, ss_off = 0, total = 0;
};


// MTP_SKL=1 forces the single-launch kernel wherever it applies, MTP_SKL=0
// turns it off. By default it runs where its 256-column tiles fill the CUs
// without a K-split (N > 128 * 256), and for at most 16 rows once W is large
// enough (>= 48 MiB) to repay a split's hand-off through the device
// coherence point (partial stores, arrival ticket, partial loads: about
// 7 us at the end of the launch). Measured, K 4096: fp8 M 64 N 131072 144
// us vs 174 us (64-column kernel), M 16 N 131072 95 us vs 153 us; with
// splits, fp8 M 8 N 28672 27.9 us vs 37.1 us (row-chunk kernel), M 16 N
// 14336 18.6 vs 21.5, M 8 N 8192 17.8 vs 14.5 (below the bound), bf16 M 16
// N 28672 51.4 vs 72.1; fp8 M 64 N 14336 (four splits) 27.8 us vs 25.7 us.
constexpr int64_t kSklSplitMinWBytes = (int64_t)48 << 20;
int skl_mode() { return tune(kTuneSkl); }

PlanSkl make_plan_skl(int ct, int wt, int64_t M, int64_t N, int64_t K, bool gam) {
  PlanSkl p;
  p.ct = ct;
  p.wt = wt;
  p.gam = gam;
  if (ct != MTP_BF16 && ct != MTP_F16) return p;
  if (wt != MTP_FP8E4M3 && wt != ct) return p;
  if (M <= 0 || M > 64 || N <= 0 || K <= 0) return p;
  const int wb = dtype_bytes(wt);
  if ((K * wb) % kSkUB != 0) return p;
  if (tune(kTuneSklWaves) > 0) p.nw = tune(kTuneSklWaves) == 4 ? 4 : 8;
  const int64_t bn = skl_bn(p.nw);
  // buffer descriptors: x, the workgroup's W rows (32-bit sizes and offsets)
  if (M * K * 2 >= ((int64_t)1 << 31) || bn * K * wb >= ((int64_t)1 << 31)) return p;
  p.mt = M <= 32 ? 1 : 2;
  p.G = (int)((N + bn - 1) / bn);
  p.nkb = (int)(K * wb / kSkUB);
  const int uk = kSkUB / wb;  // k per stage
  int S = 1;
  if (tune(kTuneSklSplits) > 0) S = tune(kTuneSklSplits);
  else S = std::max(1, device_cus() / std::max(1, p.G));
  if (S > p.nkb) S = p.nkb;
  for (;;) {
    p.kb_per = (p.nkb + S - 1) / S;
    if (!gam || (int64_t)p.kb_per * uk <= kSklGammaMax || S >= p.nkb) break;
    ++S;
  }
  if (gam && (int64_t)p.kb_per * uk > kSklGammaMax) return p;
  p.S = (p.nkb + p.kb_per - 1) / p.kb_per;
  // columns per workgroup: the tile narrowed to fill every CU (fp8 32 x
  // 14336 x 4096, 4 splits: 224 columns, 256 workgroups); tuning key
  // skl_tw sets it
  p.tw = (int)bn;
  if (tune(kTuneSklTw) > 0) {
    const int t = tune(kTuneSklTw);
    if (t > bn || t % 8 != 0) return p;
    p.tw = t;
  } else {
    // wide N without K-splits (a 64-column tile per CU at least): whole
    // rounds of one workgroup per CU where that narrows the tile by at most
    // half (bf16 8 x 151936 x 4096: 200 columns, 760 workgroups, 183.3
    // against 198.4 µs with 256 columns in 594 workgroups); otherwise one
    // round filled
    const int rw = p.S == 1 ? round_width(N, 1, (int)bn) : 0;
    p.tw = p.S == 1 && 2 * rw >= (int)bn && N >= (int64_t)device_cus() * 64
               ? rw
               : fill_width(N, p.S, (int)bn);
  }
  p.G = (int)((N + p.tw - 1) / p.tw);
  if ((int64_t)p.G * p.S > INT32_MAX) return p;
  if (p.S > 1 && p.G > kCounterSlots) return p;
  size_t off = kCounterBytes;
  if (p.S > 1) {
    const size_t part = (size_t)p.S * p.G * skl_tile_bytes(p.mt, p.nw);
    if (part >= ((size_t)1 << 31)) return p;
    p.part_off = off;
    off += align_up(part, 256);
    p.ss_off = off;
    off += align_up((size_t)p.S * p.G * 64 * sizeof(float), 256);
  }
  p.total = off;
  p.ok = skl_pick(ct, wt, p.mt, p.nw, gam) != nullptr;
  return p;
}

int launch_skl(const PlanSkl &p, SklArgs &a, void *ws, hipStream_t st) {
  SklKernel k = skl_pick(p.ct, p.wt, p.mt, p.nw, p.gam);
  if (!k) return MTP_ERR_DTYPE;
  unsigned char *w8 = (unsigned char *)ws;
  a.G = p.G;
  a.S = p.S;
  a.kb_per = p.kb_per;
  a.nkb = p.nkb;
  a.tw = p.tw;
  // the splits of a tile on one XCD from 4 splits up (fp8 24 x 14336 x
  // 4096: 19.1 -> 17.6 us); with 2 splits it loses (fp8 64 x 28672 x 4096:
  // 38.4 -> 39.9 us)
  a.xg = p.S >= 4;
  if (p.S > 1) {
    a.part = (float *)(w8 + p.part_off);
    a.part_ss = (float *)(w8 + p.ss_off);
    a.ticket = (unsigned *)w8;
  }
  hipLaunchKernelGGL(k, dim3((unsigned)(p.G * p.S)), dim3((unsigned)(64 * p.nw)), 0, st, a);
  return launch_status();
}

// ---------------------------------------------------------------------------
// x-resident skinny plan (skp.hpp): at most 64 rows of 16-bit x, W of fp8 or
// the same 16-bit type, whole 128-byte steps per W row. The x rows of a
// K-split live in LDS (<= kSkpXMaxBytes), so the split count follows from the
// rows: 1 up to 16 rows (K <= 4096 fp8 / 2048 16-bit W per 16 rows x 128 KB),
// more above. The column tile (64 TA) is the widest whose grid still covers
// 7/8 of the CUs. Workspace: counters, split-K partial tiles, sums of squares.
struct PlanSkp {
  bool ok = false;
  int ct = 0, wt = 0, mt = 0, ta = 1;
  bool gam = false, h8 = false;
  int G = 0, S = 1, kb_per = 0, nkb = 0;
  int tw = 64;  // output columns per workgroup (<= 64 ta)
  size_t lds = 0, part_off = 0, ss_off = 0, total = 0;
};

constexpr int kSkpGammaMax = kSkpGammaLoads * kSkpWaves * 256;  // gamma floats per split

// 1 forced, 0 off; by default on, unless a key forces one of the other
// skinny kernels (sweeps and tests of those)
int skp_mode() {
  const int m = tune(kTuneSkp);
  if (m >= 0) return m;
  const bool other = tune(kTuneSkl) == 1 || tune(kTuneSkSplits) > 0 ||
                     tune(kTuneSklSplits) > 0 || tune(kTuneSklWaves) > 0 ||
                     tune(kTuneWsVariant) >= 0 || tune(kTuneWsSplits) > 0;
  return other ? 0 : 1;
}

PlanSkp make_plan_skp(int ct, int wt, int64_t M, int64_t N, int64_t K, bool gam) {
  PlanSkp p;
  p.ct = ct;
  p.wt = wt;
  p.gam = gam;
  if (ct != MTP_BF16 && ct != MTP_F16) return p;
  if (wt != MTP_FP8E4M3 && wt != ct) return p;
  if (M <= 0 || M > 64 || N <= 0 || K <= 0) return p;
  const int wb = dtype_bytes(wt);
  if ((K * wb) % kSkpStageBytes != 0) return p;
  const int ks = wt == MTP_FP8E4M3 ? 4 : 2, uk = 32 * ks;
  // buffer descriptors: x, the workgroup's W rows (32-bit sizes and offsets)
  if (M * K * 2 >= ((int64_t)1 << 31) || 256 * K * wb >= ((int64_t)1 << 31)) return p;
  p.mt = (int)((M + 15) / 16);
  p.nkb = (int)(K * wb / kSkpStageBytes);
  // at most 8 rows: compact x blocks (only the parts holding rows 0 .. 7:
  // half the LDS at fp8, a quarter at 16-bit W, so longer K-splits fit)
  p.h8 = M <= 8 && tune(kTuneSkpH8) != 0;
  const int xp = p.h8 ? 8 / (1024 / (2 * uk)) : ks;  // 1 KB parts per x block
  int smax = kSkpXMaxBytes / (p.mt * xp * 1024);  // steps per split that fit
  if (gam) smax = std::min(smax, kSkpGammaMax / uk);
  const int64_t want = (int64_t)device_cus() * 7 / 8;
  int S = (p.nkb + smax - 1) / smax;
  if (tune(kTuneSkpSplits) > 0) {
    S = std::max(S, tune(kTuneSkpSplits));
  } else {
    // enough 64-column workgroups for the CUs, at least 8 steps per split
    // (beyond a workgroup per CU the split-K hand-off costs more than the x
    // copies it saves)
    const int64_t g1 = (N + 63) / 64;
    while (g1 * S < want && p.nkb / (S + 1) >= 8) ++S;
  }
  if (S > p.nkb) S = p.nkb;
  p.kb_per = (p.nkb + S - 1) / S;
  p.S = (p.nkb + p.kb_per - 1) / p.kb_per;
  // wide N without K-splits (at least a 64-column tile per CU): the width
  // that splits the columns into whole rounds of one workgroup per CU, on
  // the narrowest tile (1, 2 or 4 A tiles per wave) that holds it; bf16 K
  // 4096, 8 rows, µs per call: N 40960 53.7 against 62.5 (128-column
  // tiles, 320 workgroups), N 151936 186.4 against 200.5 (256 columns, 594
  // workgroups)
  const bool wide = tune(kTuneSkpTa) <= 0 && tune(kTuneSkpTw) <= 0 && p.S == 1 &&
                    N >= (int64_t)device_cus() * 64;
  const int rw = wide ? round_width(N, 1, 256) : 0;
  if (tune(kTuneSkpTa) > 0) {
    const int t = tune(kTuneSkpTa);
    p.ta = t >= 4 ? 4 : t >= 2 ? 2 : 1;
  } else if (wide) {
    p.ta = rw <= 64 ? 1 : rw <= 128 ? 2 : 4;
  } else {
    p.ta = 1;
    for (int t = 4; t >= 2; t /= 2)
      if ((N + 64 * t - 1) / (64 * t) * p.S >= want) {
        p.ta = t;
        break;
      }
  }
  // columns per workgroup: the tile narrowed to fill every CU (fp8 8 x
  // 14336 x 4096: 56 columns, 256 workgroups); tuning key skp_tw sets it
  p.tw = 64 * p.ta;
  if (tune(kTuneSkpTw) > 0) {
    const int t = tune(kTuneSkpTw);
    if (t > 64 * p.ta || t % 8 != 0) return p;
    p.tw = t;
  } else if (wide) {
    p.tw = rw;
  } else {
    p.tw = fill_width(N, p.S, 64 * p.ta);
  }
  p.G = (int)((N + p.tw - 1) / p.tw);
  if ((int64_t)p.G * p.S > INT32_MAX) return p;
  if (p.S > 1 && p.G > kCounterSlots) return p;
  p.lds = skp_lds_bytes(p.mt, xp, p.kb_per, uk, gam);
  if (p.lds > (size_t)kSkpXMaxBytes + kSkpStaging + (size_t)kSkpGammaMax * 4) return p;
  size_t off = kCounterBytes;
  if (p.S > 1) {
    const size_t part = (size_t)p.S * p.G * kSkpWaves * p.ta * p.mt * 1024;
    if (part >= ((size_t)1 << 31)) return p;
    p.part_off = off;
    off += align_up(part, 256);
    p.ss_off = off;
    off += align_up((size_t)p.S * p.G * 64 * sizeof(float), 256);
  }
  p.total = off;
  p.ok = skp_pick(ct, wt, p.mt, p.ta, gam, p.h8) != nullptr;
  return p;
}

int launch_skp(const PlanSkp &p, SkpArgs &a, void *ws, hipStream_t st) {
  SkpKernel k = skp_pick(p.ct, p.wt, p.mt, p.ta, p.gam, p.h8);
  if (!k) return MTP_ERR_DTYPE;
  unsigned char *w8 = (unsigned char *)ws;
  a.G = p.G;
  a.S = p.S;
  a.kb_per = p.kb_per;
  a.nkb = p.nkb;
  a.tw = p.tw;
  // the splits of a tile on one XCD with compact x blocks (fp8 8 x 4096 x
  // 4096: 10.3 -> 9.5 us); with full blocks it loses (bf16 16 x 4096 x
  // 4096: 11.1 -> 11.4 us)
  a.xg = p.h8 ? 1 : 0;
  if (p.S > 1) {
    a.part = (float *)(w8 + p.part_off);
    a.part_ss = (float *)(w8 + p.ss_off);
    a.ticket = (unsigned *)w8;
  }
  const hipError_t e = hipFuncSetAttribute((const void *)k,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)p.lds);
  if (e != hipSuccess) {
    note_hip_error(e);
    return MTP_ERR_LAUNCH;
  }
  hipLaunchKernelGGL(k, dim3((unsigned)(p.G * p.S)), dim3(64 * kSkpWaves), p.lds, st, a);
  return launch_status();
}

int launch_generic_linear(const void *x, int xt, const void *w, int wt, const float *wscale,
                          const void *i4scale, int i4dt, int group, int nib, const void *gamma,
                          int gt, const void *bias, int bt, void *y, int64_t M, int64_t N,
                          int64_t K, float eps, float scale, int norm, hipStream_t st) {
  if (M > 65535) return MTP_ERR_SHAPE;
  dim3 grid((unsigned)((N + 255) / 256), (unsigned)M, 1);
  hipLaunchKernelGGL(generic_rmsnorm_linear_kernel, grid, dim3(256), 0, st, x, xt, w, wt,
                     wscale, i4scale, i4dt, group, nib, gamma, gt, bias, bt, y, xt, (int)M,
                     (int)N, (int)K, eps, scale, norm);
  return launch_status();
}

// Shared body of the three RMSNorm -> linear entry points (float / fp8 weights).
int rmsnorm_linear_impl(const void *x, int xt, int64_t M, int64_t K, const void *w, int wt,
                        int64_t N, const float *wscale, const void *bias, int bt,
                        const void *gamma, int gt, float eps, float scale, int norm, void *y,
                        void *ws, size_t ws_bytes, void *stream) {
  if (!is_float_dt(xt)) return MTP_ERR_DTYPE;
  if (!(is_float_dt(wt) || wt == MTP_FP8E4M3)) return MTP_ERR_DTYPE;
  if (bias && !is_float_dt(bt)) return MTP_ERR_DTYPE;
  if (gamma && !is_float_dt(gt)) return MTP_ERR_DTYPE;
  if (M < 0 || N < 0 || K < 0 || N > INT32_MAX || K > INT32_MAX || M > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (M == 0 || N == 0) return MTP_OK;
  if (!x && K > 0) return MTP_ERR_NULL;
  if ((!w && K > 0) || !y) return MTP_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  const bool aligned = aligned16(x) && aligned16(w) && aligned16(y) && (!gamma || aligned16(gamma));
  WsArgs a{};
  a.x = x;
  a.w = w;
  a.wscale = wscale;
  a.gamma = (const float *)gamma;
  a.bias = bias;
  a.bias_dt = bt;
  a.y = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.eps = eps;
  a.scale = scale;
  a.norm = norm;
  // fp32 x and W, <= 32 rows: one launch of 16-column workgroups, every load
  // in one round trip or each wave's K-range streamed through LDS
  // (launch_sf32 picks; fp32 K 1024 N 4096 16 rows: the planner's tiled
  // kernel 9.9 us)
  if (xt == MTP_F32 && wt == MTP_F32 && !wscale && tune(kTuneSf32) != 0 && M <= 32 &&
      K >= 16 && K <= kSf32StreamMaxK && K % 16 == 0 && aligned && (!gamma || gt == MTP_F32) &&
      tune(kTuneWsVariant) < 0 && tune(kTuneWsSplits) <= 0) {
    Sf32Args sa{};
    sa.x = (const float *)x;
    sa.gamma = (const float *)gamma;
    sa.w = (const float *)w;
    sa.bias = bias;
    sa.bias_dt = bt;
    sa.y = (float *)y;
    sa.M = (int)M;
    sa.N = (int)N;
    sa.K = (int)K;
    sa.norm = norm;
    sa.eps = eps;
    sa.scale = scale;
    return launch_sf32(sa, st);
  }
  const int skpm = skp_mode();
  if (skpm != 0 && aligned && (!gamma || gt == MTP_F32)) {
    const PlanSkp pp = make_plan_skp(xt, wt, M, N, K, gamma != nullptr);
    // past N = 32768 with at least 48 MiB of W the single-launch kernel
    // streams W faster for these rows too (K 4096, 8 rows, µs per call:
    // bf16 N 40960 51.9 against 53.5, N 128256 155.1 against 157.0, fp8 N
    // 65536 46.6 against 47.4; at N 32768 and below the x-resident kernel
    // leads: bf16 42.7 against 57.4)
    bool to_skl = false;
    if (tune(kTuneSkp) != 1 && N > 32768 && skl_mode() != 0 &&
        N * K * dtype_bytes(wt) >= kSklSplitMinWBytes) {
      const PlanSkl pl = make_plan_skl(xt, wt, M, N, K, gamma != nullptr);
      to_skl = pl.ok;
    }
    // by default up to 16 rows (one x tile); above that the split-K
    // hand-off and the per-workgroup in-place pass cost more than the other
    // kernels' x re-reads (fp8 K 4096 N 14336: 8 rows 14.5 us vs 18.0,
    // 16 rows 16.4 vs 18.4, 32 rows 20.8 vs 19.9, 64 rows 31 vs 24; 16-bit W
    // 4096 x 4096, 16 rows: 11.1 vs 14.3)
    if (pp.ok && !to_skl && (tune(kTuneSkp) == 1 || pp.mt == 1)) {
      if (!ws || ws_bytes < pp.total) return MTP_ERR_WORKSPACE;
      SkpArgs pa{};
      pa.x = x;
      pa.gamma = (const float *)gamma;
      pa.w = w;
      pa.wscale = wscale;
      pa.bias = bias;
      pa.bias_dt = bt;
      pa.y = y;
      pa.M = (int)M;
      pa.N = (int)N;
      pa.K = (int)K;
      pa.norm = norm;
      pa.eps = eps;
      pa.scale = scale;
      return launch_skp(pp, pa, ws, st);
    }
  }
  // wave-specialised skinny GEMM (after the prep launch): by default for
  // 33 .. 64 rows with gamma where the 64-column tiles alone fill most of
  // the CUs (no K-split); tuning key skw 1 forces it wherever it applies, 0
  // turns it off. Measured, K 4096, N 14336: fp8 64 rows 21.7 us against
  // 23.4 (two-launch kernel), 48 rows 21.6 against 22.8; it ties at 24 and
  // 32 rows (single-launch kernel) and with 16-bit W and gamma (64 rows
  // 30.3 against 30.5), and loses without gamma to the raw-x form (bf16 W,
  // 48 rows: 30.0 against 27.1).
  if (aligned && (!gamma || gt == MTP_F32) && tune(kTuneSkw) != 0) {
    bool want = tune(kTuneSkw) == 1;
    if (!want && gamma && M > 32 && tune(kTuneSkl) != 1 && tune(kTuneSkSplits) <= 0) {
      const PlanSk nat = make_plan_sk(xt, wt, M, N, K, true);
      want = nat.ok && nat.S == 1;
    }
    const PlanSk ps = want ? make_plan_sk(xt, wt, M, N, K, gamma != nullptr, true) : PlanSk{};
    if (ps.ok) {
      if (!ws || ws_bytes < ps.total) return MTP_ERR_WORKSPACE;
      SkArgs sa{};
      sa.w = w;
      sa.wscale = wscale;
      sa.bias = bias;
      sa.bias_dt = bt;
      sa.y = y;
      sa.M = (int)M;
      sa.N = (int)N;
      sa.K = (int)K;
      sa.scale = scale;
      return launch_sk(ps, x, (const float *)gamma, eps, norm, sa, ws, st);
    }
  }
  const int sklm = skl_mode();
  if (sklm != 0) {
    const PlanSkl pl = make_plan_skl(xt, wt, M, N, K, gamma != nullptr);
    // with splits: <= 16 rows from 48 MiB of W; fp8 W also 17 .. 32 rows
    // from 48 MiB and 33 .. 64 rows from 96 MiB (fp8 K 4096: M 24 N 14336
    // 18.7 us vs 20.4, M 64 N 28672 37.5 vs 44.6, M 64 N 14336 27.8 vs 25.0;
    // 16-bit W above 16 rows ties or loses: M 32 N 8192 K 8192 35.0 vs 31.9)
    const bool wide = pl.S == 1;
    const int64_t wbytes = N * K * dtype_bytes(wt);
    const bool big_skinny =
        (M <= 16 && wbytes >= kSklSplitMinWBytes) ||
        (wt == MTP_FP8E4M3 && ((M <= 32 && wbytes >= kSklSplitMinWBytes) ||
                               wbytes >= 2 * kSklSplitMinWBytes));
    if (pl.ok && (sklm == 1 || wide || big_skinny) && aligned && (!gamma || gt == MTP_F32)) {
      if (!ws || ws_bytes < pl.total) return MTP_ERR_WORKSPACE;
      SklArgs la{};
      la.x = x;
      la.gamma = (const float *)gamma;
      la.w = w;
      la.wscale = wscale;
      la.bias = bias;
      la.bias_dt = bt;
      la.y = y;
      la.M = (int)M;
      la.N = (int)N;
      la.K = (int)K;
      la.norm = norm;
      la.eps = eps;
      la.scale = scale;
      return launch_skl(pl, la, ws, st);
    }
  }
  const PlanSk ps = make_plan_sk(xt, wt, M, N, K, gamma != nullptr);
  if (ps.ok && aligned && (!gamma || gt == MTP_F32)) {
    if (!ws || ws_bytes < ps.total) return MTP_ERR_WORKSPACE;
    SkArgs sa{};
    sa.w = w;
    sa.wscale = wscale;
    sa.bias = bias;
    sa.bias_dt = bt;
    sa.y = y;
    sa.M = (int)M;
    sa.N = (int)N;
    sa.K = (int)K;
    sa.scale = scale;
    return launch_sk(ps, x, (const float *)gamma, eps, norm, sa, ws, st);
  }
  PlanX p = make_plan_x(xt, wt, M, N, K, gamma != nullptr);
  // the tiled kernel reads gamma as fp32 (the Python shim upcasts it)
  if (!p.ok || !aligned || (gamma && gt != MTP_F32)) {
    return launch_generic_linear(x, xt, w, wt, wscale, nullptr, 0, 0, -1, gamma, gt, bias, bt, y,
                                 M, N, K, eps, scale, norm, st);
  }
  if (p.total > 0 && (!ws || ws_bytes < p.total)) return MTP_ERR_WORKSPACE;
  return launch_wsp(p, a, ws, st);
}


// ---------------------------------------------------------------------------
// Attention: plan and launch.
// 8-wave workgroups that fill the chip once: one per CU
int attn_target_blocks() { return device_cus(); }

struct AttnPlan {
  int qt = 0, nchunks = 1, chunk_blocks = 0;
  bool fast = false;
  size_t part_off = 0, ml_off = 0, total = 0;
};

// Key blocks of kAttnBlock (context, then dense) are split into chunks of
// chunk_blocks consecutive blocks, one workgroup each, so that the launch
// has at most one workgroup per CU where the heads allow; the
// attn_chunk_blocks tuning key overrides the chunk length.
AttnPlan make_attn_plan(int ct, int64_t B, int64_t NQ, int64_t H, int64_t D, int64_t Lc,
                        int64_t Lt) {
  AttnPlan p;
  p.fast = (ct == MTP_BF16 || ct == MTP_F16) && (D == 64 || D == 128) && NQ >= 1 && NQ <= 64;
  if (!p.fast) return p;  // the fallback needs no workspace
  p.qt = (int)((NQ + 15) / 16);
  const int64_t ntot = (Lc + kAttnBlock - 1) / kAttnBlock + (Lt + kAttnBlock - 1) / kAttnBlock;
  if (ntot == 0) return p;
  const int64_t want = std::max<int64_t>(1, attn_target_blocks() / (B * H));
  int64_t cb = (ntot + want - 1) / want;
  if (tune(kTuneAttnChunkBlocks) > 0) cb = tune(kTuneAttnChunkBlocks);
  cb = std::max(cb, (ntot + kAttnMaxChunks - 1) / kAttnMaxChunks);
  p.chunk_blocks = (int)std::min<int64_t>(cb, ntot);
  p.nchunks = (int)((ntot + p.chunk_blocks - 1) / p.chunk_blocks);
  if (p.nchunks > 1) {
    const int64_t qp = (int64_t)p.qt * 16;
    size_t off = kCounterBytes;
    p.part_off = off;
    off += align_up((size_t)(B * H) * p.nchunks * qp * D * 4, 256);
    p.ml_off = off;
    off += align_up((size_t)(B * H) * p.nchunks * qp * 2 * 4, 256);
    p.total = off;
  }
  return p;
}

// The 32-query-tile kernel takes 33 .. 64 queries at head dim 128 when its
// buffer descriptors cover the key sources: every valid context row lies in
// [0, npages * page stride) of the pages and the dense rows of a head span
// less than 2 GiB (offsets stay below the out-of-range marker).
bool attn32_usable(const AttnArgs &a, int ct, int64_t D) {
  if (tune(kTuneAttn32) == 0) return false;
  if ((ct != MTP_BF16 && ct != MTP_F16) || D != 128 || a.NQ <= 32 || a.NQ > 64) return false;
  const int64_t lim = (int64_t)1 << 31;
  if (a.Lc > 0) {
    if (a.p_sp < 0 || a.p_sb < 0 || a.p_sh < 0 || a.npages <= 0) return false;
    if ((int64_t)(a.B - 1) * a.p_sb + (int64_t)(a.H - 1) * a.p_sh + (int64_t)a.page_size * D >
        a.p_sp)
      return false;
    if ((int64_t)a.npages * a.p_sp * 2 >= lim) return false;
  }
  if (a.Lt > 0) {
    if (a.d_st < 0 || ((int64_t)(a.Lt - 1) * a.d_st + D) * 2 >= lim) return false;
  }
  return true;
}

// Shared launch path of the three attention entry points. All strides are
// in elements; the MFMA kernel needs 16-byte aligned rows (strides multiple
// of 8 elements), the fallback takes anything.
int launch_attention(AttnArgs &a, int ct, int64_t D, void *ws, size_t ws_bytes, hipStream_t st) {
  if (a.B * (int64_t)a.H > INT32_MAX || a.NQ > 65535) return MTP_ERR_SHAPE;
  AttnPlan p = make_attn_plan(ct, a.B, a.NQ, a.H, D, a.Lc, a.Lt);
  const bool strides8 = (a.q_sb | a.q_sn | a.q_sh | a.p_sp | a.p_sb | a.p_sh | a.d_sb | a.d_sh |
                         a.d_st | a.o_sb | a.o_sn | a.o_sh) % 8 == 0;
  const bool aligned = aligned16(a.q) && aligned16(a.out) && (!a.kp || aligned16(a.kp)) &&
                       (!a.vp || aligned16(a.vp)) && (!a.kd || aligned16(a.kd)) &&
                       (!a.vd || aligned16(a.vd));
  if (p.fast && strides8 && aligned && !a.kv_fp8) {
    if (p.total > 0 && (!ws || ws_bytes < p.total)) return MTP_ERR_WORKSPACE;
    AttnKernel k = attn_pick(ct, (int)D);
    AttnKernel km = attn_merge_pick(ct, (int)D);
    if (!k || !km) return MTP_ERR_DTYPE;
    unsigned char *w8 = (unsigned char *)ws;
    a.nchunks = p.nchunks;
    a.chunk_blocks = p.chunk_blocks;
    if (p.nchunks > 1) {
      a.part = (float *)(w8 + p.part_off);
      a.ml = (float *)(w8 + p.ml_off);
    }
    dim3 grid((unsigned)(a.B * a.H), (unsigned)p.nchunks, 1);
    if (attn32_usable(a, ct, D)) {
      AttnKernel k2 = attn2_pick(ct);
      const hipError_t e = hipFuncSetAttribute((const void *)k2,
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               attn2_lds_bytes());
      if (e != hipSuccess) {
        note_hip_error(e);
        return MTP_ERR_LAUNCH;
      }
      hipLaunchKernelGGL(k2, grid, dim3(512), (size_t)attn2_lds_bytes(), st, a);
    } else {
      hipLaunchKernelGGL(k, grid, dim3(512), 0, st, a);
    }
    if (p.nchunks > 1) {
      int s = launch_status();
      if (s != MTP_OK) return s;
      hipLaunchKernelGGL(km,
                         dim3((unsigned)(a.B * a.H), (unsigned)((a.NQ + kAttnMergeQ - 1) / kAttnMergeQ), 1),
                         dim3((unsigned)(D / 4 * kAttnMergeQ)), 0, st, a);
    }
    return launch_status();
  }
  dim3 grid((unsigned)(a.B * a.H), (unsigned)a.NQ, 1);
  if (D > 256) {
    auto k = attn_generic_wide((int)std::min<int64_t>(D, INT32_MAX));
    if (!k) return MTP_ERR_SHAPE;
    hipLaunchKernelGGL(k, grid, dim3(256), 0, st, a, (int)D, ct);
    return launch_status();
  }
  hipLaunchKernelGGL(attn_generic(), grid, dim3(64), 0, st, a, (int)D, ct);
  return launch_status();
}

bool mask_dt_ok(int dt) { return is_float_dt(dt) || dt == MTP_U8; }

// ---------------------------------------------------------------------------
// INT4 MFMA path: x -> (fragment-major fp16 copy, omul) in the workspace,
// then the decode-in-register GEMM. Workspace: the fp16 copy (rows padded
// to whole row groups) at 0, omul after it.
struct Int4Tiles {
  int mt, na;    // 32-row x tiles, 32-row weight subtiles per wave row group
  int layout;    // wave layout (kI4Rows4, kI4Rows4KHalves, kI4Rows2KHalves)
  int bn;        // weight rows per workgroup
  int64_t gm;    // row groups
  int64_t rows;  // padded rows
};
// Tiles and wave layout for M rows. Up to 64 rows: 4 waves on 4 row groups.
// Beyond: 8 waves (4 row groups x 2 k-halves, two waves per SIMD) by
// default (M 256, K 8192, N 28672: 127 us against 132 with 4 waves); the
// int4_waves tuning key (4 or 8) overrides.
Int4Tiles int4_tiles(int64_t M) {
  Int4Tiles t;
  t.mt = M <= 32 ? 1 : M <= 64 ? 2 : 4;
  t.layout = t.mt == 4 ? kI4Rows4KHalves : kI4Rows4;
  if (tune(kTuneInt4Waves) > 0) t.layout = tune(kTuneInt4Waves) == 8 ? kI4Rows4KHalves : kI4Rows4;
  t.na = t.mt == 4 ? 2 : 1;
  t.bn = int4_bn(t.na);
  t.gm = (M + 32 * t.mt - 1) / (32 * t.mt);
  t.rows = t.gm * 32 * t.mt;
  return t;
}
// Row stride of the transposed fp16 scales: the columns the GEMM covers.
int64_t int4_ldst(int64_t M, int64_t N) {
  const int64_t bn = int4_tiles(M).bn;
  return (N + bn - 1) / bn * bn;
}
size_t int4_xn_bytes(int64_t M, int64_t K) {
  return align_up((size_t)int4_tiles(M).rows * K * 2, 256);
}
size_t int4_omul_bytes(int64_t M) { return align_up((size_t)int4_tiles(M).rows * 4, 256); }
size_t int4_scT_bytes(int64_t M, int64_t N, int64_t ng) {
  return align_up((size_t)ng * int4_ldst(M, N) * 2, 256);
}
// Workspace: the counter region (left untouched: other entry points keep
// their arrival tickets there), then xn, omul, the transposed scales and the
// columns' normalising factors.
size_t int4_ws_bytes(int64_t M, int64_t N, int64_t K, int64_t ng) {
  return kCounterBytes + int4_xn_bytes(M, K) + int4_omul_bytes(M) + int4_scT_bytes(M, N, ng) +
         align_up((size_t)int4_ldst(M, N) * 4, 256);
}
constexpr int64_t kInt4MaxK = (int64_t)1 << 23;  // keeps every buffer offset in 32 bits
bool int4_fast(int64_t M, int64_t N, int64_t K, int64_t group) {
  if (K <= 0 || K % 128 != 0 || K > kInt4MaxK || group % 32 != 0) return false;
  const int64_t ng = (K + group - 1) / group;
  return ng * int4_ldst(M, N) * 2 < ((int64_t)1 << 31);
}

int launch_int4(const void *x, int xdt, int64_t M, int64_t K, const uint8_t *packed,
                const void *scales, int sdt, int64_t N, int64_t group, int nibble,
                const void *gamma, int gdt, float eps, int norm, void *y, void *ws,
                size_t ws_bytes, hipStream_t st) {
  const int64_t ng = (K + group - 1) / group;
  if (!ws || ws_bytes < int4_ws_bytes(M, N, K, ng)) return MTP_ERR_WORKSPACE;
  if (((uintptr_t)ws & 15u) != 0) return MTP_ERR_ALIGN;
  const Int4Tiles tl = int4_tiles(M);
  const int nw = tl.layout == kI4Rows4KHalves ? 8 : 4;
  I4Kernel gemm = int4_gemm_pick(tl.mt, tl.na, tl.layout, nibble == MTP_NIBBLE_TWOS);
  if (!gemm) return MTP_ERR_DTYPE;
  const int64_t gn = (N + tl.bn - 1) / tl.bn;
  const int64_t blocks = (gn + 7) / 8 * 8 * tl.gm;
  const int64_t sblocks = (N + 63) / 64;  // scale-transpose blocks of the prep launch
  if (blocks > INT32_MAX || tl.rows + sblocks > INT32_MAX) return MTP_ERR_SHAPE;
  unsigned char *w8 = (unsigned char *)ws + kCounterBytes;
  I4Args a;
  a.xn = w8;
  a.omul = (const float *)(w8 + int4_xn_bytes(M, K));
  uint16_t *scT = (uint16_t *)(w8 + int4_xn_bytes(M, K) + int4_omul_bytes(M));
  float *cmul = (float *)((unsigned char *)scT + int4_scT_bytes(M, N, ng));
  a.ldst = (int)int4_ldst(M, N);
  I4PrepKernel prep = int4_prep(xdt, gamma ? gdt : -1);
  if (!prep) return MTP_ERR_DTYPE;
  hipLaunchKernelGGL(prep, dim3((unsigned)(tl.rows + sblocks)), dim3(256), 0, st, x, M, K, gamma,
                     eps, norm, (void *)a.xn, (float *)a.omul, tl.rows, scales, sdt, N, ng,
                     (int64_t)a.ldst, scT, cmul);
  int s = launch_status();
  if (s != MTP_OK) return s;
  a.packed = packed;
  a.scales = scT;
  a.cmul = cmul;
  a.y = y;
  a.ydt = xdt;
  a.yvec = xdt != MTP_F32 && N % 4 == 0 && ((uintptr_t)y & 7u) == 0;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.group = (int)group;
  a.ng = (int)ng;
  a.glog = (group & (group - 1)) == 0 ? __builtin_ctzll((unsigned long long)group) : -1;
  a.nibble = nibble;
  a.gn = (int)gn;
  a.gm = (int)tl.gm;
  hipLaunchKernelGGL(gemm, dim3((unsigned)blocks), dim3((unsigned)(64 * nw)), 0, st, a);
  return launch_status();
}

}  // namespace

// ===========================================================================
extern "C" {

int mtp_abi_version(void) { return MTP_ABI_VERSION; }

const char *mtp_status_string(int status) {
  switch (status) {
    case MTP_OK: return "ok";
    case MTP_ERR_NULL: return "required pointer is NULL";
    case MTP_ERR_SHAPE: return "inconsistent or unsupported sizes";
    case MTP_ERR_DTYPE: return "unsupported dtype or dtype combination";
    case MTP_ERR_WORKSPACE: return "workspace missing or too small";
    case MTP_ERR_ALIGN: return "pointer alignment not supported";
    case MTP_ERR_LAUNCH: return "HIP launch failed";
    case MTP_ERR_ARG: return "invalid argument";
  }
  return "unknown status";
}

const char *mtp_last_hip_error(void) { return g_last_hip_error; }

int mtp_set_tuning(const char *name, int64_t value) {
  if (!name) return MTP_ERR_NULL;
  tune(kTuneSkl);  // the environment seeds the keys first
  for (int k = 0; k < kTuneCount; ++k) {
    if (std::strcmp(name, kTuneNames[k]) == 0) {
      if (value < -1 || value > INT32_MAX) return MTP_ERR_ARG;
      g_tune[k].store((int)value, std::memory_order_relaxed);
      return MTP_OK;
    }
  }
  return MTP_ERR_ARG;
}

int mtp_get_tuning(const char *name, int64_t *value) {
  if (!name || !value) return MTP_ERR_NULL;
  for (int k = 0; k < kTuneCount; ++k) {
    if (std::strcmp(name, kTuneNames[k]) == 0) {
      *value = tune((TuneKey)k);
      return MTP_OK;
    }
  }
  return MTP_ERR_ARG;
}

size_t mtp_rmsnorm_linear_workspace_bytes(int x_dtype, int w_kind, int64_t M, int64_t N,
                                          int64_t K) {
  // packed INT4: enough for every group the MFMA path takes (group >= 32)
  if (w_kind == MTP_U8) return int4_fast(M, N, K, 32) ? int4_ws_bytes(M, N, K, K / 32) : 0;
  // enough for the call with or without gamma
  size_t most = 0;
  for (int gam = 0; gam < 2; ++gam) {
    PlanX p = make_plan_x(x_dtype, w_kind, M, N, K, gam != 0);
    if (p.ok && p.total > most) most = p.total;
    PlanSk q = make_plan_sk(x_dtype, w_kind, M, N, K, gam != 0);
    if (q.ok && q.total > most) most = q.total;
    PlanSk qw = make_plan_sk(x_dtype, w_kind, M, N, K, gam != 0, true);
    if (qw.ok && qw.total > most) most = qw.total;
    PlanSkl l = make_plan_skl(x_dtype, w_kind, M, N, K, gam != 0);
    if (l.ok && l.total > most) most = l.total;
    PlanSkp q2 = make_plan_skp(x_dtype, w_kind, M, N, K, gam != 0);
    if (q2.ok && q2.total > most) most = q2.total;
  }
  return most;
}

int mtp_fused_rmsnorm_linear(const void *x, int x_dtype, int64_t M, int64_t K, const void *weight,
                             int w_dtype, int64_t N, const void *bias, int bias_dtype,
                             const void *gamma, int gamma_dtype, float eps, float scale, int norm,
                             void *y, void *workspace, size_t workspace_bytes, void *stream) {
  if (!is_float_dt(w_dtype)) return MTP_ERR_DTYPE;
  return rmsnorm_linear_impl(x, x_dtype, M, K, weight, w_dtype, N, nullptr, bias, bias_dtype,
                             gamma, gamma_dtype, eps, scale, norm, y, workspace, workspace_bytes,
                             stream);
}

int mtp_fused_rmsnorm_linear_fp8(const void *x, int x_dtype, int64_t M, int64_t K,
                                 const void *weight_fp8, int w_dtype, const float *wscale,
                                 int64_t N, const void *bias, int bias_dtype, const void *gamma,
                                 int gamma_dtype, float eps, int norm, void *y, void *workspace,
                                 size_t workspace_bytes, void *stream) {
  if (!wscale && N > 0 && M > 0) return MTP_ERR_NULL;
  return rmsnorm_linear_impl(x, x_dtype, M, K, weight_fp8, w_dtype, N, wscale, bias,
                             bias_dtype, gamma, gamma_dtype, eps, 1.0f, norm, y, workspace,
                             workspace_bytes, stream);
}

int mtp_fused_int4_matmul(const void *x, int x_dtype, int64_t M, int64_t K, const uint8_t *packed,
                          const void *scales, int scale_dtype, int64_t N, int64_t group,
                          int nibble, const void *gamma, int gamma_dtype, float eps, int norm,
                          void *y, void *workspace, size_t workspace_bytes, void *stream) {
  if (!is_float_dt(x_dtype)) return MTP_ERR_DTYPE;
  if (scale_dtype != MTP_F32 && scale_dtype != MTP_F16 && scale_dtype != MTP_BF16)
    return MTP_ERR_DTYPE;
  if (gamma && !is_float_dt(gamma_dtype)) return MTP_ERR_DTYPE;
  if (nibble != MTP_NIBBLE_OFFSET8 && nibble != MTP_NIBBLE_TWOS) return MTP_ERR_ARG;
  if (M < 0 || N < 0 || K < 0 || group <= 0 || (K & 1) || (group & 1) || M > INT32_MAX ||
      N > INT32_MAX || K > INT32_MAX || group > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (M == 0 || N == 0) return MTP_OK;
  if (!y || (K > 0 && (!x || !packed || !scales))) return MTP_ERR_NULL;
  if (int4_fast(M, N, K, group) && aligned16(packed) && aligned16(x) &&
      (!gamma || aligned16(gamma)))
    return launch_int4(x, x_dtype, M, K, packed, scales, scale_dtype, N, group, nibble, gamma,
                       gamma_dtype, eps, norm, y, workspace, workspace_bytes, (hipStream_t)stream);
  return launch_generic_linear(x, x_dtype, packed, MTP_U8, nullptr, scales, scale_dtype,
                               (int)group, nibble, gamma, gamma_dtype, nullptr, 0, y, M, N, K,
                               eps, 1.0f, norm, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
static int verify_rows_per_chunk(int64_t seq) { return (int)((64 / seq) * seq); }

// Persistent streaming verify (skv.hpp): hidden and W of one dtype (BF16,
// F16, F32), any bias; 128 bytes of a W row per stage, so K * element bytes
// a multiple of 512 (the stages of a tile are whole rounds of the 4-slot
// register ring: K % 256 for 16-bit, K % 128 for fp32); a 256-row tile of W
// within the reach of one buffer descriptor (W itself may be any size).
// MTP_VERIFY_WSTREAM selects the column-group kernel instead.
bool skv_usable(int ht, int64_t V, int64_t K) {
  if (ht != MTP_BF16 && ht != MTP_F16 && ht != MTP_F32) return false;
  const int64_t row = K * dtype_bytes(ht);
  if (K <= 0 || V <= 0 || row % 512 != 0) return false;
  if ((int64_t)kSkvBN * row >= ((int64_t)1 << 31)) return false;
  return tune(kTuneVerifyWstream) <= 0;
}

size_t mtp_verify_workspace_bytes(int h_dtype, int64_t rows, int64_t seq, int64_t V, int64_t K) {
  if (seq < 1 || seq > 64) return 0;
  Plan p = make_plan(h_dtype, h_dtype, rows, V, K, EPI_ARGMAX, verify_rows_per_chunk(seq));
  // the persistent and generic kernels need the counter prefix (keys and
  // ticket); the column-group kernel its per-tile maxima after it
  const size_t wsb = p.generic ? 0 : p.total;
  return std::max(wsb, kCounterBytes);
}

// One launch per chunk of rows_per_chunk rows (whole batch elements).
static int launch_skv(const void *hidden, int ht, int64_t rows, int64_t K, const void *w, int64_t V,
                      const void *bias, int bt, int rows_per_chunk, const WsArgs &o, void *ws,
                      size_t ws_bytes, hipStream_t st) {
  if (!aligned16(hidden) || !aligned16(w)) return MTP_ERR_ALIGN;
  if (!ws || ws_bytes < kCounterBytes) return MTP_ERR_WORKSPACE;
  unsigned char *w8 = (unsigned char *)ws;
  // columns per tile: from a 64-column tile per CU, the width that makes
  // whole rounds of one tile per CU (V 32000: 128 columns, 250 workgroups
  // instead of 125; V 151936: 200 columns, 760 tiles in three rounds
  // instead of 594 in two and a third); tuning key skv_tw sets it
  int tw = kSkvBN;
  if (tune(kTuneSkvTw) > 0) {
    tw = std::min(kSkvBN, tune(kTuneSkvTw) / 8 * 8);
    if (tw < 8) return MTP_ERR_ARG;
  } else if (V >= (int64_t)device_cus() * 64) {
    tw = round_width(V, 1, kSkvBN);
  }
  const int64_t ntiles = (V + tw - 1) / tw;
  if (ntiles > INT32_MAX) return MTP_ERR_SHAPE;
  const int grid = (int)std::min<int64_t>(ntiles, device_cus());
  for (int64_t m0 = 0; m0 < rows; m0 += rows_per_chunk) {
    const int Mloc = (int)std::min<int64_t>(rows_per_chunk, rows - m0);
    // fp32: 16-row tiles, and 8 rows after whole tiles on the 4 x 4 MFMA
    // (40 rows: 2 tiles + 8 instead of 3 tiles)
    const bool r8 = ht == MTP_F32 && Mloc > 16 && Mloc % 16 != 0 && Mloc % 16 <= 8 &&
                    tune(kTuneSkvR8) != 0;
    const int mt = ht == MTP_F32 ? (r8 ? Mloc / 16 : (Mloc + 15) / 16) : (Mloc <= 32 ? 1 : 2);
    SkvKernel k = skv_pick(ht, mt, r8);
    if (!k) return MTP_ERR_DTYPE;
    SkvArgs a{};
    a.x = (const unsigned char *)hidden + m0 * K * dtype_bytes(ht);
    a.w = w;
    a.bias = bias;
    a.bias_dt = bt;
    a.M = Mloc;
    a.N = (int)V;
    a.K = (int)K;
    a.ntiles = (int)ntiles;
    a.tw = tw;
    a.nst = (int)(K * dtype_bytes(ht) / kSkUB);  // 128-byte stages of a W row
    a.keys = (unsigned long long *)(w8 + kSkvKeysOff);
    a.ticket = (unsigned *)w8;
    a.multi = o.multi;
    a.textbook = o.textbook;
    if (!o.multi) {
      a.draft = o.draft + m0;
      a.accept = o.accept + m0;
    } else {
      const int64_t b0 = m0 / o.S_seq;
      a.S_seq = o.S_seq;
      a.D = o.D;
      a.draft = o.draft ? o.draft + b0 * o.D : nullptr;
      a.accept = o.accept ? o.accept + b0 * o.D : nullptr;
      a.accepted_n = o.accepted_n + b0;
      a.corrected = o.corrected + b0;
    }
    a.top = o.top ? o.top + m0 : nullptr;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(512), 0, st, a);
    const int s = launch_status();
    if (s != MTP_OK) return s;
  }
  return MTP_OK;
}

// Generic verify (vgen.hpp): any K, alignment and float dtypes; one launch
// per chunk of rows_per_chunk rows (whole batch elements).
constexpr int kVgenMaxBlocks = 1024;
static int launch_vgen(const void *hidden, int ht, int64_t rows, int64_t K, const void *w, int wt,
                       int64_t V, const void *bias, int bt, int rows_per_chunk, const WsArgs &o,
                       void *ws, size_t ws_bytes, hipStream_t st) {
  if (!ws || ws_bytes < kCounterBytes) return MTP_ERR_WORKSPACE;
  unsigned char *w8 = (unsigned char *)ws;
  const int grid = (int)std::min<int64_t>((V + kVgenThreads - 1) / kVgenThreads, kVgenMaxBlocks);
  for (int64_t m0 = 0; m0 < rows; m0 += rows_per_chunk) {
    const int Mloc = (int)std::min<int64_t>(rows_per_chunk, rows - m0);
    VgenKernel k = vgen_pick(Mloc);
    if (!k) return MTP_ERR_SHAPE;
    VgenArgs a{};
    a.x = (const unsigned char *)hidden + m0 * K * dtype_bytes(ht);
    a.xdt = ht;
    a.w = w;
    a.wdt = wt;
    a.bias = bias;
    a.bdt = bt;
    a.M = Mloc;
    a.N = (int)V;
    a.K = (int)K;
    a.keys = (unsigned long long *)(w8 + kSkvKeysOff);
    a.ticket = (unsigned *)w8;
    a.out.multi = o.multi;
    a.out.textbook = o.textbook;
    if (!o.multi) {
      a.out.draft = o.draft + m0;
      a.out.accept = o.accept + m0;
    } else {
      const int64_t b0 = m0 / o.S_seq;
      a.out.S_seq = o.S_seq;
      a.out.D = o.D;
      a.out.draft = o.draft ? o.draft + b0 * o.D : nullptr;
      a.out.accept = o.accept ? o.accept + b0 * o.D : nullptr;
      a.out.accepted_n = o.accepted_n + b0;
      a.out.corrected = o.corrected + b0;
    }
    a.out.top = o.top ? o.top + m0 : nullptr;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(kVgenThreads), 0, st, a);
    const int s = launch_status();
    if (s != MTP_OK) return s;
  }
  return MTP_OK;
}

// Route: the persistent streaming kernel (one dtype for hidden and W:
// BF16, F16 or F32; any bias; 128-byte stages of whole ring rounds; 16-byte
// aligned), else the column-group streaming kernel (same dtype for hidden
// and W, 16-byte rows and pointers), else the generic kernel.
static int verify_route(const void *hidden, int ht, int64_t rows, int64_t K, const void *w,
                        int wt, int64_t V, const void *bias, int rows_per_chunk, Plan *plan) {
  const bool aligned = aligned16(hidden) && aligned16(w);
  if (wt == ht && aligned && skv_usable(ht, V, K)) return MTP_VERIFY_ROUTE_STREAM;
  *plan = make_plan(ht, wt, rows, V, K, EPI_ARGMAX, rows_per_chunk);
  if (plan->generic || !aligned || wt != ht || (bias && !aligned16(bias)))
    return MTP_VERIFY_ROUTE_GENERIC;
  return MTP_VERIFY_ROUTE_COLUMN_GROUP;
}

static int verify_common(const void *hidden, int ht, int64_t rows, int64_t K, const void *w,
                         int wt, int64_t V, const void *bias, int bt, int rows_per_chunk,
                         WsArgs &a, void *ws, size_t ws_bytes, void *stream) {
  Plan p{};
  const int route = verify_route(hidden, ht, rows, K, w, wt, V, bias, rows_per_chunk, &p);
  if (route == MTP_VERIFY_ROUTE_STREAM)
    return launch_skv(hidden, ht, rows, K, w, V, bias, bt, rows_per_chunk, a, ws, ws_bytes,
                      (hipStream_t)stream);
  if (route == MTP_VERIFY_ROUTE_GENERIC)
    return launch_vgen(hidden, ht, rows, K, w, wt, V, bias, bt, rows_per_chunk, a, ws, ws_bytes,
                       (hipStream_t)stream);
  if (!ws || ws_bytes < p.total) return MTP_ERR_WORKSPACE;
  a.x = hidden;
  a.w = w;
  a.bias = bias;
  a.bias_dt = bt;
  a.M = (int)rows;
  a.N = (int)V;
  a.K = (int)K;
  a.scale = 1.0f;
  return launch_ws(p, a, EPI_ARGMAX, ws, (hipStream_t)stream);
}

int mtp_verify_route(const void *hidden, int h_dtype, int64_t rows, int64_t seq, int64_t K,
                     const void *weight, int w_dtype, int64_t V, const void *bias) {
  if (!is_float_dt(h_dtype) || !is_float_dt(w_dtype)) return MTP_ERR_DTYPE;
  if (rows < 1 || seq < 1 || seq > 64 || K <= 0 || V <= 0 || rows > INT32_MAX ||
      K > INT32_MAX || V > INT32_MAX)
    return MTP_ERR_SHAPE;
  Plan p{};
  return verify_route(hidden, h_dtype, rows, K, weight, w_dtype, V, bias,
                      seq == 1 ? 64 : verify_rows_per_chunk(seq), &p);
}

int mtp_fused_verify(const void *hidden, int h_dtype, int64_t M, int64_t K, const void *weight,
                     int w_dtype, int64_t V, const void *bias, int bias_dtype,
                     const int32_t *draft, int8_t *accept, int32_t *top, void *workspace,
                     size_t workspace_bytes, void *stream) {
  if (!is_float_dt(h_dtype) || !is_float_dt(w_dtype)) return MTP_ERR_DTYPE;
  if (bias && !is_float_dt(bias_dtype)) return MTP_ERR_DTYPE;
  if (M < 0 || K <= 0 || V <= 0 || M > INT32_MAX || K > INT32_MAX || V > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (M == 0) return MTP_OK;
  if (!hidden || !weight || !draft || !accept || !top) return MTP_ERR_NULL;
  WsArgs a{};
  a.draft = draft;
  a.accept = accept;
  a.top = top;
  a.multi = 0;
  return verify_common(hidden, h_dtype, M, K, weight, w_dtype, V, bias, bias_dtype, 64, a,
                       workspace, workspace_bytes, stream);
}

static int multi_verify_common(const void *hidden, int h_dtype, int64_t B, int64_t S, int64_t K,
                               const void *weight, int w_dtype, int64_t V, const void *bias,
                               int bias_dtype, const int32_t *draft, int64_t D, int8_t *accept,
                               int32_t *accepted_n, int32_t *corrected, int32_t *top_out,
                               void *workspace, size_t workspace_bytes, void *stream,
                               int textbook) {
  if (!is_float_dt(h_dtype) || !is_float_dt(w_dtype)) return MTP_ERR_DTYPE;
  if (bias && !is_float_dt(bias_dtype)) return MTP_ERR_DTYPE;
  if (B < 0 || S < 1 || D < 0 || S != D + 1 || K <= 0 || V <= 0 || S > 64 ||
      B * S > INT32_MAX || K > INT32_MAX || V > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (B == 0) return MTP_OK;
  if (!hidden || !weight || !accepted_n || !corrected || (D > 0 && (!draft || !accept)))
    return MTP_ERR_NULL;
  WsArgs a{};
  a.draft = draft;
  a.accept = accept;
  a.accepted_n = accepted_n;
  a.corrected = corrected;
  a.top = top_out;
  a.multi = 1;
  a.textbook = textbook;
  a.S_seq = (int)S;
  a.D = (int)D;
  const int rpc = verify_rows_per_chunk(S);
  return verify_common(hidden, h_dtype, B * S, K, weight, w_dtype, V, bias, bias_dtype, rpc, a,
                       workspace, workspace_bytes, stream);
}

int mtp_fused_multi_verify(const void *hidden, int h_dtype, int64_t B, int64_t S, int64_t K,
                           const void *weight, int w_dtype, int64_t V, const void *bias,
                           int bias_dtype, const int32_t *draft, int64_t D, int8_t *accept,
                           int32_t *accepted_n, int32_t *corrected, int32_t *top_out,
                           void *workspace, size_t workspace_bytes, void *stream) {
  return multi_verify_common(hidden, h_dtype, B, S, K, weight, w_dtype, V, bias, bias_dtype,
                             draft, D, accept, accepted_n, corrected, top_out, workspace,
                             workspace_bytes, stream, 0);
}

int mtp_fused_multi_verify_textbook(const void *hidden, int h_dtype, int64_t B, int64_t S,
                                    int64_t K, const void *weight, int w_dtype, int64_t V,
                                    const void *bias, int bias_dtype, const int32_t *draft,
                                    int64_t D, int8_t *accept, int32_t *accepted_n,
                                    int32_t *corrected, int32_t *top_out, void *workspace,
                                    size_t workspace_bytes, void *stream) {
  return multi_verify_common(hidden, h_dtype, B, S, K, weight, w_dtype, V, bias, bias_dtype,
                             draft, D, accept, accepted_n, corrected, top_out, workspace,
                             workspace_bytes, stream, 1);
}


size_t mtp_attention_workspace_bytes(int dtype, int64_t B, int64_t NQ, int64_t H, int64_t D,
                                     int64_t Lc, int64_t Lt) {
  if (B <= 0 || NQ <= 0 || H <= 0 || D <= 0 || Lc < 0 || Lt < 0) return 0;
  return make_attn_plan(dtype, B, NQ, H, D, Lc, Lt).total;
}

int mtp_fused_paged_attention(const void *q, int dtype, int64_t B, int64_t H, int64_t D,
                              const void *k_pages, const void *v_pages, int64_t num_pages,
                              const int32_t *page_table, int64_t L, int64_t page_size,
                              float scale, void *out, void *workspace, size_t workspace_bytes,
                              void *stream) {
  if (!is_float_dt(dtype)) return MTP_ERR_DTYPE;
  if (B < 0 || H < 0 || D <= 0 || L < 0 || page_size <= 0 || num_pages < 0 || L > INT32_MAX ||
      num_pages > INT32_MAX || page_size > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (B == 0 || H == 0) return MTP_OK;
  if (!q || !out || (L > 0 && (!k_pages || !v_pages || !page_table))) return MTP_ERR_NULL;
  if (L > 0 && num_pages == 0) return MTP_ERR_SHAPE;
  AttnArgs a{};
  a.q = q;
  a.q_sb = H * D;
  a.q_sn = 0;
  a.q_sh = D;
  a.kp = k_pages;
  a.vp = v_pages;
  a.table = page_table;
  a.ld_tab = L;
  a.Lc = (int)L;
  a.page_size = (int)page_size;
  a.npages = (int)num_pages;
  a.p_sh = page_size * D;
  a.p_sb = H * a.p_sh;
  a.p_sp = B * a.p_sb;
  a.out = out;
  a.o_sb = H * D;
  a.o_sn = 0;
  a.o_sh = D;
  a.B = (int)B;
  a.NQ = 1;
  a.H = (int)H;
  a.scale = scale;
  return launch_attention(a, dtype, D, workspace, workspace_bytes, (hipStream_t)stream);
}

// Single-query attention over dense keys k / v [B, H, L, D] (element type
// dtype, or fp8 with per-head scales), optional 1-D mask [L].
static int dense_attention(const void *q, int dtype, int64_t B, int64_t H, int64_t D,
                           const void *k, const void *v, int64_t L, const void *mask,
                           int mask_dtype, int kv_fp8, const float *kscale, const float *vscale,
                           float scale, void *out, void *workspace, size_t workspace_bytes,
                           void *stream) {
  if (!is_float_dt(dtype)) return MTP_ERR_DTYPE;
  if (mask && !mask_dt_ok(mask_dtype)) return MTP_ERR_DTYPE;
  if (B < 0 || H < 0 || D <= 0 || L < 0 || L > INT32_MAX) return MTP_ERR_SHAPE;
  if (B == 0 || H == 0) return MTP_OK;
  if (!q || !out || (L > 0 && (!k || !v))) return MTP_ERR_NULL;
  AttnArgs a{};
  a.q = q;
  a.q_sb = H * D;
  a.q_sh = D;
  a.kd = k;
  a.vd = v;
  a.Lt = (int)L;
  a.d_st = D;
  a.d_sh = L * D;
  a.d_sb = H * a.d_sh;
  a.mask = mask;
  a.mask_dt = mask_dtype;
  a.mask_2d = 0;
  a.out = out;
  a.o_sb = H * D;
  a.o_sh = D;
  a.B = (int)B;
  a.NQ = 1;
  a.H = (int)H;
  a.scale = scale;
  a.kv_fp8 = kv_fp8;
  a.kscale = kscale;
  a.vscale = vscale;
  return launch_attention(a, dtype, D, workspace, workspace_bytes, (hipStream_t)stream);
}

int mtp_fused_tree_attention(const void *q, int dtype, int64_t B, int64_t H, int64_t D,
                             const void *k, const void *v, int64_t L, const void *mask,
                             int mask_dtype, float scale, void *out, void *workspace,
                             size_t workspace_bytes, void *stream) {
  if (L > 0 && B > 0 && H > 0 && !mask) return MTP_ERR_NULL;
  return dense_attention(q, dtype, B, H, D, k, v, L, mask, mask_dtype, 0, nullptr, nullptr, scale,
                         out, workspace, workspace_bytes, stream);
}

int mtp_fused_causal_attention(const void *q, int dtype, int64_t B, int64_t H, int64_t D,
                               const void *k, const void *v, int64_t L, float scale, void *out,
                               void *workspace, size_t workspace_bytes, void *stream) {
  return dense_attention(q, dtype, B, H, D, k, v, L, nullptr, 0, 0, nullptr, nullptr, scale, out,
                         workspace, workspace_bytes, stream);
}

int mtp_fused_causal_attention_fp8(const void *q, int dtype, int64_t B, int64_t H, int64_t D,
                                   const void *k_fp8, const void *v_fp8, int64_t L,
                                   const float *kscale, const float *vscale, float scale,
                                   void *out, void *stream) {
  if (B > 0 && H > 0 && (!kscale || !vscale)) return MTP_ERR_NULL;
  // the fp8 fallback kernel needs no workspace
  return dense_attention(q, dtype, B, H, D, k_fp8, v_fp8, L, nullptr, 0, 1, kscale, vscale, scale,
                         out, nullptr, 0, stream);
}

// Tree monolith: attention over the masked keys into an intermediate
// [B * H, D] (q's dtype) at the end of the workspace, then RMSNorm over the
// head dimension (gamma rms_w) and the projection onto proj_w's rows.
static size_t monolith_tmp_off(int dtype, int64_t B, int64_t H, int64_t D, int64_t L, int w_kind,
                               int64_t N) {
  const size_t att = make_attn_plan(dtype, B, 1, H, D, 0, L).total;
  const size_t lin = mtp_rmsnorm_linear_workspace_bytes(dtype, w_kind, B * H, N, D);
  return align_up(std::max(kCounterBytes, std::max(att, lin)), 256);
}

size_t mtp_tree_attn_rmsnorm_linear_workspace_bytes(int dtype, int64_t B, int64_t H, int64_t D,
                                                    int64_t L, int w_kind, int64_t N) {
  if (B <= 0 || H <= 0 || D <= 0 || L < 0 || N <= 0) return 0;
  return monolith_tmp_off(dtype, B, H, D, L, w_kind, N) +
         align_up((size_t)(B * H * D) * dtype_bytes(dtype), 256);
}

int mtp_fused_tree_attn_rmsnorm_linear(const void *q, int dtype, int64_t B, int64_t H, int64_t D,
                                       const void *k, const void *v, int64_t L, const void *mask,
                                       int mask_dtype, const void *proj_w, int w_dtype, int64_t N,
                                       const void *rms_w, int rms_dtype, const void *proj_bias,
                                       int bias_dtype, const float *wscale, float scale, float eps,
                                       void *out, void *workspace, size_t workspace_bytes,
                                       void *stream) {
  if (!is_float_dt(dtype) || !mask_dt_ok(mask_dtype)) return MTP_ERR_DTYPE;
  if (!(is_float_dt(w_dtype) || w_dtype == MTP_FP8E4M3)) return MTP_ERR_DTYPE;
  if (w_dtype == MTP_FP8E4M3 && !wscale) return MTP_ERR_NULL;
  if (B < 0 || H < 0 || D <= 0 || L < 0 || N < 0 || L > INT32_MAX || N > INT32_MAX ||
      B * H > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (B == 0 || H == 0 || N == 0) return MTP_OK;
  if (!q || !out || !proj_w || (L > 0 && (!k || !v || !mask))) return MTP_ERR_NULL;
  const size_t need = mtp_tree_attn_rmsnorm_linear_workspace_bytes(dtype, B, H, D, L,
                                                                   wscale ? MTP_FP8E4M3 : w_dtype, N);
  if (!workspace || workspace_bytes < need) return MTP_ERR_WORKSPACE;
  const size_t off = monolith_tmp_off(dtype, B, H, D, L, wscale ? MTP_FP8E4M3 : w_dtype, N);
  void *tmp = (unsigned char *)workspace + off;
  int s = dense_attention(q, dtype, B, H, D, k, v, L, mask, mask_dtype, 0, nullptr, nullptr, scale,
                          tmp, workspace, off, stream);
  if (s != MTP_OK) return s;
  return rmsnorm_linear_impl(tmp, dtype, B * H, D, proj_w, w_dtype, N, wscale, proj_bias,
                             bias_dtype, rms_w, rms_dtype, eps, 1.0f, 1, out, workspace, off,
                             stream);
}

int mtp_tree_verify_attention(const void *q_nodes, int dtype, int64_t N, int64_t H, int64_t D,
                              const void *k_pages, const void *v_pages, int64_t num_pages,
                              const int32_t *page_table, int64_t Lc, int64_t page_size,
                              const void *k_tree, const void *v_tree, const void *tree_mask,
                              int mask_dtype, float scale, void *out, void *workspace,
                              size_t workspace_bytes, void *stream) {
  if (!is_float_dt(dtype) || !mask_dt_ok(mask_dtype)) return MTP_ERR_DTYPE;
  if (N < 0 || H < 0 || D <= 0 || Lc < 0 || page_size <= 0 || num_pages < 0 ||
      N > INT32_MAX || Lc > INT32_MAX || num_pages > INT32_MAX || page_size > INT32_MAX)
    return MTP_ERR_SHAPE;
  if (N == 0 || H == 0) return MTP_OK;
  if (!q_nodes || !out || !k_tree || !v_tree || !tree_mask ||
      (Lc > 0 && (!k_pages || !v_pages || !page_table)))
    return MTP_ERR_NULL;
  if (Lc > 0 && num_pages == 0) return MTP_ERR_SHAPE;
  AttnArgs a{};
  a.q = q_nodes;
  a.q_sn = H * D;
  a.q_sh = D;
  a.kp = k_pages;
  a.vp = v_pages;
  a.table = page_table;
  a.ld_tab = Lc;
  a.Lc = (int)Lc;
  a.page_size = (int)page_size;
  a.npages = (int)num_pages;
  a.p_sh = page_size * D;
  a.p_sb = H * a.p_sh;
  a.p_sp = a.p_sb;  // one batch row of pages
  a.kd = k_tree;
  a.vd = v_tree;
  a.Lt = (int)N;
  a.d_sh = D;
  a.d_st = H * D;
  a.mask = tree_mask;
  a.mask_dt = mask_dtype;
  a.mask_2d = 1;
  a.out = out;
  a.o_sn = H * D;
  a.o_sh = D;
  a.B = 1;
  a.NQ = (int)N;
  a.H = (int)H;
  a.scale = scale;
  return launch_attention(a, dtype, D, workspace, workspace_bytes, (hipStream_t)stream);
}


// ---------------------------------------------------------------------------
// Quantizers
size_t mtp_quantize_workspace_bytes(int64_t n) {
  (void)n;
  return kCounterBytes + 1024 * sizeof(float);
}

int mtp_quantize_fp8_e4m3(const void *x, int x_dtype, int64_t n, uint8_t *x_fp8, float *scale,
                          void *workspace, size_t workspace_bytes, void *stream) {
  if (!is_float_dt(x_dtype)) return MTP_ERR_DTYPE;
  if (n <= 0) return MTP_ERR_SHAPE;  // torch's max of an empty tensor raises
  if (!x || !x_fp8 || !scale) return MTP_ERR_NULL;
  if (!workspace || workspace_bytes < mtp_quantize_workspace_bytes(n)) return MTP_ERR_WORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  unsigned char *w8 = (unsigned char *)workspace;
  const unsigned blocks = (unsigned)std::min<int64_t>(1024, (n + 255) / 256);
  hipLaunchKernelGGL(fp8_tensor_scale_kernel, dim3(blocks), dim3(256), 0, st, x, x_dtype, n,
                     (float *)(w8 + kCounterBytes), (unsigned *)w8, scale);
  int rc = launch_status();
  if (rc != MTP_OK) return rc;
  const unsigned qb = (unsigned)std::min<int64_t>(8192, ((n + 1) / 2 + 255) / 256);
  hipLaunchKernelGGL(fp8_quantize_kernel, dim3(qb), dim3(256), 0, st, x, x_dtype, n, n, scale, 0,
                     x_fp8);
  return launch_status();
}

int mtp_quantize_fp8_rows(const void *w, int w_dtype, int64_t N, int64_t K, uint8_t *w_fp8,
                          float *wscale, void *stream) {
  if (!is_float_dt(w_dtype)) return MTP_ERR_DTYPE;
  if (N < 0 || K <= 0 || N > INT32_MAX) return MTP_ERR_SHAPE;
  if (N == 0) return MTP_OK;
  if (!w || !w_fp8 || !wscale) return MTP_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  // one pass per row from registers: rows of 8 c elements, c <= 2048 chunks
  // (K <= 16384), 16-byte aligned input and 8-byte aligned output rows
  const int64_t kc = K / 8;
  if (K % 8 == 0 && kc <= 2048 && aligned16(w) && ((uintptr_t)w_fp8 & 7u) == 0) {
    const int nv = kc <= 256 ? 1 : kc <= 512 ? 2 : kc <= 1024 ? 4 : 8;
    using Fn = void (*)(const void *, int64_t, uint8_t *, float *);
    static const Fn table[3][4] = {
        {fp8_rows_vec_kernel<MTP_F32, 1>, fp8_rows_vec_kernel<MTP_F32, 2>,
         fp8_rows_vec_kernel<MTP_F32, 4>, fp8_rows_vec_kernel<MTP_F32, 8>},
        {fp8_rows_vec_kernel<MTP_BF16, 1>, fp8_rows_vec_kernel<MTP_BF16, 2>,
         fp8_rows_vec_kernel<MTP_BF16, 4>, fp8_rows_vec_kernel<MTP_BF16, 8>},
        {fp8_rows_vec_kernel<MTP_F16, 1>, fp8_rows_vec_kernel<MTP_F16, 2>,
         fp8_rows_vec_kernel<MTP_F16, 4>, fp8_rows_vec_kernel<MTP_F16, 8>}};
    const int di = w_dtype == MTP_F32 ? 0 : w_dtype == MTP_BF16 ? 1 : 2;
    const int vi = nv == 1 ? 0 : nv == 2 ? 1 : nv == 4 ? 2 : 3;
    hipLaunchKernelGGL(table[di][vi], dim3((unsigned)N), dim3(256), 0, st, w, K, w_fp8, wscale);
    return launch_status();
  }
  hipLaunchKernelGGL(fp8_row_scale_kernel, dim3((unsigned)N), dim3(256), 0, st, w, w_dtype, K,
                     wscale);
  int rc = launch_status();
  if (rc != MTP_OK) return rc;
  const int64_t n = N * K;
  const unsigned qb = (unsigned)std::min<int64_t>(8192, ((n + 1) / 2 + 255) / 256);
  hipLaunchKernelGGL(fp8_quantize_kernel, dim3(qb), dim3(256), 0, st, w, w_dtype, n, K, wscale, 1,
                     w_fp8);
  return launch_status();
}

int mtp_dequantize_fp8(const uint8_t *x_fp8, int64_t n, int64_t row_len, const float *scale,
                       int per_row, float *out, void *stream) {
  if (n < 0 || (per_row && row_len <= 0)) return MTP_ERR_SHAPE;
  if (n == 0) return MTP_OK;
  if (!x_fp8 || !scale || !out) return MTP_ERR_NULL;
  const unsigned blocks = (unsigned)std::min<int64_t>(8192, (n + 255) / 256);
  hipLaunchKernelGGL(fp8_dequantize_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     x_fp8, n, per_row ? row_len : 1, scale, per_row ? 1 : 0, out);
  return launch_status();
}

int mtp_quantize_int4(const void *w, int w_dtype, int64_t N, int64_t K, int64_t group,
                      uint8_t *packed, float *scales, void *stream) {
  if (!is_float_dt(w_dtype)) return MTP_ERR_DTYPE;
  if (N < 0 || K <= 0 || (K & 1) || group <= 0 || (group & 1)) return MTP_ERR_SHAPE;
  if (N == 0) return MTP_OK;
  if (!w || !packed || !scales) return MTP_ERR_NULL;
  // vector form: groups of 8 L elements, L a power of two <= 64, whole
  // groups per row, 16-byte aligned rows
  const int64_t L = group / 8;
  if (group % 8 == 0 && L <= 64 && (L & (L - 1)) == 0 && K % group == 0 && aligned16(w) &&
      ((uintptr_t)packed & 3u) == 0 && N * K / 8 / 256 + 1 < INT32_MAX) {
    constexpr int U = 1;  // 2 and 4 chunks per thread measured no faster
    void (*k)(const void *, int64_t, int64_t, int, uint8_t *, float *) =
        w_dtype == MTP_F32    ? int4_quantize_vec_kernel<MTP_F32, U>
        : w_dtype == MTP_BF16 ? int4_quantize_vec_kernel<MTP_BF16, U>
                              : int4_quantize_vec_kernel<MTP_F16, U>;
    hipLaunchKernelGGL(k, dim3((unsigned)((N * K / 8 + 256 * U - 1) / (256 * U))), dim3(256), 0,
                       (hipStream_t)stream, w, N, K, (int)L, packed, scales);
    return launch_status();
  }
  const int64_t items = N * ((K + group - 1) / group);
  hipLaunchKernelGGL(int4_quantize_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, w, w_dtype, N, K, group, packed, scales);
  return launch_status();
}

int mtp_dequantize_int4(const uint8_t *packed, const void *scales, int scale_dtype, int64_t N,
                        int64_t K, int64_t group, float *out, void *stream) {
  if (!is_float_dt(scale_dtype)) return MTP_ERR_DTYPE;
  if (N < 0 || K <= 0 || (K & 1) || group <= 0) return MTP_ERR_SHAPE;
  if (N == 0) return MTP_OK;
  if (!packed || !scales || !out) return MTP_ERR_NULL;
  const unsigned blocks = (unsigned)std::min<int64_t>(8192, (N * K + 255) / 256);
  hipLaunchKernelGGL(int4_dequantize_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     packed, scales, scale_dtype, N, K, group, out);
  return launch_status();
}

}  // extern "C"
