// C ABI of the draft chain (RMSNorm, add + RMSNorm, greedy token + embedding
// row) and of the KV step after verify (paged-KV write, device-side
// rollback / commit, batch prefix match), plus the workspace initialiser.
// Declarations and the reference interfaces they replace are in
// include/mtp_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "abi_util.hpp"
#include "draft.hpp"
#include "kvstep.hpp"

using namespace mtp;

namespace {

// Zero fill with a kernel (a memset node in a captured graph is avoided).
__global__ void __launch_bounds__(256) zero_fill_kernel(uint32_t *p, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256)
    p[i] = 0u;
}

// Workgroups per launch the segments aim at: with the vector form a segment
// of a few thousand columns is one load round trip, and the per-row hand-off
// (publish, ticket, key reads, embedding copy) is what costs, so fewer and
// longer segments win (draft step of 8 rows x 128256 columns: 172.5 us per
// step against 175.3 with 512 and 174 with 64; 229 with one per row).
constexpr int kArgmaxTargetBlocks = 128;
constexpr int64_t kArgmaxMinSeg = 2048;   // vocabulary entries per workgroup at least

struct ArgmaxPlan {
  int S = 1;
  int64_t seg = 0;
  size_t total = 0;
};

ArgmaxPlan argmax_plan(int64_t M, int64_t V) {
  ArgmaxPlan p;
  if (M <= 0 || V <= 0) return p;
  int64_t S = (kArgmaxTargetBlocks + M - 1) / M;
  S = std::min<int64_t>(S, (V + kArgmaxMinSeg - 1) / kArgmaxMinSeg);
  if (M > kCounterSlots) S = 1;  // one ticket per row in the counter prefix
  S = std::max<int64_t>(S, 1);
  // whole 16-byte chunks per segment for the vector form (8 elements)
  p.seg = ((V + S - 1) / S + 7) / 8 * 8;
  p.S = (int)((V + p.seg - 1) / p.seg);
  p.total = p.S > 1 ? kCounterBytes + align_up((size_t)M * p.S * 8, 256) : 0;
  return p;
}

typedef void (*RmsVecKernel)(const void *, const void *, const void *, void *, int, float);

template <int DT, bool W, bool ADD>
RmsVecKernel rms_vec_nv(int nv) {
  switch (nv) {
    case 1: return rmsnorm_vec_kernel<DT, W, ADD, 1>;
    case 2: return rmsnorm_vec_kernel<DT, W, ADD, 2>;
    case 4: return rmsnorm_vec_kernel<DT, W, ADD, 4>;
    case 8: return rmsnorm_vec_kernel<DT, W, ADD, 8>;
  }
  return nullptr;
}
template <int DT>
RmsVecKernel rms_vec_dt(bool w, bool add, int nv) {
  if (w) return add ? rms_vec_nv<DT, true, true>(nv) : rms_vec_nv<DT, true, false>(nv);
  return add ? rms_vec_nv<DT, false, true>(nv) : rms_vec_nv<DT, false, false>(nv);
}
// The 16-byte form of a norm launch, or null: rows of whole 16-byte chunks
// (at most 2048 of them), 16-byte aligned x / r / y / weight, the weight
// (if any) of the rows' dtype.
RmsVecKernel rms_vec_pick(const void *x, const void *r, int dt, int64_t N, const void *w, int wdt,
                          const void *y) {
  const int64_t e = dt == MTP_F32 ? 4 : 8;
  if (N % e != 0 || N / e > 2048) return nullptr;
  if (!aligned16(x) || !aligned16(y) || (r && !aligned16(r)) || (w && !aligned16(w))) return nullptr;
  if (w && wdt != dt) return nullptr;
  const int64_t nch = N / e;
  const int nv = nch <= 256 ? 1 : nch <= 512 ? 2 : nch <= 1024 ? 4 : 8;
  switch (dt) {
    case MTP_F32: return rms_vec_dt<MTP_F32>(w != nullptr, r != nullptr, nv);
    case MTP_BF16: return rms_vec_dt<MTP_BF16>(w != nullptr, r != nullptr, nv);
    case MTP_F16: return rms_vec_dt<MTP_F16>(w != nullptr, r != nullptr, nv);
  }
  return nullptr;
}

int rmsnorm_common(const void *x, const void *r, int dt, int64_t M, int64_t N, const void *w,
                   int wdt, float eps, void *y, void *stream) {
  if (!is_float_dt(dt) || (w && !is_float_dt(wdt))) return MTP_ERR_DTYPE;
  if (M < 0 || N < 0 || N > INT32_MAX || M > INT32_MAX) return MTP_ERR_SHAPE;
  if (M == 0 || N == 0) return MTP_OK;
  if (!x || !y) return MTP_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  // 16-byte form: one round trip per row, the row held in registers
  // (RMSNorm of 8 x 4096 bf16: 8.5 -> 4.6 us under rocprofv3)
  if (RmsVecKernel kv = rms_vec_pick(x, r, dt, N, w, wdt, y)) {
    for (int64_t m0 = 0; m0 < M; m0 += 65535 * 16) {
      const int64_t rows = std::min<int64_t>(M - m0, 65535 * 16);
      const size_t off = (size_t)m0 * N * dtype_bytes(dt);
      hipLaunchKernelGGL(kv, dim3((unsigned)rows), dim3(256), 0, st,
                         (const void *)((const unsigned char *)x + off),
                         r ? (const void *)((const unsigned char *)r + off) : nullptr, w,
                         (void *)((unsigned char *)y + off), (int)N, eps);
      const int s = launch_status();
      if (s != MTP_OK) return s;
    }
    return MTP_OK;
  }
  for (int64_t m0 = 0; m0 < M; m0 += 65535 * 16) {
    const int64_t rows = std::min<int64_t>(M - m0, 65535 * 16);
    const size_t off = (size_t)m0 * N * dtype_bytes(dt);
    const void *xs = (const unsigned char *)x + off;
    void *ys = (unsigned char *)y + off;
    if (r) {
      hipLaunchKernelGGL(rmsnorm_rows_kernel<true>, dim3((unsigned)rows), dim3(256), 0, st, xs,
                         (const void *)((const unsigned char *)r + off), dt, w, wdt, ys, (int)N,
                         eps);
    } else {
      hipLaunchKernelGGL(rmsnorm_rows_kernel<false>, dim3((unsigned)rows), dim3(256), 0, st, xs,
                         (const void *)nullptr, dt, w, wdt, ys, (int)N, eps);
    }
    const int s = launch_status();
    if (s != MTP_OK) return s;
  }
  return MTP_OK;
}

}  // namespace

extern "C" {

int mtp_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
  if (workspace_bytes == 0) return MTP_OK;
  if (!workspace) return MTP_ERR_NULL;
  if (!aligned16(workspace) || workspace_bytes % 4 != 0) return MTP_ERR_ALIGN;
  const int64_t n4 = (int64_t)(workspace_bytes / 4);
  const unsigned blocks = (unsigned)std::min<int64_t>((n4 + 255) / 256, 4096);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     (uint32_t *)workspace, n4);
  return launch_status();
}

int mtp_fused_rmsnorm(const void *x, int dtype, int64_t M, int64_t N, const void *weight,
                      int w_dtype, float eps, void *y, void *stream) {
  return rmsnorm_common(x, nullptr, dtype, M, N, weight, w_dtype, eps, y, stream);
}

int mtp_fused_add_rmsnorm(const void *x, const void *residual, int dtype, int64_t M, int64_t N,
                          const void *weight, int w_dtype, float eps, void *y, void *stream) {
  if (M > 0 && N > 0 && !residual) return MTP_ERR_NULL;
  return rmsnorm_common(x, residual, dtype, M, N, weight, w_dtype, eps, y, stream);
}

size_t mtp_argmax_workspace_bytes(int64_t M, int64_t V) { return argmax_plan(M, V).total; }

int mtp_argmax(const void *logits, int dtype, int64_t M, int64_t V, int64_t ld, int64_t *tokens,
               const void *emb_table, int table_dtype, int64_t table_rows, int64_t H,
               void *emb_out, void *workspace, size_t workspace_bytes, void *stream) {
  if (!is_float_dt(dtype)) return MTP_ERR_DTYPE;
  if (emb_table && !is_float_dt(table_dtype)) return MTP_ERR_DTYPE;
  if (M < 0 || V <= 0 || ld < V || V > INT32_MAX || M > INT32_MAX) return MTP_ERR_SHAPE;
  if (emb_table && (H <= 0 || table_rows < V || H > INT32_MAX)) return MTP_ERR_SHAPE;
  if (M == 0) return MTP_OK;
  if (!logits || !tokens || (emb_table && !emb_out)) return MTP_ERR_NULL;
  const ArgmaxPlan p = argmax_plan(M, V);
  if (p.total > 0 && (!workspace || workspace_bytes < p.total)) return MTP_ERR_WORKSPACE;
  unsigned char *w8 = (unsigned char *)workspace;
  for (int64_t m0 = 0; m0 < M; m0 += 65535) {
    const int rows = (int)std::min<int64_t>(M - m0, 65535);
    ArgmaxArgs a{};
    a.logits = (const unsigned char *)logits + (size_t)m0 * ld * dtype_bytes(dtype);
    a.dt = dtype;
    a.ld = ld;
    a.M = rows;
    a.V = (int)V;
    a.S = p.S;
    a.seg = (int)p.seg;
    if (p.S > 1) {
      a.part = (unsigned long long *)(w8 + kCounterBytes);
      a.ticket = (unsigned *)w8;
    }
    a.tokens = tokens + m0;
    a.table = emb_table;
    a.tbytes = emb_table ? dtype_bytes(table_dtype) : 0;
    a.H = (int)H;
    a.emb = emb_table ? (unsigned char *)emb_out + (size_t)m0 * H * a.tbytes : nullptr;
    a.emb16 = emb_table && (H * a.tbytes) % 16 == 0 && aligned16(emb_table) && aligned16(a.emb);
    // 16-byte form: rows of whole chunks, 16-byte aligned (segments are
    // whole chunks by the plan)
    const int64_t e = dtype == MTP_F32 ? 4 : 8;
    const bool vec = ld % e == 0 && aligned16(logits);
    void (*k)(ArgmaxArgs) = argmax_rows_kernel<-1>;
    if (vec) {
      k = dtype == MTP_F32    ? argmax_rows_kernel<MTP_F32>
          : dtype == MTP_BF16 ? argmax_rows_kernel<MTP_BF16>
                              : argmax_rows_kernel<MTP_F16>;
    }
    hipLaunchKernelGGL(k, dim3((unsigned)p.S, (unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, a);
    const int s = launch_status();
    if (s != MTP_OK) return s;
  }
  return MTP_OK;
}

int mtp_paged_kv_write(const void *k_new, const void *v_new, int src_dtype, int64_t B, int64_t T,
                       int64_t H, int64_t D, int64_t s_sb, int64_t s_st, int64_t s_sh,
                       void *k_pages, void *v_pages, int dst_dtype, int64_t num_pages,
                       int64_t page_size, const int32_t *page_table, int64_t ld_tab,
                       const int64_t *start_dev, int start_per_row, int64_t start_host,
                       void *stream) {
  if (!is_float_dt(src_dtype) || !is_float_dt(dst_dtype)) return MTP_ERR_DTYPE;
  if (B < 0 || T < 0 || H < 0 || D <= 0 || num_pages < 0 || page_size <= 0 || ld_tab < 0 ||
      B > INT32_MAX || T > INT32_MAX || H > INT32_MAX || D > INT32_MAX || num_pages > INT32_MAX ||
      page_size > INT32_MAX)
    return MTP_ERR_SHAPE;
  const int64_t rows = B * T * H;
  if (rows == 0) return MTP_OK;
  if (!k_new || !v_new || !k_pages || !v_pages || !page_table) return MTP_ERR_NULL;
  KvWriteArgs a{};
  a.k_new = k_new;
  a.v_new = v_new;
  a.src_dt = src_dtype;
  a.s_sb = s_sb;
  a.s_st = s_st;
  a.s_sh = s_sh;
  a.k_pages = k_pages;
  a.v_pages = v_pages;
  a.dst_dt = dst_dtype;
  a.p_sh = page_size * D;
  a.p_sb = H * a.p_sh;
  a.p_sp = B * a.p_sb;
  a.table = page_table;
  a.ld_tab = ld_tab;
  a.start_dev = start_dev;
  a.start_per_row = start_per_row ? 1 : 0;
  a.start_host = start_host;
  a.B = (int)B;
  a.T = (int)T;
  a.H = (int)H;
  a.D = (int)D;
  a.page_size = (int)page_size;
  a.npages = (int)num_pages;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > INT32_MAX) return MTP_ERR_SHAPE;
  hipLaunchKernelGGL(paged_kv_write_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, a);
  return launch_status();
}

int mtp_verify_commit(const int8_t *accept, const int32_t *accepted_n, const int32_t *corrected,
                      const void *draft, int draft_dtype, int64_t B, int64_t D,
                      const int64_t *checkpoint, int64_t *kv_len, int64_t *tokens,
                      int32_t *width, int64_t *ids, int64_t ld_ids, int64_t *ids_len,
                      void *stream) {
  if (draft_dtype != MTP_I32 && draft_dtype != MTP_I64) return MTP_ERR_DTYPE;
  if (B <= 0 || D < 0 || B > INT32_MAX || D > INT32_MAX - 1 || (ids && ld_ids < 0))
    return MTP_ERR_SHAPE;
  if (!accepted_n || !corrected || !checkpoint || !kv_len || !tokens || !width ||
      (D > 0 && (!accept || !draft)) || (ids && !ids_len))
    return MTP_ERR_NULL;
  CommitArgs a{};
  a.accept = accept;
  a.accepted_n = accepted_n;
  a.corrected = corrected;
  a.draft = draft;
  a.draft_i64 = draft_dtype == MTP_I64;
  a.B = (int)B;
  a.D = (int)D;
  a.checkpoint = checkpoint;
  a.kv_len = kv_len;
  a.tokens = tokens;
  a.width = width;
  a.ids = ids;
  a.ld_ids = ld_ids;
  a.ids_len = ids_len;
  hipLaunchKernelGGL(verify_commit_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, a);
  return launch_status();
}

int mtp_batch_prefix_match(const int64_t *ids, int64_t R, int64_t L, int32_t *out, void *stream) {
  if (R < 0 || L < 0 || R > INT32_MAX || L > INT32_MAX) return MTP_ERR_SHAPE;
  if (R == 0) return MTP_OK;
  if (!out || (L > 0 && !ids)) return MTP_ERR_NULL;
  // a single row has nothing to share a prefix with: 0, as the reference
  const int Lk = R <= 1 ? 0 : (int)L;
  hipLaunchKernelGGL(prefix_match_kernel, dim3((unsigned)((R + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, ids, L, (int)R, Lk, out);
  return launch_status();
}

}  // extern "C"
