/*
 * mtp_hip.h — C ABI of the MI355X (gfx950) verify/draft hot path.
 *
 * One entry point per Python function of the reference's kernel layer.
 * Every entry point:
 *   - takes plain device pointers, element counts and dtype codes (no torch
 *     types), all tensors contiguous row-major in the reference's layout
 *     (nn.Linear weights are [N, K] = [out, in]);
 *   - enqueues its kernels on `stream` (a hipStream_t; NULL = the null
 *     stream) and returns without synchronising, so it can be captured into
 *     a hipGraph;
 *   - never allocates device memory: scratch comes from the caller through
 *     `workspace` / `workspace_bytes`, sized by the matching *_workspace_bytes
 *     query. The first MTP_WORKSPACE_COUNTER_BYTES of every workspace hold
 *     arrival counters: they must be zero before the first use, and every
 *     launch leaves the counters it used at zero again, so one workspace can
 *     serve any sequence of calls (any entry point, any shape) on one stream
 *     (calls that overlap on different streams need distinct workspaces);
 *   - validates its arguments on the host before any HIP call and returns a
 *     status code (MTP_OK = 0, negative on error; mtp_status_string() names
 *     it). It never aborts the process.
 */
#ifndef MTP_HIP_H
#define MTP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTP_ABI_VERSION 1

/* Bytes at the start of a workspace reserved for arrival counters. */
#define MTP_WORKSPACE_COUNTER_BYTES 65536

/* Element type codes. */
enum mtp_dtype {
  MTP_F32 = 0,
  MTP_BF16 = 1,
  MTP_F16 = 2,
  MTP_FP8E4M3 = 3, /* OCP float8_e4m3fn (torch.float8_e4m3fn) */
  MTP_U8 = 4,
  MTP_I8 = 5,
  MTP_I32 = 6,
  MTP_I64 = 7
};

/* Status codes. */
enum mtp_status {
  MTP_OK = 0,
  MTP_ERR_NULL = -1,      /* a required pointer is NULL */
  MTP_ERR_SHAPE = -2,     /* sizes inconsistent or out of the supported range */
  MTP_ERR_DTYPE = -3,     /* unsupported dtype or dtype combination */
  MTP_ERR_WORKSPACE = -4, /* workspace missing or smaller than required */
  MTP_ERR_ALIGN = -5,     /* a pointer is not aligned as the kernel requires */
  MTP_ERR_LAUNCH = -6,    /* the HIP runtime rejected a launch */
  MTP_ERR_ARG = -7        /* any other invalid argument */
};

/* INT4 nibble conventions for mtp_fused_int4_matmul. */
enum mtp_nibble {
  /* nibble n decodes to n - 8: the reference decoder (mtp_kernels.py:758-762,
   * 470-473); this is the parity contract. */
  MTP_NIBBLE_OFFSET8 = 0,
  /* nibble n is a two's-complement int4 (n >= 8 means n - 16): what the
   * reference quantizer writes (mtp_kernels.py:742-750). */
  MTP_NIBBLE_TWOS = 1
};

int mtp_abi_version(void);
const char *mtp_status_string(int status);
/* Name of the last HIP error seen by a failed launch on this thread. */
const char *mtp_last_hip_error(void);

/*
 * Launch-planning overrides, process-wide (no counterpart in the reference,
 * whose Triton launches take tile sizes from KernelTuningConfig,
 * mtp_kernels.py:54-103). Keys: "skl" (1 force / 0 disable the single-launch
 * skinny kernel), "sk_splits", "ws_variant", "ws_splits", "skl_waves" (4 or
 * 8), "skl_splits", "attn_chunk_blocks", "int4_waves" (4 or 8),
 * "verify_wstream" (1 = column-group verify kernel), "skp" (1 force / 0
 * disable the x-resident skinny kernel), "skp_splits", "skp_ta" (A tiles
 * per wave: 1, 2 or 4), "skp_h8" (0: full x blocks in the x-resident
 * kernel for at most 8 rows), "sf32" (0: no one-launch fp32 kernels for at most 32 rows), "attn32"
 * (0: 16-query-tile attention for 33 .. 64 queries), "sk_xraw" (0: the
 * skinny kernel keeps its prep launch without gamma too), "skw" (1: the
 * wave-specialised skinny GEMM wherever it applies, 0: never), "skw_tw",
 * "skp_tw", "skl_tw" (output columns per workgroup of the wave-specialised,
 * x-resident and single-launch skinny kernels, a multiple of 8 up to their
 * tile width; default: narrowed by at most a quarter so that the grid puts
 * one workgroup on every CU), "skv_r8" (0: the fp32 verify pads 8 rows
 * past whole 16-row tiles to a full tile instead of running them on the
 * 4 x 4 MFMA), "skv_tw" (columns per tile of the streaming verify, a
 * multiple of 8 up to 256; default: whole rounds of one tile per CU from
 * a 64-column tile per CU). value -1
 * restores the planner's choice. The MTP_SKL, MTP_SK_SPLITS, MTP_WS_TUNE
 * ("variant,splits"), MTP_SKL_WAVES, MTP_SKL_SPLITS, MTP_ATTN_CHUNK_BLOCKS,
 * MTP_INT4_WAVES, MTP_VERIFY_WSTREAM, MTP_SKP, MTP_SKP_SPLITS, MTP_SKP_TA,
 * MTP_SKP_H8, MTP_SF32, MTP_ATTN32, MTP_SK_XRAW, MTP_SKW, MTP_SKW_TW, MTP_SKP_TW, MTP_SKL_TW,
 * MTP_SKV_R8 and MTP_SKV_TW environment variables
 * seed the keys once, at the
 * first launch plan. MTP_ERR_ARG for an unknown key.
 */
int mtp_set_tuning(const char *name, int64_t value);
int mtp_get_tuning(const char *name, int64_t *value);

/* ------------------------------------------------------------------------- */
/* RMSNorm -> linear family                                                  */
/* ------------------------------------------------------------------------- */

/*
 * Replaces fused_rmsnorm_linear(x, weight, bias=None, eps=1e-6, scale=None)
 * (mtp_kernels.py:936-977; eager twin _eager_rmsnorm_linear 778-787):
 *   y = cast_xdtype(((x * rsqrt(mean(x^2) + eps) * gamma) @ W^T + bias) * scale)
 * x [M, K] in x_dtype (F32, BF16, F16); weight [N, K] in w_dtype (any float
 * dtype; the tiled kernels take w_dtype == x_dtype with 16-byte aligned
 * rows, everything else runs an exact fp32 fallback); bias [N] in bias_dtype or NULL (the reference casts bias to
 * x.dtype first, mtp_kernels.py:952: the caller passes it already cast);
 * gamma [K] in gamma_dtype or NULL (keyword extension; NULL = the reference);
 * norm = 0 skips the RMSNorm (the no-norm mode CachedLinear needs,
 * mtp_perf_hardening.py:150-165); y [M, N] in x_dtype.
 * Arithmetic: products exact, fp32 accumulation (TF32 off for F32).
 */
int mtp_fused_rmsnorm_linear(const void *x, int x_dtype, int64_t M, int64_t K,
                             const void *weight, int w_dtype, int64_t N,
                             const void *bias, int bias_dtype,
                             const void *gamma, int gamma_dtype, float eps,
                             float scale, int norm, void *y, void *workspace,
                             size_t workspace_bytes, void *stream);

/*
 * Replaces fused_rmsnorm_linear_fp8(x, weight_fp8, wscale, bias=None,
 * eps=1e-6) (mtp_kernels.py:1014-1044; eager 804-814):
 *   y = cast_xdtype((x * rstd * gamma) @ (fp8_to_f32(W) * wscale[:, None])^T + bias)
 * weight_fp8 [N, K] in w_dtype: MTP_FP8E4M3 (float8_e4m3fn), or a float
 * dtype (the reference accepts any weight dtype here; its self-test passes
 * fp32 values in +-448, mtp_engine.py:1792-1800); wscale [N] fp32 (per output
 * channel, a slice of the packed scale buffer of pack_scales,
 * mtp_kernels.py:1336-1353).
 */
int mtp_fused_rmsnorm_linear_fp8(const void *x, int x_dtype, int64_t M,
                                 int64_t K, const void *weight_fp8,
                                 int w_dtype, const float *wscale, int64_t N,
                                 const void *bias, int bias_dtype,
                                 const void *gamma, int gamma_dtype, float eps,
                                 int norm, void *y, void *workspace,
                                 size_t workspace_bytes, void *stream);

/*
 * Replaces fused_int4_matmul(x, packed, scales, K, group=32)
 * (mtp_kernels.py:1194-1219; eager 875-878; decoder 754-768):
 *   y = cast_xdtype(xn @ Wdq^T),  Wdq[n, k] = nib(n, k) * scales[n, k / group]
 * nib(n, k) is nibble (k & 1) of packed[n, k / 2] (low nibble for even k),
 * decoded per `nibble` (MTP_NIBBLE_OFFSET8 = the reference). packed [N, K/2]
 * u8; scales [N, ceil(K/group)] in scale_dtype (F32, F16 or BF16).
 * norm = 0 is the reference (xn = x, or x * gamma when gamma is given; no
 * RMSNorm, no bias); norm = 1 composes the RMSNorm prologue
 * xn = x * rstd * gamma (the INT4 RMSNorm+linear workload).
 * When K % 128 == 0, group % 32 == 0 and packed is 16-byte aligned, the
 * MFMA path runs: it needs the workspace of
 * mtp_rmsnorm_linear_workspace_bytes(x_dtype, MTP_U8, M, N, K) (fp16 copy
 * of xn, one float per row, the scales transposed to fp16 and one float per
 * column) and computes with weights decoded to fp16. Each column's scales
 * are first normalised by an exact power of two (undone in the fp32
 * epilogue), so any finite scale magnitude is safe: a scale is rounded once
 * to 11 bits, and only scales below 2^-21 of their column's largest lose
 * more. A non-finite scale makes its column's outputs non-finite.
 * Other shapes run a CUDA-core fallback without workspace.
 */
int mtp_fused_int4_matmul(const void *x, int x_dtype, int64_t M, int64_t K,
                          const uint8_t *packed, const void *scales,
                          int scale_dtype, int64_t N, int64_t group,
                          int nibble, const void *gamma, int gamma_dtype,
                          float eps, int norm, void *y, void *workspace,
                          size_t workspace_bytes, void *stream);

/* Workspace bytes the three entry points above need for these sizes
 * (w_kind: MTP_F32/MTP_BF16/MTP_F16 weights, MTP_FP8E4M3, or MTP_U8 for
 * packed INT4). */
size_t mtp_rmsnorm_linear_workspace_bytes(int x_dtype, int w_kind, int64_t M,
                                          int64_t N, int64_t K);

/* ------------------------------------------------------------------------- */
/* Verify: lm_head GEMM -> argmax -> acceptance -> rollback index            */
/* ------------------------------------------------------------------------- */

/*
 * Replaces fused_verify(hidden, weight, draft, bias=None) -> (accept, top)
 * (mtp_fused_verify.py:199-234; kernel 42-80; eager 159-166):
 *   top[m] = argmax_v(hidden[m] . W[v] + bias[v])  (lowest index on ties,
 *            NaN counts as the maximum, as torch.argmax)
 *   accept[m] = (top[m] == draft[m])
 * hidden [M, K] and weight [V, K] in any float dtypes (F32/BF16/F16; both
 * upcast to fp32 as the reference does), bias [V] or NULL, draft [M] int32
 * -> accept [M] int8, top [M] int32. Any K and element alignment (16-bit
 * same-dtype operands with 16-byte rows take the streaming kernels, the
 * rest a generic kernel). Logits never reach HBM.
 */
int mtp_fused_verify(const void *hidden, int h_dtype, int64_t M, int64_t K,
                     const void *weight, int w_dtype, int64_t V,
                     const void *bias, int bias_dtype, const int32_t *draft,
                     int8_t *accept, int32_t *top, void *workspace,
                     size_t workspace_bytes, void *stream);

/*
 * Replaces fused_multi_verify(hidden, weight, draft, bias=None)
 *   -> (accept, accepted_n, corrected)
 * (mtp_fused_verify.py:237-290; kernel 88-156; eager 169-196):
 *   top[b, s] = argmax_v(hidden[b, s] . W[v] + bias[v]),  s = 0..D
 *   accept[b, d] = (top[b, d+1] == draft[b, d]) and accept[b, d-1]
 *   accepted_n[b] = number of leading accepted drafts (the rollback index)
 *   corrected[b] = top[b, 0]
 * hidden [B, S, K] with S == D + 1, weight [V, K], draft [B, D] int32.
 * top_out [B, S] int32 may be NULL (keyword extension return_top).
 */
int mtp_fused_multi_verify(const void *hidden, int h_dtype, int64_t B,
                           int64_t S, int64_t K, const void *weight,
                           int w_dtype, int64_t V, const void *bias,
                           int bias_dtype, const int32_t *draft, int64_t D,
                           int8_t *accept, int32_t *accepted_n,
                           int32_t *corrected, int32_t *top_out,
                           void *workspace, size_t workspace_bytes,
                           void *stream);

/*
 * fused_multi_verify(..., convention="textbook") (keyword extension). The
 * reference's convention is mtp_fused_multi_verify's
 * (mtp_fused_verify.py:136-154, 184-195: draft d checked against the argmax
 * at s = d + 1, corrected = the anchor's argmax); this is the textbook
 * speculative-decoding chain on the same argmax tokens:
 *   accept[b, d] = (top[b, d] == draft[b, d]) and accept[b, d-1]
 *   accepted_n[b] = number of leading accepted drafts
 *   corrected[b] = top[b, accepted_n[b]]  (the replacement token, or the
 *                                          bonus token when all D accept)
 * Same arguments, kernels and workspace as mtp_fused_multi_verify.
 */
int mtp_fused_multi_verify_textbook(const void *hidden, int h_dtype, int64_t B,
                                    int64_t S, int64_t K, const void *weight,
                                    int w_dtype, int64_t V, const void *bias,
                                    int bias_dtype, const int32_t *draft,
                                    int64_t D, int8_t *accept,
                                    int32_t *accepted_n, int32_t *corrected,
                                    int32_t *top_out, void *workspace,
                                    size_t workspace_bytes, void *stream);

/*
 * Allocation-free mtp_fused_multi_verify. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results as mtp_fused_multi_verify, without the workspace:
 * the library keeps one static device array of
 * mtp_noalloc_scratch_bytes() (1 MiB) per GPU, allocated with the module,
 * and clears its counter prefix with a kernel before each call. The
 * persistent and generic verify kernels need only the counter prefix; a
 * call on the column-group kernel (mtp_verify_route) whose workspace
 * (mtp_verify_workspace_bytes) exceeds the array returns MTP_ERR_WORKSPACE.
 * Calls on one GPU share the array: calls that overlap (different streams,
 * no ordering) race. mtp_noalloc_init() looks the array's address up for
 * the current device (the first call on a device does it otherwise): call
 * it once per device before capturing calls into a graph.
 */
int mtp_fused_multi_verify_noalloc(const void *hidden, int h_dtype, int64_t B,
                                   int64_t S, int64_t K, const void *weight,
                                   int w_dtype, int64_t V, const void *bias,
                                   int bias_dtype, const int32_t *draft,
                                   int64_t D, int8_t *accept,
                                   int32_t *accepted_n, int32_t *corrected,
                                   int32_t *top_out, void *stream);
size_t mtp_noalloc_scratch_bytes(void);
int mtp_noalloc_init(void);

/*
 * The kernel a verify call with these operands takes (host only, nothing
 * launched): rows = M, seq = 1 for mtp_fused_verify; rows = B * S, seq = S
 * for the chain. No counterpart in the reference (its routes are Triton or
 * eager); for tests and tuning. Returns one of:
 *   MTP_VERIFY_ROUTE_STREAM        persistent W-streaming kernel (one dtype
 *                                  for hidden and W: BF16 / F16 / F32; any
 *                                  bias; K * element bytes % 512 == 0;
 *                                  16-byte aligned rows)
 *   MTP_VERIFY_ROUTE_COLUMN_GROUP  column-group streaming kernel
 *   MTP_VERIFY_ROUTE_GENERIC       any dtypes, K and alignment
 * or a negative status.
 */
#define MTP_VERIFY_ROUTE_STREAM 0
#define MTP_VERIFY_ROUTE_COLUMN_GROUP 1
#define MTP_VERIFY_ROUTE_GENERIC 2
int mtp_verify_route(const void *hidden, int h_dtype, int64_t rows, int64_t seq,
                     int64_t K, const void *weight, int w_dtype, int64_t V,
                     const void *bias);

/* Workspace bytes for mtp_fused_verify (rows = M, seq = 1) or
 * mtp_fused_multi_verify (rows = B * S, seq = S) at vocabulary size V. */
size_t mtp_verify_workspace_bytes(int h_dtype, int64_t rows, int64_t seq,
                                  int64_t V, int64_t K);

/* ------------------------------------------------------------------------- */
/* Tree / paged attention                                                    */
/* ------------------------------------------------------------------------- */

/*
 * Replaces fused_paged_attention(q, k_pages, v_pages, page_table, page_size,
 * scale=None) (mtp_kernels.py:1136-1162; kernel 494-554; eager 832-856):
 *   out[b, h] = softmax_t(q[b, h] . k_t * scale) @ v_t,
 *   k_t = k_pages[page_table[b, t], b, h, t % page_size]   (t < L)
 * q / out [B, H, D]; k_pages / v_pages [num_pages, B, H, page_size, D]; all
 * in dtype (F32, BF16, F16); page_table [B, L] int32 (the reference casts it,
 * 1143). scale: the caller passes 1/sqrt(D) for the reference default. A
 * page index outside [0, num_pages) masks its key instead of being read.
 */
int mtp_fused_paged_attention(const void *q, int dtype, int64_t B, int64_t H,
                              int64_t D, const void *k_pages,
                              const void *v_pages, int64_t num_pages,
                              const int32_t *page_table, int64_t L,
                              int64_t page_size, float scale, void *out,
                              void *workspace, size_t workspace_bytes,
                              void *stream);

/*
 * Replaces fused_tree_attention(q, k, v, mask, scale=None)
 * (mtp_kernels.py:1165-1191; kernel 559-613; eager 859-872):
 *   out[b, h] = softmax_l(where(mask[l] > 0.5, q[b, h] . k[b, h, l] * scale,
 *               -inf)) @ v[b, h, l]      (every key masked: NaN, as there)
 * q / out [B, H, D]; k / v [B, H, L, D]; mask [L] in mask_dtype (F32, BF16,
 * F16, or U8 for bool).
 */
int mtp_fused_tree_attention(const void *q, int dtype, int64_t B, int64_t H,
                             int64_t D, const void *k, const void *v, int64_t L,
                             const void *mask, int mask_dtype, float scale,
                             void *out, void *workspace, size_t workspace_bytes,
                             void *stream);

/*
 * The tree-verify attention step in one launch (no single reference
 * function: the reference composes it from one fused_tree_attention call per
 * node over keys = context ++ tree nodes, mtp_kernels.py:1165-1191, with the
 * SpeculativeDraftTree mask, mtp_engine.py:671-680):
 *   out[n, h] = softmax over { context tokens t < Lc } u { tree nodes m with
 *               tree_mask[n, m] > 0.5 } of q[n, h] . k * scale, @ v
 * q_nodes / k_tree / v_tree / out [N, H, D]; k_pages / v_pages
 * [num_pages, 1, H, page_size, D]; page_table [1, Lc] int32; tree_mask
 * [N, N] in mask_dtype.
 */
int mtp_tree_verify_attention(const void *q_nodes, int dtype, int64_t N,
                              int64_t H, int64_t D, const void *k_pages,
                              const void *v_pages, int64_t num_pages,
                              const int32_t *page_table, int64_t Lc,
                              int64_t page_size, const void *k_tree,
                              const void *v_tree, const void *tree_mask,
                              int mask_dtype, float scale, void *out,
                              void *workspace, size_t workspace_bytes,
                              void *stream);

/* ------------------------------------------------------------------------- */
/* Quantizers                                                                */
/* ------------------------------------------------------------------------- */

/*
 * Replaces quantize_fp8_e4m3(x) -> (x_fp8, scale) (mtp_kernels.py:704-713):
 *   scale = amax(|x|) / 448 if amax > 0 else 1   (amax keeps NaN, NaN > 0 is false)
 *   x_fp8 = e4m3fn(clamp(x / scale, -448, 448))  round to nearest even
 * x: n elements in x_dtype; x_fp8: n bytes; scale: one fp32 (device).
 * Needs mtp_quantize_workspace_bytes(n) of workspace.
 */
int mtp_quantize_fp8_e4m3(const void *x, int x_dtype, int64_t n, uint8_t *x_fp8,
                          float *scale, void *workspace, size_t workspace_bytes,
                          void *stream);
size_t mtp_quantize_workspace_bytes(int64_t n);

/*
 * Per-output-channel fp8 weights: the scale rule of
 * QuantScaleState.update_weight_scales (mtp_engine.py:617-622),
 * wscale[n] = amax(|W[n, :]|) / 448 (0 -> 1), with each row quantized as
 * quantize_fp8_e4m3 does: W_fp8[n, k] = e4m3fn(clamp(W[n, k] / wscale[n], +-448)).
 * w [N, K] in w_dtype -> w_fp8 [N, K] bytes, wscale [N] fp32.
 */
int mtp_quantize_fp8_rows(const void *w, int w_dtype, int64_t N, int64_t K,
                          uint8_t *w_fp8, float *wscale, void *stream);

/*
 * Replaces dequantize_fp8(x_fp8, scale) (mtp_kernels.py:726-727):
 *   out = fp32(x_fp8) * scale, with one scale (per_row = 0) or one scale per
 *   row of row_len elements (per_row = 1, the per-channel layout).
 */
int mtp_dequantize_fp8(const uint8_t *x_fp8, int64_t n, int64_t row_len,
                       const float *scale, int per_row, float *out,
                       void *stream);

/*
 * Replaces quantize_int4(x, group=32) -> (packed, scales)
 * (mtp_kernels.py:730-751): per row and group of `group` columns,
 *   s = amax / 7 if amax > 0 else 1,  q = clamp(round_half_even(w / s), -8, 7)
 *   packed[n, k / 2] = (q[k] & 0xF) | (q[k + 1] & 0xF) << 4   (even k low)
 * w [N, K] (K and group even) -> packed [N, K/2] u8, scales [N, ceil(K/group)] fp32.
 */
int mtp_quantize_int4(const void *w, int w_dtype, int64_t N, int64_t K,
                      int64_t group, uint8_t *packed, float *scales,
                      void *stream);

/*
 * Replaces dequantize_int4(packed, scales, K, group) (mtp_kernels.py:754-768):
 *   out[n, k] = (nibble(n, k) - 8) * scales[n, k / group]   (fp32 [N, K])
 */
int mtp_dequantize_int4(const uint8_t *packed, const void *scales,
                        int scale_dtype, int64_t N, int64_t K, int64_t group,
                        float *out, void *stream);

/*
 * Replaces fused_causal_attention(q, k, v, scale=None)
 * (mtp_kernels.py:980-1011; kernel 235-298; eager 790-801):
 *   out[b, h] = softmax_l(q[b, h] . k[b, h, l] * scale) @ v[b, h, l]
 * (a single query at the last position: every key is attended).
 * q / out [B, H, D], k / v [B, H, L, D], one float dtype. Workspace as
 * mtp_attention_workspace_bytes(dtype, B, 1, H, D, 0, L).
 */
int mtp_fused_causal_attention(const void *q, int dtype, int64_t B, int64_t H,
                               int64_t D, const void *k, const void *v,
                               int64_t L, float scale, void *out,
                               void *workspace, size_t workspace_bytes,
                               void *stream);

/*
 * Replaces fused_causal_attention_fp8(q, k_fp8, v_fp8, kscale, vscale,
 * scale=None) (mtp_kernels.py:1105-1133; kernel 373-427; eager 817-829):
 * k / v fp8 e4m3fn [B, H, L, D] dequantised per head by kscale[H] /
 * vscale[H] (fp32); q / out [B, H, D] in dtype. No workspace.
 */
int mtp_fused_causal_attention_fp8(const void *q, int dtype, int64_t B,
                                   int64_t H, int64_t D, const void *k_fp8,
                                   const void *v_fp8, int64_t L,
                                   const float *kscale, const float *vscale,
                                   float scale, void *out, void *stream);

/*
 * Replaces fused_tree_attn_rmsnorm_linear(q, k, v, mask, proj_w, rms_w=None,
 * proj_bias=None, wscale=None, scale=None, eps=1e-6)
 * (mtp_kernels.py:1222-1250; eager _eager_tree_attn_rmsnorm_linear 881-907):
 *   a[b, h] = masked single-query attention (as mtp_fused_tree_attention)
 *   out[b, h] = (a * rsqrt(mean_d(a^2) + eps) * rms_w) @ (proj_w * wscale)^T + proj_bias
 * q [B, H, D], k / v [B, H, L, D], mask [L]; proj_w [N, D] (float, or fp8
 * with wscale [N]); rms_w [D] or NULL (ones); proj_bias [N] or NULL;
 * out [B, H, N] in q's dtype. A mask that admits no key gives NaN rows,
 * like the eager twin, deterministically. Two launches (attention into the
 * workspace, then the RMSNorm -> linear kernel over the B * H rows).
 */
int mtp_fused_tree_attn_rmsnorm_linear(
    const void *q, int dtype, int64_t B, int64_t H, int64_t D, const void *k,
    const void *v, int64_t L, const void *mask, int mask_dtype,
    const void *proj_w, int w_dtype, int64_t N, const void *rms_w,
    int rms_dtype, const void *proj_bias, int bias_dtype, const float *wscale,
    float scale, float eps, void *out, void *workspace, size_t workspace_bytes,
    void *stream);
/* w_kind: proj_w's dtype, or MTP_FP8E4M3 whenever wscale is passed. */
size_t mtp_tree_attn_rmsnorm_linear_workspace_bytes(int dtype, int64_t B,
                                                    int64_t H, int64_t D,
                                                    int64_t L, int w_kind,
                                                    int64_t N);

/* Workspace bytes for the attention entry points: B batch rows, NQ queries
 * per (batch, head) (1 for the two reference functions, N for tree verify),
 * Lc context keys, Lt dense keys (L of fused_tree_attention, N of tree
 * verify). */
size_t mtp_attention_workspace_bytes(int dtype, int64_t B, int64_t NQ,
                                     int64_t H, int64_t D, int64_t Lc,
                                     int64_t Lt);

/* ------------------------------------------------------------------------- */
/* Draft chain                                                               */
/* ------------------------------------------------------------------------- */

/*
 * Replaces fused_rmsnorm(x, weight=None, eps=1e-6)
 * (mtp_kernels.py:910-933; kernel 120-146; eager _eager_rmsnorm 771-775):
 *   y = x * rsqrt(mean(x^2) + eps) * weight   (fp32, rounded to dtype)
 * x / y [M, N] contiguous in dtype; weight [N] in w_dtype or NULL (ones).
 * The reference casts weight to x's dtype first: the caller passes it cast.
 */
int mtp_fused_rmsnorm(const void *x, int dtype, int64_t M, int64_t N,
                      const void *weight, int w_dtype, float eps, void *y,
                      void *stream);

/*
 * Replaces fused_add_rmsnorm(x, residual, weight=None, eps=1e-6)
 * (mtp_kernels.py:1082-1102; kernel 1050-1070; eager 1073-1079):
 *   s = x + residual (fp32);  y = s * rsqrt(mean(s^2) + eps) * weight
 * (the draft chain's combine-norm, combine_norm(hidden + emb) at
 * mtp_engine.py:241, 757, in one pass; fp32 addition, where the module
 * rounds the sum to the hidden dtype first).
 */
int mtp_fused_add_rmsnorm(const void *x, const void *residual, int dtype,
                          int64_t M, int64_t N, const void *weight,
                          int w_dtype, float eps, void *y, void *stream);

/*
 * Replaces argmax_greedy(logits) / sample_token(logits, temperature <= 0)
 * (mtp_perf_hardening.py:170-186; the engine's _sample_tokens,
 * mtp_engine.py:722-726) and the embedding lookup of the next draft step
 * (mtp_engine.py:750, 773):
 *   tokens[m] = argmax_v logits[m, v]   (torch.argmax order, int64)
 *   emb_out[m, :] = emb_table[tokens[m], :]   (when emb_table is not NULL)
 * logits [M, V] with row stride ld elements; emb_table [table_rows, H].
 * Needs mtp_argmax_workspace_bytes(M, V) of workspace.
 */
int mtp_argmax(const void *logits, int dtype, int64_t M, int64_t V,
               int64_t ld, int64_t *tokens, const void *emb_table,
               int table_dtype, int64_t table_rows, int64_t H, void *emb_out,
               void *workspace, size_t workspace_bytes, void *stream);
size_t mtp_argmax_workspace_bytes(int64_t M, int64_t V);

/* ------------------------------------------------------------------------- */
/* KV step after verify                                                      */
/* ------------------------------------------------------------------------- */

/*
 * Batched form of PagedKVCache.write_inplace (mtp_engine.py:581-585):
 *   pages[table[b, p], b, h, p % page_size, :] = new[b, t, h, :],  p = start + t
 * for k and v. new: [B, T, H, D] by element strides (s_sb, s_st, s_sh), d
 * contiguous, in src_dtype; pages [num_pages, B, H, page_size, D] in
 * dst_dtype (converted as .to(dtype)); page_table [B, ld_tab] int32. start
 * is start_dev[b] (start_per_row = 1) or start_dev[0] (a device scalar,
 * e.g. the KV length mtp_verify_commit maintains), or start_host when
 * start_dev is NULL. Positions outside the table and pages outside
 * [0, num_pages) are skipped.
 */
int mtp_paged_kv_write(const void *k_new, const void *v_new, int src_dtype,
                       int64_t B, int64_t T, int64_t H, int64_t D,
                       int64_t s_sb, int64_t s_st, int64_t s_sh, void *k_pages,
                       void *v_pages, int dst_dtype, int64_t num_pages,
                       int64_t page_size, const int32_t *page_table,
                       int64_t ld_tab, const int64_t *start_dev,
                       int start_per_row, int64_t start_host, void *stream);

/*
 * The verify consumer of generate_fused / generate_optimized
 * (mtp_engine.py:1244-1258, 1328-1344) with its KVManager rollback / commit
 * (275-331) on the device, without the host reads of accepted_n and accept:
 *   a_n = min_b accepted_n[b];  reject = any accept[b, d] == 0
 *   width = reject ? a_n + 1 : D
 *   tokens[b, :width] = reject ? draft[b, :a_n] ++ corrected[b] : draft[b]
 *   tokens[b, width:] = -1;  *kv_len = *checkpoint + width;  *width_out = width
 * and, when ids is not NULL (contiguous rows of capacity ld_ids),
 * ids[b, *ids_len + j] = tokens[b, j] for the j < width that fit and
 * *ids_len += that count: *ids_len never passes ld_ids, so a full buffer
 * shows as an advance shorter than *width_out. tokens [B, D + 1] int64; draft
 * [B, D] int32 or int64; checkpoint / kv_len / ids_len are int64 device
 * scalars (kv_len may alias checkpoint). One workgroup.
 */
int mtp_verify_commit(const int8_t *accept, const int32_t *accepted_n,
                      const int32_t *corrected, const void *draft,
                      int draft_dtype, int64_t B, int64_t D,
                      const int64_t *checkpoint, int64_t *kv_len,
                      int64_t *tokens, int32_t *width_out, int64_t *ids,
                      int64_t ld_ids, int64_t *ids_len, void *stream);

/*
 * Replaces RadixKVCache.batch_prefix_match(ids) (mtp_radix.py:195-272,
 * kernel 254-267): out[r] = first column c with ids[r, c] != ids[0, c], or
 * L when the row equals row 0; all zeros when R <= 1. ids [R, L] int64,
 * out [R] int32.
 */
int mtp_batch_prefix_match(const int64_t *ids, int64_t R, int64_t L,
                           int32_t *out, void *stream);

/* ------------------------------------------------------------------------- */
/* Workspace                                                                 */
/* ------------------------------------------------------------------------- */

/* Zero a workspace with a kernel launch on `stream` (no memset node when the
 * stream is being captured). workspace 16-byte aligned, bytes % 4 == 0.
 * No counterpart in the reference (whose wrappers allocate per call). */
int mtp_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MTP_HIP_H */
