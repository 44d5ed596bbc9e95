"""Drop-in for the reference module ``mtp_kernels`` on MI355X.

Same names, argument order, defaults and return values as the reference's
public functions (mtp_kernels.py:704-768, 910-1250, 1336-1353, 1426-1457);
every compute entry point launches a hand-written gfx950 kernel through
libmtp_hip.so. ``_HAS_TRITON`` is False: nothing here (or in a caller that
tests the flag) takes a Triton route. Keyword-only extensions: ``gamma``
(RMSNorm weight, default None = the reference) and ``norm`` (False = plain
linear, the mode CachedLinear needs) on the RMSNorm -> linear entry points;
``nibble``, ``gamma``, ``norm`` and ``eps`` on fused_int4_matmul (default =
the reference: offset-8 nibbles, no norm).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from . import ops


@dataclass(frozen=True)
class KernelTuningConfig:
    """Launch defaults of the reference (mtp_kernels.py:54-65). Only
    ``fp8_scale`` (the default ``scale`` of fused_rmsnorm_linear) is read;
    tile shapes come from the library's own tables."""
    BLOCK_M: int = 64
    BLOCK_N: int = 64
    BLOCK_K: int = 32
    BLOCK_DHEAD: int = 64
    num_warps: int = 4
    num_stages: int = 2
    fp8_scale: float = 1.0


TUNING = KernelTuningConfig()
MAX_FP8 = 448.0

# No Triton anywhere on this path (callers such as the radix cache and the
# stream pipelines read this flag to pick their route).
_HAS_TRITON = False


def build_tuning_config() -> KernelTuningConfig:
    """The reference picks Triton block sizes per CUDA architecture
    (mtp_kernels.py:91-103); the gfx950 kernels plan their own tiles, so
    this returns the defaults (fp8_scale = 1.0, the one field callers read)."""
    return KernelTuningConfig()


def fused_rmsnorm(x: torch.Tensor, weight: Optional[torch.Tensor] = None,
                  eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * weight in x.dtype, weight cast to x.dtype
    first (mtp_kernels.py:910-933)."""
    return ops.rmsnorm(x, weight, eps)


def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor,
                      weight: Optional[torch.Tensor] = None, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm of x + residual (summed in fp32), in x.dtype
    (mtp_kernels.py:1082-1102)."""
    return ops.rmsnorm(x, weight, eps, residual=residual)


def fused_rmsnorm_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
    scale: Optional[float] = None,
    *,
    gamma: Optional[torch.Tensor] = None,
    norm: bool = True,
) -> torch.Tensor:
    """((x * rsqrt(mean(x^2) + eps) [* gamma]) @ weight.T + bias) * scale in
    x.dtype (mtp_kernels.py:936-977). The bias is cast to x.dtype first, as
    the reference does (line 952)."""
    if scale is None:
        scale = TUNING.fp8_scale
    if bias is not None:
        bias = bias.to(dtype=x.dtype, device=x.device)
    return ops.rmsnorm_linear(x, weight, bias, eps, scale, gamma=gamma, norm=norm)


def fused_rmsnorm_linear_fp8(
    x: torch.Tensor,
    weight_fp8: torch.Tensor,
    wscale: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
    *,
    gamma: Optional[torch.Tensor] = None,
    norm: bool = True,
) -> torch.Tensor:
    """(x * rstd [* gamma]) @ (float(W) * wscale[:, None]).T + bias in
    x.dtype (mtp_kernels.py:1014-1044)."""
    return ops.rmsnorm_linear_fp8(x, weight_fp8, wscale, bias, eps, gamma=gamma, norm=norm)


def fused_int4_matmul(
    x: torch.Tensor,
    packed: torch.Tensor,
    scales: torch.Tensor,
    K: int,
    group: int = 32,
    *,
    nibble: str = "ref",
    gamma: Optional[torch.Tensor] = None,
    norm: bool = False,
    eps: float = 1e-6,
) -> torch.Tensor:
    """x @ dequantize_int4(packed, scales, K, group).T in x.dtype
    (mtp_kernels.py:1194-1219). nibble="ref" decodes nibble n as n - 8 (the
    reference decoder); "twos" reads two's-complement nibbles."""
    return ops.int4_matmul(x, packed, scales, K, group, nibble=nibble, gamma=gamma, norm=norm,
                           eps=eps)


def fused_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           scale: Optional[float] = None) -> torch.Tensor:
    """Single-query decode attention over every key (mtp_kernels.py:980-1011):
    q [B, H, D]; k / v [B, H, L, D]; scale defaults to 1/sqrt(D)."""
    return ops.causal_attention(q, k, v, scale)


def fused_causal_attention_fp8(q: torch.Tensor, k_fp8: torch.Tensor, v_fp8: torch.Tensor,
                               kscale: torch.Tensor, vscale: torch.Tensor,
                               scale: Optional[float] = None) -> torch.Tensor:
    """fused_causal_attention with fp8 K / V and per-head scales
    (mtp_kernels.py:1105-1133)."""
    return ops.causal_attention_fp8(q, k_fp8, v_fp8, kscale, vscale, scale)


def fused_causal_attention_autotuned(q, k, v, scale=None):
    """The reference autotunes Triton tiles over L (mtp_kernels.py:1256-1331);
    here it is the same gfx950 kernel as fused_causal_attention."""
    return ops.causal_attention(q, k, v, scale)


def fused_bitmask_attention(q, k, v, scale=None):
    """A single query at the last position sees every key, so the causal
    bitmask admits all of them; the reference delegates to
    fused_causal_attention as well (mtp_kernels.py:1426-1440)."""
    return ops.causal_attention(q, k, v, scale)


_AUTOTUNER_CACHE: dict = {}


def prewarm_autotuner(geometries: List[Tuple[int, int, int, int]]) -> None:
    """Nothing to tune (no Triton autotuner); kept for callers
    (mtp_kernels.py:1445-1457)."""
    _AUTOTUNER_CACHE["warmed"] = True


def fused_tree_attn_rmsnorm_linear(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: torch.Tensor,
    proj_w: torch.Tensor,
    rms_w: Optional[torch.Tensor] = None,
    proj_bias: Optional[torch.Tensor] = None,
    wscale: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    eps: float = 1e-6,
) -> torch.Tensor:
    """Masked single-query attention -> RMSNorm over the head dim -> linear
    (mtp_kernels.py:1222-1250, eager 881-907): out [B, H, N] in q.dtype. A
    mask with no valid key gives NaN rows, as the eager twin does, on every
    run (the reference routes to eager because its fused kernel was not
    deterministic there)."""
    return ops.tree_attn_rmsnorm_linear(q, k, v, mask, proj_w, rms_w, proj_bias, wscale, scale,
                                        eps)


def fused_paged_attention(
    q: torch.Tensor,
    k_pages: torch.Tensor,
    v_pages: torch.Tensor,
    page_table: torch.Tensor,
    page_size: int,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Single-query attention over a paged KV cache (mtp_kernels.py:1136-1162):
    q [B, H, D]; pages [P, B, H, page_size, D]; page_table [B, L]; scale
    defaults to 1/sqrt(D). Returns [B, H, D] in q's dtype."""
    return ops.paged_attention(q, k_pages, v_pages, page_table, page_size, scale)


def fused_tree_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mask: torch.Tensor,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Single-query attention with a 1-D key mask (mtp_kernels.py:1165-1191):
    q [B, H, D]; k / v [B, H, L, D]; mask [L] (> 0.5 attends)."""
    return ops.tree_attention(q, k, v, mask, scale)


def tree_verify_attention(
    q_nodes: torch.Tensor,
    k_pages: torch.Tensor,
    v_pages: torch.Tensor,
    page_table: torch.Tensor,
    page_size: int,
    k_tree: torch.Tensor,
    v_tree: torch.Tensor,
    tree_mask: torch.Tensor,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Extension: the tree-verify attention step in one launch — every
    tree node's query over the paged context and its ancestors (tree_mask
    [N, N] from SpeculativeDraftTree), one softmax per node. The reference
    composes the same result from one fused_tree_attention call per node."""
    return ops.tree_verify_attention(q_nodes, k_pages, v_pages, page_table, page_size, k_tree,
                                     v_tree, tree_mask, scale)


def quantize_fp8_e4m3(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(x_fp8, scale) with scale = amax(|x|) / 448 (1 when amax is not > 0)
    (mtp_kernels.py:704-713)."""
    return ops.quantize_fp8_tensor(x)


def quantize_fp8_rows(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Extension: per-output-channel fp8 weights, the scale rule of
    QuantScaleState.update_weight_scales (mtp_engine.py:617-622):
    (w_fp8 [N, K], wscale [N])."""
    return ops.quantize_fp8_rows(w)


def dequantize_fp8(x_fp8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32(x_fp8) * scale (mtp_kernels.py:726-727)."""
    return ops.dequantize_fp8(x_fp8, scale)


def quantize_int4(x: torch.Tensor, group: int = 32) -> Tuple[torch.Tensor, torch.Tensor]:
    """(packed uint8 [N, K/2], scales fp32 [N, ceil(K/group)]) (mtp_kernels.py:730-751)."""
    return ops.quantize_int4(x, group)


def dequantize_int4(packed: torch.Tensor, scales: torch.Tensor, K: int, group: int) -> torch.Tensor:
    """(nibble - 8) * scale as fp32 [N, K] (mtp_kernels.py:754-768)."""
    return ops.dequantize_int4(packed, scales, K, group)


def pack_scales(weight_scales: List[torch.Tensor],
                kv_scales: Optional[List[torch.Tensor]] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """One flat fp32 buffer holding every scale tensor back to back, plus the
    int64 offsets [0, n0, n0+n1, ...] (mtp_kernels.py:1336-1346)."""
    all_scales = list(weight_scales) + list(kv_scales or [])
    sizes = [int(s.numel()) for s in all_scales]
    offs = [0]
    for n in sizes:
        offs.append(offs[-1] + n)
    flat = torch.cat([s.reshape(-1).to(torch.float32) for s in all_scales])
    return flat, torch.tensor(offs, dtype=torch.int64, device=flat.device)


def unpack_scale_tensor(flat: torch.Tensor, offsets: torch.Tensor, idx: int,
                        shape: Tuple[int, ...]) -> torch.Tensor:
    """View of scale tensor ``idx`` inside the packed buffer
    (mtp_kernels.py:1349-1353)."""
    start, end = int(offsets[idx]), int(offsets[idx + 1])
    return flat[start:end].view(*shape)


__all__ = [
    "KernelTuningConfig",
    "TUNING",
    "MAX_FP8",
    "build_tuning_config",
    "fused_rmsnorm",
    "fused_add_rmsnorm",
    "fused_rmsnorm_linear",
    "fused_causal_attention",
    "fused_causal_attention_autotuned",
    "fused_rmsnorm_linear_fp8",
    "fused_causal_attention_fp8",
    "fused_paged_attention",
    "fused_tree_attention",
    "fused_tree_attn_rmsnorm_linear",
    "fused_int4_matmul",
    "fused_bitmask_attention",
    "pack_scales",
    "unpack_scale_tensor",
    "prewarm_autotuner",
    "quantize_fp8_e4m3",
    "dequantize_fp8",
    "quantize_int4",
    "dequantize_int4",
    "_HAS_TRITON",
]
