"""Drop-in for the reference module ``mtp_kernels`` (RMSNorm -> linear family)
on MI355X.

Same names, argument order, defaults and return values as the reference's
wrappers (mtp_kernels.py:936-977, 1014-1044, 1194-1219, 1336-1353); every
entry point launches a hand-written gfx950 kernel through libmtp_hip.so.
Keyword-only extensions: ``gamma`` (RMSNorm weight, default None = the
reference) and ``norm`` (False = plain linear, the mode CachedLinear needs)
on the RMSNorm -> linear entry points; ``nibble``, ``gamma``, ``norm`` and
``eps`` on fused_int4_matmul (default = the reference: offset-8 nibbles, no
norm).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from mtp_hip import ops


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
    "fused_rmsnorm_linear",
    "fused_rmsnorm_linear_fp8",
    "fused_int4_matmul",
    "pack_scales",
    "unpack_scale_tensor",
]
