"""Tensor-level entry points over the C ABI.

Each function canonicalises its inputs the way the reference's wrapper does
(.contiguous(), dtype of the output = dtype of x, draft ids as int32),
allocates the outputs with the torch allocator, takes the per-stream
workspace and enqueues the kernel on torch's current stream without
synchronising. Inputs must live on a HIP device.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import check, code, ptr

_FLOATS = (torch.float32, torch.bfloat16, torch.float16)


def _on_device(name: str, t: torch.Tensor, **others) -> None:
    """Every tensor handed to the library must live on the same HIP device:
    a host tensor's data_ptr() is not a device address."""
    if t.device.type != "cuda":
        raise RuntimeError(f"mtp_hip: {name} must be on a HIP device (got {t.device})")
    for k, o in others.items():
        if o is not None and o.device != t.device:
            raise RuntimeError(f"mtp_hip: {k} is on {o.device}, expected {t.device} like {name}")


def rmsnorm_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                   eps: float = 1e-6, scale: float = 1.0, gamma: Optional[torch.Tensor] = None,
                   norm: bool = True) -> torch.Tensor:
    """y = ((x * rstd * gamma) @ weight.T + bias) * scale, cast to x.dtype."""
    lib = _lib.load()
    x = x.contiguous()
    weight = weight.contiguous()
    assert x.dim() == 2 and weight.dim() == 2, "fused_rmsnorm_linear: x and weight must be 2-D"
    M, K = x.shape
    N, K2 = weight.shape
    assert K == K2, f"fused_rmsnorm_linear: K mismatch {K} vs {K2}"
    if bias is not None:
        bias = bias.contiguous()
        assert bias.numel() == N, f"fused_rmsnorm_linear: bias has {bias.numel()} != {N}"
    if gamma is not None:
        gamma = gamma.contiguous().to(torch.float32)
        assert gamma.numel() == K, f"fused_rmsnorm_linear: gamma has {gamma.numel()} != {K}"
    _on_device("x", x, weight=weight, bias=bias, gamma=gamma)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    nbytes = lib.mtp_rmsnorm_linear_workspace_bytes(code(x.dtype), code(weight.dtype), M, N, K)
    ws = _lib.workspace(x.device, nbytes)
    st = lib.mtp_fused_rmsnorm_linear(
        ptr(x), code(x.dtype), M, K, ptr(weight), code(weight.dtype), N,
        ptr(bias), code(bias.dtype) if bias is not None else 0,
        ptr(gamma), code(gamma.dtype) if gamma is not None else 0,
        float(eps), float(scale), int(bool(norm)), ptr(y), ptr(ws), nbytes,
        _lib.stream_handle(x.device))
    check(st, "fused_rmsnorm_linear")
    return y


def rmsnorm_linear_fp8(x: torch.Tensor, weight_fp8: torch.Tensor, wscale: torch.Tensor,
                       bias: Optional[torch.Tensor] = None, eps: float = 1e-6,
                       gamma: Optional[torch.Tensor] = None, norm: bool = True) -> torch.Tensor:
    """y = ((x * rstd * gamma) @ (W * wscale[:, None]).T + bias), cast to x.dtype."""
    lib = _lib.load()
    x = x.contiguous()
    weight_fp8 = weight_fp8.contiguous()
    wscale = wscale.contiguous().to(torch.float32)
    assert x.dim() == 2 and weight_fp8.dim() == 2, "fused_rmsnorm_linear_fp8: 2-D x and weight"
    M, K = x.shape
    N, K2 = weight_fp8.shape
    assert K == K2, f"fused_rmsnorm_linear_fp8: K mismatch {K} vs {K2}"
    assert wscale.numel() == N, f"fused_rmsnorm_linear_fp8: wscale has {wscale.numel()} != {N}"
    if bias is not None:
        bias = bias.contiguous()
        assert bias.numel() == N, f"fused_rmsnorm_linear_fp8: bias has {bias.numel()} != {N}"
    if gamma is not None:
        gamma = gamma.contiguous().to(torch.float32)
        assert gamma.numel() == K, f"fused_rmsnorm_linear_fp8: gamma has {gamma.numel()} != {K}"
    _on_device("x", x, weight=weight_fp8, wscale=wscale, bias=bias, gamma=gamma)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    # The reference accepts any weight dtype here (its self-test passes fp32
    # values in +-448); the library takes the weight dtype as given.
    wcode = code(weight_fp8.dtype)
    nbytes = lib.mtp_rmsnorm_linear_workspace_bytes(code(x.dtype), wcode, M, N, K)
    ws = _lib.workspace(x.device, nbytes)
    st = lib.mtp_fused_rmsnorm_linear_fp8(
        ptr(x), code(x.dtype), M, K, ptr(weight_fp8), wcode, ptr(wscale), N,
        ptr(bias), code(bias.dtype) if bias is not None else 0,
        ptr(gamma), code(gamma.dtype) if gamma is not None else 0,
        float(eps), int(bool(norm)), ptr(y), ptr(ws), nbytes, _lib.stream_handle(x.device))
    check(st, "fused_rmsnorm_linear_fp8")
    return y


def int4_matmul(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, K: int,
                group: int = 32, nibble: str = "ref", gamma: Optional[torch.Tensor] = None,
                norm: bool = False, eps: float = 1e-6) -> torch.Tensor:
    """y = (xn @ dequant(packed, scales).T) cast to x.dtype; xn = x (norm=False)."""
    lib = _lib.load()
    x = x.contiguous()
    packed = packed.contiguous()
    scales = scales.contiguous()
    assert x.dim() == 2 and packed.dim() == 2 and scales.dim() == 2, "fused_int4_matmul: 2-D inputs"
    M, K2 = x.shape
    assert K2 == K, f"fused_int4_matmul: K mismatch {K2} vs {K}"
    N = packed.shape[0]
    assert packed.dtype == torch.uint8 and packed.shape[1] == K // 2, \
        f"fused_int4_matmul: packed must be uint8 [N, K/2], got {tuple(packed.shape)}"
    ng = (K + group - 1) // group
    assert tuple(scales.shape) == (N, ng), \
        f"fused_int4_matmul: scales must be [N, ceil(K/group)] = {(N, ng)}, got {tuple(scales.shape)}"
    if gamma is not None:
        gamma = gamma.contiguous()
        assert gamma.numel() == K, f"fused_int4_matmul: gamma has {gamma.numel()} != {K}"
    _on_device("x", x, packed=packed, scales=scales, gamma=gamma)
    mode = {"ref": _lib.NIBBLE_OFFSET8, "offset": _lib.NIBBLE_OFFSET8,
            "twos": _lib.NIBBLE_TWOS}[nibble]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    nbytes = lib.mtp_rmsnorm_linear_workspace_bytes(code(x.dtype), _lib.U8, M, N, K)
    ws = _lib.workspace(x.device, nbytes)
    st = lib.mtp_fused_int4_matmul(
        ptr(x), code(x.dtype), M, K, ptr(packed), ptr(scales), code(scales.dtype), N, int(group),
        mode, ptr(gamma), code(gamma.dtype) if gamma is not None else 0, float(eps),
        int(bool(norm)), ptr(y), ptr(ws), nbytes, _lib.stream_handle(x.device))
    check(st, "fused_int4_matmul")
    return y


def verify(hidden: torch.Tensor, weight: torch.Tensor, draft: torch.Tensor,
           bias: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(accept int8 [M], top int32 [M]) with top = argmax(hidden @ W.T + bias)."""
    lib = _lib.load()
    hidden = hidden.contiguous()
    weight = weight.contiguous()
    draft = draft.contiguous().to(torch.int32)
    assert hidden.dim() == 2 and weight.dim() == 2, "fused_verify: 2-D hidden and weight"
    M, K = hidden.shape
    V = weight.shape[0]
    assert weight.shape[1] == K, f"fused_verify: K mismatch {K} vs {weight.shape[1]}"
    assert draft.numel() == M, f"fused_verify: draft has {draft.numel()} != {M}"
    if bias is not None:
        bias = bias.contiguous()
        assert bias.numel() == V, f"fused_verify: bias has {bias.numel()} != {V}"
    _on_device("hidden", hidden, weight=weight, draft=draft, bias=bias)
    accept = torch.empty(M, dtype=torch.int8, device=hidden.device)
    top = torch.empty(M, dtype=torch.int32, device=hidden.device)
    nbytes = lib.mtp_verify_workspace_bytes(code(hidden.dtype), M, 1, V, K)
    ws = _lib.workspace(hidden.device, nbytes)
    st = lib.mtp_fused_verify(
        ptr(hidden), code(hidden.dtype), M, K, ptr(weight), code(weight.dtype), V,
        ptr(bias), code(bias.dtype) if bias is not None else 0, ptr(draft), ptr(accept), ptr(top),
        ptr(ws), nbytes, _lib.stream_handle(hidden.device))
    check(st, "fused_verify")
    return accept, top


def multi_verify(hidden: torch.Tensor, weight: torch.Tensor, draft: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, return_top: bool = False):
    """(accept int8 [B, D], accepted_n int32 [B], corrected int32 [B][, top int32 [B, S]])."""
    lib = _lib.load()
    hidden = hidden.contiguous()
    weight = weight.contiguous()
    draft = draft.contiguous().to(torch.int32)
    assert hidden.dim() == 3 and weight.dim() == 2 and draft.dim() == 2, \
        "fused_multi_verify: hidden [B, S, K], weight [V, K], draft [B, D]"
    B, S, K = hidden.shape
    V = weight.shape[0]
    D = draft.shape[1]
    assert S == D + 1, f"expected S == D + 1, got S={S} D={D}"
    assert weight.shape[1] == K, f"fused_multi_verify: K mismatch {K} vs {weight.shape[1]}"
    assert draft.shape[0] == B, f"fused_multi_verify: draft rows {draft.shape[0]} != B={B}"
    if bias is not None:
        bias = bias.contiguous()
        assert bias.numel() == V, f"fused_multi_verify: bias has {bias.numel()} != {V}"
    _on_device("hidden", hidden, weight=weight, draft=draft, bias=bias)
    dev = hidden.device
    accept = torch.empty((B, D), dtype=torch.int8, device=dev)
    accepted_n = torch.empty((B,), dtype=torch.int32, device=dev)
    corrected = torch.empty((B,), dtype=torch.int32, device=dev)
    top = torch.empty((B, S), dtype=torch.int32, device=dev) if return_top else None
    nbytes = lib.mtp_verify_workspace_bytes(code(hidden.dtype), B * S, S, V, K)
    ws = _lib.workspace(dev, nbytes)
    st = lib.mtp_fused_multi_verify(
        ptr(hidden), code(hidden.dtype), B, S, K, ptr(weight), code(weight.dtype), V,
        ptr(bias), code(bias.dtype) if bias is not None else 0, ptr(draft), D, ptr(accept),
        ptr(accepted_n), ptr(corrected), ptr(top), ptr(ws), nbytes, _lib.stream_handle(dev))
    check(st, "fused_multi_verify")
    if return_top:
        return accept, accepted_n, corrected, top
    return accept, accepted_n, corrected


def _mask_arg(mask: torch.Tensor) -> torch.Tensor:
    mask = mask.contiguous()
    if mask.dtype == torch.bool:
        mask = mask.to(torch.uint8)
    if mask.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.uint8):
        mask = mask.to(torch.float32)
    return mask


def _attn_call(fn_name: str, q: torch.Tensor, B: int, NQ: int, H: int, D: int, Lc: int, Lt: int,
               *args) -> None:
    lib = _lib.load()
    nbytes = lib.mtp_attention_workspace_bytes(code(q.dtype), B, NQ, H, D, Lc, Lt)
    ws = _lib.workspace(q.device, nbytes)
    st = getattr(lib, fn_name)(*args, ptr(ws), nbytes, _lib.stream_handle(q.device))
    check(st, fn_name[4:])


def paged_attention(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                    page_table: torch.Tensor, page_size: int, scale: Optional[float] = None):
    """out[b, h] = softmax_t(q . k_t * scale) @ v_t over the paged keys of b."""
    q = q.contiguous()
    k_pages = k_pages.contiguous()
    v_pages = v_pages.contiguous()
    page_table = page_table.contiguous().to(torch.int32)
    assert q.dim() == 3, "fused_paged_attention: q [B, H, D]"
    B, H, D = q.shape
    L = page_table.shape[-1]
    assert k_pages.dim() == 5 and tuple(k_pages.shape[1:3]) == (B, H) and \
        k_pages.shape[3] == page_size and k_pages.shape[4] == D, \
        f"fused_paged_attention: pages must be [P, {B}, {H}, {page_size}, {D}], got {tuple(k_pages.shape)}"
    assert v_pages.shape == k_pages.shape, "fused_paged_attention: k_pages / v_pages differ"
    assert page_table.dim() == 2 and page_table.shape[0] == B, \
        f"fused_paged_attention: page_table must be [{B}, L]"
    assert k_pages.dtype == q.dtype and v_pages.dtype == q.dtype, "fused_paged_attention: dtypes differ"
    _on_device("q", q, k_pages=k_pages, v_pages=v_pages, page_table=page_table)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    _attn_call("mtp_fused_paged_attention", q, B, 1, H, D, L, 0,
               ptr(q), code(q.dtype), B, H, D, ptr(k_pages), ptr(v_pages), k_pages.shape[0],
               ptr(page_table), L, int(page_size), float(scale), ptr(out))
    return out


def tree_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor,
                   scale: Optional[float] = None):
    """out[b, h] = softmax_l(q . k_l * scale where mask[l] > 0.5 else -inf) @ v_l."""
    q = q.contiguous()
    k = k.contiguous()
    v = v.contiguous()
    mask = _mask_arg(mask)
    assert q.dim() == 3 and k.dim() == 4, "fused_tree_attention: q [B, H, D], k / v [B, H, L, D]"
    B, H, D = q.shape
    L = k.shape[2]
    assert tuple(k.shape) == (B, H, L, D) and v.shape == k.shape, \
        f"fused_tree_attention: k / v must be [{B}, {H}, L, {D}], got {tuple(k.shape)}"
    assert mask.numel() == L, f"fused_tree_attention: mask has {mask.numel()} != {L}"
    assert k.dtype == q.dtype and v.dtype == q.dtype, "fused_tree_attention: dtypes differ"
    _on_device("q", q, k=k, v=v, mask=mask)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    _attn_call("mtp_fused_tree_attention", q, B, 1, H, D, 0, L,
               ptr(q), code(q.dtype), B, H, D, ptr(k), ptr(v), L, ptr(mask), code(mask.dtype),
               float(scale), ptr(out))
    return out


def tree_verify_attention(q_nodes: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                          page_table: torch.Tensor, page_size: int, k_tree: torch.Tensor,
                          v_tree: torch.Tensor, tree_mask: torch.Tensor,
                          scale: Optional[float] = None):
    """Every tree node's query over the paged context plus its masked tree
    nodes, under one softmax: out [N, H, D]."""
    q_nodes = q_nodes.contiguous()
    k_tree = k_tree.contiguous()
    v_tree = v_tree.contiguous()
    k_pages = k_pages.contiguous()
    v_pages = v_pages.contiguous()
    page_table = page_table.contiguous().to(torch.int32)
    tree_mask = _mask_arg(tree_mask)
    assert q_nodes.dim() == 3, "tree_verify_attention: q_nodes [N, H, D]"
    N, H, D = q_nodes.shape
    Lc = page_table.shape[-1]
    assert tuple(k_tree.shape) == (N, H, D) and v_tree.shape == k_tree.shape, \
        "tree_verify_attention: k_tree / v_tree must be [N, H, D]"
    assert tuple(tree_mask.shape) == (N, N), "tree_verify_attention: tree_mask must be [N, N]"
    assert k_pages.dim() == 5 and k_pages.shape[1] == 1 and k_pages.shape[2] == H and \
        k_pages.shape[3] == page_size and k_pages.shape[4] == D and v_pages.shape == k_pages.shape, \
        "tree_verify_attention: pages must be [P, 1, H, page_size, D]"
    assert page_table.numel() == Lc, "tree_verify_attention: page_table [1, Lc]"
    for t in (k_tree, v_tree, k_pages, v_pages):
        assert t.dtype == q_nodes.dtype, "tree_verify_attention: dtypes differ"
    _on_device("q_nodes", q_nodes, k_tree=k_tree, v_tree=v_tree, k_pages=k_pages,
               v_pages=v_pages, page_table=page_table, tree_mask=tree_mask)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q_nodes)
    _attn_call("mtp_tree_verify_attention", q_nodes, 1, N, H, D, Lc, N,
               ptr(q_nodes), code(q_nodes.dtype), N, H, D, ptr(k_pages), ptr(v_pages),
               k_pages.shape[0], ptr(page_table), Lc, int(page_size), ptr(k_tree), ptr(v_tree),
               ptr(tree_mask), code(tree_mask.dtype), float(scale), ptr(out))
    return out


def quantize_fp8_tensor(x: torch.Tensor):
    """(x_fp8, scale): per-tensor amax / 448 scale and e4m3fn values."""
    lib = _lib.load()
    x = x.contiguous()
    _on_device("x", x)
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    n = x.numel()
    assert n > 0, "quantize_fp8_e4m3: empty tensor"
    nbytes = lib.mtp_quantize_workspace_bytes(n)
    ws = _lib.workspace(x.device, nbytes)
    st = lib.mtp_quantize_fp8_e4m3(ptr(x), code(x.dtype), n, ptr(q), ptr(scale), ptr(ws), nbytes,
                                   _lib.stream_handle(x.device))
    check(st, "quantize_fp8_e4m3")
    return q, scale


def quantize_fp8_rows(w: torch.Tensor):
    """(w_fp8 [N, K], wscale [N]): per-row amax / 448 scales (0 -> 1)."""
    lib = _lib.load()
    w = w.contiguous()
    assert w.dim() == 2, "quantize_fp8_rows: w [N, K]"
    _on_device("w", w)
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.float8_e4m3fn, device=w.device)
    s = torch.empty((N,), dtype=torch.float32, device=w.device)
    st = lib.mtp_quantize_fp8_rows(ptr(w), code(w.dtype), N, K, ptr(q), ptr(s),
                                   _lib.stream_handle(w.device))
    check(st, "quantize_fp8_rows")
    return q, s


def dequantize_fp8(x_fp8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32(x_fp8) * scale for a one-element scale or a per-row [rows, 1] scale."""
    lib = _lib.load()
    x_fp8 = x_fp8.contiguous()
    scale = scale.contiguous().to(torch.float32)
    _on_device("x_fp8", x_fp8, scale=scale)
    out = torch.empty(x_fp8.shape, dtype=torch.float32, device=x_fp8.device)
    if scale.numel() == 1:
        per_row, row_len = 0, 1
    else:
        assert x_fp8.dim() >= 2 and scale.dim() == x_fp8.dim() and scale.shape[-1] == 1 and \
            scale.numel() == x_fp8.numel() // x_fp8.shape[-1], \
            "dequantize_fp8: scale must be one value or [rows, 1]"
        per_row, row_len = 1, x_fp8.shape[-1]
    st = lib.mtp_dequantize_fp8(ptr(x_fp8), x_fp8.numel(), row_len, ptr(scale), per_row, ptr(out),
                                _lib.stream_handle(x_fp8.device))
    check(st, "dequantize_fp8")
    return out


def quantize_int4(x: torch.Tensor, group: int = 32):
    """(packed u8 [N, K/2], scales fp32 [N, ceil(K/group)])."""
    lib = _lib.load()
    x = x.contiguous()
    assert x.dim() == 2, "quantize_int4: x [N, K]"
    _on_device("x", x)
    N, K = x.shape
    ng = (K + group - 1) // group
    packed = torch.empty((N, K // 2), dtype=torch.uint8, device=x.device)
    scales = torch.empty((N, ng), dtype=torch.float32, device=x.device)
    st = lib.mtp_quantize_int4(ptr(x), code(x.dtype), N, K, int(group), ptr(packed), ptr(scales),
                               _lib.stream_handle(x.device))
    check(st, "quantize_int4")
    return packed, scales


def dequantize_int4(packed: torch.Tensor, scales: torch.Tensor, K: int, group: int) -> torch.Tensor:
    """(nibble - 8) * scales[n, k // group] as fp32 [N, K]."""
    lib = _lib.load()
    packed = packed.contiguous()
    scales = scales.contiguous()
    _on_device("packed", packed, scales=scales)
    N = packed.shape[0]
    assert packed.dtype == torch.uint8 and packed.shape[1] == K // 2, \
        f"dequantize_int4: packed must be uint8 [N, {K // 2}]"
    assert tuple(scales.shape) == (N, (K + group - 1) // group), "dequantize_int4: scales shape"
    out = torch.empty((N, K), dtype=torch.float32, device=packed.device)
    st = lib.mtp_dequantize_int4(ptr(packed), ptr(scales), code(scales.dtype), N, K, int(group),
                                 ptr(out), _lib.stream_handle(packed.device))
    check(st, "dequantize_int4")
    return out
