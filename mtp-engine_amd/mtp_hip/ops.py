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


def verify_route(hidden: torch.Tensor, weight: torch.Tensor,
                 bias: Optional[torch.Tensor] = None) -> str:
    """Which kernel a verify call on these tensors takes: "stream" (the
    persistent W-streaming kernel), "column_group" or "generic". hidden is
    [M, K] (fused_verify) or [B, S, K] (fused_multi_verify); nothing runs."""
    lib = _lib.load()
    if hidden.dim() == 3:
        B, S, K = hidden.shape
        rows, seq = B * S, S
    else:
        (rows, K), seq = hidden.shape, 1
    r = lib.mtp_verify_route(ptr(hidden), code(hidden.dtype), rows, seq, K, ptr(weight),
                             code(weight.dtype), weight.shape[0], ptr(bias))
    if r < 0:
        check(r, "verify_route")
    return {_lib.VERIFY_ROUTE_STREAM: "stream", _lib.VERIFY_ROUTE_COLUMN_GROUP: "column_group",
            _lib.VERIFY_ROUTE_GENERIC: "generic"}[r]


_CONVENTIONS = ("reference", "textbook")


def multi_verify(hidden: torch.Tensor, weight: torch.Tensor, draft: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, return_top: bool = False,
                 convention: str = "reference"):
    """(accept int8 [B, D], accepted_n int32 [B], corrected int32 [B][, top int32 [B, S]]).
    convention: "reference" (draft d against top[:, d + 1], corrected =
    top[:, 0]) or "textbook" (draft d against top[:, d], corrected =
    top[b, accepted_n[b]])."""
    if convention not in _CONVENTIONS:
        raise ValueError(f"fused_multi_verify: convention must be one of {_CONVENTIONS}")
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
    fn = lib.mtp_fused_multi_verify if convention == "reference" else \
        lib.mtp_fused_multi_verify_textbook
    st = fn(
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


# ---------------------------------------------------------------------------
# Draft chain
def rmsnorm(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6,
            residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """(x [+ residual]) * rsqrt(mean(.^2) + eps) * weight over the last dim of
    a 2-D x, in x.dtype. The weight is cast to x.dtype first, as the
    reference's wrappers do (mtp_kernels.py:918-920, 1088-1090)."""
    lib = _lib.load()
    x = x.contiguous()
    assert x.dim() == 2, "fused_rmsnorm: x must be 2-D [M, N]"
    M, N = x.shape
    if weight is not None:
        weight = weight.contiguous().to(dtype=x.dtype, device=x.device)
        assert weight.numel() == N, f"fused_rmsnorm: weight has {weight.numel()} != {N}"
    if residual is not None:
        residual = residual.contiguous()
        assert residual.shape == x.shape, "fused_add_rmsnorm: residual shape differs from x"
        if residual.dtype != x.dtype:
            residual = residual.to(x.dtype)
    _on_device("x", x, weight=weight, residual=residual)
    y = torch.empty_like(x)
    wcode = code(weight.dtype) if weight is not None else 0
    st = _lib.stream_handle(x.device)
    if residual is None:
        s = lib.mtp_fused_rmsnorm(ptr(x), code(x.dtype), M, N, ptr(weight), wcode, float(eps),
                                  ptr(y), st)
        check(s, "fused_rmsnorm")
    else:
        s = lib.mtp_fused_add_rmsnorm(ptr(x), ptr(residual), code(x.dtype), M, N, ptr(weight),
                                      wcode, float(eps), ptr(y), st)
        check(s, "fused_add_rmsnorm")
    return y


def argmax(logits: torch.Tensor, emb_table: Optional[torch.Tensor] = None):
    """torch.argmax(logits, dim=-1) (int64; NaN is the maximum, the lowest
    index wins ties) over a 2-D (or 1-D) float tensor; with emb_table
    [V', H] also returns emb_table[tokens] from the same launch."""
    lib = _lib.load()
    one_d = logits.dim() == 1
    lg = logits.reshape(1, -1) if one_d else logits
    assert lg.dim() == 2, "argmax: logits must be 1-D or 2-D"
    if lg.stride(-1) != 1:
        lg = lg.contiguous()
    M, V = lg.shape
    ld = lg.stride(0) if M > 1 else V
    _on_device("logits", lg, emb_table=emb_table)
    tokens = torch.empty((M,), dtype=torch.int64, device=lg.device)
    emb = None
    if emb_table is not None:
        emb_table = emb_table.contiguous()
        assert emb_table.dim() == 2, "argmax: emb_table must be [V, H]"
        emb = torch.empty((M, emb_table.shape[1]), dtype=emb_table.dtype, device=lg.device)
    nbytes = lib.mtp_argmax_workspace_bytes(M, V)
    ws = _lib.workspace(lg.device, nbytes)
    s = lib.mtp_argmax(ptr(lg), code(lg.dtype), M, V, ld, ptr(tokens), ptr(emb_table),
                       code(emb_table.dtype) if emb_table is not None else 0,
                       emb_table.shape[0] if emb_table is not None else 0,
                       emb_table.shape[1] if emb_table is not None else 0, ptr(emb), ptr(ws),
                       nbytes, _lib.stream_handle(lg.device))
    check(s, "argmax")
    if one_d:
        tokens = tokens.reshape(())
        emb = emb.reshape(-1) if emb is not None else None
    return tokens if emb_table is None else (tokens, emb)


# ---------------------------------------------------------------------------
# Decode attention and the tree monolith
def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     scale: Optional[float] = None) -> torch.Tensor:
    """out[b, h] = softmax_l(q . k_l * scale) @ v_l (a single query that
    attends every key): q [B, H, D], k / v [B, H, L, D]."""
    lib = _lib.load()
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    B, H, D = q.shape
    _B, _H, L, _D = k.shape
    assert B == _B and H == _H and D == _D
    assert v.shape == k.shape and k.dtype == q.dtype and v.dtype == q.dtype, \
        "fused_causal_attention: k / v shape or dtype differs"
    _on_device("q", q, k=k, v=v)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    nbytes = lib.mtp_attention_workspace_bytes(code(q.dtype), B, 1, H, D, 0, L)
    ws = _lib.workspace(q.device, nbytes)
    s = lib.mtp_fused_causal_attention(ptr(q), code(q.dtype), B, H, D, ptr(k), ptr(v), L,
                                       float(scale), ptr(out), ptr(ws), nbytes,
                                       _lib.stream_handle(q.device))
    check(s, "fused_causal_attention")
    return out


def causal_attention_fp8(q: torch.Tensor, k_fp8: torch.Tensor, v_fp8: torch.Tensor,
                         kscale: torch.Tensor, vscale: torch.Tensor,
                         scale: Optional[float] = None) -> torch.Tensor:
    """causal_attention with fp8 e4m3fn K / V dequantised per head by kscale
    [H] / vscale [H]."""
    lib = _lib.load()
    q, k_fp8, v_fp8 = q.contiguous(), k_fp8.contiguous(), v_fp8.contiguous()
    kscale = kscale.contiguous().to(torch.float32)
    vscale = vscale.contiguous().to(torch.float32)
    B, H, D = q.shape
    _B, _H, L, _D = k_fp8.shape
    assert (B, H, D) == (_B, _H, _D)
    assert v_fp8.shape == k_fp8.shape, "fused_causal_attention_fp8: v shape differs from k"
    assert k_fp8.dtype == torch.float8_e4m3fn and v_fp8.dtype == torch.float8_e4m3fn, \
        "fused_causal_attention_fp8: k / v must be float8_e4m3fn"
    assert kscale.numel() == H and vscale.numel() == H, "fused_causal_attention_fp8: scales [H]"
    _on_device("q", q, k_fp8=k_fp8, v_fp8=v_fp8, kscale=kscale, vscale=vscale)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    s = lib.mtp_fused_causal_attention_fp8(ptr(q), code(q.dtype), B, H, D, ptr(k_fp8),
                                           ptr(v_fp8), L, ptr(kscale), ptr(vscale), float(scale),
                                           ptr(out), _lib.stream_handle(q.device))
    check(s, "fused_causal_attention_fp8")
    return out


def tree_attn_rmsnorm_linear(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             mask: torch.Tensor, proj_w: torch.Tensor,
                             rms_w: Optional[torch.Tensor] = None,
                             proj_bias: Optional[torch.Tensor] = None,
                             wscale: Optional[torch.Tensor] = None,
                             scale: Optional[float] = None, eps: float = 1e-6) -> torch.Tensor:
    """Masked single-query attention, RMSNorm over the head dim (gamma
    rms_w), projection onto proj_w [N, D] (times wscale [N]) plus proj_bias:
    out [B, H, N] in q's dtype."""
    lib = _lib.load()
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    mask = _mask_arg(mask)
    proj_w = proj_w.contiguous()
    B, H, D = q.shape
    L = k.shape[2]
    N = proj_w.shape[0]
    assert tuple(k.shape) == (B, H, L, D) and v.shape == k.shape, \
        "fused_tree_attn_rmsnorm_linear: k / v must be [B, H, L, D]"
    assert k.dtype == q.dtype and v.dtype == q.dtype, "fused_tree_attn_rmsnorm_linear: dtypes"
    assert mask.numel() == L, f"fused_tree_attn_rmsnorm_linear: mask has {mask.numel()} != {L}"
    assert proj_w.dim() == 2 and proj_w.shape[1] == D, "fused_tree_attn_rmsnorm_linear: proj_w [N, D]"
    if rms_w is not None:
        rms_w = rms_w.contiguous().to(torch.float32)
        assert rms_w.numel() == D
    if proj_bias is not None:
        proj_bias = proj_bias.contiguous()
        assert proj_bias.numel() == N
    if wscale is not None:
        wscale = wscale.contiguous().to(torch.float32)
        assert wscale.numel() == N
    _on_device("q", q, k=k, v=v, mask=mask, proj_w=proj_w, rms_w=rms_w, proj_bias=proj_bias,
               wscale=wscale)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty((B, H, N), dtype=q.dtype, device=q.device)
    wkind = _lib.FP8E4M3 if wscale is not None else code(proj_w.dtype)
    nbytes = lib.mtp_tree_attn_rmsnorm_linear_workspace_bytes(code(q.dtype), B, H, D, L, wkind, N)
    ws = _lib.workspace(q.device, nbytes)
    s = lib.mtp_fused_tree_attn_rmsnorm_linear(
        ptr(q), code(q.dtype), B, H, D, ptr(k), ptr(v), L, ptr(mask), code(mask.dtype),
        ptr(proj_w), code(proj_w.dtype), N, ptr(rms_w), _lib.F32 if rms_w is not None else 0,
        ptr(proj_bias), code(proj_bias.dtype) if proj_bias is not None else 0, ptr(wscale),
        float(scale), float(eps), ptr(out), ptr(ws), nbytes, _lib.stream_handle(q.device))
    check(s, "fused_tree_attn_rmsnorm_linear")
    return out


# ---------------------------------------------------------------------------
# KV step after verify
def paged_kv_write(k_new: torch.Tensor, v_new: torch.Tensor, k_pages: torch.Tensor,
                   v_pages: torch.Tensor, page_table: torch.Tensor, start) -> None:
    """Write the K / V rows of T new tokens into their pages, in place:
    pages[table[b, p], b, h, p % page_size] = new[b, h, t], p = start + t.
    k_new / v_new [B, H, T, D] (any strides with d contiguous); pages
    [P, B, H, page_size, D]; page_table [B, L] int32; start an int, or an
    int64 device tensor of one element (shared) or [B] (per row)."""
    lib = _lib.load()
    assert k_new.dim() == 4 and v_new.shape == k_new.shape, "paged_kv_write: new K / V [B, H, T, D]"
    if k_new.stride(-1) != 1:
        k_new = k_new.contiguous()
    if v_new.stride(-1) != 1 or v_new.stride() != k_new.stride():
        v_new = v_new.contiguous()
        k_new = k_new.contiguous()
    B, H, T, D = k_new.shape
    assert k_pages.is_contiguous() and v_pages.is_contiguous() and v_pages.shape == k_pages.shape, \
        "paged_kv_write: pages must be contiguous [P, B, H, page_size, D]"
    P, _B, _H, ps, _D = k_pages.shape
    assert (_B, _H, _D) == (B, H, D), "paged_kv_write: pages do not match the new rows"
    page_table = page_table.contiguous().to(torch.int32)
    assert page_table.dim() == 2 and page_table.shape[0] == B, "paged_kv_write: page_table [B, L]"
    start_dev, per_row, start_host = None, 0, 0
    if torch.is_tensor(start):
        start_dev = start.contiguous().to(torch.int64)
        assert start_dev.numel() in (1, B), "paged_kv_write: start must hold 1 or B positions"
        per_row = int(start_dev.numel() == B and B > 1)
    else:
        start_host = int(start)
    _on_device("k_new", k_new, v_new=v_new, k_pages=k_pages, v_pages=v_pages,
               page_table=page_table, start=start_dev)
    sb, sh, st_, _ = k_new.stride()
    s = lib.mtp_paged_kv_write(ptr(k_new), ptr(v_new), code(k_new.dtype), B, T, H, D, sb, st_, sh,
                               ptr(k_pages), ptr(v_pages), code(k_pages.dtype), P, ps,
                               ptr(page_table), page_table.shape[1], ptr(start_dev), per_row,
                               start_host, _lib.stream_handle(k_new.device))
    check(s, "paged_kv_write")


def verify_commit(accept: torch.Tensor, accepted_n: torch.Tensor, corrected: torch.Tensor,
                  draft: torch.Tensor, checkpoint: torch.Tensor, kv_len: torch.Tensor,
                  ids: Optional[torch.Tensor] = None, ids_len: Optional[torch.Tensor] = None):
    """The engine's verify consumer on the device (no host reads): returns
    (tokens [B, D + 1] int64, -1 past the width; width int32 [1]) and sets
    kv_len = checkpoint + width (int64 device scalars; they may be the same
    tensor); with ids [B, cap] int64 (contiguous) and ids_len (int64
    scalar) the tokens are appended at ids_len, which advances by the width,
    or by fewer where the buffer is full (ids_len never passes cap)."""
    lib = _lib.load()
    B, D = draft.shape
    accept = accept.contiguous().to(torch.int8)
    accepted_n = accepted_n.contiguous().to(torch.int32)
    corrected = corrected.contiguous().to(torch.int32)
    draft = draft.contiguous()
    if draft.dtype not in (torch.int32, torch.int64):
        draft = draft.to(torch.int64)
    for name, t in (("checkpoint", checkpoint), ("kv_len", kv_len)):
        assert t.dtype == torch.int64 and t.numel() == 1 and t.is_contiguous(), \
            f"verify_commit: {name} must be a contiguous int64 device scalar"
    if ids is not None:
        assert ids.dtype == torch.int64 and ids.dim() == 2 and ids.shape[0] == B and \
            ids.is_contiguous(), "verify_commit: ids must be a contiguous int64 [B, cap]"
        assert ids_len is not None and ids_len.dtype == torch.int64 and ids_len.numel() == 1
    _on_device("accepted_n", accepted_n, accept=accept, corrected=corrected, draft=draft,
               checkpoint=checkpoint, kv_len=kv_len, ids=ids, ids_len=ids_len)
    dev = accepted_n.device
    tokens = torch.empty((B, D + 1), dtype=torch.int64, device=dev)
    width = torch.empty((1,), dtype=torch.int32, device=dev)
    s = lib.mtp_verify_commit(ptr(accept), ptr(accepted_n), ptr(corrected), ptr(draft),
                              code(draft.dtype), B, D, ptr(checkpoint), ptr(kv_len), ptr(tokens),
                              ptr(width), ptr(ids), ids.stride(0) if ids is not None else 0,
                              ptr(ids_len), _lib.stream_handle(dev))
    check(s, "verify_commit")
    return tokens, width


def batch_prefix_match(ids: torch.Tensor) -> torch.Tensor:
    """int32 [R]: per row the length of the prefix it shares with row 0 (L
    for a full match; zeros when R <= 1)."""
    lib = _lib.load()
    ids = ids.contiguous().to(torch.int64)
    assert ids.dim() == 2, "batch_prefix_match: ids [R, L]"
    R, L = ids.shape
    _on_device("ids", ids)
    out = torch.empty((R,), dtype=torch.int32, device=ids.device)
    s = lib.mtp_batch_prefix_match(ptr(ids), R, L, ptr(out), _lib.stream_handle(ids.device))
    check(s, "batch_prefix_match")
    return out
