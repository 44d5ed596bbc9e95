"""Tensor-level entry points over the C ABI.

Each function canonicalises its inputs the way the reference's wrapper does
(.contiguous(), dtype of the output = dtype of x, draft ids as int32),
allocates the outputs with the torch allocator, takes the per-stream
workspace and enqueues the kernel on torch's current stream without
synchronising. Inputs must live on a HIP device.
"""
from __future__ import annotations

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
