"""Install the gfx950 kernels into already-imported reference modules.

For a process that imports the reference's own ``mtp_kernels``,
``mtp_fused_verify``, ``mtp_perf_hardening`` (and optionally ``mtp_radix``
and ``mtp_engine``), ``install(...)`` replaces only the hot-path attributes
of those module objects with the gfx950 implementations; everything else in
them (the engine loop, TP layer, pipelines, radix tree) stays the
reference's. Call it before ``import mtp_engine`` (whose ``from mtp_kernels
import ...`` binds names at import time), or pass ``engine_mod`` to patch the
names it already bound. Nothing here imports a reference module: the caller
hands them in.
"""
from __future__ import annotations

from types import ModuleType
from typing import Dict, List, Optional, Tuple

import torch

from . import fused_verify as _fv
from . import kernels as _k
from . import ops
from . import perf_hardening as _ph

# Attributes replaced in the caller's mtp_kernels: the compute entry points
# of the verify / draft path (RMSNorm -> linear in every weight format, the
# quantizers, tree / paged attention and the tree monolith, the draft
# chain's norms). Everything else in the module stays the reference's.
KERNELS_NAMES = (
    "fused_rmsnorm", "fused_add_rmsnorm", "fused_rmsnorm_linear", "fused_rmsnorm_linear_fp8",
    "fused_int4_matmul", "fused_paged_attention", "fused_tree_attention",
    "fused_tree_attn_rmsnorm_linear", "quantize_fp8_e4m3", "dequantize_fp8", "quantize_int4",
    "dequantize_int4",
)
VERIFY_NAMES = ("fused_verify", "fused_multi_verify")
HARDENING_NAMES = ("argmax_greedy", "sample_token", "CachedLinear")


def _radix_prefix_match(original):
    def batch_prefix_match(self, ids: torch.Tensor) -> torch.Tensor:
        ids = ids.to(device=self.device, dtype=torch.long)
        if ids.device.type != "cuda":
            return original(self, ids)
        return ops.batch_prefix_match(ids)

    batch_prefix_match.__doc__ = ("RadixKVCache.batch_prefix_match (mtp_radix.py:195-236) on "
                                  "the gfx950 prefix-match kernel for device ids.")
    return batch_prefix_match


class Installed:
    """What install() replaced, for uninstall()."""

    def __init__(self):
        self.saved: List[Tuple[object, str, object, bool]] = []

    def set(self, obj, name: str, value) -> None:
        had = hasattr(obj, name)
        self.saved.append((obj, name, getattr(obj, name, None), had))
        setattr(obj, name, value)

    def names(self) -> Dict[str, List[str]]:
        out: Dict[str, List[str]] = {}
        for obj, name, _, _ in self.saved:
            out.setdefault(getattr(obj, "__name__", repr(obj)), []).append(name)
        return out


def install(kernels_mod: Optional[ModuleType] = None, verify_mod: Optional[ModuleType] = None,
            hardening_mod: Optional[ModuleType] = None, radix_mod: Optional[ModuleType] = None,
            engine_mod: Optional[ModuleType] = None) -> Installed:
    """Replace the hot-path attributes of the given (already imported)
    reference modules with the gfx950 implementations. Returns a record
    that uninstall() reverts."""
    rec = Installed()
    ours = {n: getattr(_k, n) for n in KERNELS_NAMES}
    ours.update({n: getattr(_fv, n) for n in VERIFY_NAMES})
    ours.update({n: getattr(_ph, n) for n in HARDENING_NAMES})
    if kernels_mod is not None:
        for n in KERNELS_NAMES:
            rec.set(kernels_mod, n, ours[n])
    if verify_mod is not None:
        for n in VERIFY_NAMES:
            rec.set(verify_mod, n, ours[n])
    if hardening_mod is not None:
        for n in HARDENING_NAMES:
            rec.set(hardening_mod, n, ours[n])
    if radix_mod is not None and hasattr(radix_mod, "RadixKVCache"):
        cls = radix_mod.RadixKVCache
        rec.set(cls, "batch_prefix_match", _radix_prefix_match(cls.batch_prefix_match))
    if engine_mod is not None:
        # names the engine bound with `from mtp_... import ...` at its import
        for n, fn in ours.items():
            if hasattr(engine_mod, n):
                rec.set(engine_mod, n, fn)
    return rec


def uninstall(rec: Installed) -> None:
    """Put back what install() replaced (in reverse order)."""
    for obj, name, old, had in reversed(rec.saved):
        if had:
            setattr(obj, name, old)
        else:
            delattr(obj, name)
    rec.saved.clear()


__all__ = ["install", "uninstall", "Installed", "KERNELS_NAMES", "VERIFY_NAMES",
           "HARDENING_NAMES"]
