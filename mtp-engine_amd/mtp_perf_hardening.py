"""Drop-in ``CachedLinear`` (mtp_perf_hardening.py:150-165) on MI355X.

Same constructor and forward contract as the reference (an nn.Linear that
caches its weight/bias views); forward runs the no-norm mode of the gfx950
RMSNorm -> linear kernel instead of F.linear. Leading dimensions of x are
flattened and restored, as F.linear does.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from mtp_hip import ops


class CachedLinear(nn.Linear):
    def __init__(self, in_features: int, out_features: int, bias: bool = True):
        super().__init__(in_features, out_features, bias=bias)
        self._w = self.weight.data
        self._b = self.bias.data if bias and self.bias is not None else None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        b = None if self._b is None else self._b.to(x2.dtype)
        y = ops.rmsnorm_linear(x2, self._w, b, 0.0, 1.0, norm=False)
        return y.reshape(*lead, y.shape[-1])

    def _refresh_cache(self) -> None:
        self._w = self.weight.data
        self._b = self.bias.data if self.bias is not None else None

    def _apply(self, fn, *args, **kwargs):
        # .to() / .cuda() replace the parameters' storage: re-point the cached
        # views, or they would keep referring to the old (e.g. host) tensors.
        out = super()._apply(fn, *args, **kwargs)
        self._refresh_cache()
        return out


__all__ = ["CachedLinear"]
