"""Hot-path members of the reference module ``mtp_perf_hardening`` on MI355X.

``CachedLinear`` (mtp_perf_hardening.py:150-165) runs the no-norm mode of
the gfx950 RMSNorm -> linear kernel; ``argmax_greedy`` and the greedy branch
of ``sample_token`` (mtp_perf_hardening.py:170-186) run the multi-workgroup
argmax kernel. The module's other helpers (shape padding, pinned staging
buffers, the page table, stream helpers) are host-side code off the verify /
draft path: ``mtp_hip.install(hardening_mod=...)`` replaces only these three
names in the caller's own ``mtp_perf_hardening`` and leaves the rest there.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import ops


# --------------------------------------------------------------------------- #
# CachedLinear (mtp_perf_hardening.py:150-165)
# --------------------------------------------------------------------------- #
class CachedLinear(nn.Linear):
    """nn.Linear with its weight / bias views cached at construction;
    forward runs the no-norm mode of the gfx950 RMSNorm -> linear kernel.
    Leading dimensions of x are flattened and restored, as F.linear does."""

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


# --------------------------------------------------------------------------- #
# Token selection (mtp_perf_hardening.py:170-186)
# --------------------------------------------------------------------------- #
def argmax_greedy(logits: torch.Tensor) -> torch.Tensor:
    """argmax over the last dim (int64, torch.argmax's order) on the GPU."""
    if logits.dim() <= 2:
        return ops.argmax(logits)
    lead = logits.shape[:-1]
    return ops.argmax(logits.reshape(-1, logits.shape[-1])).reshape(lead)


def sample_token(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    """temperature <= 0: the greedy argmax kernel. Otherwise a draw from
    softmax(logits / temperature) with torch's multinomial, as the
    reference does (a random draw has no bit-exact counterpart to match)."""
    if temperature <= 0.0:
        return argmax_greedy(logits)
    probs = torch.softmax(logits * (1.0 / temperature), dim=-1)
    return torch.multinomial(probs, num_samples=1).squeeze(-1)


__all__ = ["CachedLinear", "argmax_greedy", "sample_token"]
