"""Drop-in for the reference module ``mtp_perf_hardening`` on MI355X.

The names the engine imports (mtp_engine.py:49-57) and the ones the
reference's perf tests use, with the same constructors and call contracts
(mtp_perf_hardening.py:33-248). The hot-path members run gfx950 kernels:
``CachedLinear.forward`` is the no-norm mode of the RMSNorm -> linear
kernel, ``argmax_greedy`` and the greedy branch of ``sample_token`` are the
multi-workgroup argmax kernel. The rest are host-side helpers (shape
padding, pinned staging buffers, a device page table); ``maybe_compile``
returns the module unchanged, because this build has no tracing compiler
(launch-bound loops are captured into HIP graphs instead).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import ops


# --------------------------------------------------------------------------- #
# Shape padding (mtp_perf_hardening.py:33-57)
# --------------------------------------------------------------------------- #
def next_pow2(n: int) -> int:
    """Smallest power of two >= n (1 for n <= 1)."""
    return 1 if n <= 1 else 1 << (int(n) - 1).bit_length()


def align_vocab(vocab_size: int, alignment: int = 128) -> int:
    """vocab_size rounded up to a multiple of alignment, at least alignment."""
    return max(-(-int(vocab_size) // alignment) * alignment, alignment)


def pad_seq_len(seq_len: int, alignment: int = 32) -> int:
    return -(-int(seq_len) // alignment) * alignment


def pad_batch(batch: int, alignment: int = 8) -> int:
    return -(-int(batch) // alignment) * alignment


# --------------------------------------------------------------------------- #
# Constants computed once per engine (mtp_perf_hardening.py:62-91)
# --------------------------------------------------------------------------- #
class PrecomputedConstants:
    """Per-engine scalar constants as Python floats: attention scale
    1/sqrt(head_dim), RMSNorm 1/dim, inverse temperature (0 for greedy), the
    fp8 scale and the padded vocabulary."""

    def __init__(self, head_dim: int, hidden_dim: int, vocab_size: int, dtype: torch.dtype,
                 temperature: float = 1.0, eps: float = 1e-6, fp8_scale: float = 1.0 / 448.0):
        self.head_dim = head_dim
        self.hidden_dim = hidden_dim
        self.vocab_size = vocab_size
        self.dtype = dtype
        self.eps = eps
        self.attn_scale = 1.0 / math.sqrt(max(head_dim, 1))
        self.rms_inv = 1.0 / max(hidden_dim, 1)
        self.inv_temperature = (1.0 / temperature) if temperature > 0.0 else 0.0
        self.fp8_scale = fp8_scale
        self.vocab_padded = align_vocab(vocab_size)


def fast_check(actual: Tuple[int, ...], expected: Tuple[int, ...]) -> bool:
    """Shape equality on plain ints (mtp_perf_hardening.py:97-105)."""
    return len(actual) == len(expected) and all(a == b for a, b in zip(actual, expected))


# --------------------------------------------------------------------------- #
# Pinned staging buffers (mtp_perf_hardening.py:110-144)
# --------------------------------------------------------------------------- #
class PinnedBufferPool:
    """Page-locked host buffers for prompt ids and output tokens, allocated
    pinned from the start (no registration of existing memory), so copies
    to the GPU can run asynchronously."""

    def __init__(self, max_batch: int, max_seq_len: int, dtype: torch.dtype = torch.long):
        self.max_batch = max_batch
        self.max_seq_len = max_seq_len
        self.use_pin = torch.cuda.is_available()
        shape = (max_batch, max_seq_len)
        self.prompt = torch.empty(shape, dtype=dtype, pin_memory=self.use_pin)
        self.tokens = torch.empty(shape, dtype=dtype, pin_memory=self.use_pin)

    def stage_prompt(self, ids: torch.Tensor) -> torch.Tensor:
        B, S = ids.shape
        view = self.prompt[:B, :S]
        view.copy_(ids.to(self.prompt.dtype))
        return view

    def to_device_non_blocking(self, x: torch.Tensor, device: torch.device) -> torch.Tensor:
        if self.use_pin and torch.device(device).type == "cuda":
            return x.to(device, non_blocking=True)
        return x.to(device)


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


# --------------------------------------------------------------------------- #
# Device page table (mtp_perf_hardening.py:188-213)
# --------------------------------------------------------------------------- #
class FlatPageTable:
    """One contiguous int32 [batch, max_logical] logical -> physical page map
    on the device (-1 = unmapped), updated in place; the [B, L] page-table
    layout the paged attention and KV-write kernels read."""

    def __init__(self, batch: int, max_logical: int, device: torch.device):
        self.batch = batch
        self.max_logical = max_logical
        self.device = device
        self.table = torch.full((batch, max_logical), -1, dtype=torch.int32, device=device)

    def set_logical(self, batch_idx: int, logical: int, physical: int) -> None:
        self.table[batch_idx, logical] = physical

    def swap_pointers(self, a: int, b: int) -> None:
        col = self.table[:, a].clone()
        self.table[:, a] = self.table[:, b]
        self.table[:, b] = col

    def physical_of(self, batch_idx: int, logical: int) -> int:
        return int(self.table[batch_idx, logical].item())


# --------------------------------------------------------------------------- #
# Streams and compilation (mtp_perf_hardening.py:218-248)
# --------------------------------------------------------------------------- #
def get_stream() -> Optional["torch.cuda.Stream"]:
    return torch.cuda.current_stream() if torch.cuda.is_available() else None


def change_allocator_to_stream() -> None:
    """No-op: the kernels take torch's current stream and allocate nothing."""


def maybe_compile(module: nn.Module, enabled: bool = True):
    """Returns the module unchanged: there is no tracing compiler on this
    path; capture launch-bound loops into a HIP graph (torch.cuda.graph)."""
    return module


__all__ = [
    "next_pow2",
    "align_vocab",
    "pad_seq_len",
    "pad_batch",
    "PrecomputedConstants",
    "fast_check",
    "PinnedBufferPool",
    "CachedLinear",
    "argmax_greedy",
    "sample_token",
    "FlatPageTable",
    "get_stream",
    "change_allocator_to_stream",
    "maybe_compile",
]
