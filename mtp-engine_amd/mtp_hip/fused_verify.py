"""Drop-in for the reference module ``mtp_fused_verify`` on MI355X.

Same names, argument order, defaults and return tuples as
mtp_fused_verify.py:199-290; the work runs in one gfx950 kernel launch
(lm_head GEMM -> argmax -> acceptance -> rollback index, logits never written
to HBM). Keyword-only extensions on fused_multi_verify: ``return_top`` and
``convention`` ("reference", the default, or "textbook").
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ops


def fused_verify(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    draft: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(accept int8 [M], top int32 [M]); mtp_fused_verify.py:199-234."""
    return ops.verify(hidden, weight, draft, bias)


def fused_multi_verify(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    draft: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    *,
    return_top: bool = False,
    convention: str = "reference",
):
    """(accept int8 [B, D], accepted_n int32 [B], corrected int32 [B]).

    mtp_fused_verify.py:237-290: top[b, s] = argmax over the vocabulary of
    hidden[b, s] @ weight.T + bias; corrected = top[:, 0]; accept[b, d] =
    (top[b, d+1] == draft[b, d]) while every earlier draft was accepted;
    accepted_n = length of the accepted prefix (the rollback index).
    convention="textbook" checks draft d against top[b, d] instead and
    returns corrected = top[b, accepted_n] (the replacement token, or the
    bonus token when every draft is accepted).
    With return_top=True the [B, S] argmax ids are returned fourth.
    """
    return ops.multi_verify(hidden, weight, draft, bias, return_top=return_top,
                            convention=convention)


__all__ = ["fused_verify", "fused_multi_verify"]
