"""Seeded synthetic inputs of the five verify/draft workloads.

All data is drawn on the CPU with torch.Generator("cpu").manual_seed(seed) in
the API layout (nn.Linear weights [N, K]), so a CPU check and the GPU see
identical bits. Workload i uses seed i - 1. Draw order is part of the
definition and is listed per function.

  1  fp32 RMSNorm+linear   x[16,1024], gamma[1024], W[4096,1024]        seed 0
  2  fp8-e4m3 weights       x bf16 [M,4096] (M in 8/32/64), gamma, W fp8
                            [14336,4096] with per-channel scale amax/448  seed 1
  3  multi-verify chain     hidden bf16 [8,5,4096], W bf16 [128256,4096]  seed 2
  4  tree-verify step       64-node tree attention over 2048 paged ctx +
                            bf16 RMSNorm+linear 4096 -> 4096             seed 3
  5  INT4 RMSNorm+linear    x bf16 [256,8192], gamma, W int4 (group 128,
                            fp16 scales) [28672,8192]                    seed 4
"""
from __future__ import annotations

import math
from typing import Dict

import numpy as np
import torch

MAX_FP8 = 448.0


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator("cpu")
    g.manual_seed(seed)
    return g


def _randn(g, *shape, chunk_rows: int = 0) -> torch.Tensor:
    return torch.randn(*shape, generator=g)


# --------------------------------------------------------------------------- #
def fp32_linear(seed: int = 0, M: int = 16, K: int = 1024, N: int = 4096) -> Dict:
    """Workload 1. Draws: x, gamma, W."""
    g = _gen(seed)
    x = _randn(g, M, K)
    gamma = 1.0 + 0.1 * _randn(g, K)
    W = 0.02 * _randn(g, N, K)
    return dict(x=x, gamma=gamma, weight=W, eps=1e-6)


def quantize_fp8_rows(W: torch.Tensor):
    """Per-output-row e4m3fn quantisation: s = amax(|W[n]|) / 448 (0 -> 1),
    q = clamp(W / s, +-448) cast with round-to-nearest-even."""
    amax = W.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / MAX_FP8, torch.ones_like(amax))
    q = (W / s[:, None]).clamp(-MAX_FP8, MAX_FP8).to(torch.float8_e4m3fn)
    return q, s.to(torch.float32)


def fp8_linear(M: int, seed: int = 1, K: int = 4096, N: int = 14336) -> Dict:
    """Workload 2. Draws: W (fp32), gamma, x (fp32 then bf16)."""
    g = _gen(seed)
    W = 0.02 * _randn(g, N, K)
    gamma = 1.0 + 0.1 * _randn(g, K)
    x = _randn(g, M, K).to(torch.bfloat16)
    wq, ws = quantize_fp8_rows(W)
    del W
    return dict(x=x, gamma=gamma, weight_fp8=wq, wscale=ws, eps=1e-6)


def _weight(g, N: int, K: int, std: float = 0.02, rows: int = 8192,
            dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    out = torch.empty((N, K), dtype=dtype)
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        out[r0:r1] = (std * torch.randn(r1 - r0, K, generator=g)).to(dtype)
    return out


def _bf16_weight(g, N: int, K: int, std: float = 0.02, rows: int = 8192) -> torch.Tensor:
    return _weight(g, N, K, std, rows)


def multi_verify(seed: int = 2, B: int = 8, D: int = 4, K: int = 4096, V: int = 128256,
                 dtype: torch.dtype = torch.bfloat16, bias: bool = False) -> Dict:
    """Workload 3 inputs without the drafts. Draws: hidden (fp32 -> dtype),
    W (0.02 N(0, 1) -> dtype, generated in 8192-row chunks), then with
    bias=True a bias 0.5 N(0, 1) -> dtype (the engine's lm_head carries one,
    mtp_engine.py:198). dtype=float32 is the engine's default head dtype.
    Drafts need the target argmax: see make_chain_drafts."""
    g = _gen(seed)
    hidden = _randn(g, B, D + 1, K).to(dtype)
    W = _weight(g, V, K, dtype=dtype)
    b = (0.5 * _randn(g, V)).to(dtype) if bias else None
    return dict(hidden=hidden, weight=W, bias=b, B=B, D=D, seed=seed)


def make_chain_drafts(top: torch.Tensor, V: int, seed: int, alpha: float = 0.6) -> torch.Tensor:
    """Drafts for a [B, D+1] target argmax `top`: k_b ~ Geometric (P(k) =
    (1 - alpha) alpha^k, capped at D); draft[b, d] = top[b, d+1] for d < k_b;
    draft[b, k_b] is a random id != top[b, k_b+1]; later drafts uniform.
    Draws (generator seed + 1000): u[B], then per b the random ids."""
    g = _gen(seed + 1000)
    top = top.to(torch.int64).cpu()
    B, S = top.shape
    D = S - 1
    u = torch.rand(B, generator=g, dtype=torch.float64)
    draft = torch.empty((B, D), dtype=torch.int64)
    ks = []
    for b in range(B):
        k = int(math.floor(math.log(max(float(u[b]), 1e-300)) / math.log(alpha)))
        k = min(max(k, 0), D)
        ks.append(k)
        rnd = torch.randint(0, V, (D,), generator=g)
        for d in range(D):
            if d < k:
                draft[b, d] = top[b, d + 1]
            elif d == k:
                v = int(rnd[d])
                draft[b, d] = v if v != int(top[b, d + 1]) else (v + 1) % V
            else:
                draft[b, d] = rnd[d]
    return draft


def quantize_int4_groups(W: torch.Tensor, group: int = 128, nibble: str = "ref"):
    """Per (row, group): s = amax / 7 (0 -> 1) stored as fp16; q =
    round_half_even(W / s16).clamp(-8, 7); nibbles packed two per byte, even
    k in the low nibble; "ref" stores q & 0xF, "offset" stores q + 8."""
    N, K = W.shape
    ng = K // group
    Wg = W.reshape(N, ng, group)
    amax = Wg.abs().amax(dim=-1)
    s = torch.where(amax > 0, amax / 7.0, torch.ones_like(amax)).to(torch.float16)
    q = torch.round(Wg / s.to(torch.float32)[..., None]).clamp(-8, 7).to(torch.int8)
    qn = q.reshape(N, K).numpy().astype(np.int16)
    nib = ((qn & 0xF) if nibble == "ref" else (qn + 8)).astype(np.uint8)
    packed = nib[:, 0::2] | (nib[:, 1::2] << 4)
    return torch.from_numpy(np.ascontiguousarray(packed)), s


def int4_linear(seed: int = 4, M: int = 256, K: int = 8192, N: int = 28672, group: int = 128,
                nibble: str = "ref") -> Dict:
    """Workload 5. Draws: W (fp32, 4096-row chunks, quantised chunk by chunk),
    gamma, x (fp32 -> bf16)."""
    g = _gen(seed)
    packed = torch.empty((N, K // 2), dtype=torch.uint8)
    scales = torch.empty((N, K // group), dtype=torch.float16)
    rows = 4096
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        Wc = 0.02 * torch.randn(r1 - r0, K, generator=g)
        packed[r0:r1], scales[r0:r1] = quantize_int4_groups(Wc, group, nibble)
    gamma = 1.0 + 0.1 * _randn(g, K)
    x = _randn(g, M, K).to(torch.bfloat16)
    return dict(x=x, gamma=gamma, packed=packed, scales=scales, group=group, K=K, eps=1e-6)


# --------------------------------------------------------------------------- #
# Algorithmic work per launch (bytes moved at least once, flops of the GEMM)
def linear_bytes(M, N, K, x_bytes, w_bytes_per_elem, y_bytes, extra=0):
    return int(M * K * x_bytes + N * K * w_bytes_per_elem + M * N * y_bytes + extra)


# --------------------------------------------------------------------------- #
def draft_tree_mask(depth: int, max_branches: int) -> torch.Tensor:
    """Ancestor-or-self mask [n, n] float32 of the breadth-first draft tree
    with depth * max_branches nodes (SpeculativeDraftTree,
    mtp_engine.py:651-680): row n is 1 on n and on every ancestor of n."""
    n = depth * max_branches
    parent = [-1] * n
    frontier, idx = [0], 1
    for _ in range(1, depth):
        nxt = []
        for p in frontier:
            for _ in range(max_branches):
                if idx < n:
                    parent[idx] = p
                    nxt.append(idx)
                    idx += 1
        frontier = nxt
    mask = torch.zeros(n, n)
    for i in range(n):
        mask[i, i] = 1.0
        p = parent[i]
        while p >= 0:
            mask[i, p] = 1.0
            p = parent[p]
    return mask


def tree_verify(seed: int = 3, depth: int = 16, branches: int = 4, H: int = 32, D: int = 128,
                Lc: int = 2048, page_size: int = 16, pages: int = 160, hidden: int = 4096,
                N_out: int = 4096) -> Dict:
    """Workload 4. Draws: q, k_tree, v_tree [N, H, D]; k_pages, v_pages
    [pages, 1, H, page_size, D]; a permutation of the physical pages (the
    first Lc / page_size of it hold the context, in order); W [N_out,
    hidden] ~ 0.02 N(0, 1). All bf16 except the int32 table and the fp32
    tree mask."""
    g = _gen(seed)
    mask = draft_tree_mask(depth, branches)
    N = mask.shape[0]
    q = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    k_tree = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    v_tree = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    k_pages = torch.randn(pages, 1, H, page_size, D, generator=g).to(torch.bfloat16)
    v_pages = torch.randn(pages, 1, H, page_size, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(pages, generator=g)[: Lc // page_size]
    table = perm.repeat_interleave(page_size).to(torch.int32)[None, :]
    W = (0.02 * torch.randn(N_out, hidden, generator=g)).to(torch.bfloat16)
    return dict(q=q, k_tree=k_tree, v_tree=v_tree, k_pages=k_pages, v_pages=v_pages,
                page_table=table, page_size=page_size, tree_mask=mask, weight=W, eps=1e-6,
                seed=seed)
