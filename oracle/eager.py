"""Eager CPU restatement of the reference's hot-path functions (oracle).

Test infrastructure only; see oracle/__init__.py for who may import it and
how each function is pinned.
"""
from __future__ import annotations

import math
from typing import List, Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

MAX_FP8 = 448.0  # mtp_kernels.py:66


def _cpu(t):
    return None if t is None else t.detach().to("cpu")


# --------------------------------------------------------------------------- #
# RMSNorm -> linear family
# --------------------------------------------------------------------------- #
def rmsnorm_rstd(x: torch.Tensor, eps: float) -> torch.Tensor:
    """rsqrt(mean(x^2) + eps) over the last dim in fp32 (mtp_kernels.py:780-782)."""
    xf = x.to(torch.float32)
    ms = (xf * xf).mean(dim=-1, keepdim=True)
    return torch.rsqrt(ms + eps)


def rmsnorm_linear(x, weight, bias=None, eps=1e-6, scale=1.0, gamma=None, norm=True):
    """_eager_rmsnorm_linear (mtp_kernels.py:778-787) with the wrapper's
    canonicalisation (936-958: bias cast to x.dtype). Extensions: gamma
    multiplies the normalised x (as _eager_rmsnorm does, 771-775); norm=False
    skips the RMSNorm (plain F.linear, mtp_perf_hardening.py:159-160)."""
    x, weight, bias, gamma = _cpu(x), _cpu(weight), _cpu(bias), _cpu(gamma)
    xf = x.to(torch.float32)
    xn = xf * rmsnorm_rstd(x, eps) if norm else xf
    if gamma is not None:
        xn = xn * gamma.to(torch.float32)
    b = None if bias is None else bias.to(x.dtype).to(torch.float32)
    y = F.linear(xn, weight.to(torch.float32), b)
    return (y * scale).to(x.dtype)


def rmsnorm_linear_fp8(x, weight_fp8, wscale, bias=None, eps=1e-6, gamma=None, norm=True):
    """_eager_rmsnorm_linear_fp8 (mtp_kernels.py:804-814): weight decoded to
    fp32 and scaled per output row, then the fp32 RMSNorm -> linear."""
    x, weight_fp8, wscale, bias, gamma = map(_cpu, (x, weight_fp8, wscale, bias, gamma))
    w = weight_fp8.to(torch.float32) * wscale.to(torch.float32)[:, None]
    xf = x.to(torch.float32)
    xn = xf * rmsnorm_rstd(x, eps) if norm else xf
    if gamma is not None:
        xn = xn * gamma.to(torch.float32)
    y = F.linear(xn, w, None if bias is None else bias.to(torch.float32))
    return y.to(x.dtype)


# --------------------------------------------------------------------------- #
# FP8 producers
# --------------------------------------------------------------------------- #
def fp8_e4m3fn_decode_table() -> np.ndarray:
    """Value of every float8_e4m3fn code (OCP spec: bias 7, no inf, 0x7f/0xff
    NaN), computed from the format definition."""
    out = np.empty(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            out[c] = np.nan
        elif e == 0:
            out[c] = s * (m / 8.0) * 2.0 ** (-6)
        else:
            out[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


def quantize_fp8_per_tensor(x):
    """quantize_fp8_e4m3 (mtp_kernels.py:704-713): one scale amax/448."""
    xf = _cpu(x).to(torch.float32)
    amax = xf.abs().max()
    scale = amax / MAX_FP8 if amax > 0 else torch.tensor(1.0, dtype=torch.float32)
    q = (xf / scale).clamp(-MAX_FP8, MAX_FP8).to(torch.float8_e4m3fn)
    return q, scale.to(torch.float32)


def quantize_fp8_per_channel(w):
    """Per-output-row fp8: s[n] = amax(|W[n, :]|) / 448 (0 -> 1), as
    QuantScaleState.update_weight_scales (mtp_engine.py:617-622); values
    clamp(W / s, +-448) cast to float8_e4m3fn (mtp_engine.py:1792-1795,
    mtp_kernels.py:708-710)."""
    wf = _cpu(w).to(torch.float32)
    amax = wf.abs().max(dim=1, keepdim=True).values.squeeze(1)
    s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (wf / s[:, None]).clamp(-MAX_FP8, MAX_FP8).to(torch.float8_e4m3fn)
    return q, s


def dequantize_fp8(x_fp8, scale):
    """mtp_kernels.py:726-727."""
    return _cpu(x_fp8).to(torch.float32) * _cpu(scale).to(torch.float32)


def pack_scales(weight_scales, kv_scales=None):
    """mtp_kernels.py:1336-1346."""
    all_scales = list(weight_scales) + list(kv_scales or [])
    offs = [0]
    for s in all_scales:
        offs.append(offs[-1] + s.numel())
    flat = torch.cat([_cpu(s).reshape(-1).float() for s in all_scales])
    return flat, torch.tensor(offs, dtype=torch.int64)


# --------------------------------------------------------------------------- #
# INT4 producers / decoder
# --------------------------------------------------------------------------- #
def quantize_int4(w, group: int = 32, scale_dtype=torch.float32, nibble: str = "ref"):
    """quantize_int4 (mtp_kernels.py:730-751), vectorised with numpy: per
    (row, group) s = amax / 7 (0 -> 1); q = round_half_even(W / s) clamped to
    [-8, 7]; element k goes to byte k // 2, low nibble for even k. The
    reference stores q & 0xF (two's complement, nibble="ref"); "offset"
    stores q + 8 (what the decoder, 758-762, expects). K and group must be
    even: the reference's loop writes past the packed row for odd K and
    overlaps bytes for odd groups. With scale_dtype=float16 the scale is
    rounded first and q is computed against the stored scale."""
    wf = _cpu(w).to(torch.float32)
    N, K = wf.shape
    if K % 2 or group % 2:
        raise ValueError("quantize_int4 needs even K and even group")
    ng = (K + group - 1) // group
    scales = torch.empty((N, ng), dtype=torch.float32)
    q_all = torch.empty((N, K), dtype=torch.int8)
    for g in range(ng):
        c0, c1 = g * group, min((g + 1) * group, K)
        chunk = wf[:, c0:c1]
        amax = chunk.abs().max(dim=-1, keepdim=True).values
        s = torch.where(amax > 0, amax / 7.0, torch.ones_like(amax))
        s = s.to(scale_dtype).to(torch.float32)
        q_all[:, c0:c1] = torch.round(chunk / s).clamp(-8, 7).to(torch.int8)
        scales[:, g] = s.squeeze(-1)
    q = q_all.numpy().astype(np.int16)
    nib = (q & 0xF) if nibble == "ref" else (q + 8)
    nib = nib.astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return torch.from_numpy(packed), scales.to(scale_dtype)


def int4_nibbles(packed) -> np.ndarray:
    """[N, K] nibble values of a packed [N, K/2] u8 tensor (even k = low)."""
    p = _cpu(packed).numpy().astype(np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 2), dtype=np.int16)
    out[:, 0::2] = p & 0xF
    out[:, 1::2] = p >> 4
    return out


def dequantize_int4(packed, scales, K: int, group: int, nibble: str = "ref"):
    """dequantize_int4 (mtp_kernels.py:754-768): nibble - 8 (nibble="ref" /
    "offset"; "twos" reads two's-complement nibbles), times the group scale,
    in fp32."""
    nib = int4_nibbles(packed)[:, :K]
    q = (nib - 8) if nibble in ("ref", "offset") else ((nib ^ 8) - 8)
    w = torch.from_numpy(q.astype(np.float32))
    sc = _cpu(scales).to(torch.float32)
    ng = (K + group - 1) // group
    for g in range(ng):
        c0, c1 = g * group, min((g + 1) * group, K)
        w[:, c0:c1] = w[:, c0:c1] * sc[:, g:g + 1]
    return w


def int4_matmul(x, packed, scales, K: int, group: int, nibble="ref", gamma=None, norm=False,
                eps=1e-6):
    """_eager_int4_matmul (mtp_kernels.py:875-878): F.linear(x fp32,
    dequantized W) cast to x.dtype. norm/gamma compose the RMSNorm prologue
    (the INT4 RMSNorm+linear workload); norm=False is the reference."""
    x = _cpu(x)
    w = dequantize_int4(packed, scales, K, group, nibble)
    return rmsnorm_linear(x, w, None, eps, 1.0, gamma=gamma, norm=norm) if (norm or gamma is not None) \
        else F.linear(x.to(torch.float32), w).to(x.dtype)


# --------------------------------------------------------------------------- #
# Verify
# --------------------------------------------------------------------------- #
def logits_top(hidden2d, weight, bias=None, chunk: int = 16384):
    """argmax over V of hidden @ W.T + bias in fp32 (lowest index on ties,
    NaN is the maximum, as torch.argmax), plus the top-2 gap per row.
    Processes the vocabulary in chunks so a 1 GB weight never needs a full
    fp32 copy; every logit is the same fp32 F.linear the reference runs
    (mtp_fused_verify.py:163, 180-182)."""
    h = _cpu(hidden2d).to(torch.float32)
    W = _cpu(weight)
    b = _cpu(bias)
    V = W.shape[0]
    best_v = torch.full((h.shape[0],), -math.inf)
    best_i = torch.zeros((h.shape[0],), dtype=torch.int64)
    second = torch.full((h.shape[0],), -math.inf)
    for v0 in range(0, V, chunk):
        v1 = min(V, v0 + chunk)
        lg = F.linear(h, W[v0:v1].to(torch.float32), None if b is None else b[v0:v1].to(torch.float32))
        top2 = torch.topk(lg, k=min(2, v1 - v0), dim=-1)
        am = lg.argmax(dim=-1)
        cv = lg.gather(1, am[:, None]).squeeze(1)
        c2 = top2.values[:, 1] if v1 - v0 > 1 else torch.full_like(cv, -math.inf)
        better = (cv > best_v) | torch.isnan(cv) & ~torch.isnan(best_v)
        new_second = torch.where(better, torch.maximum(best_v, c2), torch.maximum(second, cv))
        best_i = torch.where(better, am + v0, best_i)
        best_v = torch.where(better, cv, best_v)
        second = new_second
    return best_i.to(torch.int32), (best_v - second)


def fused_verify(hidden, weight, draft, bias=None):
    """_eager_fused_verify (mtp_fused_verify.py:159-166) with the wrapper's
    draft -> int32 (207)."""
    top, _ = logits_top(hidden, weight, bias)
    accept = (top == _cpu(draft).to(torch.int32)).to(torch.int8)
    return accept, top


def chain_accept(top, draft):
    """The B x D acceptance loop of _eager_fused_multi_verify
    (mtp_fused_verify.py:184-195): accept[b, d] = top[b, d+1] == draft[b, d]
    until the first rejection (later entries stay 0); accepted_n = number of
    leading accepts; corrected = top[:, 0]."""
    top = _cpu(top).to(torch.int32)
    draft = _cpu(draft).to(torch.int32)
    B, D = draft.shape
    accept = torch.zeros((B, D), dtype=torch.int8)
    accepted_n = torch.zeros((B,), dtype=torch.int32)
    for b in range(B):
        n = 0
        for d in range(D):
            accept[b, d] = int(top[b, d + 1] == draft[b, d])
            if accept[b, d]:
                n = d + 1
            else:
                break
        accepted_n[b] = n
    corrected = top[:, 0].to(torch.int32)
    return accept, accepted_n, corrected


def chain_accept_textbook(top, draft):
    """The textbook speculative-decoding chain on the same argmax tokens
    (the correct-semantics option next to the reference's convention of
    chain_accept, mtp_fused_verify.py:136-154): accept[b, d] = top[b, d] ==
    draft[b, d] until the first rejection; accepted_n = leading accepts;
    corrected = top[b, accepted_n] (the replacement token, or the bonus
    token after D accepts)."""
    top = _cpu(top).to(torch.int32)
    draft = _cpu(draft).to(torch.int32)
    B, D = draft.shape
    accept = torch.zeros((B, D), dtype=torch.int8)
    accepted_n = torch.zeros((B,), dtype=torch.int32)
    corrected = torch.zeros((B,), dtype=torch.int32)
    for b in range(B):
        n = 0
        while n < D and int(top[b, n]) == int(draft[b, n]):
            accept[b, n] = 1
            n += 1
        accepted_n[b] = n
        corrected[b] = top[b, n]
    return accept, accepted_n, corrected


def fused_multi_verify(hidden, weight, draft, bias=None, convention: str = "reference"):
    """_eager_fused_multi_verify (mtp_fused_verify.py:169-196) with the
    wrapper's checks (237-265); convention="textbook" runs
    chain_accept_textbook on the same argmax tokens. Returns (accept,
    accepted_n, corrected, top [B, S], top-2 gap [B, S])."""
    hidden = _cpu(hidden)
    B, S, K = hidden.shape
    D = draft.shape[1]
    assert S == D + 1, f"expected S == D + 1, got S={S} D={D}"
    top, gap = logits_top(hidden.reshape(B * S, K), weight, bias)
    top = top.reshape(B, S)
    chain = chain_accept if convention == "reference" else chain_accept_textbook
    accept, accepted_n, corrected = chain(top, draft)
    return accept, accepted_n, corrected, top, gap.reshape(B, S)


def engine_rollback(accept, accepted_n, corrected, draft):
    """generate_fused's consumer of the verify outputs (mtp_engine.py:1244-1258):
    a_n = min over the batch of accepted_n; on any rejection the KV length
    rolls back to checkpoint + a_n + 1 and the step emits draft[:, :a_n] ++
    corrected; otherwise the whole draft is committed."""
    accept, accepted_n, corrected, draft = map(_cpu, (accept, accepted_n, corrected, draft))
    B, D = draft.shape
    a_n = int(accepted_n.to(torch.int64).min().item())
    has_reject = bool(accept.to(torch.bool).sum().item() < D * B)
    if has_reject:
        new_tokens = torch.cat([draft[:, :a_n], corrected.to(draft.dtype).unsqueeze(1)], dim=1)
        kv_advance = a_n + 1
    else:
        new_tokens = draft
        kv_advance = D
    return a_n, has_reject, new_tokens, kv_advance


# --------------------------------------------------------------------------- #
# Draft tree (producer of the tree-verify mask)
# --------------------------------------------------------------------------- #
def draft_tree(depth: int, max_branches: int = 8, mode: str = "tree") -> Tuple[torch.Tensor, torch.Tensor]:
    """SpeculativeDraftTree parent index and mask (mtp_engine.py:651-680):
    breadth-first, max_nodes = depth * max_branches, mask[n] = 1 on n's
    ancestors and on n itself."""
    max_nodes = depth * max_branches
    parent = torch.full((max_nodes,), -1, dtype=torch.int32)
    if mode == "trunk":
        for i in range(1, depth):
            parent[i] = i - 1
    else:
        frontier = [0]
        idx = 1
        for _ in range(1, depth):
            new_frontier: List[int] = []
            for p in frontier:
                for _ in range(max_branches):
                    if idx < max_nodes:
                        parent[idx] = p
                        new_frontier.append(idx)
                        idx += 1
            frontier = new_frontier
    mask = torch.zeros((max_nodes, max_nodes), dtype=torch.float32)
    for n in range(1, max_nodes):
        p = int(parent[n])
        while p >= 0:
            mask[n, p] = 1.0
            p = int(parent[p])
        mask[n, n] = 1.0
    mask[0, 0] = 1.0
    return parent, mask


# --------------------------------------------------------------------------- #
# Attention (tree / paged) and the composed tree-verify step
# --------------------------------------------------------------------------- #
def _softmax_attend(qf, kf, vf, scale, valid=None):
    """Single-query softmax attention in fp32 as the reference's eager twins
    compute it (mtp_kernels.py:849-855, 865-871): scores = q.k * scale,
    masked scores = -inf, m = amax, p = exp(s - m), out = (p / sum p) @ v.
    qf [..., D], kf / vf [..., L, D], valid [..., L] bool or None."""
    scores = torch.einsum("...d,...ld->...l", qf, kf) * scale
    if valid is not None:
        scores = torch.where(valid, scores, torch.full_like(scores, float("-inf")))
    m = torch.amax(scores, dim=-1, keepdim=True)
    p = torch.exp(scores - m)
    l = p.sum(dim=-1, keepdim=True)
    return torch.einsum("...l,...ld->...d", p / l, vf)


def paged_attention(q, k_pages, v_pages, page_table, page_size: int, scale=None):
    """_eager_paged_attention (mtp_kernels.py:832-856) with the wrapper's
    defaults (1136-1149): q [B, H, D]; pages [P, B, H, page_size, D]; key t of
    (b, h) is pages[page_table[b, t], b, h, t % page_size]; no mask; output in
    q's dtype."""
    q, k_pages, v_pages, page_table = map(_cpu, (q, k_pages, v_pages, page_table))
    B, H, D = q.shape
    L = page_table.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    page = page_table.long()
    slot = torch.arange(L) % page_size
    bi = torch.arange(B)[:, None]
    kg = k_pages[page, bi, :, slot[None, :]]   # [B, L, H, D]
    vg = v_pages[page, bi, :, slot[None, :]]
    kf = kg.permute(0, 2, 1, 3).float()
    vf = vg.permute(0, 2, 1, 3).float()
    return _softmax_attend(q.float(), kf, vf, scale).to(q.dtype)


def tree_attention(q, k, v, mask, scale=None):
    """_eager_tree_attention (mtp_kernels.py:859-872) with the wrapper's
    defaults (1165-1178): q [B, H, D]; k / v [B, H, L, D]; mask [L], key l is
    attended where mask[l] > 0.5 (a fully masked row is NaN, as there)."""
    q, k, v, mask = map(_cpu, (q, k, v, mask))
    B, H, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    valid = (mask > 0.5)[None, None, :].expand(B, H, -1)
    return _softmax_attend(q.float(), k.float(), v.float(), scale, valid).to(q.dtype)


def tree_verify_attention(q_nodes, k_pages, v_pages, page_table, page_size: int, k_tree, v_tree,
                          tree_mask, scale=None):
    """The tree-verify attention step of the 64-node workload, as the
    reference composes it from single-query calls: node n's query attends,
    under one softmax, to the Lc context tokens of the paged cache (batch 0)
    and to the tree nodes m with tree_mask[n, m] > 0.5 — i.e. one
    _eager_tree_attention call per node (mtp_kernels.py:859-872) over
    keys = context ++ tree with mask = ones(Lc) ++ tree_mask[n]
    (tree mask from SpeculativeDraftTree, mtp_engine.py:671-680).
    q_nodes / k_tree / v_tree [N, H, D]; pages [P, 1, H, page_size, D];
    page_table [1, Lc] -> out [N, H, D] in q's dtype."""
    q_nodes, k_pages, v_pages, page_table, k_tree, v_tree, tree_mask = map(
        _cpu, (q_nodes, k_pages, v_pages, page_table, k_tree, v_tree, tree_mask))
    N, H, D = q_nodes.shape
    Lc = page_table.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    page = page_table[0].long()
    slot = torch.arange(Lc) % page_size
    kc = k_pages[page, 0, :, slot]                      # [Lc, H, D]
    vc = v_pages[page, 0, :, slot]
    keys = torch.cat([kc, k_tree], 0).permute(1, 0, 2).float()   # [H, Lc + N, D]
    vals = torch.cat([vc, v_tree], 0).permute(1, 0, 2).float()
    valid = torch.cat([torch.ones(N, Lc, dtype=torch.bool), tree_mask > 0.5], 1)  # [N, Lc + N]
    qf = q_nodes.float().permute(1, 0, 2)               # [H, N, D]
    scores = torch.einsum("hnd,hld->hnl", qf, keys) * scale
    scores = torch.where(valid[None], scores, torch.full_like(scores, float("-inf")))
    m = torch.amax(scores, dim=-1, keepdim=True)
    p = torch.exp(scores - m)
    l = p.sum(dim=-1, keepdim=True)
    out = torch.einsum("hnl,hld->hnd", p / l, vals)
    return out.permute(1, 0, 2).to(q_nodes.dtype)


# --------------------------------------------------------------------------- #
# Draft chain: RMSNorm, add + RMSNorm, greedy token + embedding
# --------------------------------------------------------------------------- #
def rmsnorm(x, weight=None, eps: float = 1e-6):
    """fused_rmsnorm's eager route (mtp_kernels.py:910-933 -> _eager_rmsnorm
    771-775): the weight is cast to x.dtype by the wrapper (918-920), then
    (fp32(x) * rsqrt(mean(x^2) + eps) * fp32(weight)) cast to x.dtype."""
    x = _cpu(x).contiguous()
    N = x.shape[-1]
    w = torch.ones(N, dtype=x.dtype) if weight is None else _cpu(weight).to(x.dtype)
    xf = x.to(torch.float32)
    ms = (xf * xf).mean(dim=-1, keepdim=True)
    return (xf * torch.rsqrt(ms + eps) * w.to(torch.float32)).to(x.dtype)


def add_rmsnorm(x, residual, weight=None, eps: float = 1e-6):
    """fused_add_rmsnorm's eager route (mtp_kernels.py:1082-1102 ->
    _eager_add_rmsnorm 1073-1079): s = fp32(x) + fp32(residual), then the
    RMSNorm of s with the weight cast to x.dtype, cast to x.dtype."""
    x, residual = _cpu(x).contiguous(), _cpu(residual).contiguous()
    N = x.shape[-1]
    w = torch.ones(N, dtype=x.dtype) if weight is None else _cpu(weight).to(x.dtype)
    s = x.to(torch.float32) + residual.to(torch.float32)
    ms = (s * s).mean(dim=-1, keepdim=True)
    return (s * torch.rsqrt(ms + eps) * w.to(torch.float32)).to(x.dtype)


def argmax_tokens(logits, emb_table=None):
    """argmax_greedy / sample_token(temperature <= 0)
    (mtp_perf_hardening.py:170-186) = logits.argmax(dim=-1) (int64), and
    the next step's embedding rows token_embedding(token)
    (mtp_engine.py:750, 773) when a table is given."""
    tok = _cpu(logits).argmax(dim=-1)
    if emb_table is None:
        return tok
    return tok, _cpu(emb_table)[tok]


# --------------------------------------------------------------------------- #
# Decode attention (causal, fp8 KV) and the tree monolith
# --------------------------------------------------------------------------- #
def causal_attention(q, k, v, scale=None):
    """fused_causal_attention's eager route (mtp_kernels.py:980-1011 ->
    _eager_causal_attention 790-801): one query attending every key."""
    q, k, v = map(_cpu, (q, k, v))
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    return _softmax_attend(q.float(), k.float(), v.float(), scale).to(q.dtype)


def causal_attention_fp8(q, k_fp8, v_fp8, kscale, vscale, scale=None):
    """fused_causal_attention_fp8's eager route (mtp_kernels.py:1105-1133 ->
    _eager_causal_attention_fp8 817-829): K / V decoded to fp32 and scaled
    per head (kscale[h], vscale[h]) before the attention."""
    q, k_fp8, v_fp8, kscale, vscale = map(_cpu, (q, k_fp8, v_fp8, kscale, vscale))
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    kf = k_fp8.to(torch.float32) * kscale.float()[None, :, None, None]
    vf = v_fp8.to(torch.float32) * vscale.float()[None, :, None, None]
    return _softmax_attend(q.float(), kf, vf, scale).to(q.dtype)


def tree_attn_rmsnorm_linear(q, k, v, mask, proj_w, rms_w=None, proj_bias=None, wscale=None,
                             scale=None, eps: float = 1e-6):
    """_eager_tree_attn_rmsnorm_linear (mtp_kernels.py:881-907), the route
    fused_tree_attn_rmsnorm_linear always takes (1222-1250): masked
    single-query attention in fp32, RMSNorm over the head dim with rms_w
    (ones when None), projection onto fp32(proj_w) * wscale[:, None], plus
    fp32(proj_bias), cast to q.dtype: out [B, H, N]."""
    q, k, v, mask, proj_w, rms_w, proj_bias, wscale = map(
        _cpu, (q, k, v, mask, proj_w, rms_w, proj_bias, wscale))
    B, H, D = q.shape
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    valid = (mask > 0.5)[None, None, :].expand(B, H, -1)
    attn = _softmax_attend(q.float(), k.float(), v.float(), scale, valid)
    g = torch.ones(D, dtype=torch.float32) if rms_w is None else rms_w.to(torch.float32)
    ms = (attn * attn).mean(dim=-1, keepdim=True)
    attn = attn * torch.rsqrt(ms + eps) * g
    w = proj_w.to(torch.float32)
    if wscale is not None:
        w = w * wscale.to(torch.float32)[:, None]
    out = torch.einsum("bhd,nd->bhn", attn, w)
    if proj_bias is not None:
        out = out + proj_bias.to(torch.float32)
    return out.to(q.dtype)


# --------------------------------------------------------------------------- #
# KV step after verify
# --------------------------------------------------------------------------- #
def paged_kv_write(k_new, v_new, k_pages, v_pages, page_table, start):
    """PagedKVCache.write_inplace (mtp_engine.py:581-585) for every (b, h)
    and the T new tokens at logical positions start + t: pages[table[b, p],
    b, h, p % page_size] = new[b, h, t].to(pages.dtype). Returns the updated
    copies. Positions outside the table or with a page outside [0, P) are
    skipped (the reference would index page -1, i.e. the last page)."""
    k_new, v_new, kp, vp, table = map(_cpu, (k_new, v_new, k_pages, v_pages, page_table))
    kp, vp = kp.clone(), vp.clone()
    B, H, T, D = k_new.shape
    P, ps = kp.shape[0], kp.shape[3]
    st = _cpu(start) if torch.is_tensor(start) else torch.tensor([int(start)])
    st = st.reshape(-1).to(torch.int64)
    for b in range(B):
        s0 = int(st[b] if st.numel() == B and B > 1 else st[0])
        for t in range(T):
            p = s0 + t
            if p < 0 or p >= table.shape[1]:
                continue
            pid = int(table[b, p])
            if pid < 0 or pid >= P:
                continue
            kp[pid, b, :, p % ps] = k_new[b, :, t].to(kp.dtype)
            vp[pid, b, :, p % ps] = v_new[b, :, t].to(vp.dtype)
    return kp, vp


def verify_commit(accept, accepted_n, corrected, draft, checkpoint: int):
    """generate_fused's verify consumer (mtp_engine.py:1244-1258) with the
    KVManager bookkeeping it drives (checkpoint, rollback, append,
    commit_front; 275-331): returns (tokens [B, D + 1] int64 padded with -1,
    width, new KV length = checkpoint + width)."""
    a_n, has_reject, new_tokens, kv_advance = engine_rollback(accept, accepted_n, corrected, draft)
    B, D = _cpu(draft).shape
    tokens = torch.full((B, D + 1), -1, dtype=torch.int64)
    w = new_tokens.shape[1]
    tokens[:, :w] = new_tokens.to(torch.int64)
    return tokens, w, int(checkpoint) + kv_advance


def batch_prefix_match(ids):
    """RadixKVCache.batch_prefix_match's eager route (mtp_radix.py:195-236):
    per row the first column differing from row 0, L when none; zeros for
    R <= 1."""
    ids = _cpu(ids).to(torch.long)
    R, L = ids.shape
    if R <= 1:
        return torch.zeros((R,), dtype=torch.int32)
    diff = ids != ids[0:1, :]
    # a False sentinel column keeps argmax defined for L == 0
    padded = torch.cat([diff, torch.zeros((R, 1), dtype=torch.bool)], dim=1)
    first = padded.to(torch.int32).argmax(dim=1)
    full = torch.full((R,), L, dtype=first.dtype)
    return torch.where(diff.any(dim=1), first, full).to(torch.int32)
