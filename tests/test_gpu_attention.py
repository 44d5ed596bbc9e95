"""GPU parity of the tree / paged attention family and the tree-verify step
against the oracle's restatement of the reference's eager attention
(mtp_kernels.py:832-872). Outputs are in the input dtype: 2e-2 for bf16 /
f16 (the attention probabilities enter the second MFMA rounded to that
type), 1e-5 for fp32 (fallback kernel), with |y - ref| <= rtol * (|ref| +
RMS(ref))."""
from __future__ import annotations

import math

import pytest
import torch

from conftest import close
from oracle import eager as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RTOL = {torch.bfloat16: 2e-2, torch.float16: 2e-2, torch.float32: 1e-5}


def _paged(g, B, H, L, D, ps, dtype, extra_pages=3):
    """Random pages [P, B, H, ps, D] and a table placing the L keys of each
    batch row on a random permutation of pages (last page partial)."""
    npg = (L + ps - 1) // ps
    P = npg + extra_pages
    kp = torch.randn(P, B, H, ps, D, generator=g).to(dtype)
    vp = torch.randn(P, B, H, ps, D, generator=g).to(dtype)
    table = torch.stack([torch.randperm(P, generator=g)[:npg].repeat_interleave(ps)[:L]
                         for _ in range(B)]).to(torch.int32)
    return kp, vp, table


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,H,L,D", [(2, 4, 37, 128), (1, 3, 100, 64), (3, 2, 5, 128),
                                     (2, 2, 33, 96)])
def test_tree_attention(B, H, L, D, dtype):
    from mtp_kernels import fused_tree_attention
    g = torch.Generator().manual_seed(B * 100 + L + D)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k = torch.randn(B, H, L, D, generator=g).to(dtype)
    v = torch.randn(B, H, L, D, generator=g).to(dtype)
    mask = (torch.rand(L, generator=g) > 0.3).float()
    mask[L // 2] = 1.0
    print(f"case tree B={B} H={H} L={L} D={D} {dtype}", flush=True)
    out = fused_tree_attention(q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV)).cpu()
    ref = O.tree_attention(q, k, v, mask)
    assert out.dtype == dtype and out.shape == (B, H, D)
    ok, worst = close(out, ref, RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"


def test_tree_attention_masks_as_bool_and_all_masked_is_nan():
    from mtp_kernels import fused_tree_attention
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 20, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 2, 20, 128, generator=g).to(torch.bfloat16)
    m = torch.rand(20, generator=g) > 0.5
    m[0] = True
    out = fused_tree_attention(q.to(DEV), k.to(DEV), v.to(DEV), m.to(DEV)).cpu()
    ok, worst = close(out, O.tree_attention(q, k, v, m.float()), 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"
    nan = fused_tree_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.zeros(20, device=DEV)).cpu()
    assert torch.isnan(nan.float()).all()


@pytest.mark.parametrize("B,H,L,D,ps", [(2, 3, 50, 128, 16), (1, 8, 2048, 128, 16),
                                        (4, 2, 300, 64, 8), (1, 1, 1, 128, 16)])
def test_paged_attention(B, H, L, D, ps):
    from mtp_kernels import fused_paged_attention
    g = torch.Generator().manual_seed(L + B)
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    kp, vp, table = _paged(g, B, H, L, D, ps, torch.bfloat16)
    print(f"case paged B={B} H={H} L={L} D={D} ps={ps}", flush=True)
    out = fused_paged_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps).cpu()
    ref = O.paged_attention(q, kp, vp, table, ps)
    ok, worst = close(out, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("N,H,Lc,depth,br", [(5, 2, 40, 3, 2), (21, 4, 300, 6, 4),
                                             (40, 2, 0, 5, 8), (64, 3, 1000, 16, 4)])
def test_tree_verify_attention_small(N, H, Lc, depth, br):
    from mtp_kernels import tree_verify_attention
    from mtp_hip import workloads
    g = torch.Generator().manual_seed(N + Lc)
    D, ps = 128, 16
    tm = workloads.draft_tree_mask(depth, br)[:N, :N]
    q = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kp, vp, table = _paged(g, 1, H, max(Lc, 1), D, ps, torch.bfloat16)
    table = table[:, :Lc]
    print(f"case tree-verify N={N} H={H} Lc={Lc}", flush=True)
    out = tree_verify_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps,
                                kt.to(DEV), vt.to(DEV), tm.to(DEV)).cpu()
    ref = O.tree_verify_attention(q, kp, vp, table, ps, kt, vt, tm)
    ok, worst = close(out, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"


def test_tree_verify_step_full_size():
    """The 64-node tree-verify step: attention over 2048 paged context tokens
    plus the ancestors, then RMSNorm+linear 4096 -> 4096 (bf16, no gamma)."""
    from mtp_kernels import fused_rmsnorm_linear, tree_verify_attention
    from mtp_hip import workloads
    d = workloads.tree_verify()
    print("case tree-verify workload", flush=True)
    dv = {k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in d.items()}
    att = tree_verify_attention(dv["q"], dv["k_pages"], dv["v_pages"], dv["page_table"],
                                d["page_size"], dv["k_tree"], dv["v_tree"], dv["tree_mask"])
    y = fused_rmsnorm_linear(att.reshape(64, -1), dv["weight"], None, d["eps"]).cpu()
    att_ref = O.tree_verify_attention(d["q"], d["k_pages"], d["v_pages"], d["page_table"],
                                      d["page_size"], d["k_tree"], d["v_tree"], d["tree_mask"])
    ok, worst = close(att.cpu(), att_ref, 2e-2)
    assert ok, f"attention worst err/bound = {worst:.3g}"
    y_ref = O.rmsnorm_linear(att_ref.reshape(64, -1), d["weight"], None, d["eps"], 1.0)
    ok, worst = close(y, y_ref, 2e-2)
    assert ok, f"linear worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("chunk_blocks", [1, 3, 5, 20, 36])
def test_tree_verify_attention_chunkings(chunk_blocks, tune):
    """Forced chunk lengths (blocks of 64 keys per workgroup) over 35 context
    blocks plus 1 tree block: one block per chunk (36 partials merged), a
    chunk that straddles the context / tree boundary (3), a tree-only chunk
    (5), and chunks longer than the 1024-key page-table window (20, 36: the
    window is reloaded mid-chunk)."""
    from mtp_kernels import tree_verify_attention
    from mtp_hip import workloads
    tune(attn_chunk_blocks=chunk_blocks)
    g = torch.Generator().manual_seed(chunk_blocks)
    N, H, Lc, D, ps = 64, 3, 2200, 128, 16
    tm = workloads.draft_tree_mask(16, 4)[:N, :N]
    q = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kp, vp, table = _paged(g, 1, H, Lc, D, ps, torch.bfloat16)
    print(f"case tree-verify chunk_blocks={chunk_blocks}", flush=True)
    out = tree_verify_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps,
                                kt.to(DEV), vt.to(DEV), tm.to(DEV)).cpu()
    ref = O.tree_verify_attention(q, kp, vp, table, ps, kt, vt, tm)
    ok, worst = close(out, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("N,H,Lc,D,dtype", [(40, 2, 500, 64, torch.bfloat16),
                                            (33, 4, 777, 128, torch.float16),
                                            (17, 2, 64, 64, torch.float16)])
def test_tree_verify_attention_head_dims_and_fp16(N, H, Lc, D, dtype):
    from mtp_kernels import tree_verify_attention
    from mtp_hip import workloads
    g = torch.Generator().manual_seed(N * D + Lc)
    ps = 16
    tm = workloads.draft_tree_mask(16, 4)[:N, :N]
    q = torch.randn(N, H, D, generator=g).to(dtype)
    kt = torch.randn(N, H, D, generator=g).to(dtype)
    vt = torch.randn(N, H, D, generator=g).to(dtype)
    kp, vp, table = _paged(g, 1, H, Lc, D, ps, dtype)
    print(f"case tree-verify N={N} H={H} Lc={Lc} D={D} {dtype}", flush=True)
    out = tree_verify_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps,
                                kt.to(DEV), vt.to(DEV), tm.to(DEV)).cpu()
    ref = O.tree_verify_attention(q, kp, vp, table, ps, kt, vt, tm)
    ok, worst = close(out, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("N,H,Lc,ps", [(33, 2, 130, 16), (48, 3, 1500, 16), (64, 2, 0, 16),
                                       (64, 2, 100, 5), (57, 1, 4000, 32)])
def test_tree_verify_attention_query_tilings(N, H, Lc, ps, tune):
    """33 .. 64 queries at head dim 128 take the 32-query-tile kernel by
    default; the 16-query-tile kernel (attn32=0) gives the oracle's answer on
    the same inputs too: context only up to a partial page, odd page sizes,
    a tree-only key set and a context longer than the page-table window."""
    from mtp_kernels import tree_verify_attention
    from mtp_hip import workloads
    g = torch.Generator().manual_seed(N * 7 + Lc + ps)
    D = 128
    tm = workloads.draft_tree_mask(16, 4)[:N, :N]
    q = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kp, vp, table = _paged(g, 1, H, max(Lc, 1), D, ps, torch.bfloat16)
    table = table[:, :Lc]
    ref = O.tree_verify_attention(q, kp, vp, table, ps, kt, vt, tm)
    outs = []
    for attn32 in (-1, 0):
        tune(attn32=attn32)
        print(f"case tree-verify tiling N={N} H={H} Lc={Lc} ps={ps} attn32={attn32}", flush=True)
        out = tree_verify_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps,
                                    kt.to(DEV), vt.to(DEV), tm.to(DEV)).cpu()
        ok, worst = close(out, ref, 2e-2)
        assert ok, f"attn32={attn32}: worst err/bound = {worst:.3g}"
        outs.append(out)
    # deterministic: the default kernel repeats itself bit for bit
    tune(attn32=-1)
    again = tree_verify_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps,
                                  kt.to(DEV), vt.to(DEV), tm.to(DEV)).cpu()
    assert torch.equal(again, outs[0])


def test_tree_verify_attention_fully_masked_node_is_nan():
    """A tree node whose mask row is all zero with no context keys: NaN, as
    the reference's softmax of an all -inf row, on both query tilings."""
    from mtp_kernels import tree_verify_attention
    from mtp_hip import _lib, workloads
    g = torch.Generator().manual_seed(11)
    N, H, D, ps = 40, 2, 128, 16
    tm = workloads.draft_tree_mask(16, 4)[:N, :N].clone()
    tm[5] = 0.0
    q = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kp, vp, table = _paged(g, 1, H, 1, D, ps, torch.bfloat16)
    table = table[:, :0]
    ref = O.tree_verify_attention(q, kp, vp, table, ps, kt, vt, tm)
    try:
        for attn32 in (-1, 0):
            _lib.set_tuning(attn32=attn32)
            print(f"case tree-verify masked node attn32={attn32}", flush=True)
            out = tree_verify_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps,
                                        kt.to(DEV), vt.to(DEV), tm.to(DEV)).cpu()
            assert torch.isnan(out[5].float()).all()
            keep = torch.ones(N, dtype=torch.bool)
            keep[5] = False
            ok, worst = close(out[keep], ref[keep], 2e-2)
            assert ok, f"attn32={attn32}: worst err/bound = {worst:.3g}"
    finally:
        _lib.set_tuning(attn32=-1)
