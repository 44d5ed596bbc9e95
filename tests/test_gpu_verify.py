"""GPU parity of fused_verify / fused_multi_verify against the CPU oracle.

Token ids, accepted lengths, rollback indices and corrected tokens must be
bit-exact wherever the oracle's top-2 logit gap exceeds TAU (logits that
close can legitimately swap under a different fp32 summation order); rows
whose first low-gap position is at or before the first rejection are
excluded from the chain checks and counted."""
import pytest
import torch

from oracle import eager as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check_tokens(top_gpu, top_ref, gap, tau):
    top_gpu = top_gpu.cpu().reshape(-1)
    top_ref = top_ref.reshape(-1)
    sure = (gap.reshape(-1) > tau)
    assert sure.float().mean() > 0.9, "too many near-ties for a meaningful check"
    assert torch.equal(top_gpu[sure], top_ref[sure].to(top_gpu.dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,V", [(4, 64, 256), (1, 128, 1000), (70, 256, 3000), (9, 512, 50257)])
def test_fused_verify_matches_oracle(dtype, M, K, V):
    import mtp_fused_verify as FV
    g = torch.Generator().manual_seed(M + K + V)
    h = torch.randn(M, K, generator=g).to(dtype)
    W = (0.05 * torch.randn(V, K, generator=g)).to(dtype)
    b = (0.1 * torch.randn(V, generator=g)).to(dtype)
    _, top_ref = O.fused_verify(h, W, torch.zeros(M), b)
    top_ref_i, gap = O.logits_top(h, W, b)
    draft = top_ref.clone().to(torch.int64)
    draft[::2] = (draft[::2] + 1) % V  # half the rows rejected
    print(f"case verify dtype={dtype} M={M} K={K} V={V}", flush=True)
    acc, top = FV.fused_verify(h.to(DEV), W.to(DEV), draft.to(DEV), b.to(DEV))
    torch.cuda.synchronize()
    assert acc.dtype == torch.int8 and top.dtype == torch.int32
    _check_tokens(top, top_ref_i, gap, 1e-3)
    sure = gap > 1e-3
    exp_acc = (top_ref == draft.to(torch.int32)).to(torch.int8)
    assert torch.equal(acc.cpu()[sure], exp_acc[sure])


def test_verify_planted_ties_and_nan():
    from mtp_hip import ops
    V, K = 700, 64
    W = torch.zeros(V, K)
    W[10, :] = 1.0
    W[650, :] = 1.0  # tie with row 10 across column groups: 10 must win
    h = torch.ones(3, K)
    h[2] = -1.0
    acc, top = ops.verify(h.to(DEV), W.to(DEV), torch.tensor([10, 0, 0]).to(DEV))
    assert top.cpu().tolist()[:2] == [10, 10]
    assert int(top.cpu()[2]) == 0  # all others 0, rows 10/650 at -K: the first zero wins
    assert acc.cpu().tolist() == [1, 0, 1]
    Wn = W.clone()
    Wn[333, 0] = float("nan")
    _, topn = ops.verify(h.to(DEV), Wn.to(DEV), torch.zeros(3, dtype=torch.int64).to(DEV))
    assert topn.cpu().tolist() == [333, 333, 333]  # NaN is the maximum


def test_reference_multi_verify_check_seeded():
    """test_new_features.py:34-56 on the same seeded inputs."""
    import mtp_fused_verify as FV
    torch.manual_seed(1)
    B, S, K, V, D = 2, 5, 64, 256, 4
    hidden = torch.randn(B, S, K)
    W = torch.randn(V, K)
    b = torch.randn(V)
    draft = torch.randint(0, V, (B, D))
    accept, accepted_n, corrected = FV.fused_multi_verify(hidden.to(DEV), W.to(DEV),
                                                          draft.to(DEV), b.to(DEV))
    top = torch.nn.functional.linear(hidden, W, b).argmax(-1)
    for i in range(B):
        ref_n = 0
        for d in range(D):
            if top[i, d + 1] == draft[i, d]:
                ref_n = d + 1
            else:
                break
        assert accepted_n[i].item() == ref_n
        assert corrected[i].item() == top[i, 0].item()
        # prefix-masked: ones on the accepted prefix, zeros from the first rejection on
        assert accept[i].tolist() == [1] * ref_n + [0] * (D - ref_n)


def _chain_case(B, D, K, V, dtype, seed, bias):
    from mtp_hip import workloads
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(B, D + 1, K, generator=g).to(dtype)
    W = (0.05 * torch.randn(V, K, generator=g)).to(dtype)
    b = (0.1 * torch.randn(V, generator=g)).to(dtype) if bias else None
    top, gap = O.logits_top(hidden.reshape(-1, K), W, b)
    draft = workloads.make_chain_drafts(top.reshape(B, D + 1), V, seed)
    return hidden, W, b, draft, top.reshape(B, D + 1), gap.reshape(B, D + 1)


def _check_chain(out, hidden, W, b, draft, tau):
    accept, accepted_n, corrected, top = [t.cpu() for t in out]
    ra, rn, rc, rtop, gap = O.fused_multi_verify(hidden, W, draft, b)
    B, S = rtop.shape
    excluded = 0
    for i in range(B):
        first_bad = next((s for s in range(S) if not gap[i, s] > tau), S)
        if first_bad < S and first_bad <= int(rn[i]) + 1:  # near-tie at/before the first rejection
            excluded += 1
            continue
        assert int(accepted_n[i]) == int(rn[i]), i
        assert int(corrected[i]) == int(rc[i]), i
        assert torch.equal(accept[i], ra[i]), i
    assert excluded <= B // 4 + 1, f"excluded {excluded} of {B}"
    sure = gap > tau
    assert torch.equal(top[sure], rtop[sure])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,D,K,V,bias", [(2, 4, 64, 256, True), (20, 4, 128, 5000, False),
                                          (3, 0, 64, 300, True), (7, 8, 256, 20000, True)])
def test_multi_verify_matches_oracle(dtype, B, D, K, V, bias):
    from mtp_hip import ops
    hidden, W, b, draft, _, _ = _chain_case(B, D, K, V, dtype, seed=B * 31 + V, bias=bias)
    print(f"case multi dtype={dtype} B={B} D={D} K={K} V={V}", flush=True)
    out = ops.multi_verify(hidden.to(DEV), W.to(DEV), draft.to(DEV),
                           None if b is None else b.to(DEV), return_top=True)
    torch.cuda.synchronize()
    _check_chain(out, hidden, W, b, draft, 1e-3)


@pytest.mark.parametrize("B,D", [(8, 4), (6, 3), (14, 3), (10, 1), (9, 1)])
@pytest.mark.parametrize("bias", [False, True])
def test_fp32_verify_eight_row_remainder(B, D, bias, tune):
    """fp32 rows past whole 16-row tiles (40 = 2 x 16 + 8, 24, 56, 20 and
    18: 4 and 6 padding rows) on the 4 x 4 MFMA form of the streaming
    kernel, against the oracle, and against the padded form (tuning key
    skv_r8 = 0) wherever the top-2 gap is clear."""
    from mtp_hip import ops
    K, V = 256, 20000
    hidden, W, b, draft, top, gap = _chain_case(B, D, K, V, torch.float32, seed=B * 17 + D,
                                                bias=bias)
    hd, Wd, dd = hidden.to(DEV), W.to(DEV), draft.to(DEV)
    bd = None if b is None else b.to(DEV)
    assert ops.verify_route(hd, Wd, bd) == "stream"
    print(f"case fp32 remainder B={B} D={D} bias={bias}", flush=True)
    out = ops.multi_verify(hd, Wd, dd, bd, return_top=True)
    torch.cuda.synchronize()
    _check_chain(out, hidden, W, b, draft, 1e-3)
    tune(skv_r8=0)
    pad = ops.multi_verify(hd, Wd, dd, bd, return_top=True)
    torch.cuda.synchronize()
    sure = (gap > 1e-3).reshape(-1)
    assert torch.equal(out[3].cpu().reshape(-1)[sure], pad[3].cpu().reshape(-1)[sure])


@pytest.mark.parametrize("tw", [8, 40, 200, 256])
@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 20000), (torch.float32, 3001)])
def test_streaming_verify_tile_widths(tw, dtype, V, tune):
    """The streaming verify kernel with tw columns per tile (tuning key
    skv_tw; columns past tw read zeros and stay out of the argmax), a bias
    and a ragged last tile: against the oracle wherever the top-2 gap is
    clear."""
    from mtp_hip import ops
    B, D, K = 6, 4, 256
    hidden, W, b, draft, top, gap = _chain_case(B, D, K, V, dtype, seed=tw + V, bias=True)
    hd, Wd, dd, bd = hidden.to(DEV), W.to(DEV), draft.to(DEV), b.to(DEV)
    assert ops.verify_route(hd, Wd, bd) == "stream"
    tune(skv_tw=tw)
    print(f"case skv tw={tw} dtype={dtype} V={V}", flush=True)
    out = ops.multi_verify(hd, Wd, dd, bd, return_top=True)
    torch.cuda.synchronize()
    _check_chain(out, hidden, W, b, draft, 1e-3)


def test_workspace_shared_across_kernels_and_shapes():
    """Split-K linear, verify and multi-verify calls of different shapes share
    one per-stream workspace; each must still match the oracle (the arrival
    counters live in a fixed prefix that every launch leaves at zero)."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(99)
    x = torch.randn(48, 1024, generator=g).to(torch.bfloat16)
    W = (0.05 * torch.randn(3000, 1024, generator=g)).to(torch.bfloat16)
    h = torch.randn(3, 5, 256, generator=g).to(torch.bfloat16)
    Wv = (0.05 * torch.randn(6000, 256, generator=g)).to(torch.bfloat16)
    ref_y = O.rmsnorm_linear(x, W, None, 1e-6)
    top, gap = O.logits_top(h.reshape(-1, 256), Wv)
    draft = top.reshape(3, 5)[:, 1:].to(torch.int64)
    for rep in range(3):
        y = ops.rmsnorm_linear(x.to(DEV), W.to(DEV), None, 1e-6)
        _, _, _, t = ops.multi_verify(h.to(DEV), Wv.to(DEV), draft.to(DEV), return_top=True)
        _, t1 = ops.verify(h.reshape(-1, 256).to(DEV), Wv.to(DEV), top.to(DEV))
        torch.cuda.synchronize()
        from conftest import close
        assert close(y, ref_y, 2e-2)[0], rep
        sure = gap > 1e-3
        assert torch.equal(t.cpu().reshape(-1)[sure], top[sure]), rep
        assert torch.equal(t1.cpu()[sure], top[sure]), rep


def test_multi_verify_workload_full_size():
    """The multi-verify workload: 8 x (4+1) hidden bf16 [40,4096], lm_head
    [128256,4096] bf16, geometric(0.6) accepted prefixes."""
    from mtp_hip import ops, workloads
    d = workloads.multi_verify()
    hidden, W = d["hidden"], d["weight"]
    top, gap = O.logits_top(hidden.reshape(-1, hidden.shape[-1]), W)
    draft = workloads.make_chain_drafts(top.reshape(d["B"], d["D"] + 1), W.shape[0], d["seed"])
    print("case multi-verify workload", flush=True)
    Wd = W.to(DEV)
    out = ops.multi_verify(hidden.to(DEV), Wd, draft.to(DEV), None, return_top=True)
    torch.cuda.synchronize()
    _check_chain(out, hidden, W, None, draft, 1e-4)
    # rollback consumer on device outputs equals the oracle's
    ra, rn, rc, _, _ = O.fused_multi_verify(hidden, W, draft)
    got = O.engine_rollback(out[0], out[1], out[2], draft)
    exp = O.engine_rollback(ra, rn, rc, draft)
    assert got[:2] == exp[:2] and torch.equal(got[2], exp[2])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_multi_verify_engine_call_full_size(dtype):
    """The engine's own verify call, fused_multi_verify(hidden_all,
    proj.weight, draft, bias=proj.bias) (mtp_engine.py:1237-1242,
    1320-1322), at the multi-verify workload's size: 8 x (4+1) hidden rows,
    lm_head [128256, 4096] with a bias [128256], in bf16 and in the
    engine's default fp32 (2.1 GB of W). Both take the persistent
    W-streaming kernel; tokens, accepted_n and corrected equal the oracle's
    wherever the top-2 gap is clear."""
    from mtp_hip import ops, workloads
    d = workloads.multi_verify(dtype=dtype, bias=True)
    hidden, W, b = d["hidden"], d["weight"], d["bias"]
    top, gap = O.logits_top(hidden.reshape(-1, hidden.shape[-1]), W, b)
    draft = workloads.make_chain_drafts(top.reshape(d["B"], d["D"] + 1), W.shape[0], d["seed"])
    print(f"case engine verify call dtype={dtype}", flush=True)
    hd, Wd, bd = hidden.to(DEV), W.to(DEV), b.to(DEV)
    assert ops.verify_route(hd, Wd, bd) == "stream"
    out = ops.multi_verify(hd, Wd, draft.to(DEV), bd, return_top=True)
    torch.cuda.synchronize()
    _check_chain(out, hidden, W, b, draft, 1e-4)
    # without the bias the tokens differ on some rows: the bias is applied
    nb = ops.multi_verify(hd, Wd, draft.to(DEV), None, return_top=True)[3]
    torch.cuda.synchronize()
    top_nb, gap_nb = O.logits_top(hidden.reshape(-1, hidden.shape[-1]), W)
    sure = (gap_nb > 1e-4).reshape(-1)
    assert torch.equal(nb.cpu().reshape(-1)[sure], top_nb[sure].to(torch.int32))
    assert not torch.equal(top_nb, top)


def test_verify_weights_past_4gib():
    """W of 4.4 GB (fp32 [270000, 4096]): the persistent kernel addresses W
    through one buffer descriptor per 256-row tile, so tiles past 2 and 4
    GiB read their own rows (the last tile starts at 4.42e9 bytes)."""
    from mtp_hip import ops, workloads
    g = torch.Generator().manual_seed(270000)
    V, K, M = 270000, 4096, 8
    W = workloads._weight(g, V, K, dtype=torch.float32)
    h = torch.randn(M, K, generator=g)
    b = 0.5 * torch.randn(V, generator=g)
    # the winners of some rows planted in the last tiles
    for m, n in enumerate((V - 1, V - 200, V // 2 + 7, 262144 + 5)):
        W[n] = 0.05 * h[m]
    top, gap = O.logits_top(h, W, b)
    assert int(top[0]) == V - 1 and int(top[3]) == 262144 + 5
    print("case verify W 4.4 GB", flush=True)
    hd, Wd, bd = h.to(DEV), W.to(DEV), b.to(DEV)
    del W
    assert ops.verify_route(hd, Wd, bd) == "stream"
    draft = top.clone().to(torch.int64)
    draft[1::2] = (draft[1::2] + 1) % V
    acc, t = ops.verify(hd, Wd, draft.to(DEV), bd)
    torch.cuda.synchronize()
    _check_tokens(t, top, gap, 1e-3)
    sure = gap > 1e-3
    assert torch.equal(acc.cpu()[sure], (top == draft.to(torch.int32)).to(torch.int8)[sure])


@pytest.mark.parametrize("route", ["stream", "column_group", "generic"])
def test_multi_verify_textbook_convention(route, tune):
    """convention="textbook": draft d is checked against top[b, d] and
    corrected = top[b, accepted_n] (the bonus token after D accepts), on
    each verify kernel, against the oracle's textbook chain; drafts built
    from top[b, :D] so that whole chains, partial chains and immediate
    rejections all occur."""
    from mtp_hip import ops
    B, D, V = 12, 4, 20000
    K = 250 if route == "generic" else 512
    g = torch.Generator().manual_seed(41)
    hidden = torch.randn(B, D + 1, K, generator=g).to(torch.bfloat16)
    W = (0.05 * torch.randn(V, K, generator=g)).to(torch.bfloat16)
    b = (0.1 * torch.randn(V, generator=g)).to(torch.bfloat16)
    top, gap = O.logits_top(hidden.reshape(-1, K), W, b)
    top, gap = top.reshape(B, D + 1), gap.reshape(B, D + 1)
    draft = top[:, :D].clone().to(torch.int64)
    for i in range(B):  # row i rejects at position i % (D + 1) (D + 1: accepts all)
        j = i % (D + 1)
        if j < D:
            draft[i, j] = (draft[i, j] + 1) % V
    if route == "column_group":
        tune(verify_wstream=1)
    hd, Wd, bd = hidden.to(DEV), W.to(DEV), b.to(DEV)
    assert ops.verify_route(hd, Wd, bd) == route
    print(f"case textbook route={route}", flush=True)
    acc, n, corr, t = ops.multi_verify(hd, Wd, draft.to(DEV), bd, return_top=True,
                                       convention="textbook")
    torch.cuda.synchronize()
    ra, rn, rc, rtop, rgap = O.fused_multi_verify(hidden, W, draft, b, convention="textbook")
    assert bool((rgap > 1e-3).all()), "a near-tie in this seeded case"
    assert torch.equal(t.cpu(), rtop.to(torch.int32))
    assert torch.equal(acc.cpu(), ra) and torch.equal(n.cpu(), rn) and torch.equal(corr.cpu(), rc)
    assert rn.tolist() == [i % (D + 1) for i in range(B)]
    # the reference convention on the same call differs
    _, n_ref, corr_ref = ops.multi_verify(hd, Wd, draft.to(DEV), bd)
    torch.cuda.synchronize()
    assert torch.equal(corr_ref.cpu(), rtop[:, 0].to(torch.int32))


# --- the persistent streaming path: 16-bit, no bias, K % 512 == 0 ---------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,K,V", [(1, 512, 3000), (33, 1024, 50257), (64, 512, 20000),
                                   (70, 512, 128), (5, 2048, 70000)])
def test_fused_verify_streaming_path(dtype, M, K, V):
    """Row chunks of 64 (70 rows: two launches), tiles past V (V % 64 != 0),
    grids smaller than the persistent 256 (V = 128, 3000)."""
    import mtp_fused_verify as FV
    g = torch.Generator().manual_seed(M * 7 + V)
    h = torch.randn(M, K, generator=g).to(dtype)
    W = (0.05 * torch.randn(V, K, generator=g)).to(dtype)
    top_ref, gap = O.logits_top(h, W)
    draft = top_ref.clone().to(torch.int64)
    draft[::3] = (draft[::3] + 1) % V
    print(f"case verify-stream dtype={dtype} M={M} K={K} V={V}", flush=True)
    acc, top = FV.fused_verify(h.to(DEV), W.to(DEV), draft.to(DEV))
    torch.cuda.synchronize()
    _check_tokens(top, top_ref, gap, 1e-3)
    sure = gap > 1e-3
    exp_acc = (top_ref == draft.to(torch.int32)).to(torch.int8)
    assert torch.equal(acc.cpu()[sure], exp_acc[sure])


def test_verify_streaming_planted_ties_and_nan():
    """Ties between columns handled by different workgroups and tiles: the
    lowest index wins; a NaN logit is the maximum; all-zero logits give 0."""
    from mtp_hip import ops
    V, K = 40000, 512
    W = torch.zeros(V, K)
    W[10, :] = 1.0 / 64
    W[650, :] = 1.0 / 64     # another tile of another workgroup
    W[39999, :] = 1.0 / 64   # the last, partial tile
    h = torch.ones(3, K)
    h[2] = -1.0
    Wb = W.to(torch.bfloat16)
    acc, top = ops.verify(h.to(torch.bfloat16).to(DEV), Wb.to(DEV), torch.tensor([10, 0, 0]).to(DEV))
    assert top.cpu().tolist() == [10, 10, 0]
    assert acc.cpu().tolist() == [1, 0, 1]
    Wn = Wb.clone()
    Wn[33333, 7] = float("nan")
    _, topn = ops.verify(h.to(torch.bfloat16).to(DEV), Wn.to(DEV), torch.zeros(3, dtype=torch.int64).to(DEV))
    assert topn.cpu().tolist() == [33333, 33333, 33333]
    z = torch.zeros(2, K, dtype=torch.bfloat16)
    _, topz = ops.verify(z.to(DEV), Wn.to(DEV), torch.zeros(2, dtype=torch.int64).to(DEV))
    assert topz.cpu().tolist() == [33333, 33333]  # 0 * NaN is NaN
    _, topz = ops.verify(z.to(DEV), Wb.to(DEV), torch.zeros(2, dtype=torch.int64).to(DEV))
    assert topz.cpu().tolist() == [0, 0]


@pytest.mark.parametrize("B,D,K,V", [(8, 4, 1024, 30000), (13, 4, 512, 5000), (4, 0, 512, 777)])
def test_multi_verify_streaming_path(B, D, K, V):
    """13 x 5 = 65 rows: two row chunks (60 + 5) in two launches."""
    from mtp_hip import ops
    hidden, W, b, draft, _, _ = _chain_case(B, D, K, V, torch.bfloat16, seed=B + K + V, bias=False)
    print(f"case multi-stream B={B} D={D} K={K} V={V}", flush=True)
    out = ops.multi_verify(hidden.to(DEV), W.to(DEV), draft.to(DEV), None, return_top=True)
    torch.cuda.synchronize()
    _check_chain(out, hidden, W, b, draft, 1e-3)


def test_verify_streaming_and_column_group_paths_agree(tune):
    """The persistent streaming kernel and the column-group kernel
    (tuning key verify_wstream) give the same tokens wherever the top-2 gap is clear."""
    from mtp_hip import ops
    hidden, W, _, draft, top, gap = _chain_case(6, 4, 1024, 60000, torch.bfloat16, seed=5,
                                                bias=False)
    hd, Wd, dd = hidden.to(DEV), W.to(DEV), draft.to(DEV)
    a = ops.multi_verify(hd, Wd, dd, None, return_top=True)
    tune(verify_wstream=1)
    b = ops.multi_verify(hd, Wd, dd, None, return_top=True)
    torch.cuda.synchronize()
    sure = (gap > 1e-3).reshape(-1)
    assert torch.equal(a[3].cpu().reshape(-1)[sure], b[3].cpu().reshape(-1)[sure])
    assert torch.equal(a[3].cpu().reshape(-1)[sure], top.reshape(-1)[sure].to(torch.int32))


# --- any K, any alignment, mixed dtypes: the generic kernel -------------------

GEN_CASES = [
    # name, hidden dtype, weight dtype, K, bias dtype
    ("odd_k", torch.bfloat16, torch.bfloat16, 100, None),
    ("mixed_f32_bf16", torch.float32, torch.bfloat16, 256, None),
    ("mixed_bf16_f32", torch.bfloat16, torch.float32, 64, torch.float32),
    ("f16_bias_f32", torch.float16, torch.float16, 96, torch.float32),
    ("unaligned", torch.bfloat16, torch.bfloat16, 512, None),
]


@pytest.mark.parametrize("name,hdt,wdt,K,bdt", GEN_CASES)
def test_verify_generic_path(name, hdt, wdt, K, bdt):
    """Inputs the reference accepts that the streaming kernels do not take:
    K % 8 != 0, hidden and W of different float dtypes (both upcast as in
    mtp_fused_verify.py:163), a bias of another dtype, and rows that start
    2 bytes past a 16-byte boundary (an offset view)."""
    from mtp_hip import ops
    M, V = 9, 7000
    g = torch.Generator().manual_seed(K + V)
    h = torch.randn(M, K, generator=g).to(hdt)
    W = (0.05 * torch.randn(V, K, generator=g)).to(wdt)
    b = None if bdt is None else (0.1 * torch.randn(V, generator=g)).to(bdt)
    top, gap = O.logits_top(h, W, b)
    draft = top.clone().to(torch.int64)
    draft[1::2] = (draft[1::2] + 1) % V
    hd, Wd = h.to(DEV), W.to(DEV)
    if name == "unaligned":
        buf = torch.empty(M * K + 1, dtype=hdt, device=DEV)
        buf[1:].copy_(hd.reshape(-1))
        hd = buf[1:].view(M, K)
        assert hd.data_ptr() % 16 == 2
        bufw = torch.empty(V * K + 1, dtype=wdt, device=DEV)
        bufw[1:].copy_(Wd.reshape(-1))
        Wd = bufw[1:].view(V, K)
    print(f"case verify-generic {name}", flush=True)
    acc, t = ops.verify(hd, Wd, draft.to(DEV), None if b is None else b.to(DEV))
    torch.cuda.synchronize()
    _check_tokens(t, top, gap, 1e-3)
    sure = gap > 1e-3
    assert torch.equal(acc.cpu()[sure], (top == draft.to(torch.int32)).to(torch.int8)[sure])
    # the chain variant over the same rows
    B, S = 3, 3
    hh = h[: B * S].reshape(B, S, K)
    dd = top[: B * S].reshape(B, S)[:, 1:].clone().to(torch.int64)
    dd[1, 1] = (dd[1, 1] + 1) % V
    out = ops.multi_verify(hh.to(DEV), W.to(DEV), dd.to(DEV), None if b is None else b.to(DEV),
                           return_top=True)
    torch.cuda.synchronize()
    _check_chain(out, hh, W, b, dd, 1e-3)


@pytest.mark.parametrize("K", [256, 768])
def test_verify_streaming_path_k_multiple_of_256(K):
    """The persistent kernel takes K % 256 == 0 (whole rounds of its 4-slot
    register ring over the 64-k stages of a tile)."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(K)
    h = torch.randn(12, K, generator=g).to(torch.bfloat16)
    W = (0.05 * torch.randn(9000, K, generator=g)).to(torch.bfloat16)
    top, gap = O.logits_top(h, W)
    _, t = ops.verify(h.to(DEV), W.to(DEV), top.to(DEV))
    torch.cuda.synchronize()
    _check_tokens(t, top, gap, 1e-3)


def test_persistent_verify_after_other_kernels_with_negative_logits():
    """The persistent verify kernel after a split-K linear, an INT4 call and
    a chunked attention on the same stream's workspace (all of which leave
    scratch data behind the counter prefix), on rows whose logits are all
    negative (h = -1, W > 0): a stale key would win the atomic max there.
    Its row keys live in the counter prefix, which every launch leaves at
    zero."""
    from mtp_hip import _lib, ops, workloads
    g = torch.Generator().manual_seed(123)
    x = torch.randn(48, 1024, generator=g).to(torch.bfloat16)
    Wl = (0.05 * torch.randn(3000, 1024, generator=g)).to(torch.bfloat16)
    K, V = 512, 20000
    h = -torch.ones(6, K).to(torch.bfloat16)
    Wv = (0.001 + 0.05 * torch.rand(V, K, generator=g)).to(torch.bfloat16)
    top, gap = O.logits_top(h, Wv)
    hb = h.reshape(2, 3, K)
    dr = top.reshape(2, 3)[:, 1:].to(torch.int64)
    N, H, D, Lc, ps = 64, 4, 128, 1500, 16
    q = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    kt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(N, H, D, generator=g).to(torch.bfloat16)
    npg = (Lc + ps - 1) // ps
    kp = torch.randn(npg, 1, H, ps, D, generator=g).to(torch.bfloat16)
    vp = torch.randn(npg, 1, H, ps, D, generator=g).to(torch.bfloat16)
    table = torch.arange(npg).repeat_interleave(ps)[:Lc].reshape(1, Lc).to(torch.int32)
    tm = workloads.draft_tree_mask(16, 4)[:N, :N]
    W4 = 0.02 * torch.randn(256, 1024, generator=g)
    pk, sc = O.quantize_int4(W4, 128, torch.float16, "ref")
    for rep in range(2):
        with _lib.tuning(sk_splits=3):
            ops.rmsnorm_linear(x.to(DEV), Wl.to(DEV), None, 1e-6)
        ops.int4_matmul(x.to(DEV), pk.to(DEV), sc.to(DEV), 1024, 128, norm=True)
        from mtp_kernels import tree_verify_attention
        tree_verify_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), table.to(DEV), ps, kt.to(DEV),
                              vt.to(DEV), tm.to(DEV))
        _, t1 = ops.verify(h.to(DEV), Wv.to(DEV), top.to(DEV))
        out = ops.multi_verify(hb.to(DEV), Wv.to(DEV), dr.to(DEV), return_top=True)
        torch.cuda.synchronize()
        t1 = t1.cpu()
        assert int(t1.min()) >= 0 and int(t1.max()) < V, rep
        _check_tokens(t1, top, gap, 1e-4)
        _check_tokens(out[3], top, gap, 1e-4)
