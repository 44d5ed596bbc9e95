"""HIP-graph capture of the hot path: a draft step (RMSNorm, RMSNorm ->
linear head, greedy token + embedding, combine-norm), the fp32 linear
routes (one launch, streaming, row-chunk with K-splits), the fp8 skinny
routes (prep + wave-specialised GEMM, prep + split-K GEMM, single launch),
the tree-verify attention (chunk launch + merge launch),
the persistent multi-verify and the device-side
commit are each captured once on a warmed-up stream and replayed with new
input contents; every replay equals the eager result bit for bit (the
kernels re-arm their tickets and keys themselves), with eager work and
synchronisation between replays."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _capture(fn, warm=3):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = fn()
    return graph, out


def _replays(graph, out, fill_inputs, eager, n=4):
    for i in range(n):
        fill_inputs(i)
        graph.replay()
        torch.cuda.synchronize()
        ref = eager()
        torch.cuda.synchronize()
        outs = out if isinstance(out, tuple) else (out,)
        refs = ref if isinstance(ref, tuple) else (ref,)
        for o, r in zip(outs, refs):
            assert torch.equal(o, r), f"replay {i}"
        _ = torch.ones(1000, device=DEV).sum().item()  # eager work between replays


def test_draft_step_graph_replay():
    from mtp_hip import ops
    g = torch.Generator().manual_seed(1)
    B, Hd, V = 4, 1024, 32000
    dt = torch.bfloat16
    hidden = torch.randn(B, Hd, generator=g).to(dt).to(DEV)
    W = (0.05 * torch.randn(V, Hd, generator=g)).to(dt).to(DEV)
    bias = (0.1 * torch.randn(V, generator=g)).to(dt).to(DEV)
    head_w = (1 + 0.1 * torch.randn(Hd, generator=g)).to(dt).to(DEV)
    comb_w = (1 + 0.1 * torch.randn(Hd, generator=g)).to(dt).to(DEV)
    table = torch.randn(V, Hd, generator=g).to(dt).to(DEV)

    def step():
        h_norm = ops.rmsnorm(hidden, head_w, 1e-6)
        logits = ops.rmsnorm_linear(hidden, W, bias, 1e-6)
        tok, emb = ops.argmax(logits, table)
        comb = ops.rmsnorm(h_norm, comb_w, 1e-6, residual=emb)
        return logits, tok, emb, comb

    graph, out = _capture(step)
    seeds = [torch.randn(B, Hd, generator=g).to(dt).to(DEV) for _ in range(4)]
    _replays(graph, out, lambda i: hidden.copy_(seeds[i]), step)


@pytest.mark.parametrize("route", ["small", "stream", "tiled"])
def test_fp32_linear_graph_replay(route):
    """The fp32 TF32-off routes under capture: the one-launch kernel (x [16,
    1024]), the streaming kernel at the fp32 head's shape (x [8, 4096], W
    [4096, 4096]) and the tiled row-chunk kernel with grid K-splits (tuning
    key sf32 = 0; its split-K tickets are re-armed on every replay)."""
    from mtp_hip import _lib as L, ops, workloads
    if route == "stream":
        d = workloads.fp32_linear(M=8, K=4096, N=4096)
    else:
        d = workloads.fp32_linear()
    print(f"case fp32 graph route={route} x={tuple(d['x'].shape)}", flush=True)
    x = d["x"].to(DEV)
    W = d["weight"].to(DEV)
    gm = d["gamma"].to(DEV)
    L.set_tuning(sf32=0 if route == "tiled" else -1)
    try:
        fn = lambda: ops.rmsnorm_linear(x, W, None, d["eps"], 1.0, gamma=gm)  # noqa: E731
        graph, out = _capture(fn)
        g = torch.Generator().manual_seed(2)
        xs = [torch.randn(x.shape, generator=g).to(DEV) for _ in range(4)]
        _replays(graph, out, lambda i: x.copy_(xs[i]), fn)
    finally:
        L.set_tuning(sf32=-1)


@pytest.mark.parametrize("M,N,keys", [(64, 14336, {}), (48, 4096, {}), (32, 14336, {}),
                                      (64, 4096, {"sk_splits": 3})])
def test_fp8_linear_graph_replay(M, N, keys):
    """The fp8 RMSNorm -> linear routes under capture at K = 4096 with gamma:
    the prep launch + wave-specialised GEMM (64 rows x 14336), the
    two-launch GEMM with planned and forced K-splits (48 / 64 rows x 4096:
    split tickets re-armed on every replay) and the single-launch kernel
    (32 rows x 14336)."""
    from mtp_hip import _lib as L, ops, workloads
    d = workloads.fp8_linear(M)
    K = d["x"].shape[1]
    g = torch.Generator().manual_seed(M + N)
    wq = d["weight_fp8"][:N].to(DEV)
    ws = d["wscale"][:N].to(DEV)
    x = d["x"].to(DEV)
    gm = d["gamma"].to(DEV)
    print(f"case fp8 graph M={M} N={N} K={K} keys={keys}", flush=True)
    L.set_tuning(**keys)
    try:
        fn = lambda: ops.rmsnorm_linear_fp8(x, wq, ws, None, d["eps"], gamma=gm)  # noqa: E731
        graph, out = _capture(fn)
        xs = [torch.randn(x.shape, generator=g).to(x.dtype).to(DEV) for _ in range(4)]
        _replays(graph, out, lambda i: x.copy_(xs[i]), fn)
    finally:
        L.set_tuning(**{k: -1 for k in keys})


def test_tree_verify_attention_graph_replay():
    """The tree-verify attention (64 nodes, 4 heads, 700 paged context keys
    and the tree keys in one-block chunks: 12 chunks per head) under capture:
    the chunk launch and the merge launch replay with new queries."""
    from mtp_hip import _lib as L, ops, workloads
    g = torch.Generator().manual_seed(7)
    N, H, D, Lc, ps = 64, 4, 128, 700, 16
    dt = torch.bfloat16
    npg = (Lc + ps - 1) // ps
    tm = workloads.draft_tree_mask(16, 4)[:N, :N].to(DEV)
    q = torch.randn(N, H, D, generator=g).to(dt).to(DEV)
    kt = torch.randn(N, H, D, generator=g).to(dt).to(DEV)
    vt = torch.randn(N, H, D, generator=g).to(dt).to(DEV)
    kp = torch.randn(npg + 2, 1, H, ps, D, generator=g).to(dt).to(DEV)
    vp = torch.randn(npg + 2, 1, H, ps, D, generator=g).to(dt).to(DEV)
    table = torch.randperm(npg + 2, generator=g)[:npg].repeat_interleave(ps)[:Lc]
    table = table.to(torch.int32)[None, :].to(DEV)
    print("case tree-verify attention graph", flush=True)
    L.set_tuning(attn_chunk_blocks=1)
    try:
        fn = lambda: ops.tree_verify_attention(q, kp, vp, table, ps, kt, vt, tm)  # noqa: E731
        graph, out = _capture(fn)
        qs = [torch.randn(q.shape, generator=g).to(dt).to(DEV) for _ in range(4)]
        _replays(graph, out, lambda i: q.copy_(qs[i]), fn)
    finally:
        L.set_tuning(attn_chunk_blocks=-1)


@pytest.mark.parametrize("dtype,bias", [(torch.bfloat16, None), (torch.bfloat16, torch.bfloat16),
                                        (torch.float32, torch.float32)])
def test_multi_verify_graph_replay(dtype, bias):
    """The persistent verify kernel under capture, without and with the
    engine's lm_head bias and in the engine's default fp32: keys and ticket
    are reset by the last workgroup of each replay."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(3)
    B, D, K, V = 8, 4, 1024, 50000
    hidden = torch.randn(B, D + 1, K, generator=g).to(dtype).to(DEV)
    W = (0.05 * torch.randn(V, K, generator=g)).to(dtype).to(DEV)
    b = None if bias is None else (0.5 * torch.randn(V, generator=g)).to(bias).to(DEV)
    draft = torch.randint(0, V, (B, D), generator=g).to(DEV)
    assert ops.verify_route(hidden, W, b) == "stream"
    print(f"case multi-verify graph dtype={dtype} bias={bias}", flush=True)
    fn = lambda: ops.multi_verify(hidden, W, draft, b, return_top=True)  # noqa: E731
    graph, out = _capture(fn)
    hs = [torch.randn(hidden.shape, generator=g).to(dtype).to(DEV) for _ in range(4)]

    def fill(i):
        hidden.copy_(hs[i])
        # drafts that accept a prefix of the new argmax, so accepted_n varies
        top = ops.multi_verify(hidden, W, draft, b, return_top=True)[3]
        draft.copy_(top[:, 1:].to(draft.dtype))
        draft[i % B, i % D] += 1
        torch.cuda.synchronize()

    _replays(graph, out, fill, fn)


def test_commit_graph_replay_advances_device_lengths():
    """The device-side commit captured: each replay advances the id buffer
    and the KV length on the device, as consecutive eager steps would."""
    from mtp_hip import ops
    B, D = 2, 3
    acc = torch.tensor([[1, 1, 0], [1, 0, 0]], dtype=torch.int8, device=DEV)
    n = torch.tensor([2, 1], dtype=torch.int32, device=DEV)
    corr = torch.tensor([9, 8], dtype=torch.int32, device=DEV)
    draft = torch.tensor([[1, 2, 3], [4, 5, 6]], device=DEV)
    kv = torch.tensor([10], dtype=torch.int64, device=DEV)
    ids = torch.zeros(B, 32, dtype=torch.int64, device=DEV)
    ids_len = torch.tensor([0], dtype=torch.int64, device=DEV)
    fn = lambda: ops.verify_commit(acc, n, corr, draft, kv, kv, ids, ids_len)  # noqa: E731
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up step: width 2
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        fn()  # captured (this records, it does not run)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert int(kv.item()) == 10 + 2 * (i + 2)
        assert int(ids_len.item()) == 2 * (i + 2)
    assert ids[:, :8].tolist() == [[1, 9] * 4, [4, 8] * 4]


def _norm_linear_case(g, M, K, N):
    dt = torch.bfloat16
    x = torch.randn(M, K, generator=g).to(dt).to(DEV)
    W = (0.02 * torch.randn(N, K, generator=g)).to(dt).to(DEV)
    gm = (1 + 0.1 * torch.randn(K, generator=g)).to(dt).to(DEV)
    return x, W, gm


def test_captured_workspace_survives_growth():
    """A graph keeps the address of the workspace it was captured with. A
    later, larger eager call on the capture stream gets a new buffer; the
    old one stays allocated, so a tensor allocated afterwards (the canary,
    the old buffer's size) is never written by a replay, and every replay
    still equals eager."""
    from mtp_hip import _lib as L, ops
    g = torch.Generator().manual_seed(5)
    x, W, gm = _norm_linear_case(g, 64, 1024, 2048)
    fn = lambda: ops.rmsnorm_linear(x, W, None, 1e-6, 1.0, gamma=gm)  # noqa: E731
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.synchronize()
    key = (torch.device(DEV).index or 0, s.cuda_stream)
    old = L._workspaces[key]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = fn()
    xb, Wb, gb = _norm_linear_case(g, 64, 16384, 2048)
    with torch.cuda.stream(s):
        ops.rmsnorm_linear(xb, Wb, None, 1e-6, 1.0, gamma=gb)  # grows s's workspace
    torch.cuda.synchronize()
    assert L._workspaces[key].data_ptr() != old.data_ptr(), "the larger call did not grow it"
    canary = torch.full((old.numel() // 4,), 0x5A5A5A5A, dtype=torch.int32, device=DEV)
    xs = [torch.randn(x.shape, generator=g).to(x.dtype).to(DEV) for _ in range(3)]
    _replays(graph, out, lambda i: x.copy_(xs[i]), fn, n=3)
    assert bool((canary == 0x5A5A5A5A).all()), "a replay wrote into memory it does not own"


def test_capture_on_fresh_stream_then_eager():
    """A stream whose first call is captured: the capture's workspace is
    zeroed only by its recorded fill kernel, so eager calls on that stream
    afterwards must get a buffer of their own (and be correct before the
    graph ever replays)."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(6)
    x, W, gm = _norm_linear_case(g, 64, 1024, 2048)
    fn = lambda: ops.rmsnorm_linear(x, W, None, 1e-6, 1.0, gamma=gm)  # noqa: E731
    ref = fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = fn()
    with torch.cuda.stream(s):
        eager = fn()
    torch.cuda.synchronize()
    assert torch.equal(eager, ref)
    xs = [torch.randn(x.shape, generator=g).to(x.dtype).to(DEV) for _ in range(3)]
    _replays(graph, out, lambda i: x.copy_(xs[i]), fn, n=3)
