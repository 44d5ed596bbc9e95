"""HIP-graph capture of the hot path: a draft step (RMSNorm, RMSNorm ->
linear head, greedy token + embedding, combine-norm), the fp32 linear
routes (one launch, streaming, row-chunk with K-splits), the persistent multi-verify and the device-side
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


def test_multi_verify_graph_replay():
    """The persistent verify kernel under capture: keys and ticket are
    reset by the last workgroup of each replay."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(3)
    B, D, K, V = 8, 4, 1024, 50000
    hidden = torch.randn(B, D + 1, K, generator=g).to(torch.bfloat16).to(DEV)
    W = (0.05 * torch.randn(V, K, generator=g)).to(torch.bfloat16).to(DEV)
    draft = torch.randint(0, V, (B, D), generator=g).to(DEV)
    fn = lambda: ops.multi_verify(hidden, W, draft, return_top=True)  # noqa: E731
    graph, out = _capture(fn)
    hs = [torch.randn(hidden.shape, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4)]

    def fill(i):
        hidden.copy_(hs[i])
        # drafts that accept a prefix of the new argmax, so accepted_n varies
        top = ops.multi_verify(hidden, W, draft, return_top=True)[3]
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
