"""The allocation-free multi-verify entry point (mtp_fused_multi_verify_noalloc,
workspace in the library's static device array) against the existing entry
point with a caller workspace, through the C ABI: identical accept,
accepted_n, corrected and top on calls in a row, the last smaller, with a
column-group case (per-tile maxima in the array) and an fp32 case with a
bias between; and a call captured into a HIP graph, replayed with new
inputs."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _noalloc_fn(lib):
    return lib.mtp_fused_multi_verify_noalloc  # ctypes signature set by mtp_hip._lib


def _case(seed, B, D, K, V, dtype, bias):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(B, D + 1, K, generator=g).to(dtype).to(DEV)
    W = (0.05 * torch.randn(V, K, generator=g)).to(dtype).to(DEV)
    b = (0.1 * torch.randn(V, generator=g)).to(dtype).to(DEV) if bias else None
    top = torch.nn.functional.linear(h.float(), W.float(),
                                     None if b is None else b.float()).argmax(-1)
    draft = top[:, 1:].clone().to(torch.int32)
    draft[0, D // 2] = (draft[0, D // 2] + 1) % V
    return h, W, b, draft.contiguous()


def _outs(B, D):
    return (torch.full((B, D), -1, dtype=torch.int8, device=DEV),
            torch.full((B,), -1, dtype=torch.int32, device=DEV),
            torch.full((B,), -1, dtype=torch.int32, device=DEV),
            torch.full((B, D + 1), -1, dtype=torch.int32, device=DEV))


def _run_both(lib, noalloc, h, W, b, draft):
    from mtp_hip import _lib as L
    B, S, K = h.shape
    V = W.shape[0]
    D = S - 1
    code = L.code(h.dtype)
    st = torch.cuda.current_stream().cuda_stream
    bp, bc = (None, 0) if b is None else (b.data_ptr(), L.code(b.dtype))
    ref = _outs(B, D)
    nws = lib.mtp_verify_workspace_bytes(code, B * S, S, V, K)
    ws = torch.zeros(nws, dtype=torch.uint8, device=DEV)
    s = lib.mtp_fused_multi_verify(h.data_ptr(), code, B, S, K, W.data_ptr(), code, V, bp, bc,
                                   draft.data_ptr(), D, *[t.data_ptr() for t in ref],
                                   ws.data_ptr(), nws, st)
    assert s == 0, s
    got = _outs(B, D)
    s = noalloc(h.data_ptr(), code, B, S, K, W.data_ptr(), code, V, bp, bc, draft.data_ptr(), D,
                *[t.data_ptr() for t in got], st)
    assert s == 0, s
    torch.cuda.synchronize()
    for r, o, name in zip(ref, got, ("accept", "accepted_n", "corrected", "top")):
        assert torch.equal(r, o), name
    return ref


def test_noalloc_multi_verify_matches_workspace_entry_point():
    from mtp_hip import _lib
    lib = _lib.load()
    noalloc = _noalloc_fn(lib)
    assert lib.mtp_noalloc_scratch_bytes() == 1 << 20
    print("case noalloc 1: B=8 D=4 K=1024 V=50000 bf16 (persistent kernel)", flush=True)
    r1 = _run_both(lib, noalloc, *_case(1, 8, 4, 1024, 50000, torch.bfloat16, False))
    assert int(r1[1].min()) >= 0
    print("case noalloc 2: B=5 D=3 K=448 V=20000 bf16 + bias (column-group kernel)", flush=True)
    c2 = _case(2, 5, 3, 448, 20000, torch.bfloat16, True)
    from mtp_hip import ops
    assert ops.verify_route(c2[0], c2[1], c2[2]) == "column_group"
    _run_both(lib, noalloc, *c2)
    print("case noalloc 3: B=4 D=4 K=1024 V=30000 fp32 + bias (persistent kernel)", flush=True)
    _run_both(lib, noalloc, *_case(5, 4, 4, 1024, 30000, torch.float32, True))
    print("case noalloc 4: B=2 D=2 K=256 V=3000 f16 (smaller)", flush=True)
    _run_both(lib, noalloc, *_case(3, 2, 2, 256, 3000, torch.float16, False))


def test_noalloc_multi_verify_under_graph_capture():
    """The allocation-free call captured into a HIP graph (its clear kernel
    and the verify launch are kernel nodes) and replayed with new hidden
    rows: every replay equals the workspace entry point's eager result, with
    eager work and synchronisation between replays."""
    from mtp_hip import _lib as L
    lib = L.load()
    noalloc = _noalloc_fn(lib)
    assert lib.mtp_noalloc_init() == 0  # address looked up before the capture
    h, W, b, draft = _case(6, 8, 4, 1024, 50000, torch.bfloat16, True)
    B, S, K = h.shape
    D, V = S - 1, W.shape[0]
    code = L.code(h.dtype)
    got = _outs(B, D)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    # one eager call first (the library caches the device's properties on
    # its first launch plan, outside the capture)
    st = noalloc(h.data_ptr(), code, B, S, K, W.data_ptr(), code, V, b.data_ptr(),
                 L.code(b.dtype), draft.data_ptr(), D, *[t.data_ptr() for t in got],
                 s.cuda_stream)
    assert st == 0, st
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("case noalloc captured: B=8 D=4 K=1024 V=50000 bf16 + bias", flush=True)
    with torch.cuda.graph(graph, stream=s):
        st = noalloc(h.data_ptr(), code, B, S, K, W.data_ptr(), code, V, b.data_ptr(),
                     L.code(b.dtype), draft.data_ptr(), D, *[t.data_ptr() for t in got],
                     s.cuda_stream)
    assert st == 0, st
    g = torch.Generator().manual_seed(60)
    for i in range(3):
        h.copy_(torch.randn(h.shape, generator=g).to(h.dtype))
        top = torch.nn.functional.linear(h.float(), W.float(), b.float()).argmax(-1)
        draft.copy_(top[:, 1:].to(torch.int32))
        draft[i % B, i % D] = (draft[i % B, i % D] + 1) % V
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = _outs(B, D)
        nws = lib.mtp_verify_workspace_bytes(code, B * S, S, V, K)
        ws = torch.zeros(nws, dtype=torch.uint8, device=DEV)
        st = lib.mtp_fused_multi_verify(h.data_ptr(), code, B, S, K, W.data_ptr(), code, V,
                                        b.data_ptr(), L.code(b.dtype), draft.data_ptr(), D,
                                        *[t.data_ptr() for t in ref], ws.data_ptr(), nws,
                                        torch.cuda.current_stream().cuda_stream)
        assert st == 0, st
        torch.cuda.synchronize()
        for r, o, name in zip(ref, got, ("accept", "accepted_n", "corrected", "top")):
            assert torch.equal(r, o), (i, name)
        assert int(ref[1][i % B]) <= i % D
        _ = torch.ones(1000, device=DEV).sum().item()  # eager work between replays


def test_noalloc_rejects_what_does_not_fit():
    from mtp_hip import _lib
    lib = _lib.load()
    noalloc = _noalloc_fn(lib)
    fake = 4096
    # a shape on the column-group kernel (bf16 rows of 896 bytes) whose
    # per-tile maxima, 64 rows x 2M columns, exceed the 1 MiB array: the
    # check runs on the host before any launch
    assert lib.mtp_verify_route(fake, _lib.BF16, 64, 4, 448, fake, _lib.BF16, 2 ** 21,
                                fake) == _lib.VERIFY_ROUTE_COLUMN_GROUP
    s = noalloc(fake, _lib.BF16, 16, 4, 448, fake, _lib.BF16, 2 ** 21, fake, _lib.BF16, fake, 3,
                fake, fake, fake, None, None)
    assert s == _lib.ERR_WORKSPACE
    assert noalloc(fake, _lib.BF16, 2, 5, 512, fake, _lib.BF16, 100, None, 0, fake, 3, fake, fake,
                   fake, None, None) == _lib.ERR_SHAPE
