"""GPU parity of the draft chain kernels against the CPU oracle: RMSNorm,
add + RMSNorm (the combine-norm), the greedy argmax with the embedding
gather; plus the reference's own RMSNorm check (test_engine.py:4) through
the drop-in module. Tolerance |y - ref| <= rtol (|ref| + RMS(ref)), rtol
1e-5 for fp32 and 2e-2 for bf16 / f16; tokens and embedding rows bit-exact."""
import math

import pytest
import torch

from conftest import close
from oracle import eager as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N", [(7, 32), (4, 4096), (3, 1000), (1000, 256), (1, 1)])
@pytest.mark.parametrize("weighted", [True, False])
def test_rmsnorm_matches_oracle(dtype, M, N, weighted):
    from mtp_hip import ops
    g = torch.Generator().manual_seed(M * 7 + N)
    x = (3 * torch.randn(M, N, generator=g)).to(dtype)
    w = torch.randn(N, generator=g) if weighted else None
    print(f"case rmsnorm dtype={dtype} M={M} N={N} w={weighted}", flush=True)
    y = ops.rmsnorm(x.to(DEV), None if w is None else w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    ref = O.rmsnorm(x, w, 1e-6)
    assert y.dtype == dtype and y.shape == x.shape
    ok, worst = close(y, ref, RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N", [(8, 4096), (5, 777)])
def test_add_rmsnorm_matches_oracle(dtype, M, N):
    import mtp_kernels as mk
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, N, generator=g).to(dtype)
    r = torch.randn(M, N, generator=g).to(dtype)
    w = 1 + 0.1 * torch.randn(N, generator=g)
    print(f"case add_rmsnorm dtype={dtype} M={M} N={N}", flush=True)
    y = mk.fused_add_rmsnorm(x.to(DEV), r.to(DEV), w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    ok, worst = close(y, O.add_rmsnorm(x, r, w, 1e-6), RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"


def test_reference_rmsnorm_check_through_dropin():
    """test_engine.py:4: seed 0, x [7, 32], weight [32], max error < 1e-4."""
    import mtp_kernels as mk
    torch.manual_seed(0)
    A = torch.randn(7, 32)
    B = torch.randn(32)
    E = mk.fused_rmsnorm(A.to(DEV), B.to(DEV), 1e-6).cpu()
    F = A * torch.rsqrt((A * A).mean(-1, keepdim=True) + 1e-6) * B
    assert (E - F).abs().max().item() < 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,V", [(1, 1), (1, 100), (8, 32000), (8, 128256), (40, 5000),
                                 (3000, 300)])
def test_argmax_matches_torch_argmax(dtype, M, V):
    from mtp_hip import ops
    g = torch.Generator().manual_seed(M + V)
    lg = torch.randn(M, V, generator=g).to(dtype)
    print(f"case argmax dtype={dtype} M={M} V={V}", flush=True)
    tok = ops.argmax(lg.to(DEV))
    torch.cuda.synchronize()
    assert tok.dtype == torch.int64
    assert torch.equal(tok.cpu(), O.argmax_tokens(lg))


def test_argmax_ties_nan_inf_across_segments_and_gather():
    """Ties between columns in different workgroups of a row (the lowest
    index wins), NaN as the maximum, an all -inf row (index 0), and the
    embedding rows of the chosen tokens, bit-exact."""
    from mtp_hip import ops
    M, V, H = 5, 128256, 96
    lg = torch.zeros(M, V)
    lg[0, 70000] = 5.0
    lg[0, 100000] = 5.0
    lg[0, 127999] = 5.0
    lg[1, 3] = float("nan")
    lg[1, 90000] = float("nan")
    lg[1, 500] = float("inf")
    lg[2] = -math.inf
    lg[3, 128255] = 1.0
    lg[4] = 0.0
    g = torch.Generator().manual_seed(3)
    table = torch.randn(V, H, generator=g).to(torch.bfloat16)
    for dtype in (torch.float32, torch.bfloat16):
        tok, emb = ops.argmax(lg.to(dtype).to(DEV), table.to(DEV))
        torch.cuda.synchronize()
        ref_tok, ref_emb = O.argmax_tokens(lg.to(dtype), table)
        assert tok.cpu().tolist() == [70000, 3, 0, 128255, 0] == ref_tok.tolist()
        assert torch.equal(emb.cpu(), ref_emb)


def test_argmax_strided_rows_and_1d():
    from mtp_hip import ops
    g = torch.Generator().manual_seed(9)
    big = torch.randn(6, 1000, generator=g)
    view = big[:, 100:900]  # row stride 1000, unit column stride
    tok = ops.argmax(big.to(DEV)[:, 100:900])
    torch.cuda.synchronize()
    assert torch.equal(tok.cpu(), view.argmax(-1))
    one = ops.argmax(big[2].to(DEV))
    assert int(one) == int(big[2].argmax())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_argmax_partial_last_chunk(dtype):
    """Row stride a whole number of 16-byte chunks but V not (the last
    elements of each row read one at a time): the maximum placed in the
    partial chunk, tied with an earlier column, NaN there, and a maximum
    just before it; tokens bit-exact against torch.argmax, with the
    embedding gather."""
    from mtp_hip import ops
    g = torch.Generator().manual_seed(17)
    big = torch.randn(6, 4096, generator=g).to(dtype)
    V = 4093  # 4093 % 8 == 5 and 4093 % 4 == 1
    big[0, 4092] = 50.0                       # maximum in the partial chunk
    big[1, 4090] = 40.0
    big[1, 100] = 40.0                        # tie: the lower index wins
    big[2, 4091] = float("nan")               # NaN in the partial chunk
    big[3, 4087] = 30.0                       # last column of the last full chunk
    big[4, 4088] = 30.0                       # first column of the partial chunk
    big[5, 4095] = 99.0                       # past V: never chosen
    view = big.to(DEV)[:, :V]
    table = torch.randn(V, 64, generator=g).to(dtype)
    tok, emb = ops.argmax(view, table.to(DEV))
    torch.cuda.synchronize()
    ref = big[:, :V].float().argmax(-1)
    ref[2] = 4091
    assert tok.cpu().tolist() == ref.tolist()
    assert tok.cpu().tolist()[:5] == [4092, 100, 4091, 4087, 4088]
    assert torch.equal(emb.cpu(), table[tok.cpu()])


def test_perf_hardening_greedy_routes():
    from mtp_hip import perf_hardening as mh
    g = torch.Generator().manual_seed(10)
    lg = torch.randn(2, 3, 500, generator=g)
    d = lg.to(DEV)
    assert torch.equal(mh.argmax_greedy(d).cpu(), lg.argmax(-1))
    assert torch.equal(mh.sample_token(d[0], 0.0).cpu(), lg[0].argmax(-1))
    s = mh.sample_token(d[0], 1.0)
    assert s.shape == (3,) and int(s.max()) < 500
