"""GPU parity of the grouped INT4 weight-only matmul (fused_int4_matmul and
its RMSNorm-composed form) against the CPU oracle on identical seeded
inputs. Tolerance: |y - ref| <= 2e-2 * (|ref| + RMS(ref)) for every output
dtype (the INT4 bar), 1e-5 would not hold because the MFMA path decodes the
weights and the activations to fp16.

Shapes with K % 128 == 0 and group % 32 == 0 run the MFMA kernel (1, 2, 4
and 8 row tiles, one and several row groups, ragged N and M); the others run
the CUDA-core fallback."""
import pytest
import torch

from conftest import close
from oracle import eager as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL = 2e-2


def _case(M, N, K, group, xdtype, sdtype, nibble, seed, xscale=1.0):
    g = torch.Generator().manual_seed(seed)
    W = 0.02 * torch.randn(N, K, generator=g)
    # "offset" packs q + 8 (what the reference decoder reads), "ref" packs
    # q & 0xF (what the reference quantizer writes, read back as "twos")
    packed, scales = O.quantize_int4(W, group, nibble="offset" if nibble == "ref" else "ref")
    scales = scales.to(sdtype)
    x = (xscale * torch.randn(M, K, generator=g)).to(xdtype)
    gamma = 1.0 + 0.1 * torch.randn(K, generator=g)
    return x, packed, scales, gamma


def _run(x, packed, scales, K, group, nibble, gamma, norm):
    from mtp_hip import ops
    y = ops.int4_matmul(x.to(DEV), packed.to(DEV), scales.to(DEV), K, group, nibble=nibble,
                        gamma=None if gamma is None else gamma.to(DEV), norm=norm)
    torch.cuda.synchronize()
    return y


MFMA_SHAPES = [(1, 128, 128, 32), (5, 200, 256, 128), (17, 300, 512, 64), (33, 96, 384, 32),
               (64, 512, 1024, 128), (100, 130, 256, 32), (256, 1024, 1024, 128),
               (300, 260, 512, 128)]


@pytest.mark.parametrize("M,N,K,group", MFMA_SHAPES)
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_int4_rmsnorm_linear_matches_oracle(M, N, K, group, xdtype):
    print(f"case M={M} N={N} K={K} group={group} x={xdtype}", flush=True)
    x, packed, scales, gamma = _case(M, N, K, group, xdtype, torch.float16, "ref", M + N + K)
    y = _run(x, packed, scales, K, group, "ref", gamma, True)
    ref = O.int4_matmul(x, packed, scales, K, group, gamma=gamma, norm=True)
    assert y.dtype == xdtype and y.shape == (M, N)
    ok, worst = close(y, ref, RTOL)
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("sdtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("factor", ["tiny", "huge", "mixed"])
@pytest.mark.parametrize("M,N,K,group", [(33, 300, 512, 128), (256, 260, 1024, 64)])
def test_int4_extreme_group_scales(M, N, K, group, sdtype, factor):
    """The MFMA path decodes the weights to fp16 after normalising each
    column's scales by a power of two: group scales near 1e-6 (fp16
    subnormal on their own), near 1e3 (decoded weights up to 1.3e5, past the
    fp16 limit without the normalisation), and columns of both kinds in one
    matrix, in every scale dtype, against the oracle on the same scales."""
    print(f"case M={M} N={N} K={K} group={group} s={sdtype} {factor}", flush=True)
    x, packed, scales, gamma = _case(M, N, K, group, torch.bfloat16, torch.float32, "ref",
                                     M + N + K)
    # quantizer scales of 0.02-normal weights are about 1e-2
    col = torch.arange(N)[:, None]
    if factor == "tiny":
        mul = torch.full((N, 1), 1e-4)
    elif factor == "huge":
        mul = torch.full((N, 1), 1e5)
    else:
        mul = torch.where(col % 2 == 0, torch.tensor(1e-4), torch.tensor(1e5))
    scales = (scales.float() * mul).to(sdtype)
    assert torch.isfinite(scales.float()).all()
    y = _run(x, packed, scales, K, group, "ref", gamma, True)
    ref = O.int4_matmul(x, packed, scales, K, group, gamma=gamma, norm=True)
    assert torch.isfinite(y.float()).all()
    if factor == "mixed":
        # columns differ by 1e9 in magnitude: each column against its own RMS
        for sel in (col[:, 0] % 2 == 0, col[:, 0] % 2 == 1):
            ok, worst = close(y[:, sel], ref[:, sel], RTOL)
            assert ok, f"worst err/bound = {worst:.3g}"
    else:
        ok, worst = close(y, ref, RTOL)
        assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("nibble", ["ref", "twos"])
@pytest.mark.parametrize("sdtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,group", [(8, 256, 512, 128), (70, 136, 256, 32)])
def test_int4_reference_mode_scales_and_nibbles(M, N, K, group, sdtype, nibble):
    """norm=False, no gamma: the reference's plain x @ dequant(W).T."""
    print(f"case M={M} N={N} K={K} group={group} scales={sdtype} nibble={nibble}", flush=True)
    x, packed, scales, _ = _case(M, N, K, group, torch.bfloat16, sdtype, nibble, 11 * M + K)
    y = _run(x, packed, scales, K, group, nibble, None, False)
    ref = O.int4_matmul(x, packed, scales, K, group, nibble=nibble)
    ok, worst = close(y, ref, RTOL)
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("sdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,group", [(40, 200, 8192, 64), (40, 130, 4352, 32),
                                         (70, 90, 1024, 32)])
def test_int4_scale_transpose_paths(M, N, K, group, sdtype):
    """The prep's scale transpose at the edges of its one-pass form: 128
    groups per row (the largest it takes), 136 groups (the two-pass form),
    ragged N (a last block of 26 columns) with 32 groups per row; x rows of
    8192 and 4352 (registers / loop)."""
    print(f"case int4 scales M={M} N={N} K={K} group={group} s={sdtype}", flush=True)
    x, packed, scales, gamma = _case(M, N, K, group, torch.bfloat16, sdtype, "ref", M * N + K)
    y = _run(x, packed, scales, K, group, "ref", gamma, True)
    ref = O.int4_matmul(x, packed, scales, K, group, gamma=gamma, norm=True)
    ok, worst = close(y, ref, RTOL)
    assert ok, f"worst err/bound = {worst:.3g}"


def test_int4_no_norm_row_ranges():
    """norm=False rows of very different magnitude (1e-6 .. 1e4, a zero row):
    each row is brought to fp16 with its own power of two."""
    M, N, K, group = 6, 192, 256, 64
    x, packed, scales, gamma = _case(M, N, K, group, torch.float32, torch.float16, "ref", 5)
    for i, s in enumerate([1e-6, 1e-3, 1.0, 30.0, 1e4]):
        x[i] *= s
    x[5] = 0.0
    for gm in (None, gamma):
        y = _run(x, packed, scales, K, group, "ref", gm, False)
        ref = O.int4_matmul(x, packed, scales, K, group, gamma=gm, norm=False)
        for i in range(M):  # per row: each row has its own scale
            ok, worst = close(y[i], ref[i], RTOL)
            assert ok, f"row {i}: worst err/bound = {worst:.3g}"
        assert torch.equal(y[5].cpu(), torch.zeros(N))


@pytest.mark.parametrize("M,N,K,group", [(4, 32, 64, 32), (3, 50, 96, 32), (9, 64, 256, 16),
                                         (2, 40, 130, 26)])
def test_int4_fallback_shapes(M, N, K, group):
    """K % 128 != 0 or group % 32 != 0: the CUDA-core path (including the
    reference self-test's W[32, 64], group 32)."""
    x, packed, scales, gamma = _case(M, N, K, group, torch.float32, torch.float32, "ref", K)
    y = _run(x, packed, scales, K, group, "ref", None, False)
    ref = O.int4_matmul(x, packed, scales, K, group)
    ok, worst = close(y, ref, 1e-5)
    assert ok, f"worst err/bound = {worst:.3g}"
    y = _run(x, packed, scales, K, group, "ref", gamma, True)
    ok, worst = close(y, O.int4_matmul(x, packed, scales, K, group, gamma=gamma, norm=True), 1e-5)
    assert ok, f"worst err/bound = {worst:.3g}"


def test_int4_workload_full_size():
    """The INT4 RMSNorm+linear workload at full size (x bf16 [256, 8192],
    W [28672, 8192] group 128, fp16 scales, gamma): every output row checked
    on 2048 columns spread over all of N (the oracle on those columns is the
    same per-column computation)."""
    from mtp_hip import workloads
    d = workloads.int4_linear()
    print("case int4 workload M=256 K=8192 N=28672", flush=True)
    y = _run(d["x"], d["packed"], d["scales"], d["K"], d["group"], "ref", d["gamma"], True)
    N = d["packed"].shape[0]
    cols = torch.cat([torch.arange(0, 128), torch.arange(N - 128, N),
                      torch.randperm(N, generator=torch.Generator().manual_seed(0))[:1792]])
    ref = O.int4_matmul(d["x"], d["packed"][cols], d["scales"][cols], d["K"], d["group"],
                        gamma=d["gamma"], norm=True, eps=d["eps"])
    ok, worst = close(y.cpu()[:, cols], ref, RTOL)
    assert ok, f"worst err/bound = {worst:.3g}"


def test_int4_leaves_shared_workspace_counters_zero():
    """INT4 calls and split-K calls share the per-stream workspace: after an
    INT4 call (its x fragments and scales sit past the counter region) the
    arrival counters are still zero and a split-K RMSNorm -> linear is exact
    to the oracle."""
    import os
    from mtp_hip import _lib, ops
    x, packed, scales, gamma = _case(64, 512, 1024, 128, torch.bfloat16, torch.float16, "ref", 3)
    _run(x, packed, scales, 1024, 128, "ref", gamma, True)
    ws = _lib._workspaces[(0, torch.cuda.current_stream().cuda_stream)]
    counters = ws[:65536]  # MTP_WORKSPACE_COUNTER_BYTES (include/mtp_hip.h)
    assert int(counters.count_nonzero()) == 0
    g = torch.Generator().manual_seed(11)
    xl = torch.randn(33, 1024, generator=g).to(torch.bfloat16)
    W = (0.05 * torch.randn(260, 1024, generator=g)).to(torch.bfloat16)
    gm = 1 + 0.1 * torch.randn(1024, generator=g)
    with _lib.tuning(sk_splits=3):
        y = ops.rmsnorm_linear(xl.to(DEV), W.to(DEV), None, 1e-6, 1.0, gamma=gm.to(DEV))
    torch.cuda.synchronize()
    ok, worst = close(y, O.rmsnorm_linear(xl, W, None, 1e-6, 1.0, gamma=gm), 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"
    assert int(counters.count_nonzero()) == 0
