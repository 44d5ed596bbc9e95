"""GPU parity of the RMSNorm -> linear family (fp32 / bf16 / f16 / fp8
weights) against the CPU oracle on identical seeded inputs.

Tolerance: |y - ref| <= rtol * (|ref| + RMS(ref)) with rtol 1e-5 for fp32
(TF32 off) and 2e-2 for bf16 / f16 / fp8 outputs."""
import os

import pytest
import torch

from conftest import close
from oracle import eager as O

pytestmark = pytest.mark.gpu

RTOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}
DEV = "cuda"


@pytest.fixture(autouse=True)
def _tune_reset():
    """Every test starts and ends with the planner's own launch choices."""
    from mtp_hip import _lib
    _lib.set_tuning(**{k: -1 for k in _lib.TUNING_KEYS})
    yield
    _lib.set_tuning(**{k: -1 for k in _lib.TUNING_KEYS})


def _ws_tune(spec: str) -> None:
    from mtp_hip import _lib
    v, sp = (int(t) for t in spec.split(","))
    _lib.set_tuning(ws_variant=v, ws_splits=sp)


def _set(**keys) -> None:
    from mtp_hip import _lib
    _lib.set_tuning(**keys)


def _inputs(M, N, K, dtype, seed, bias=True, gamma=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    W = (0.05 * torch.randn(N, K, generator=g)).to(dtype)
    b = (0.1 * torch.randn(N, generator=g)).to(dtype) if bias else None
    gm = (1 + 0.1 * torch.randn(K, generator=g)) if gamma else None
    return x, W, b, gm


def _dev(t):
    return None if t is None else t.to(DEV)


SHAPES = [(16, 4096, 1024), (1, 64, 64), (5, 128, 64), (17, 100, 256), (33, 1000, 136),
          (64, 512, 1024), (70, 256, 512), (130, 96, 64)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_rmsnorm_linear_matches_oracle(dtype, M, N, K):
    from mtp_hip import ops
    x, W, b, gm = _inputs(M, N, K, dtype, seed=M * 7 + N + K)
    print(f"case dtype={dtype} M={M} N={N} K={K}", flush=True)
    y = ops.rmsnorm_linear(_dev(x), _dev(W), _dev(b), 1e-6, 0.75, gamma=_dev(gm))
    torch.cuda.synchronize()
    ref = O.rmsnorm_linear(x, W, b, 1e-6, 0.75, gamma=gm)
    assert y.dtype == dtype and y.shape == (M, N)
    ok, worst = close(y, ref, RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("tune", ["0,1", "0,3", "1,1", "1,4", "2,2", "3,5", "4,1", "5,2",
                                  "6,3", "7,1", "7,4"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_tile_variants_and_splits(tune, dtype):
    from mtp_hip import ops
    _ws_tune(tune)
    M, N, K = 40, 1040, 1536
    x, W, b, gm = _inputs(M, N, K, dtype, seed=11)
    print(f"case tune={tune} dtype={dtype}", flush=True)
    y = ops.rmsnorm_linear(_dev(x), _dev(W), _dev(b), 1e-6, 1.0, gamma=_dev(gm))
    torch.cuda.synchronize()
    ref = O.rmsnorm_linear(x, W, b, 1e-6, 1.0, gamma=gm)
    ok, worst = close(y, ref, RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"


def test_no_norm_no_gamma_no_bias_and_generic_path():
    from mtp_hip import ops
    # K = 100 is not a multiple of the 16-byte vector: the generic kernel runs.
    for (M, N, K) in [(7, 48, 64), (7, 48, 100)]:
        x, W, _, _ = _inputs(M, N, K, torch.bfloat16, seed=3, bias=False, gamma=False)
        y = ops.rmsnorm_linear(_dev(x), _dev(W), None, 1e-6, 1.0, norm=False)
        ref = O.rmsnorm_linear(x, W, None, 1e-6, 1.0, norm=False)
        ok, worst = close(y, ref, 2e-2)
        assert ok, (M, N, K, worst)


def test_reference_self_checks():
    """The reference's own checks on its seeded inputs: fused linear max abs
    error < 1e-4 (test_engine.py:5, mtp_engine.py:1644-1651) and the fp8
    entry with fp32 weights in +-448 (mtp_engine.py:1792-1800)."""
    import mtp_kernels as MK
    torch.manual_seed(1)
    x = torch.randn(5, 64)
    W = torch.randn(128, 64)
    b = torch.randn(128)
    y = MK.fused_rmsnorm_linear(x.to(DEV), W.to(DEV), b.to(DEV), 1e-6).cpu()
    xn = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6)
    assert (y - torch.nn.functional.linear(xn, W, b)).abs().max().item() < 1e-4
    Wsw = torch.randn(32, 64)
    row_scale = Wsw.abs().max(dim=-1, keepdim=True).values.squeeze(-1) / 448.0
    Wf8 = (Wsw / row_scale[:, None]).clamp(-448, 448)
    xq = torch.randn(4, 64)
    y8 = MK.fused_rmsnorm_linear_fp8(xq.to(DEV), Wf8.to(DEV), row_scale.to(DEV)).cpu()
    xn = xq * torch.rsqrt((xq * xq).mean(-1, keepdim=True) + 1e-6)
    y8_ref = torch.nn.functional.linear(xn, Wf8.float() * row_scale[:, None])
    assert (y8 - y8_ref).abs().max().item() < 1e-4


@pytest.mark.parametrize("M,N,K", [(3, 48, 64), (20, 272, 528), (64, 1024, 2048), (9, 40, 80)])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fp8_weights_match_oracle(M, N, K, xdtype):
    from mtp_hip import ops
    g = torch.Generator().manual_seed(M + N)
    W = 0.02 * torch.randn(N, K, generator=g)
    wq, ws = O.quantize_fp8_per_channel(W)
    x = torch.randn(M, K, generator=g).to(xdtype)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = 0.1 * torch.randn(N, generator=g)
    print(f"case fp8 M={M} N={N} K={K} x={xdtype}", flush=True)
    y = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6, gamma=_dev(gm))
    ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
    ok, worst = close(y, ref, RTOL[xdtype])
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("tune", ["0,1", "1,2", "2,3", "3,1", "4,2", "5,1", "6,2", "7,3"])
@pytest.mark.parametrize("M", [40, 64])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float32])
def test_fp8_tile_variants_and_splits(tune, M, xdtype):
    """Every tile variant with fp8 weights: two x fragments per W chunk at
    16-bit x (four at fp32 x), so some variants stage several x blocks per
    wave and others leave waves without one."""
    from mtp_hip import ops
    _ws_tune(tune)
    N, K = 592, 1216
    g = torch.Generator().manual_seed(M * 3 + 1)
    W = 0.02 * torch.randn(N, K, generator=g)
    wq, ws = O.quantize_fp8_per_channel(W)
    x = torch.randn(M, K, generator=g).to(xdtype)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    print(f"case fp8 tune={tune} M={M} x={xdtype}", flush=True)
    y = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), None, 1e-6, gamma=_dev(gm))
    ref = O.rmsnorm_linear_fp8(x, wq, ws, None, 1e-6, gamma=gm)
    ok, worst = close(y, ref, RTOL[xdtype])
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("splits", ["1", "2", "3", "5"])
@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (7, 300, 512), (33, 260, 1024), (64, 1000, 2048)])
@pytest.mark.parametrize("wkind", ["fp8", "same"])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
def test_skinny_kernel_splits(splits, M, N, K, wkind, xdtype):
    """The skinny weight-streaming kernel (M <= 64, 16-bit x, fp8 or 16-bit
    W): every forced K-split count, ragged M and N, with and without gamma
    and norm, against the oracle. Without gamma it can read the raw x rows
    and apply rs to the fp32 sums (no prep launch; the default, sk_xraw=1);
    the prep form (sk_xraw=0) gives the oracle's answer on the same inputs
    too."""
    _set(sk_splits=int(splits))
    from mtp_hip import ops
    print(f"case splits={splits} M={M} N={N} K={K} w={wkind} x={xdtype}", flush=True)
    g = torch.Generator().manual_seed(M * 131 + N + K)
    x = torch.randn(M, K, generator=g).to(xdtype)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(xdtype)
    if wkind == "fp8":
        wq, ws = O.quantize_fp8_per_channel(W)
        y = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6, gamma=_dev(gm))
        ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
        y2 = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), None, 1e-6, norm=False)
        ref2 = O.rmsnorm_linear_fp8(x, wq, ws, None, 1e-6, norm=False)
    else:
        Wc = W.to(xdtype)
        y = ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5, gamma=_dev(gm))
        ref = O.rmsnorm_linear(x, Wc, b, 1e-6, 0.5, gamma=gm)
        y2 = ops.rmsnorm_linear(_dev(x), _dev(Wc), None, 1e-6, 1.0, norm=False)
        ref2 = O.rmsnorm_linear(x, Wc, None, 1e-6, 1.0, norm=False)
    torch.cuda.synchronize()
    for out, r in ((y, ref), (y2, ref2)):
        ok, worst = close(out, r, 2e-2)
        assert ok, f"worst err/bound = {worst:.3g}"
    # no gamma, norm and bias: the raw-x form (forced: also for two x
    # tiles), then the prep form
    for xraw in (1, 0):
        _set(sk_xraw=xraw)
        if wkind == "fp8":
            y3 = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6)
            ref3 = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6)
        else:
            y3 = ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5)
            ref3 = O.rmsnorm_linear(x, Wc, b, 1e-6, 0.5)
        torch.cuda.synchronize()
        ok, worst = close(y3, ref3, 2e-2)
        assert ok, f"sk_xraw={xraw}: worst err/bound = {worst:.3g}"
        if xraw == 1:
            assert torch.equal(y3, ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6)
                               if wkind == "fp8" else
                               ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5))


SKW_SHAPES = [(17, 300, 512), (33, 260, 1024), (64, 1000, 2048), (40, 100, 128),
              (64, 64, 256), (24, 520, 768), (57, 130, 8192), (32, 4100, 384)]


@pytest.mark.parametrize("M,N,K", SKW_SHAPES)
@pytest.mark.parametrize("wkind", ["fp8", "same"])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
def test_wave_specialised_skinny_kernel(M, N, K, wkind, xdtype):
    """The wave-specialised skinny kernel after the prep launch (forced with
    the tuning key skw=1): ragged M (one or two 32-row tiles) and N, K from
    one stage (128 fp8 / 64 16-bit k, fewer stages than its ring) to 8192;
    with gamma, norm and bias, without norm, and without gamma, against the
    oracle, and bit for bit on a second call."""
    _set(skw=1)
    from mtp_hip import ops
    print(f"case skw M={M} N={N} K={K} w={wkind} x={xdtype}", flush=True)
    g = torch.Generator().manual_seed(M * 977 + N + K)
    x = torch.randn(M, K, generator=g).to(xdtype)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(xdtype)
    if wkind == "fp8":
        if K % 128:
            pytest.skip("fp8 stages are 128 k")
        wq, ws = O.quantize_fp8_per_channel(W)
        run = lambda **kw: ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), kw.get("b"), 1e-6,
                                                  gamma=kw.get("gm"), norm=kw.get("norm", True))
        oracle = lambda **kw: O.rmsnorm_linear_fp8(x, wq, ws, kw.get("b"), 1e-6,
                                                   gamma=kw.get("gm"), norm=kw.get("norm", True))
    else:
        Wc = W.to(xdtype)
        run = lambda **kw: ops.rmsnorm_linear(_dev(x), _dev(Wc), kw.get("b"), 1e-6, 0.5,
                                              gamma=kw.get("gm"), norm=kw.get("norm", True))
        oracle = lambda **kw: O.rmsnorm_linear(x, Wc, kw.get("b"), 1e-6, 0.5,
                                               gamma=kw.get("gm"), norm=kw.get("norm", True))
    cases = [dict(gm=gm, b=b), dict(norm=False), dict(b=b)]
    for kw in cases:
        dev_kw = {k: (_dev(v) if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}
        y = run(**dev_kw)
        ref = oracle(**kw)
        torch.cuda.synchronize()
        ok, worst = close(y, ref, 2e-2)
        assert ok, f"{sorted(kw)}: worst err/bound = {worst:.3g}"
        assert torch.equal(y, run(**dev_kw))  # fixed order: bit for bit


@pytest.mark.parametrize("tw", [56, 40, 8])
@pytest.mark.parametrize("M,N,K,wkind", [(64, 1000, 1024, "fp8"), (33, 260, 384, "same"),
                                         (48, 4100, 2048, "fp8"), (17, 57, 128, "fp8")])
def test_wave_specialised_column_widths(M, N, K, wkind, tw):
    """The wave-specialised kernel with fewer output columns per workgroup
    than its 64-wide MFMA tile (tuning key skw_tw): the tile's last columns
    read zeros and are not stored, N ragged against the width; gamma, norm
    and bias, against the oracle and bit for bit on a second call."""
    _set(skw=1, skw_tw=tw)
    from mtp_hip import ops
    print(f"case skw tw={tw} M={M} N={N} K={K} w={wkind}", flush=True)
    g = torch.Generator().manual_seed(M * 31 + N + K + tw)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
    if wkind == "fp8":
        wq, ws = O.quantize_fp8_per_channel(W)
        y = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6, gamma=_dev(gm))
        again = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6, gamma=_dev(gm))
        ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
    else:
        Wc = W.to(torch.bfloat16)
        y = ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5, gamma=_dev(gm))
        again = ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5, gamma=_dev(gm))
        ref = O.rmsnorm_linear(x, Wc, b, 1e-6, 0.5, gamma=gm)
    torch.cuda.synchronize()
    ok, worst = close(y, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"
    assert torch.equal(y, again)


SKL_CASES = [(None, "8", (40, 40000, 512)), (None, "8", (3, 33024, 256)),
             ("1", "4", (64, 1000, 2048)), ("1", "8", (7, 300, 512)),
             ("2", "8", (33, 260, 1024)), ("3", "4", (1, 128, 1280)),
             ("5", "8", (64, 2000, 2048)), (None, "4", (17, 520, 768))]


@pytest.mark.parametrize("splits,waves,shape", SKL_CASES)
@pytest.mark.parametrize("wkind", ["fp8", "same"])
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
def test_single_launch_skinny_kernel(splits, waves, shape, wkind, xdtype):
    """The single-launch skinny kernel (norm applied to the fp32 sums,
    gamma applied while x is staged, 32 * waves columns per workgroup):
    forced everywhere (tuning key skl=1) for the small shapes, by default for the
    wide ones (no K-split), with forced and planned K-splits, ragged M and
    N, with and without gamma, bias and norm, against the oracle."""
    M, N, K = shape
    if N <= 32768:
        _set(skl=1)
    if splits is not None:
        _set(skl_splits=int(splits))
    _set(skl_waves=int(waves))
    from mtp_hip import ops
    print(f"case skl splits={splits} waves={waves} M={M} N={N} K={K} w={wkind} x={xdtype}",
          flush=True)
    g = torch.Generator().manual_seed(M * 17 + N + K)
    x = torch.randn(M, K, generator=g).to(xdtype)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(xdtype)
    if wkind == "fp8":
        wq, ws = O.quantize_fp8_per_channel(W)
        y = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6, gamma=_dev(gm))
        ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
        y2 = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), None, 1e-6, norm=False)
        ref2 = O.rmsnorm_linear_fp8(x, wq, ws, None, 1e-6, norm=False)
    else:
        Wc = W.to(xdtype)
        y = ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5, gamma=_dev(gm))
        ref = O.rmsnorm_linear(x, Wc, b, 1e-6, 0.5, gamma=gm)
        y2 = ops.rmsnorm_linear(_dev(x), _dev(Wc), None, 1e-6, 1.0, norm=False)
        ref2 = O.rmsnorm_linear(x, Wc, None, 1e-6, 1.0, norm=False)
    torch.cuda.synchronize()
    for out, r in ((y, ref), (y2, ref2)):
        ok, worst = close(out, r, 2e-2)
        assert ok, f"worst err/bound = {worst:.3g}"
    # deterministic: fixed split and row-sum orders
    y3 = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6, gamma=_dev(gm)) \
        if wkind == "fp8" else ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5,
                                                  gamma=_dev(gm))
    assert torch.equal(y, y3)


@pytest.mark.parametrize("M,N", [(64, 13000), (48, 16000), (8, 13000), (32, 13000),
                                 (16, 15000), (8, 40960), (4, 50257)])
def test_default_routes_fill_widths(M, N):
    """The planner's own routes and column widths at N other than 14336
    (fp8 W, K 4096, gamma and bias): the wave-specialised kernel at 64 / 48
    rows, the x-resident kernel at 8 / 16 rows, the single-launch kernel at
    32 rows, each with the width that fills the CUs and a ragged last
    workgroup; 8 and 4 rows at N past 32768 on the single-launch kernel
    with the widths that make whole rounds (160 and 200 columns); against
    the oracle."""
    from mtp_hip import ops
    K = 4096
    print(f"case fill width M={M} N={N}", flush=True)
    g = torch.Generator().manual_seed(M * 13 + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = 0.02 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
    wq, ws = O.quantize_fp8_per_channel(W)
    y = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6, gamma=_dev(gm))
    ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
    torch.cuda.synchronize()
    ok, worst = close(y, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"


# (columns per workgroup, K-splits, waves, (M, N, K), W kind)
SKL_TW_CASES = [(224, "4", "8", (32, 3000, 2048), "fp8"), (200, None, "8", (24, 1000, 1024), "fp8"),
                (64, "2", "4", (40, 300, 512), "same"), (8, None, "8", (7, 100, 256), "fp8"),
                (120, "3", "4", (64, 520, 1536), "fp8")]


@pytest.mark.parametrize("tw,splits,waves,shape,wkind", SKL_TW_CASES)
def test_single_launch_column_widths(tw, splits, waves, shape, wkind):
    """The single-launch kernel with fewer output columns per workgroup than
    its 32 x waves-wide tile (tuning key skl_tw): the tile's last columns
    read zeros and are not stored; with and without K-splits, 4 and 8
    waves, ragged N; against the oracle and bit for bit on a second call."""
    M, N, K = shape
    _set(skl=1, skl_tw=tw, skl_waves=int(waves))
    if splits is not None:
        _set(skl_splits=int(splits))
    from mtp_hip import ops
    print(f"case skl tw={tw} splits={splits} waves={waves} M={M} N={N} K={K} w={wkind}",
          flush=True)
    g = torch.Generator().manual_seed(M * 41 + N + K + tw)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
    if wkind == "fp8":
        wq, ws = O.quantize_fp8_per_channel(W)
        run = lambda: ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6,
                                             gamma=_dev(gm))
        ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
    else:
        Wc = W.to(torch.bfloat16)
        run = lambda: ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5, gamma=_dev(gm))
        ref = O.rmsnorm_linear(x, Wc, b, 1e-6, 0.5, gamma=gm)
    y = run()
    torch.cuda.synchronize()
    ok, worst = close(y, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"
    assert torch.equal(y, run())


# (K-splits, A tiles per wave, compact <= 8-row blocks, (M, N, K)); None: planned
SKP_CASES = [(None, None, None, (1, 64, 128)), (None, None, None, (5, 200, 384)),
             (None, None, None, (16, 300, 4096)),
             ("2", "1", None, (17, 140, 256)), ("3", "2", None, (33, 130, 512)),
             (None, "4", None, (64, 300, 1024)),
             (None, None, None, (48, 1000, 2048)), ("5", None, None, (64, 2000, 2048)),
             (None, None, None, (64, 136, 8192)), (None, "2", None, (9, 520, 1280)),
             (None, None, None, (40, 70, 1344)), (None, None, None, (40, 70, 1280)),
             (None, None, None, (8, 700, 4096)), ("3", "2", None, (7, 130, 1536)),
             ("1", "4", None, (2, 300, 1024)), (None, None, None, (8, 1000, 8192)),
             (None, None, "0", (8, 300, 2048)), ("2", None, "0", (3, 200, 1024))]


# 16-bit W at K = 8192 would repeat the split counts of fp8 W at K = 4096
# (same bytes per row), so those pairs are not generated
SKP_PARAMS = [c + (wk,) for c in SKP_CASES for wk in ("fp8", "same")
              if not (wk == "same" and c[3][2] >= 8192)]


@pytest.mark.parametrize("splits,ta,h8,shape,wkind", SKP_PARAMS)
@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
def test_x_resident_skinny_kernel(splits, ta, h8, shape, wkind, xdtype):
    """The x-resident skinny kernel (tuning key skp=1): x rows of a K-split
    copied into LDS once, gamma applied there, norm applied to the fp32
    sums; planned and forced K-splits and A tiles per wave, compact and full
    x blocks for at most 8 rows, ragged M, N and split lengths, with and
    without gamma, bias and norm, against the oracle, and deterministic bit
    for bit."""
    M, N, K = shape
    _set(skp=1)
    if splits is not None:
        _set(skp_splits=int(splits))
    if ta is not None:
        _set(skp_ta=int(ta))
    if h8 is not None:
        _set(skp_h8=int(h8))
    from mtp_hip import ops
    print(f"case skp splits={splits} ta={ta} h8={h8} M={M} N={N} K={K} w={wkind} x={xdtype}",
          flush=True)
    g = torch.Generator().manual_seed(M * 29 + N + K)
    x = torch.randn(M, K, generator=g).to(xdtype)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(xdtype)
    if wkind == "fp8":
        wq, ws = O.quantize_fp8_per_channel(W)
        run = lambda: ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6,
                                             gamma=_dev(gm))
        ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
        y2 = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), None, 1e-6, norm=False)
        ref2 = O.rmsnorm_linear_fp8(x, wq, ws, None, 1e-6, norm=False)
    else:
        Wc = W.to(xdtype)
        run = lambda: ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5, gamma=_dev(gm))
        ref = O.rmsnorm_linear(x, Wc, b, 1e-6, 0.5, gamma=gm)
        y2 = ops.rmsnorm_linear(_dev(x), _dev(Wc), None, 1e-6, 1.0, norm=False)
        ref2 = O.rmsnorm_linear(x, Wc, None, 1e-6, 1.0, norm=False)
    y = run()
    torch.cuda.synchronize()
    for out, r in ((y, ref), (y2, ref2)):
        ok, worst = close(out, r, 2e-2)
        assert ok, f"worst err/bound = {worst:.3g}"
    assert torch.equal(y, run())


# (columns per workgroup, K-splits, A tiles per wave, (M, N, K), W kind)
SKP_TW_CASES = [(56, None, None, (8, 1000, 4096), "fp8"), (40, "2", None, (5, 300, 1024), "fp8"),
                (8, None, None, (16, 57, 512), "same"), (112, None, "2", (9, 700, 2048), "fp8"),
                (48, "3", "1", (33, 260, 1536), "fp8"), (24, None, None, (2, 100, 256), "same"),
                (160, None, "4", (8, 1000, 1024), "same"), (200, "2", "4", (3, 1500, 2048), "fp8")]


@pytest.mark.parametrize("tw,splits,ta,shape,wkind", SKP_TW_CASES)
def test_x_resident_column_widths(tw, splits, ta, shape, wkind):
    """The x-resident kernel with fewer output columns per workgroup than
    its 64 TA-wide tile (tuning key skp_tw): the tile's last columns read
    zeros and are not stored; with and without K-splits, one or two A tiles
    per wave, ragged N; against the oracle and bit for bit on a second
    call."""
    M, N, K = shape
    _set(skp=1, skp_tw=tw)
    if splits is not None:
        _set(skp_splits=int(splits))
    if ta is not None:
        _set(skp_ta=int(ta))
    from mtp_hip import ops
    print(f"case skp tw={tw} splits={splits} ta={ta} M={M} N={N} K={K} w={wkind}", flush=True)
    g = torch.Generator().manual_seed(M * 37 + N + K + tw)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.bfloat16)
    if wkind == "fp8":
        wq, ws = O.quantize_fp8_per_channel(W)
        run = lambda: ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), _dev(b), 1e-6,
                                             gamma=_dev(gm))
        ref = O.rmsnorm_linear_fp8(x, wq, ws, b, 1e-6, gamma=gm)
    else:
        Wc = W.to(torch.bfloat16)
        run = lambda: ops.rmsnorm_linear(_dev(x), _dev(Wc), _dev(b), 1e-6, 0.5, gamma=_dev(gm))
        ref = O.rmsnorm_linear(x, Wc, b, 1e-6, 0.5, gamma=gm)
    y = run()
    torch.cuda.synchronize()
    ok, worst = close(y, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"
    assert torch.equal(y, run())


@pytest.mark.parametrize("M,N,K,wkind", [(3, 8192, 4096, "same"), (13, 12288, 4096, "fp8")])
def test_single_launch_default_route_few_rows(M, N, K, wkind):
    """At most 16 rows with at least 48 MiB of W take the single-launch
    kernel with K-splits by default (no environment override)."""
    from mtp_hip import ops
    print(f"case skl default few rows M={M} N={N} K={K} w={wkind}", flush=True)
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    if wkind == "fp8":
        wq, ws = O.quantize_fp8_per_channel(W)
        y = ops.rmsnorm_linear_fp8(_dev(x), _dev(wq), _dev(ws), None, 1e-6, gamma=_dev(gm))
        ref = O.rmsnorm_linear_fp8(x, wq, ws, None, 1e-6, gamma=gm)
    else:
        Wc = W.to(torch.bfloat16)
        y = ops.rmsnorm_linear(_dev(x), _dev(Wc), None, 1e-6, 1.0, gamma=_dev(gm))
        ref = O.rmsnorm_linear(x, Wc, None, 1e-6, 1.0, gamma=gm)
    torch.cuda.synchronize()
    ok, worst = close(y, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("M,N,K", [(16, 4096, 1024), (1, 5, 16), (3, 17, 1008), (16, 130, 512),
                                   (9, 64, 272), (12, 1000, 48), (16, 4096, 4096), (7, 130, 1040),
                                   (16, 200, 8192), (1, 17, 2064), (17, 130, 1024),
                                   (32, 4096, 4096), (24, 200, 1040), (32, 64, 48),
                                   (8, 8192, 1024)])
@pytest.mark.parametrize("bias_dt", [None, torch.float32, torch.bfloat16, torch.float16])
def test_small_fp32_kernel(M, N, K, bias_dt):
    """fp32 x and W with at most 32 rows take the one-launch fp32 kernels by
    default (at most 16 rows, 512 < K <= 1024 and at most one workgroup per
    CU: every load of the launch in one round trip, here at N 4096 and 17;
    otherwise each wave's K-range streamed through LDS, one or two
    16-row tiles, ragged last blocks at K 1040 and 2064): ragged N (scalar stores), K not
    a multiple of the 256-k wave range,
    gamma / norm / bias (fp32, bf16, f16) / scale on and off, rtol 1e-5
    against the oracle; tuning key sf32=0 gives the tiled kernel the same answer."""
    from mtp_hip import ops
    print(f"case sf32 M={M} N={N} K={K} bias={bias_dt}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g)
    W = 0.05 * torch.randn(N, K, generator=g)
    gm = 1 + 0.1 * torch.randn(K, generator=g)
    b = None if bias_dt is None else (0.1 * torch.randn(N, generator=g)).to(bias_dt)
    y = ops.rmsnorm_linear(_dev(x), _dev(W), _dev(b), 1e-6, 0.75, gamma=_dev(gm))
    ref = O.rmsnorm_linear(x, W, b, 1e-6, 0.75, gamma=gm)
    y2 = ops.rmsnorm_linear(_dev(x), _dev(W), _dev(b), 1e-6, 1.0, norm=False)
    ref2 = O.rmsnorm_linear(x, W, b, 1e-6, 1.0, norm=False)
    torch.cuda.synchronize()
    for out, r in ((y, ref), (y2, ref2)):
        ok, worst = close(out, r, 1e-5)
        assert ok, f"worst err/bound = {worst:.3g}"
    _set(sf32=0)
    y3 = ops.rmsnorm_linear(_dev(x), _dev(W), _dev(b), 1e-6, 0.75, gamma=_dev(gm))
    torch.cuda.synchronize()
    ok, worst = close(y3, ref, 1e-5)
    assert ok, f"tiled kernel: worst err/bound = {worst:.3g}"


@pytest.mark.parametrize("M", [8, 32, 64])
def test_fp8_workload_full_size(M):
    """The fp8-e4m3 RMSNorm+linear workload: x bf16 [M,4096], W [14336,4096]."""
    from mtp_hip import ops, workloads
    d = workloads.fp8_linear(M)
    print(f"case fp8 workload M={M}", flush=True)
    y = ops.rmsnorm_linear_fp8(_dev(d["x"]), _dev(d["weight_fp8"]), _dev(d["wscale"]), None,
                               d["eps"], gamma=_dev(d["gamma"]))
    ref = O.rmsnorm_linear_fp8(d["x"], d["weight_fp8"], d["wscale"], None, d["eps"],
                               gamma=d["gamma"])
    ok, worst = close(y, ref, 2e-2)
    assert ok, f"worst err/bound = {worst:.3g}"
    # size-independent property: deterministic (fixed split order) bit for bit
    y2 = ops.rmsnorm_linear_fp8(_dev(d["x"]), _dev(d["weight_fp8"]), _dev(d["wscale"]), None,
                                d["eps"], gamma=_dev(d["gamma"]))
    assert torch.equal(y, y2)


def test_fp32_workload_full_size():
    """fp32 RMSNorm+linear workload (x[16,1024], W[4096,1024]), rtol 1e-5."""
    from mtp_hip import ops, workloads
    d = workloads.fp32_linear()
    y = ops.rmsnorm_linear(_dev(d["x"]), _dev(d["weight"]), None, d["eps"], 1.0,
                           gamma=_dev(d["gamma"]))
    ref = O.rmsnorm_linear(d["x"], d["weight"], None, d["eps"], 1.0, gamma=d["gamma"])
    ok, worst = close(y, ref, 1e-5)
    assert ok, f"worst err/bound = {worst:.3g}"


def test_graph_replay_matches_eager():
    """Captured into a HIP graph, every replay equals the eager result (the
    kernel re-arms its split-K tickets itself)."""
    from mtp_hip import ops
    M, N, K = 32, 2048, 2048
    x, W, b, gm = _inputs(M, N, K, torch.bfloat16, seed=5)
    x, W, b, gm = _dev(x), _dev(W), _dev(b), _dev(gm)
    eager = ops.rmsnorm_linear(x, W, b, 1e-6, 1.0, gamma=gm)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            ops.rmsnorm_linear(x, W, b, 1e-6, 1.0, gamma=gm)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.rmsnorm_linear(x, W, b, 1e-6, 1.0, gamma=gm)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        _ = (x.float() * 2).sum()  # eager work between replays
        torch.cuda.synchronize()


def test_cached_linear_drop_in():
    from mtp_hip.perf_hardening import CachedLinear
    torch.manual_seed(0)
    lin = CachedLinear(64, 96).to(DEV)
    x = torch.randn(2, 3, 64, device=DEV)
    y = lin(x)
    ref = torch.nn.functional.linear(x.cpu(), lin.weight.detach().cpu(), lin.bias.detach().cpu())
    ok, worst = close(y.reshape(-1, 96), ref.reshape(-1, 96), 1e-5)
    assert ok and y.shape == (2, 3, 96), worst
