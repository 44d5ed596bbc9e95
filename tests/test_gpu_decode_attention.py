"""GPU parity of the decode attention entry points the engine imports
(fused_causal_attention, its fp8-KV variant) and of the tree monolith
fused_tree_attn_rmsnorm_linear against the CPU oracle. Tolerance |y - ref|
<= rtol (|ref| + RMS(ref)): 2e-2 for bf16 / f16 outputs, 1e-5 for fp32;
an all-masked monolith gives NaN rows exactly where the eager twin does."""
import pytest
import torch

from conftest import close
from oracle import eager as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL = {torch.bfloat16: 2e-2, torch.float16: 2e-2, torch.float32: 1e-5}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,H,L,D", [(2, 4, 300, 128), (1, 8, 1, 64), (3, 2, 65, 96),
                                     (1, 32, 2048, 128)])
def test_causal_attention_matches_oracle(dtype, B, H, L, D):
    import mtp_kernels as mk
    g = torch.Generator().manual_seed(B + H + L + D)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k = torch.randn(B, H, L, D, generator=g).to(dtype)
    v = torch.randn(B, H, L, D, generator=g).to(dtype)
    print(f"case causal {dtype} B={B} H={H} L={L} D={D}", flush=True)
    out = mk.fused_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    ok, worst = close(out, O.causal_attention(q, k, v), RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"
    out2 = mk.fused_bitmask_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    assert torch.equal(out2, out)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_causal_attention_fp8_matches_oracle(dtype):
    import mtp_kernels as mk
    g = torch.Generator().manual_seed(8)
    B, H, L, D = 2, 4, 77, 128
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k = torch.randn(B, H, L, D, generator=g)
    v = torch.randn(B, H, L, D, generator=g)
    ks = k.abs().amax(dim=(0, 2, 3)) / 448
    vs = v.abs().amax(dim=(0, 2, 3)) / 448
    k8 = (k / ks[None, :, None, None]).to(torch.float8_e4m3fn)
    v8 = (v / vs[None, :, None, None]).to(torch.float8_e4m3fn)
    out = mk.fused_causal_attention_fp8(q.to(DEV), k8.to(DEV), v8.to(DEV), ks.to(DEV), vs.to(DEV))
    torch.cuda.synchronize()
    ok, worst = close(out, O.causal_attention_fp8(q, k8, v8, ks, vs), RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"


MONO = [
    # B, H, D, L, N, dtype, wkind, bias, gamma
    (2, 4, 128, 64, 1000, torch.bfloat16, "same", True, True),
    (3, 2, 64, 37, 300, torch.float16, "same", False, True),
    (2, 3, 128, 20, 520, torch.float32, "same", True, False),
    (2, 4, 128, 64, 1000, torch.bfloat16, "fp8", True, True),
    (4, 1, 1024, 32, 32000, torch.bfloat16, "same", True, True),  # the engine's shape family
]


@pytest.mark.parametrize("B,H,D,L,N,dtype,wkind,bias,gamma", MONO)
def test_tree_monolith_matches_oracle(B, H, D, L, N, dtype, wkind, bias, gamma):
    import mtp_kernels as mk
    g = torch.Generator().manual_seed(B * H + D + L + N)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k = torch.randn(B, H, L, D, generator=g).to(dtype)
    v = torch.randn(B, H, L, D, generator=g).to(dtype)
    mask = (torch.rand(L, generator=g) > 0.4).float()
    mask[0] = 1.0
    W = 0.05 * torch.randn(N, D, generator=g)
    rms_w = (1 + 0.1 * torch.randn(D, generator=g)) if gamma else None
    pb = (0.1 * torch.randn(N, generator=g)).to(dtype) if bias else None
    if wkind == "fp8":
        W, ws = O.quantize_fp8_per_channel(W)
    else:
        W, ws = W.to(dtype), None
    dv = lambda t: None if t is None else t.to(DEV)  # noqa: E731
    print(f"case monolith B={B} H={H} D={D} L={L} N={N} {dtype} w={wkind}", flush=True)
    out = mk.fused_tree_attn_rmsnorm_linear(dv(q), dv(k), dv(v), dv(mask), dv(W), rms_w=dv(rms_w),
                                            proj_bias=dv(pb), wscale=dv(ws))
    torch.cuda.synchronize()
    ref = O.tree_attn_rmsnorm_linear(q, k, v, mask, W, rms_w, pb, ws)
    assert out.shape == (B, H, N) and out.dtype == dtype
    ok, worst = close(out, ref, RTOL[dtype])
    assert ok, f"worst err/bound = {worst:.3g}"
    # deterministic bit for bit
    out2 = mk.fused_tree_attn_rmsnorm_linear(dv(q), dv(k), dv(v), dv(mask), dv(W),
                                             rms_w=dv(rms_w), proj_bias=dv(pb), wscale=dv(ws))
    assert torch.equal(out, out2)


def test_tree_monolith_all_masked_is_nan_and_partial_blocks_are_finite():
    """A mask that admits no key: NaN everywhere, as the eager twin. A mask
    whose first blocks are all masked (the case the reference's fused kernel
    got wrong) stays finite and matches."""
    import mtp_kernels as mk
    g = torch.Generator().manual_seed(2)
    B, H, D, L, N = 2, 2, 128, 200, 256
    q = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, L, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, L, D, generator=g).to(torch.bfloat16)
    W = (0.05 * torch.randn(N, D, generator=g)).to(torch.bfloat16)
    none = mk.fused_tree_attn_rmsnorm_linear(q.to(DEV), k.to(DEV), v.to(DEV),
                                             torch.zeros(L).to(DEV), W.to(DEV))
    assert bool(torch.isnan(none.cpu()).all())
    late = torch.zeros(L)
    late[190:] = 1.0
    out = mk.fused_tree_attn_rmsnorm_linear(q.to(DEV), k.to(DEV), v.to(DEV), late.to(DEV),
                                            W.to(DEV))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.cpu()).all())
    ok, worst = close(out, O.tree_attn_rmsnorm_linear(q, k, v, late, W), 2e-2)
    assert ok, worst


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [512, 1024, 4096])
def test_wide_head_dim_attention(dtype, D):
    """Head dims above 256 (the monolith's single-head shape, D = hidden
    size) run the workgroup-per-query fallback."""
    import mtp_kernels as mk
    g = torch.Generator().manual_seed(D)
    B, H, L = 3, 1, 40
    q = torch.randn(B, H, D, generator=g).to(dtype)
    k = torch.randn(B, H, L, D, generator=g).to(dtype)
    v = torch.randn(B, H, L, D, generator=g).to(dtype)
    mask = (torch.rand(L, generator=g) > 0.5).float()
    mask[3] = 1.0
    out = mk.fused_causal_attention(q.to(DEV), k.to(DEV), v.to(DEV))
    out_t = mk.fused_tree_attention(q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV))
    torch.cuda.synchronize()
    ok, worst = close(out, O.causal_attention(q, k, v), RTOL[dtype])
    assert ok, f"causal worst err/bound = {worst:.3g}"
    ok, worst = close(out_t, O.tree_attention(q, k, v, mask), RTOL[dtype])
    assert ok, f"tree worst err/bound = {worst:.3g}"
