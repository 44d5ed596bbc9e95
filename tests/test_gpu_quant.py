"""GPU quantizers against the oracle, bit-exact: fp8-e4m3 per tensor and per
channel (including every rounding tie between adjacent e4m3 values), the fp8
dequantizer, grouped INT4 (including half-integer ties, which torch.round
sends to the even neighbour) and the INT4 dequantizer."""
from __future__ import annotations

import pytest
import torch

from oracle import eager as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _fp8_midpoints() -> torch.Tensor:
    """Every positive finite e4m3fn value, every midpoint between neighbours,
    and their negatives (scale stays 1: the largest value is 448)."""
    t = torch.from_numpy(O.fp8_e4m3fn_decode_table()).float()
    pos = torch.unique(t[torch.isfinite(t) & (t >= 0)]).sort().values
    mids = (pos[1:] + pos[:-1]) / 2
    v = torch.cat([pos, mids])
    return torch.cat([v, -v])


def test_fp8_per_tensor_is_bit_exact_including_ties():
    from mtp_kernels import quantize_fp8_e4m3
    g = torch.Generator().manual_seed(0)
    for x in (_fp8_midpoints(), torch.randn(3, 1000, generator=g) * 3,
              torch.randn(257, generator=g).to(torch.bfloat16), torch.zeros(10)):
        q, s = quantize_fp8_e4m3(x.to(DEV))
        qr, sr = O.quantize_fp8_per_tensor(x)
        assert float(s) == float(sr)
        assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))


def test_fp8_per_channel_is_bit_exact():
    from mtp_kernels import quantize_fp8_rows
    g = torch.Generator().manual_seed(1)
    w = 0.02 * torch.randn(300, 520, generator=g)
    w[7] = 0.0
    q, s = quantize_fp8_rows(w.to(DEV))
    qr, sr = O.quantize_fp8_per_channel(w)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))
    # the fp8 RMSNorm+linear workload's weights come from this producer
    from mtp_hip import workloads
    d = workloads.fp8_linear(8)
    assert d["weight_fp8"].dtype == torch.float8_e4m3fn


@pytest.mark.parametrize("K", [8, 520, 2056, 4096, 8192, 16384, 522, 16392])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fp8_per_channel_row_widths(K, dtype):
    """Rows of 8 c elements up to 16384 take the one-pass kernel (1, 2, 4 or
    8 chunks of 8 per thread); 522 and 16392 take the two-pass kernels. Row
    0 holds every e4m3 value and every midpoint at scale 1 where it fits."""
    from mtp_kernels import quantize_fp8_rows
    g = torch.Generator().manual_seed(K)
    w = 0.02 * torch.randn(12, K, generator=g)
    mids = _fp8_midpoints()
    if K >= mids.numel():
        w[0] = 0.0
        w[0, : mids.numel()] = mids
    w[3] = 0.0
    w = w.to(dtype)
    q, s = quantize_fp8_rows(w.to(DEV))
    qr, sr = O.quantize_fp8_per_channel(w)
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))


def test_fp8_dequantize_is_exact():
    from mtp_kernels import dequantize_fp8
    g = torch.Generator().manual_seed(2)
    x = torch.randn(64, 96, generator=g)
    q, s = O.quantize_fp8_per_tensor(x)
    assert torch.equal(dequantize_fp8(q.to(DEV), s.to(DEV)).cpu(), O.dequantize_fp8(q, s))
    qr, sr = O.quantize_fp8_per_channel(x)
    out = dequantize_fp8(qr.to(DEV), sr[:, None].to(DEV)).cpu()
    assert torch.equal(out, O.dequantize_fp8(qr, sr[:, None]))


@pytest.mark.parametrize("group", [8, 32, 128, 512])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", ["whole", "ragged"])
def test_int4_quantize_is_bit_exact_including_ties(group, dtype, shape):
    """Whole groups per row take the vector kernel (8 elements per lane, the
    group's amax by lane shuffles); a ragged last group takes the
    per-group kernel. Both must give the oracle's bytes and scales."""
    from mtp_kernels import quantize_int4
    g = torch.Generator().manual_seed(group)
    N, K = 40, 4 * group + (0 if shape == "whole" else 4)
    w = (0.02 * torch.randn(N, K, generator=g)).to(dtype)
    # rows whose groups have amax 7 (scale 1) and half-integer entries
    ties = torch.tensor([-7.5, -6.5, -2.5, -1.5, -0.5, 0.5, 1.5, 2.5, 3.5, 6.5])
    w[0, :group] = 0.0
    w[0, :10] = ties.to(dtype)
    w[0, 10] = 7.0
    w[1] = 0.0
    packed, scales = quantize_int4(w.to(DEV), group)
    pr, sr = O.quantize_int4(w, group)
    assert torch.equal(scales.cpu(), sr)
    assert torch.equal(packed.cpu(), pr)


def test_int4_dequantize_is_exact():
    from mtp_kernels import dequantize_int4
    g = torch.Generator().manual_seed(9)
    packed = torch.randint(0, 256, (33, 64), generator=g, dtype=torch.uint8)
    for sdt, group in ((torch.float32, 32), (torch.float16, 128)):
        scales = torch.rand(33, (128 + group - 1) // group, generator=g).to(sdt)
        out = dequantize_int4(packed.to(DEV), scales.to(DEV), 128, group).cpu()
        assert torch.equal(out, O.dequantize_int4(packed, scales, 128, group))


def test_quantizers_at_workload_sizes():
    """The weight producers at the workloads' full sizes, bit for bit: the
    per-channel fp8 quantizer on the fp8 linear's W [14336, 4096] and the
    grouped INT4 quantizer (group 128) on the INT4 linear's W [28672,
    8192], both fp32, both through the vector kernels."""
    from mtp_kernels import quantize_fp8_rows, quantize_int4
    g = torch.Generator(device=DEV).manual_seed(11)
    print("case fp8 rows 14336 x 4096", flush=True)
    w = 0.02 * torch.randn(14336, 4096, generator=g, device=DEV)
    q, s = quantize_fp8_rows(w)
    qr, sr = O.quantize_fp8_per_channel(w.cpu())
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))
    del w, q, s, qr, sr
    print("case int4 28672 x 8192 group 128", flush=True)
    w = 0.02 * torch.randn(28672, 8192, generator=g, device=DEV)
    packed, scales = quantize_int4(w, 128)
    pr, sr = O.quantize_int4(w.cpu(), 128)
    assert torch.equal(scales.cpu(), sr)
    assert torch.equal(packed.cpu(), pr)

