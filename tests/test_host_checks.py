"""Host-side guards of the Python shim (CPU): tensors that are not on a HIP
device, or whose shapes disagree, are refused before any library call, and
CachedLinear's cached views follow its parameters through .to()."""
import pytest
import torch

from mtp_hip import ops


def test_host_tensors_are_refused():
    x = torch.randn(4, 64)
    W = torch.randn(32, 64)
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.rmsnorm_linear(x, W)
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.rmsnorm_linear_fp8(x, W.to(torch.float8_e4m3fn), torch.ones(32))
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.verify(x, W, torch.zeros(4, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.multi_verify(x.reshape(1, 4, 64), W, torch.zeros(1, 3, dtype=torch.int64))


def test_shape_mismatches_are_assertions():
    x = torch.randn(4, 64)
    with pytest.raises(AssertionError):
        ops.rmsnorm_linear(x, torch.randn(32, 63))
    with pytest.raises(AssertionError):
        ops.rmsnorm_linear(x, torch.randn(32, 64), torch.randn(31))
    with pytest.raises(AssertionError):
        ops.rmsnorm_linear(x, torch.randn(32, 64), gamma=torch.randn(65))
    with pytest.raises(AssertionError):
        ops.multi_verify(torch.randn(2, 5, 64), torch.randn(10, 64), torch.zeros(2, 3))
    with pytest.raises(AssertionError):
        ops.int4_matmul(x, torch.zeros(8, 31, dtype=torch.uint8), torch.ones(8, 2), 64, 32)
    with pytest.raises(AssertionError):
        ops.int4_matmul(x, torch.zeros(8, 32, dtype=torch.uint8), torch.ones(8, 3), 64, 32)


def test_cached_linear_follows_module_moves():
    from mtp_hip.perf_hardening import CachedLinear
    lin = CachedLinear(8, 4)
    lin = lin.to(torch.float64)
    assert lin._w.dtype == torch.float64 and lin._w.data_ptr() == lin.weight.data_ptr()
    assert lin._b.data_ptr() == lin.bias.data_ptr()
