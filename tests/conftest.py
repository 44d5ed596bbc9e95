import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mtp-engine_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built libmtp_hip.so")


def has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if has_gpu():
        return
    skip = pytest.mark.skip(reason="no HIP GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def close(y, ref, rtol):
    """|y - ref| <= rtol * (|ref| + RMS(ref)) elementwise, in fp64."""
    import torch
    y = y.detach().cpu().to(torch.float64)
    ref = ref.detach().cpu().to(torch.float64)
    rms = ref.pow(2).mean().sqrt() if ref.numel() else torch.tensor(0.0, dtype=torch.float64)
    err = (y - ref).abs()
    bound = rtol * (ref.abs() + rms)
    ok = bool((err <= bound).all())
    worst = float((err / (bound + 1e-300)).max()) if ref.numel() else 0.0
    return ok, worst


@pytest.fixture
def tune():
    """Set library tuning keys (mtp_set_tuning) for one test; every key goes
    back to the planner's choice afterwards."""
    from mtp_hip import _lib

    def setter(**keys):
        _lib.set_tuning(**keys)

    yield setter
    _lib.set_tuning(**{k: -1 for k in _lib.TUNING_KEYS})
