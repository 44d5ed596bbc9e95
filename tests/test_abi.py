"""The C-ABI library loads, exports every symbol include/mtp_hip.h declares,
and validates arguments on the host (status codes, no GPU call)."""
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mtp_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mtp_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from mtp_hip import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmtp_hip.so not built: run python mtp-engine_amd/build.py")
    return _lib.load()


def test_every_declared_symbol_is_exported(lib):
    from mtp_hip import _lib
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in mtp_hip.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_status_strings(lib):
    assert lib.mtp_abi_version() == 1
    assert lib.mtp_status_string(0) == b"ok"
    for s in range(-7, 0):
        assert lib.mtp_status_string(s) not in (b"ok", b"unknown status")


def test_validation_without_gpu(lib):
    from mtp_hip import _lib as L
    fake = 4096  # never dereferenced: every call below returns before any HIP call
    # unsupported x dtype
    assert lib.mtp_fused_rmsnorm_linear(fake, 99, 4, 64, fake, L.F32, 8, None, 0, None, 0,
                                        1e-6, 1.0, 1, fake, None, 0, None) == L.ERR_DTYPE
    # empty batch is a no-op
    assert lib.mtp_fused_rmsnorm_linear(None, L.F32, 0, 64, None, L.F32, 8, None, 0, None, 0,
                                        1e-6, 1.0, 1, None, None, 0, None) == L.OK
    # missing output
    assert lib.mtp_fused_rmsnorm_linear(fake, L.F32, 4, 64, fake, L.F32, 8, None, 0, None, 0,
                                        1e-6, 1.0, 1, None, None, 0, None) == L.ERR_NULL
    # fp8 entry needs the channel scale
    assert lib.mtp_fused_rmsnorm_linear_fp8(fake, L.BF16, 4, 64, fake, L.FP8E4M3, None, 8, None, 0,
                                            None, 0, 1e-6, 1, fake, None, 0, None) == L.ERR_NULL
    # int4: odd K / odd group / bad nibble mode
    args = dict(x=fake, xt=L.BF16, M=4, K=63, pk=fake, sc=fake, sct=L.F16, N=8, g=32, nib=0)
    assert lib.mtp_fused_int4_matmul(fake, L.BF16, 4, 63, fake, fake, L.F16, 8, 32, 0, None, 0,
                                     1e-6, 0, fake, None, 0, None) == L.ERR_SHAPE
    assert lib.mtp_fused_int4_matmul(fake, L.BF16, 4, 64, fake, fake, L.F16, 8, 33, 0, None, 0,
                                     1e-6, 0, fake, None, 0, None) == L.ERR_SHAPE
    assert lib.mtp_fused_int4_matmul(fake, L.BF16, 4, 64, fake, fake, L.F16, 8, 32, 5, None, 0,
                                     1e-6, 0, fake, None, 0, None) == L.ERR_ARG
    del args
    # multi-verify: S must equal D + 1
    assert lib.mtp_fused_multi_verify(fake, L.BF16, 2, 5, 64, fake, L.BF16, 256, None, 0, fake, 3,
                                      fake, fake, fake, None, fake, 1 << 20, None) == L.ERR_SHAPE
    # verify: a weight dtype that is not a float
    assert lib.mtp_fused_verify(fake, L.BF16, 4, 64, fake, L.I32, 256, None, 0, fake, fake, fake,
                                fake, 1 << 20, None) == L.ERR_DTYPE
    # verify: workspace too small
    need = lib.mtp_verify_workspace_bytes(L.BF16, 4, 1, 256, 64)
    assert need > 0
    assert lib.mtp_fused_verify(fake, L.BF16, 4, 64, fake, L.BF16, 256, None, 0, fake, fake, fake,
                                fake, need - 1, None) == L.ERR_WORKSPACE


def test_workspace_queries_are_host_only(lib):
    from mtp_hip import _lib as L
    # fp8 workload at M = 64: split-K partials are needed
    assert lib.mtp_rmsnorm_linear_workspace_bytes(L.BF16, L.FP8E4M3, 64, 14336, 4096) > 0
    # shapes the tiled kernel does not take need no workspace
    assert lib.mtp_rmsnorm_linear_workspace_bytes(L.BF16, L.BF16, 4, 64, 63) == 0
    assert lib.mtp_verify_workspace_bytes(L.BF16, 40, 5, 128256, 4096) > 0
    assert lib.mtp_verify_workspace_bytes(L.BF16, 40, 0, 128256, 4096) == 0


def test_new_entry_points_validate_without_gpu(lib):
    from mtp_hip import _lib as L
    fake = 4096
    # draft chain
    assert lib.mtp_fused_rmsnorm(fake, 99, 4, 64, None, 0, 1e-6, fake, None) == L.ERR_DTYPE
    assert lib.mtp_fused_rmsnorm(None, L.BF16, 0, 64, None, 0, 1e-6, None, None) == L.OK
    assert lib.mtp_fused_add_rmsnorm(fake, None, L.BF16, 4, 64, None, 0, 1e-6, fake,
                                     None) == L.ERR_NULL
    assert lib.mtp_argmax(fake, L.BF16, 4, 100, 50, fake, None, 0, 0, 0, None, None, 0,
                          None) == L.ERR_SHAPE  # ld < V
    assert lib.mtp_argmax(fake, L.BF16, 4, 100, 100, fake, fake, L.BF16, 99, 8, fake, None, 0,
                          None) == L.ERR_SHAPE  # table smaller than the vocabulary
    assert lib.mtp_argmax_workspace_bytes(8, 128256) > 65536
    assert lib.mtp_argmax_workspace_bytes(100000, 50) == 0  # one workgroup per row
    # KV step
    assert lib.mtp_batch_prefix_match(None, 0, 5, None, None) == L.OK
    assert lib.mtp_batch_prefix_match(fake, 3, 5, None, None) == L.ERR_NULL
    assert lib.mtp_verify_commit(fake, fake, fake, fake, L.F32, 2, 3, fake, fake, fake, fake,
                                 None, 0, None, None) == L.ERR_DTYPE
    assert lib.mtp_verify_commit(fake, fake, fake, fake, L.I64, 0, 3, fake, fake, fake, fake,
                                 None, 0, None, None) == L.ERR_SHAPE
    assert lib.mtp_paged_kv_write(fake, fake, L.BF16, 1, 2, 3, 128, 0, 0, 0, None, fake, L.BF16,
                                  4, 16, fake, 64, None, 0, 0, None) == L.ERR_NULL
    # decode attention / monolith
    assert lib.mtp_fused_causal_attention_fp8(fake, L.BF16, 1, 2, 64, fake, fake, 8, None, fake,
                                              0.1, fake, None) == L.ERR_NULL
    assert lib.mtp_fused_tree_attn_rmsnorm_linear(
        fake, L.BF16, 1, 2, 64, fake, fake, 8, fake, L.F32, fake, L.FP8E4M3, 10, None, 0, None,
        0, None, 0.1, 1e-6, fake, fake, 1 << 24, None) == L.ERR_NULL  # fp8 W needs wscale
    assert lib.mtp_tree_attn_rmsnorm_linear_workspace_bytes(L.BF16, 4, 1, 4096, 64, L.BF16,
                                                           128256) > 65536
    # workspace initialiser
    assert lib.mtp_workspace_init(None, 0, None) == L.OK
    assert lib.mtp_workspace_init(fake + 4, 256, None) == L.ERR_ALIGN


def test_tuning_keys_round_trip(lib):
    from mtp_hip import _lib as L
    for k in L.TUNING_KEYS:
        with L.tuning(**{k: 3}):
            assert L.get_tuning(k) == 3
    assert lib.mtp_set_tuning(b"no_such_key", 1) == L.ERR_ARG
    assert lib.mtp_set_tuning(b"skl", -2) == L.ERR_ARG
