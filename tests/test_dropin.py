"""The drop-in boundary on the CPU (no kernel runs): every name the
reference's engine, pipelines, radix cache, tests and benches import from
mtp_kernels / mtp_fused_verify / mtp_perf_hardening resolves in this build's
modules (sys.path mode), and install() replaces exactly the hot-path names
of stand-in reference modules with the gfx950 functions and puts them back.
The name lists are data transcribed from the reference's import statements
(tests/golden/reference_imports.json)."""
import importlib
import json
import os
import types

import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
DATA = json.load(open(os.path.join(HERE, "golden", "reference_imports.json")))


def _needed():
    need = {}
    for imp in DATA["imports"]:
        need.setdefault(imp["module"], set()).update(imp["names"])
    for mod, names in DATA["module_all"].items():
        need.setdefault(mod, set()).update(names)
    return need


@pytest.mark.parametrize("module", sorted(_needed()))
def test_sys_path_modules_export_every_imported_name(module):
    mod = importlib.import_module(module)  # this build's module (tests put it first)
    assert os.path.dirname(os.path.abspath(mod.__file__)).endswith("mtp-engine_amd")
    missing = sorted(n for n in _needed()[module] if not hasattr(mod, n))
    assert not missing, f"{module} lacks {missing}"
    # `from mtp_x import *` must not name anything undefined
    for n in getattr(mod, "__all__", []):
        assert hasattr(mod, n), f"{module}.__all__ names {n}, which is undefined"


def test_no_triton_route_and_hot_path_names_are_the_hip_functions():
    import mtp_kernels
    import mtp_fused_verify
    import mtp_perf_hardening
    from mtp_hip import fused_verify as fv, kernels as k, perf_hardening as ph
    assert mtp_kernels._HAS_TRITON is False
    ours = {"mtp_kernels": (mtp_kernels, k), "mtp_fused_verify": (mtp_fused_verify, fv),
            "mtp_perf_hardening": (mtp_perf_hardening, ph)}
    for mod, names in DATA["hot_path"].items():
        shim, impl = ours[mod]
        for n in names:
            assert getattr(shim, n) is getattr(impl, n), (mod, n)


def _stand_in(name, names):
    m = types.ModuleType(name)
    for n in names:
        setattr(m, n, ("reference", name, n))
    return m


def test_install_replaces_exactly_the_hot_path_and_uninstall_restores():
    import mtp_hip
    from mtp_hip import dropin, fused_verify as fv, kernels as k, ops, perf_hardening as ph
    need = _needed()
    km = _stand_in("mtp_kernels", need["mtp_kernels"] | set(dropin.KERNELS_NAMES))
    vm = _stand_in("mtp_fused_verify", need["mtp_fused_verify"] | {"_HAS_TRITON"})
    hm = _stand_in("mtp_perf_hardening", need["mtp_perf_hardening"])

    class RadixKVCache:
        def __init__(self):
            self.device = torch.device("cpu")

        def batch_prefix_match(self, ids):
            return "reference eager"

    rm = types.ModuleType("mtp_radix")
    rm.RadixKVCache = RadixKVCache
    em = _stand_in("mtp_engine", need["mtp_kernels"] | need["mtp_fused_verify"] |
                   need["mtp_perf_hardening"] | {"DEVICE", "SpeculativeDecodingEngine"})
    before = {id(m): dict(vars(m)) for m in (km, vm, hm, em)}

    rec = mtp_hip.install(km, vm, hm, rm, em)
    for n in DATA["hot_path"]["mtp_kernels"]:
        assert getattr(km, n) is getattr(k, n), n
    for n in DATA["hot_path"]["mtp_fused_verify"]:
        assert getattr(vm, n) is getattr(fv, n), n
    for n in DATA["hot_path"]["mtp_perf_hardening"]:
        assert getattr(hm, n) is getattr(ph, n), n
    assert km._HAS_TRITON is False and vm._HAS_TRITON is False
    # the engine's own bindings of hot-path names are redirected, the rest kept
    assert em.fused_rmsnorm_linear is k.fused_rmsnorm_linear
    assert em.fused_multi_verify is fv.fused_multi_verify
    assert em.argmax_greedy is ph.argmax_greedy
    assert em.SpeculativeDecodingEngine == ("reference", "mtp_engine", "SpeculativeDecodingEngine")
    # everything not on the hot path still resolves to the reference object
    replaced = set(dropin.KERNELS_NAMES) | set(dropin.VERIFY_NAMES) | set(dropin.HARDENING_NAMES)
    for n in need["mtp_kernels"] - replaced:
        assert getattr(km, n) == ("reference", "mtp_kernels", n), n
    for n in need["mtp_perf_hardening"] - replaced:
        assert getattr(hm, n) == ("reference", "mtp_perf_hardening", n), n
    # every import statement of the reference resolves against the patched modules
    mods = {"mtp_kernels": km, "mtp_fused_verify": vm, "mtp_perf_hardening": hm}
    for imp in DATA["imports"]:
        for n in imp["names"]:
            assert hasattr(mods[imp["module"]], n), (imp["site"], n)
    # radix: device ids take the kernel, host ids keep the reference's route
    cache = rm.RadixKVCache()
    assert cache.batch_prefix_match(torch.zeros(2, 3, dtype=torch.long)) == "reference eager"
    mtp_hip.uninstall(rec)
    for m in (km, vm, hm, em):
        assert dict(vars(m)) == before[id(m)]
    assert rm.RadixKVCache().batch_prefix_match(None) == "reference eager"
    assert ops.batch_prefix_match is not None


def test_host_helpers_match_reference_contracts():
    import mtp_perf_hardening as mh
    assert [mh.next_pow2(n) for n in (0, 1, 2, 3, 17, 64)] == [1, 1, 2, 4, 32, 64]
    assert mh.align_vocab(128256) == 128256 and mh.align_vocab(1) == 128
    assert mh.align_vocab(130, 64) == 192
    assert mh.pad_seq_len(33) == 64 and mh.pad_batch(9) == 16
    assert mh.fast_check((2, 3), (2, 3)) and not mh.fast_check((2, 3), (2,))
    c = mh.PrecomputedConstants(128, 4096, 1000, torch.bfloat16, temperature=0.0)
    assert c.inv_temperature == 0.0 and c.vocab_padded == 1024
    assert abs(c.attn_scale - 128 ** -0.5) < 1e-12
    pool = mh.PinnedBufferPool(2, 8)
    v = pool.stage_prompt(torch.tensor([[1, 2, 3]]))
    assert v.tolist() == [[1, 2, 3]]
    assert mh.maybe_compile(torch.nn.Linear(2, 2)).__class__ is torch.nn.Linear
    import mtp_kernels as mk
    assert mk.build_tuning_config().fp8_scale == 1.0
