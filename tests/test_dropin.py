"""The drop-in boundary on the CPU (no kernel runs).

* install() replaces exactly the hot-path names (the fixture's `hot_path`
  lists, the RMSNorm -> linear family, quantizers, tree / paged attention,
  the verify entry points and the draft chain's argmax / norms, plus the
  radix cache's prefix match) in stand-in reference modules, leaves every
  other attribute alone, and uninstall() puts them back.
* The sys.path drop-in modules mtp_kernels / mtp_fused_verify export every
  name the reference's engine, pipelines, radix cache, parity tests and
  benches import from them.
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
SYS_PATH_MODULES = ("mtp_kernels", "mtp_fused_verify")


def _needed():
    need = {}
    for imp in DATA["imports"]:
        need.setdefault(imp["module"], set()).update(imp["names"])
    for mod, names in DATA["module_all"].items():
        need.setdefault(mod, set()).update(names)
    return need


@pytest.mark.parametrize("module", SYS_PATH_MODULES)
def test_sys_path_modules_export_every_imported_name(module):
    mod = importlib.import_module(module)  # this build's module (tests put it first)
    assert os.path.dirname(os.path.abspath(mod.__file__)).endswith("mtp-engine_amd")
    missing = sorted(n for n in _needed()[module] if not hasattr(mod, n))
    assert not missing, f"{module} lacks {missing}"
    # `from mtp_x import *` must not name anything undefined
    for n in getattr(mod, "__all__", []):
        assert hasattr(mod, n), f"{module}.__all__ names {n}, which is undefined"


def test_no_perf_hardening_shim():
    # the reference's own mtp_perf_hardening supplies its host helpers;
    # install() patches its three hot-path names
    root = os.path.join(os.path.dirname(HERE), "mtp-engine_amd")
    assert not os.path.exists(os.path.join(root, "mtp_perf_hardening.py"))
    from mtp_hip import perf_hardening as ph
    assert sorted(ph.__all__) == sorted(DATA["hot_path"]["mtp_perf_hardening"])


def test_no_triton_route_and_hot_path_names_are_the_hip_functions():
    import mtp_kernels
    import mtp_fused_verify
    from mtp_hip import fused_verify as fv, kernels as k
    assert mtp_kernels._HAS_TRITON is False
    ours = {"mtp_kernels": (mtp_kernels, k), "mtp_fused_verify": (mtp_fused_verify, fv)}
    for mod in SYS_PATH_MODULES:
        shim, impl = ours[mod]
        for n in DATA["hot_path"][mod]:
            assert getattr(shim, n) is getattr(impl, n), (mod, n)


def test_install_names_are_the_hot_path():
    from mtp_hip import dropin
    assert set(dropin.KERNELS_NAMES) == set(DATA["hot_path"]["mtp_kernels"])
    assert set(dropin.VERIFY_NAMES) == set(DATA["hot_path"]["mtp_fused_verify"])
    assert set(dropin.HARDENING_NAMES) == set(DATA["hot_path"]["mtp_perf_hardening"])


def _stand_in(name, names):
    m = types.ModuleType(name)
    for n in names:
        setattr(m, n, ("reference", name, n))
    return m


def test_install_replaces_exactly_the_hot_path_and_uninstall_restores():
    import mtp_hip
    from mtp_hip import dropin, fused_verify as fv, kernels as k, ops, perf_hardening as ph
    need = _needed()
    km = _stand_in("mtp_kernels", need["mtp_kernels"] | set(dropin.KERNELS_NAMES) |
                   {"fused_bitmask_attention", "prewarm_autotuner"})
    vm = _stand_in("mtp_fused_verify", need["mtp_fused_verify"] | {"_HAS_TRITON"})
    hm = _stand_in("mtp_perf_hardening", need["mtp_perf_hardening"] | set(dropin.HARDENING_NAMES) |
                   {"next_pow2", "pad_batch", "maybe_compile", "get_stream"})

    class RadixKVCache:
        def __init__(self):
            self.device = torch.device("cpu")

        def batch_prefix_match(self, ids):
            return "reference eager"

    rm = types.ModuleType("mtp_radix")
    rm.RadixKVCache = RadixKVCache
    em = _stand_in("mtp_engine", need["mtp_kernels"] | need["mtp_fused_verify"] |
                   need["mtp_perf_hardening"] | {"DEVICE", "SpeculativeDecodingEngine"})
    mods = (km, vm, hm, em)
    before = {id(m): dict(vars(m)) for m in mods}

    rec = mtp_hip.install(km, vm, hm, rm, em)
    impl = {"mtp_kernels": (km, k), "mtp_fused_verify": (vm, fv), "mtp_perf_hardening": (hm, ph)}
    hot = set()
    for mod, (patched, ours) in impl.items():
        for n in DATA["hot_path"][mod]:
            assert getattr(patched, n) is getattr(ours, n), (mod, n)
            hot.add(n)
    # exactly the hot-path names changed, in every module
    for m in mods:
        changed = {n for n, v in vars(m).items() if before[id(m)].get(n, object()) is not v}
        expect = {n for n in hot if n in before[id(m)]}
        assert changed == expect, (m.__name__, sorted(changed ^ expect))
    assert km._HAS_TRITON == ("reference", "mtp_kernels", "_HAS_TRITON")
    assert vm._HAS_TRITON == ("reference", "mtp_fused_verify", "_HAS_TRITON")
    # the engine's own bindings of hot-path names are redirected, the rest kept
    assert em.fused_rmsnorm_linear is k.fused_rmsnorm_linear
    assert em.fused_multi_verify is fv.fused_multi_verify
    assert em.argmax_greedy is ph.argmax_greedy
    assert em.fused_causal_attention == ("reference", "mtp_engine", "fused_causal_attention")
    assert em.SpeculativeDecodingEngine == ("reference", "mtp_engine", "SpeculativeDecodingEngine")
    assert set(rec.names()) == {"mtp_kernels", "mtp_fused_verify", "mtp_perf_hardening",
                                "mtp_engine", "RadixKVCache"}
    # every import statement of the reference resolves against the patched modules
    by_name = {"mtp_kernels": km, "mtp_fused_verify": vm, "mtp_perf_hardening": hm}
    for imp in DATA["imports"]:
        for n in imp["names"]:
            assert hasattr(by_name[imp["module"]], n), (imp["site"], n)
    # radix: device ids take the kernel, host ids keep the reference's route
    cache = rm.RadixKVCache()
    assert cache.batch_prefix_match(torch.zeros(2, 3, dtype=torch.long)) == "reference eager"
    mtp_hip.uninstall(rec)
    for m in mods:
        assert dict(vars(m)) == before[id(m)]
    assert rm.RadixKVCache().batch_prefix_match(None) == "reference eager"
    assert ops.batch_prefix_match is not None


def test_tuning_config_default():
    import mtp_kernels as mk
    assert mk.build_tuning_config().fp8_scale == 1.0
