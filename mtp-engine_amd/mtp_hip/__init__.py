"""MI355X (gfx950) verify/draft hot path of the mtp-engine speculative decoder.

Kernels are hand-written HIP in ../csrc, exported through the C ABI of
include/mtp_hip.h as libmtp_hip.so and bound here with ctypes. ``ops`` holds
the tensor-level entry points; ``kernels``, ``fused_verify`` and
``perf_hardening`` keep the reference modules' names and signatures on top
of it. ``install(...)`` puts the hot-path names into reference modules the
caller already imported; the modules ``mtp_kernels`` / ``mtp_fused_verify``
one directory up (that directory first on sys.path) are the other way in
for those two modules.
"""
from . import ops
from ._lib import LIB_PATH, MtpHipError, load, reserve_workspace
from .dropin import install, uninstall

__all__ = ["ops", "load", "LIB_PATH", "MtpHipError", "reserve_workspace", "install", "uninstall"]
