"""MI355X (gfx950) verify/draft hot path of the mtp-engine speculative decoder.

Kernels are hand-written HIP in ../csrc, exported through the C ABI of
include/mtp_hip.h as libmtp_hip.so and bound here with ctypes. ``ops`` holds
the tensor-level entry points; ``kernels``, ``fused_verify`` and
``perf_hardening`` keep the reference modules' names and signatures on top
of it. Two ways in: the modules ``mtp_kernels`` / ``mtp_fused_verify`` /
``mtp_perf_hardening`` one directory up (put that directory first on
sys.path), or ``install(...)`` into reference modules already imported.
"""
from . import ops
from ._lib import LIB_PATH, MtpHipError, load, reserve_workspace
from .dropin import install, uninstall

__all__ = ["ops", "load", "LIB_PATH", "MtpHipError", "reserve_workspace", "install", "uninstall"]
