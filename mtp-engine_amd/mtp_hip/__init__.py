"""MI355X (gfx950) verify/draft hot path of the mtp-engine speculative decoder.

Kernels are hand-written HIP in ../csrc, exported through the C ABI of
include/mtp_hip.h as libmtp_hip.so and bound here with ctypes. The drop-in
modules ``mtp_kernels`` and ``mtp_fused_verify`` (one directory up) keep the
reference's function names and signatures on top of ``mtp_hip.ops``.
"""
from . import ops
from ._lib import LIB_PATH, MtpHipError, load

__all__ = ["ops", "load", "LIB_PATH", "MtpHipError"]
