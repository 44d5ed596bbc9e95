"""Drop-in module ``mtp_fused_verify`` (sys.path mode): fused_verify and
fused_multi_verify (mtp_engine.py:47) are the gfx950 implementation in
mtp_hip/fused_verify.py."""
from mtp_hip.fused_verify import *  # noqa: F401,F403
from mtp_hip.fused_verify import __all__  # noqa: F401
