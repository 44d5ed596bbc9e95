"""Drop-in module ``mtp_kernels`` (sys.path mode): with this directory ahead
of the reference on sys.path, ``import mtp_kernels`` resolves here and every
name the reference engine imports from it (mtp_engine.py:21-36, 1628-1633,
1787-1791; mtp_pipeline.py:7; mtp_radix.py:241) is the gfx950
implementation in mtp_hip/kernels.py."""
from mtp_hip.kernels import *  # noqa: F401,F403
from mtp_hip.kernels import (  # noqa: F401
    _HAS_TRITON,
    quantize_fp8_rows,
    tree_verify_attention,
    __all__,
)
