"""Drop-in module ``mtp_perf_hardening`` (sys.path mode): the names the
engine imports (mtp_engine.py:49-57) and CachedLinear come from
mtp_hip/perf_hardening.py."""
from mtp_hip.perf_hardening import *  # noqa: F401,F403
from mtp_hip.perf_hardening import __all__  # noqa: F401
