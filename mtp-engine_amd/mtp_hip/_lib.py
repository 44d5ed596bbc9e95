"""ctypes binding of libmtp_hip.so (the C ABI in include/mtp_hip.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already loaded (both carry the soname libamdhip64.so.7); the kernels then run
on torch's streams and memory. A missing library is an error, never a silent
fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime first)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmtp_hip.so")

# dtype codes (enum mtp_dtype)
F32, BF16, F16, FP8E4M3, U8, I8, I32, I64 = range(8)
# status codes (enum mtp_status)
OK = 0
ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_WORKSPACE, ERR_ALIGN, ERR_LAUNCH, ERR_ARG = range(-1, -8, -1)
NIBBLE_OFFSET8, NIBBLE_TWOS = 0, 1
# verify routes (mtp_verify_route)
VERIFY_ROUTE_STREAM, VERIFY_ROUTE_COLUMN_GROUP, VERIFY_ROUTE_GENERIC = 0, 1, 2

_TORCH_CODES = {
    torch.float32: F32,
    torch.bfloat16: BF16,
    torch.float16: F16,
    torch.float8_e4m3fn: FP8E4M3,
    torch.uint8: U8,
    torch.int8: I8,
    torch.int32: I32,
    torch.int64: I64,
}

# Every symbol include/mtp_hip.h declares, with its ctypes signature.
_vp, _i, _i64, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "mtp_abi_version": (_i, []),
    "mtp_status_string": (ctypes.c_char_p, [_i]),
    "mtp_last_hip_error": (ctypes.c_char_p, []),
    "mtp_fused_rmsnorm_linear": (
        _i, [_vp, _i, _i64, _i64, _vp, _i, _i64, _vp, _i, _vp, _i, _f, _f, _i, _vp, _vp, _sz, _vp]),
    "mtp_fused_rmsnorm_linear_fp8": (
        _i, [_vp, _i, _i64, _i64, _vp, _i, _vp, _i64, _vp, _i, _vp, _i, _f, _i, _vp, _vp, _sz, _vp]),
    "mtp_fused_int4_matmul": (
        _i, [_vp, _i, _i64, _i64, _vp, _vp, _i, _i64, _i64, _i, _vp, _i, _f, _i, _vp, _vp, _sz, _vp]),
    "mtp_rmsnorm_linear_workspace_bytes": (_sz, [_i, _i, _i64, _i64, _i64]),
    "mtp_fused_verify": (
        _i, [_vp, _i, _i64, _i64, _vp, _i, _i64, _vp, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "mtp_fused_multi_verify": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp, _i, _vp, _i64, _vp, _vp, _vp, _vp,
             _vp, _sz, _vp]),
    "mtp_fused_multi_verify_textbook": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp, _i, _vp, _i64, _vp, _vp, _vp, _vp,
             _vp, _sz, _vp]),
    "mtp_verify_route": (_i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp]),
    "mtp_verify_workspace_bytes": (_sz, [_i, _i64, _i64, _i64, _i64]),
    "mtp_fused_paged_attention": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _f, _vp, _vp, _sz, _vp]),
    "mtp_fused_tree_attention": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i, _f, _vp, _vp, _sz, _vp]),
    "mtp_tree_verify_attention": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _i, _f,
             _vp, _vp, _sz, _vp]),
    "mtp_attention_workspace_bytes": (_sz, [_i, _i64, _i64, _i64, _i64, _i64, _i64]),
    "mtp_quantize_fp8_e4m3": (_i, [_vp, _i, _i64, _vp, _vp, _vp, _sz, _vp]),
    "mtp_quantize_workspace_bytes": (_sz, [_i64]),
    "mtp_quantize_fp8_rows": (_i, [_vp, _i, _i64, _i64, _vp, _vp, _vp]),
    "mtp_dequantize_fp8": (_i, [_vp, _i64, _i64, _vp, _i, _vp, _vp]),
    "mtp_quantize_int4": (_i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _vp]),
    "mtp_dequantize_int4": (_i, [_vp, _vp, _i, _i64, _i64, _i64, _vp, _vp]),
    "mtp_fused_causal_attention": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _i64, _f, _vp, _vp, _sz, _vp]),
    "mtp_fused_causal_attention_fp8": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _f, _vp, _vp]),
    "mtp_fused_tree_attn_rmsnorm_linear": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i, _vp, _i, _i64, _vp, _i, _vp, _i,
             _vp, _f, _f, _vp, _vp, _sz, _vp]),
    "mtp_tree_attn_rmsnorm_linear_workspace_bytes": (_sz, [_i, _i64, _i64, _i64, _i64, _i, _i64]),
    "mtp_fused_rmsnorm": (_i, [_vp, _i, _i64, _i64, _vp, _i, _f, _vp, _vp]),
    "mtp_fused_add_rmsnorm": (_i, [_vp, _vp, _i, _i64, _i64, _vp, _i, _f, _vp, _vp]),
    "mtp_argmax": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _vp, _i, _i64, _i64, _vp, _vp, _sz, _vp]),
    "mtp_argmax_workspace_bytes": (_sz, [_i64, _i64]),
    "mtp_paged_kv_write": (
        _i, [_vp, _vp, _i, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i, _i64, _i64,
             _vp, _i64, _vp, _i, _i64, _vp]),
    "mtp_verify_commit": (
        _i, [_vp, _vp, _vp, _vp, _i, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp]),
    "mtp_batch_prefix_match": (_i, [_vp, _i64, _i64, _vp, _vp]),
    "mtp_workspace_init": (_i, [_vp, _sz, _vp]),
    "mtp_fused_multi_verify_noalloc": (
        _i, [_vp, _i, _i64, _i64, _i64, _vp, _i, _i64, _vp, _i, _vp, _i64, _vp, _vp, _vp, _vp,
             _vp]),
    "mtp_noalloc_scratch_bytes": (_sz, []),
    "mtp_noalloc_init": (_i, []),
    "mtp_set_tuning": (_i, [ctypes.c_char_p, _i64]),
    "mtp_get_tuning": (_i, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
}

_lib = None
_lock = threading.Lock()


class MtpHipError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the library (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise MtpHipError(
                    f"{LIB_PATH} is missing: build it with `python mtp-engine_amd/build.py`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def check(status: int, what: str) -> None:
    """Map a status code to the exception the reference's wrappers raise."""
    if status == OK:
        return
    lib = load()
    msg = lib.mtp_status_string(status).decode()
    if status == ERR_LAUNCH:
        msg += ": " + lib.mtp_last_hip_error().decode()
    if status == ERR_SHAPE:
        raise AssertionError(f"{what}: {msg}")
    if status == ERR_DTYPE:
        raise TypeError(f"{what}: {msg}")
    raise MtpHipError(f"{what}: {msg} (status {status})")


# Launch-planning overrides of the library (mtp_set_tuning): -1 = the plan's.
TUNING_KEYS = ("skl", "sk_splits", "ws_variant", "ws_splits", "skl_waves", "skl_splits",
               "attn_chunk_blocks", "int4_waves", "verify_wstream", "skp", "skp_splits",
               "skp_ta", "sf32", "skp_h8", "attn32", "sk_xraw",
               "skw", "skw_tw", "skp_tw", "skl_tw", "skv_r8", "skv_tw")


def set_tuning(**keys: int) -> None:
    lib = load()
    for k, v in keys.items():
        check(lib.mtp_set_tuning(k.encode(), int(v)), f"set_tuning({k})")


def get_tuning(name: str) -> int:
    v = ctypes.c_int64(0)
    check(load().mtp_get_tuning(name.encode(), ctypes.byref(v)), f"get_tuning({name})")
    return int(v.value)


class tuning:
    """Context manager: set tuning keys, restore the previous values on exit."""

    def __init__(self, **keys: int):
        self.keys = keys
        self.old = {}

    def __enter__(self):
        self.old = {k: get_tuning(k) for k in self.keys}
        set_tuning(**self.keys)
        return self

    def __exit__(self, *exc):
        set_tuning(**self.old)
        return False


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# ---------------------------------------------------------------------------
# Workspace: one buffer per (device, stream), grown on demand and zeroed by
# the library's own fill kernel (a kernel node, never a memset, if it is
# recorded). Kernels leave their counters at zero, so a buffer is reused as
# is. reserve_workspace() sizes it ahead of a graph capture, so the capture
# allocates nothing.
#
# A captured graph keeps the device address of every buffer it used, so no
# buffer is ever freed: one that a larger buffer replaces is retired, not
# dropped. A buffer first needed while the stream is being captured lives
# in the graph's memory pool and is zeroed only when its recorded fill
# kernel runs on replay; it serves that capture alone (kept alive here) and
# never becomes the stream's eager workspace.
_workspaces: dict = {}
_captured: dict = {}
_retired: list = []
_MIN_WORKSPACE = MTP_COUNTER_BYTES = 65536


def _new_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    nbytes = (nbytes + 255) // 256 * 256
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    check(load().mtp_workspace_init(ws.data_ptr(), nbytes, stream_handle(device)),
          "workspace init")
    return ws


def _grown(ws, nbytes: int) -> int:
    return max(nbytes, _MIN_WORKSPACE, 0 if ws is None else 2 * ws.numel())


def workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _workspaces.get(key)
    if ws is not None and ws.numel() >= nbytes:
        return ws
    if torch.cuda.is_current_stream_capturing():
        cap = _captured.get(key)
        if cap is None or cap.numel() < nbytes:
            cap = _new_workspace(device, _grown(cap if cap is not None else ws, nbytes))
            _captured[key] = cap
            _retired.append(cap)
        return cap
    _captured.pop(key, None)
    if ws is not None:
        _retired.append(ws)
    ws = _new_workspace(device, _grown(ws, nbytes))
    _workspaces[key] = ws
    return ws


def reserve_workspace(device: torch.device, nbytes: int, stream=None) -> torch.Tensor:
    """Make the workspace of (device, stream) at least nbytes now (default:
    the current stream), e.g. before capturing calls on that stream."""
    device = torch.device(device)
    st = stream if stream is not None else torch.cuda.current_stream(device)
    with torch.cuda.stream(st):
        return workspace(device, max(int(nbytes), _MIN_WORKSPACE))
