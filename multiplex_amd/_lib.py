"""ctypes binding of ``libgdn.so`` (the C ABI declared in ``include/gdn.h``).

Loading fails loudly: there is no CPU or eager fallback behind this module.
"""

from __future__ import annotations

import ctypes
import os
import threading
from ctypes import POINTER, Structure, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libgdn.so"

GDN_ABI_VERSION = 4

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

GATES_RAW = 0
GATES_PRE = 1

OK = 0
ERR_LAUNCH = -5
ERR_INVALID = -22
ERR_UNSUPPORTED = -95

# Every symbol include/gdn.h declares.
EXPORTS = (
    "gdn_abi_version",
    "gdn_last_error",
    "gdn_gated_delta_update",
    "gdn_gated_delta_kernel",
    "gdn_recurrent",
    "gdn_chunk_workspace_bytes",
    "gdn_chunk_fwd",
    "gdn_chunk_prep",
    "gdn_chunk_scan",
    "gdn_chunk_fwd_noalloc",
    "gdn_chunk_conv_workspace_bytes",
    "gdn_chunk_fwd_conv",
    "gdn_conv_prologue",
    "gdn_conv_state_commit",
    "gdn_gated_rmsnorm",
    "gdn_attn_qk",
    "gdn_attn_workspace_bytes",
    "gdn_attn_fwd",
    "gdn_rms_norm",
    "gdn_silu_mul",
    "gdn_linear_decode_workspace_bytes",
    "gdn_linear_decode",
)


class RecurrentArgs(Structure):
    """Mirror of ``gdn_recurrent_args`` (field order and types must match)."""

    _fields_ = [
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("qkv_dtype", c_int32),
        ("gate_mode", c_int32),
        ("gx", c_void_p),
        ("gy", c_void_p),
        ("gate_dtype", c_int32),
        ("param_dtype", c_int32),
        ("A_log", c_void_p),
        ("dt_bias", c_void_p),
        ("state_in", c_void_p),
        ("state_out", c_void_p),
        ("snapshots", c_void_p),
        ("y", c_void_p),
        ("mask", c_void_p),
        ("cu_seqlens", c_void_p),
        ("commit_len", c_void_p),
        ("state_index", c_void_p),
        ("B", c_int64),
        ("T", c_int64),
        ("Hk", c_int64),
        ("Hv", c_int64),
        ("Dk", c_int64),
        ("Dv", c_int64),
        ("n_slots", c_int64),
        ("gate_stride", c_int64),
        ("stream", c_void_p),
        ("y_from", c_int64),
    ]


class GDNError(RuntimeError):
    """A libgdn call returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


_lock = threading.Lock()
_lib = None

_P = c_void_p
_I64 = c_int64

_SIGNATURES = {
    "gdn_abi_version": (c_int, []),
    "gdn_last_error": (c_char_p, []),
    "gdn_gated_delta_update": (
        c_int,
        [_P, _P, _P, c_int, _P, _P, c_int, _P, _P, c_int, _P, _P, _P, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _P],
    ),
    "gdn_gated_delta_kernel": (
        c_int,
        [_P, _P, _P, c_int, _P, _P, c_int, _P, _P, _P, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _P],
    ),
    "gdn_recurrent": (c_int, [POINTER(RecurrentArgs)]),
    "gdn_chunk_workspace_bytes": (c_size_t, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "gdn_chunk_fwd": (
        c_int,
        [_P, _P, _P, c_int, c_int, _P, _P, c_int, _I64, _P, _P, c_int, _P, _P, _P, _P, _P, _I64, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, c_size_t, _P],
    ),
    "gdn_chunk_prep": (
        c_int,
        [_P, _P, _P, c_int, c_int, _P, _P, c_int, _I64, _P, _P, c_int, _P, _P, _P, _P, _P, _I64, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, c_size_t, _P],
    ),
    "gdn_chunk_scan": (
        c_int,
        [_P, _P, _P, c_int, c_int, _P, _P, c_int, _I64, _P, _P, c_int, _P, _P, _P, _P, _P, _I64, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, c_size_t, _P],
    ),
    "gdn_chunk_fwd_noalloc": (
        c_int,
        [_P, _P, _P, c_int, c_int, _P, _P, c_int, _I64, _P, _P, c_int, _P, _P, _P, _P, _P, _I64, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    ),
    "gdn_chunk_conv_workspace_bytes": (c_size_t, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "gdn_chunk_fwd_conv": (
        c_int,
        [_P, _I64, _P, c_int, _P, _P, c_float, c_int, _P, _P, c_int, _I64, _P, _P, c_int, _P, _P, _P, _P, _I64, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, c_size_t, _P],
    ),
    "gdn_conv_prologue": (
        c_int,
        [_P, c_int, _I64, _P, _P, c_int, _P, _P, _P, _P, _P, _P,
         _I64, _I64, _I64, _I64, _I64, _I64, _I64, c_float, _P],
    ),
    "gdn_conv_state_commit": (
        c_int,
        [_P, _P, c_int, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    ),
    "gdn_gated_rmsnorm": (
        c_int,
        [_P, _P, c_int, _I64, _I64, _P, c_int, _P, _I64, _I64, c_float, _P],
    ),
    "gdn_attn_qk": (
        c_int,
        [_P, _I64, _P, _P, _I64, _P, _P, c_int, c_float, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
         c_float, _P],
    ),
    "gdn_attn_workspace_bytes": (c_size_t, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "gdn_attn_fwd": (
        c_int,
        [_P, _P, _I64, _P, _P, _P, _P, c_float, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, c_size_t, _P],
    ),
    "gdn_rms_norm": (c_int, [_P, _P, _P, _P, c_int, _P, _I64, _I64, _I64, c_float, _P]),
    "gdn_silu_mul": (c_int, [_P, _P, _I64, _I64, _P]),
    "gdn_linear_decode_workspace_bytes": (c_size_t, [_I64, _I64, _I64]),
    "gdn_linear_decode": (
        c_int,
        [_P, _I64, _P, _I64, _P, c_int, c_float, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, c_size_t, _P],
    ),
}


def lib_path() -> Path:
    return Path(os.environ.get("MULTIPLEX_AMD_LIB", str(LIB_PATH)))


def load() -> ctypes.CDLL:
    """Loads libgdn.so once; raises if it is missing or its ABI differs."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not path.exists():
            raise RuntimeError(
                f"{path} is not built: run `python -m multiplex_amd.build` "
                "(the GDN path has no fallback without its HIP library)"
            )
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.gdn_abi_version()
        if ver != GDN_ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {ver}, expected {GDN_ABI_VERSION}")
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().gdn_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(fn: str, status: int) -> None:
    """Raises ValueError for argument errors and GDNError for the rest."""
    if status == OK:
        return
    msg = last_error()
    if status in (ERR_INVALID, ERR_UNSUPPORTED):
        raise ValueError(f"{fn}: {msg} (status {status})")
    raise GDNError(fn, status, msg)


def call(name: str, *args) -> None:
    lib = load()
    check(name, getattr(lib, name)(*args))
