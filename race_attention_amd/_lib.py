"""ctypes binding of librace_attention.so (include/race_attention.h).

The library is the only compute path: if it is missing or a tensor is not on a
ROCm device, the calls raise -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
# RACE_ATTENTION_LIB selects another build of the library (e.g. the host-side
# sanitizer build of `python race_attention_amd/build.py --sanitize`)
LIB_PATH = os.environ.get("RACE_ATTENTION_LIB") or os.path.join(HERE, "librace_attention.so")

RACE_OK = 0
RACE_DTYPE_F32 = 0
RACE_PHASE_REDUCE, RACE_PHASE_SCAN, RACE_PHASE_OUT = 1, 2, 4
RACE_DTYPE_BF16 = 1

I64x4 = ctypes.c_int64 * 4


class RaceDesc(ctypes.Structure):
    """Mirror of race_desc (include/race_attention.h)."""
    _fields_ = [
        ("M", ctypes.c_int64), ("B", ctypes.c_int64), ("T", ctypes.c_int64),
        ("H", ctypes.c_int64), ("D", ctypes.c_int64),
        ("L", ctypes.c_int32), ("K", ctypes.c_int32),
        ("causal", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("eps", ctypes.c_float), ("inv_temp", ctypes.c_float),
        ("planes_m_stride", ctypes.c_int64),
        ("q_stride", I64x4), ("k_stride", I64x4), ("v_stride", I64x4),
        ("o_stride", I64x4), ("do_stride", I64x4), ("g_stride", I64x4),
        ("seg_tiles", ctypes.c_int32), ("phases", ctypes.c_int32),
        ("inv_temp_ptr", ctypes.c_void_p),
    ]


# every symbol include/race_attention.h declares
EXPORTS = (
    "race_state_bytes", "race_fwd_workspace_bytes", "race_bwd_workspace_bytes",
    "race_fwd", "race_bwd",
    "race_fwd_ex_workspace_bytes", "race_fwd_ex", "race_bwd_ex",
    "race_probs_bwd_workspace_bytes", "race_probs", "race_probs_bwd",
    "race_fwd_global_workspace_bytes", "race_bwd_global_workspace_bytes", "race_fwd_global", "race_bwd_global",
    "race_prefix_mean_workspace_bytes", "race_prefix_mean_fwd", "race_prefix_mean_bwd",
    "race_fwd_noalloc",
    "race_last_error", "race_abi_version",
)

_lock = threading.Lock()
_lib = None


class RaceError(RuntimeError):
    pass


def load():
    """Load librace_attention.so (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RaceError(f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                            "or `python race_attention_amd/build.py`")
        lib = ctypes.CDLL(LIB_PATH)
        vp, sz, i64, dbl = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_double
        dp = ctypes.POINTER(RaceDesc)
        for name in ("race_state_bytes", "race_fwd_workspace_bytes", "race_bwd_workspace_bytes", "race_fwd_ex_workspace_bytes",
                     "race_probs_bwd_workspace_bytes",
                     "race_fwd_global_workspace_bytes", "race_bwd_global_workspace_bytes"):
            getattr(lib, name).argtypes = [dp]
            getattr(lib, name).restype = sz
        lib.race_fwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.race_fwd.restype = ctypes.c_int
        lib.race_bwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.race_bwd.restype = ctypes.c_int
        lib.race_probs.argtypes = [dp, vp, vp, vp, vp]
        lib.race_probs.restype = ctypes.c_int
        lib.race_probs_bwd.argtypes = [dp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.race_probs_bwd.restype = ctypes.c_int
        lib.race_fwd_ex.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.race_fwd_ex.restype = ctypes.c_int
        lib.race_bwd_ex.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.race_bwd_ex.restype = ctypes.c_int
        lib.race_fwd_global.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.race_fwd_global.restype = ctypes.c_int
        lib.race_bwd_global.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.race_bwd_global.restype = ctypes.c_int
        lib.race_prefix_mean_workspace_bytes.argtypes = [i64, i64, i64]
        lib.race_prefix_mean_workspace_bytes.restype = sz
        lib.race_prefix_mean_fwd.argtypes = [vp, vp, vp, i64, i64, i64, dbl, vp, sz, vp]
        lib.race_prefix_mean_fwd.restype = ctypes.c_int
        lib.race_prefix_mean_bwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, dbl, vp, sz, vp]
        lib.race_prefix_mean_bwd.restype = ctypes.c_int
        lib.race_fwd_noalloc.argtypes = [dp, vp, vp, vp, vp, vp, vp]
        lib.race_fwd_noalloc.restype = ctypes.c_int
        lib.race_last_error.argtypes = []
        lib.race_last_error.restype = ctypes.c_char_p
        lib.race_abi_version.argtypes = []
        lib.race_abi_version.restype = ctypes.c_int
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != RACE_OK:
        msg = load().race_last_error().decode(errors="replace")
        raise RaceError(f"{what} failed ({rc}): {msg}")


def last_error() -> str:
    return load().race_last_error().decode(errors="replace")
