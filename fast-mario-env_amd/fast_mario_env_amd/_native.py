"""ctypes bindings for libmario_hip.so (the gfx950 kernels + C ABI declared in include/mario_hip.h).

Mirrors the reference's src/fast_mario_env/_native.py:30-60 (ctypes over a C ABI), but the library
is the HIP one and every buffer argument is a device pointer. There is no CPU fallback: if the
library is missing or cannot be loaded, import of the env classes fails with an error that says how
to build it.
"""
from __future__ import annotations

import ctypes
import os

LIB_ENV_VAR = "MARIO_HIP_LIB"
HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libmario_hip.so"

_P = ctypes.c_void_p
_i64, _i32, _dbl = ctypes.c_int64, ctypes.c_int, ctypes.c_double
_lib = None


def lib_path() -> str:
    return os.environ.get(LIB_ENV_VAR) or os.path.join(HERE, LIB_NAME)


class NativeLibraryError(ImportError):
    pass


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.isfile(path):
        raise NativeLibraryError(
            f"fast_mario_env_amd: {path} is missing. Build it with `python -c \"import __graft_entry__ as g; "
            f"g.build()\"` from the repository root (needs hipcc with gfx950 support).")
    L = ctypes.CDLL(path)
    L.mh_last_error.restype = ctypes.c_char_p
    L.mh_create.restype = _P
    L.mh_create.argtypes = [_P, _i64, _i32, _P, _P, _i32, _i32, _dbl, _i32, _i32, _i32, _P, _i32]
    L.mh_create_roms.restype = _P
    L.mh_create_roms.argtypes = [_P, _P, _i32, _P, _i32, _P, _P, _i32, _i32, _dbl, _i32, _i32, _i32, _P, _i32]
    L.mh_set_buffers.argtypes = [_P] * 9
    for f in ("mh_reset", "mh_step_wait"):
        getattr(L, f).argtypes = [_P, _P]
    L.mh_step_async.argtypes = [_P, _P, _P]
    L.mh_destroy.argtypes = [_P]
    for f in ("mh_frames", "mh_bad_ops", "mh_instructions", "mh_ff_instructions", "mh_env_bytes", "mh_hack_redraws"):
        getattr(L, f).restype = _i64
        getattr(L, f).argtypes = [_P]
    for f in ("mh_env_ram", "mh_env_canon", "mh_level_canon", "mh_level_obs"):
        getattr(L, f).argtypes = [_P, _P, _P]
    L.mh_num_levels.argtypes = [_P]
    L.mh_state_bytes.restype = _i64
    L.mh_raw_create.restype = _P
    L.mh_raw_create.argtypes = [_P, _i64, _i32, _i32]
    L.mh_raw_frame.argtypes = [_P, _P, _i32, _P]
    for f in ("mh_raw_ram", "mh_raw_screen", "mh_raw_canon"):
        getattr(L, f).argtypes = [_P, _P, _P]
    L.mh_raw_screen_rgb.argtypes = [_P, _P, _P, _P]
    for f in ("mh_raw_backup", "mh_raw_restore"):
        getattr(L, f).argtypes = [_P, _P]
    for f in ("mh_raw_bad_ops", "mh_raw_instructions", "mh_raw_ff_instructions"):
        getattr(L, f).restype = _i64
        getattr(L, f).argtypes = [_P]
    L.mh_raw_destroy.argtypes = [_P]
    L.mh_resize.argtypes = [_P, _P, _i32, _P]
    L.mh_resize_noalloc.argtypes = [_P, _P, _i32, _P]
    L.mh_policy_input.argtypes = [_P, _P, _i64, _i32, _P]
    L.mh_policy_conv1.argtypes = [_P, _P, _P, _P, _i64, _P]
    L.mh_policy_conv.argtypes = [_P, _P, _P, _P, _i64, _i32, _P]
    L.mh_reemulations.argtypes = [_P, _P]
    L.mh_replay_add.argtypes = [_P] * 7 + [_i32] * 4 + [_P] * 7
    L.mh_replay_gather.argtypes = [_P] * 5 + [_i32] * 4 + [_P, _P, _i32, _i32] + [_P] * 10
    L.mh_timing.argtypes = [_P, _i32]
    L.mh_timing_read.argtypes = [_P, _P, _P]
    _lib = L
    return L


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {lib().mh_last_error().decode(errors='replace')}")


def last_error() -> str:
    return lib().mh_last_error().decode(errors="replace")
