"""ctypes bindings for the two CPU checkers (test infrastructure only).

* ``oracle/liboracle.so``: this repository's restatement of the reference algorithm.
* ``oracle/_ref/libfastmario_ref.so``: the reference C++ FastVecEnv compiled from its own sources
  (``make -C oracle``); present wherever it was built, absent otherwise (tests then use the
  committed golden traces instead).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libfastmario_ref.so")
# the same reference sources built with their own -DFM_PROF counters (nes_core.hpp:23-26)
REF_PROF_SO = os.path.join(ROOT, "oracle", "_ref", "libfastmario_ref_prof.so")
CANON_BYTES = 4464
GRAY = 240 * 256
OBS = 84 * 84

_P = ctypes.c_void_p
_i64, _i32, _dbl = ctypes.c_int64, ctypes.c_int, ctypes.c_double
_libs: dict[str, ctypes.CDLL] = {}


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_P)


def have_ref() -> bool:
    return os.path.isfile(REF_SO)


def have_ref_prof() -> bool:
    return os.path.isfile(REF_PROF_SO)


def oracle() -> ctypes.CDLL:
    if "or" not in _libs:
        L = ctypes.CDLL(ORACLE_SO)
        L.or_raw_create.restype = _P
        L.or_raw_create.argtypes = [_P, _i64]
        L.or_raw_frame.argtypes = [_P, _i32, _i32]
        L.or_raw_ram.restype = L.or_raw_screen.restype = _P
        L.or_raw_ram.argtypes = L.or_raw_screen.argtypes = [_P]
        for f in ("or_raw_backup", "or_raw_restore", "or_raw_destroy", "or_reset", "or_destroy"):
            getattr(L, f).argtypes = [_P]
        for f in ("or_raw_bad_ops", "or_raw_instructions", "or_frames", "or_bad_ops", "or_instructions"):
            getattr(L, f).restype = _i64
            getattr(L, f).argtypes = [_P]
        L.or_raw_canon.argtypes = [_P, _P]
        L.or_create.restype = _P
        L.or_create.argtypes = [_P, _i64, _i32, _P, _P, _i32, _i32, _dbl, _i32, _i32, _i32, _P]
        L.or_set_buffers.argtypes = [_P] * 9
        L.or_step.argtypes = [_P, _P]
        for f in ("or_env_ram", "or_env_canon", "or_env_gray", "or_level_canon", "or_level_obs"):
            getattr(L, f).argtypes = [_P, _i32, _P]
        L.or_palette.argtypes = [_P]
        L.or_reemulations.argtypes = [_P, _P]
        L.or_pcg_run.argtypes = [_P, _P, _i32, _P, _P]
        L.or_resize.argtypes = [_P, _P]
        L.or_area_tab.restype = _i32
        L.or_area_tab.argtypes = [_i32, _i32, _P, _P, _P]
        _libs["or"] = L
    return _libs["or"]


def reference(prof: bool = False) -> ctypes.CDLL:
    key = "ref_prof" if prof else "ref"
    if key not in _libs:
        L = ctypes.CDLL(REF_PROF_SO if prof else REF_SO)
        L.fm_create.restype = _P
        L.fm_create.argtypes = [_P, _i64, _i32, _P, _P, _i32, _i32, _dbl, _i32, _i32, _i32, _P, _i32]
        L.fm_set_buffers.argtypes = [_P] * 9
        for f in ("fm_reset", "fm_step_wait", "fm_destroy"):
            getattr(L, f).argtypes = [_P]
        L.fm_step_async.argtypes = [_P, _P]
        L.fm_frames.restype = L.fm_bad_ops.restype = _i64
        L.fm_frames.argtypes = L.fm_bad_ops.argtypes = [_P]
        L.fm_env_ram.argtypes = [_P, _i32, _P]
        L.fm_palette.argtypes = [_P]
        L.fm_resize_ref.argtypes = [_P, _i32, _i32, _P, _i32, _i32]
        L.fm_resize_fast.argtypes = [_P, _P]
        L.fm_raw_create.restype = _P
        L.fm_raw_create.argtypes = [_P, _i64]
        L.fm_raw_frame.argtypes = [_P, _i32, _i32]
        L.fm_raw_ram.restype = L.fm_raw_screen.restype = _P
        L.fm_raw_ram.argtypes = L.fm_raw_screen.argtypes = [_P]
        L.fm_raw_backup.argtypes = L.fm_raw_restore.argtypes = L.fm_raw_destroy.argtypes = [_P]
        L.fm_raw_bad_ops.restype = _i64
        L.fm_raw_bad_ops.argtypes = [_P]
        _libs[key] = L
    return _libs[key]


def prof_counter(name: str = "prof_cpu_instr") -> ctypes.c_uint64:
    """A uint64 FM_PROF counter of the profiling reference build (a C++ inline variable fm::<name>),
    readable and writable in place."""
    mangled = f"_ZN2fm{len(name)}{name}E"
    return ctypes.c_uint64.in_dll(reference(prof=True), mangled)


# ---------------------------------------------------------------- raw consoles
class _RawBase:
    def __init__(self, rom: bytes):
        self._rom = np.frombuffer(rom, np.uint8).copy()
        self.h = self._create(_ptr(self._rom), len(self._rom))
        if not self.h:
            raise ValueError("unsupported ROM")
        u8p = ctypes.POINTER(ctypes.c_uint8)
        self.ram = np.ctypeslib.as_array(ctypes.cast(self._ram(self.h), u8p), (0x800,))
        self.screen = np.ctypeslib.as_array(ctypes.cast(self._screen(self.h), u8p), (240, 256))


class OracleRaw(_RawBase):
    def __init__(self, rom):
        L = self.L = oracle()
        self._create, self._ram, self._screen = L.or_raw_create, L.or_raw_ram, L.or_raw_screen
        super().__init__(rom)

    def frame(self, buttons, render):
        self.L.or_raw_frame(self.h, int(buttons), int(bool(render)))

    def backup(self):
        self.L.or_raw_backup(self.h)

    def restore(self):
        self.L.or_raw_restore(self.h)

    def bad_ops(self):
        return int(self.L.or_raw_bad_ops(self.h))

    def instructions(self):
        return int(self.L.or_raw_instructions(self.h))

    def canon(self):
        out = np.zeros(CANON_BYTES, np.uint8)
        self.L.or_raw_canon(self.h, _ptr(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            self.L.or_raw_destroy(self.h)
            self.h = None


class RefRaw(_RawBase):
    def __init__(self, rom, prof=False):
        L = self.L = reference(prof)
        self._create, self._ram, self._screen = L.fm_raw_create, L.fm_raw_ram, L.fm_raw_screen
        super().__init__(rom)

    def frame(self, buttons, render):
        self.L.fm_raw_frame(self.h, int(buttons), int(bool(render)))

    def backup(self):
        self.L.fm_raw_backup(self.h)

    def restore(self):
        self.L.fm_raw_restore(self.h)

    def bad_ops(self):
        return int(self.L.fm_raw_bad_ops(self.h))

    def __del__(self):
        if getattr(self, "h", None):
            self.L.fm_raw_destroy(self.h)
            self.h = None


# ---------------------------------------------------------------- vector envs
def rng_state(seed: int) -> list[int]:
    """numpy PCG64 state of default_rng(seed) as (state_hi, state_lo, inc_hi, inc_lo, has_uint32, uinteger)."""
    st = np.random.default_rng(seed).bit_generator.state
    s, inc = st["state"]["state"], st["state"]["inc"]
    m = (1 << 64) - 1
    return [s >> 64, s & m, inc >> 64, inc & m, st["has_uint32"], st["uinteger"]]


def gray_lut() -> np.ndarray:
    """palette value -> gray: cv2 RGB2GRAY's 14-bit fixed point on the nes-py palette (env.py:42-47)."""
    p = np.zeros(64, np.uint32)
    oracle().or_palette(_ptr(p))
    rgb = np.stack([(p >> 16) & 255, (p >> 8) & 255, p & 255], -1).astype(np.int64)
    g = (rgb[:, 0] * 4899 + rgb[:, 1] * 9617 + rgb[:, 2] * 1868 + (1 << 13)) >> 14
    return np.ascontiguousarray(g[np.arange(256) & 63], np.uint8)


class _VecBase:
    """FastVecEnv-shaped driver over a C vector env (numpy outputs, no infos list)."""

    def __init__(self, rom, levels, n, seed=0, frame_stack=4, sticky=0.0, noop_max=0, max_steps=2000,
                 maxpool=False, skip=4, env_offset=0):
        self.n, self.k = n, frame_stack
        self._rom = np.frombuffer(rom, np.uint8).copy()
        self._lv = np.array(levels, np.int32).reshape(-1)
        assert self._lv.size == 3 * n
        self._lut = gray_lut()
        self._rng = np.array([rng_state(seed * 1000 + env_offset + i) for i in range(n)], np.uint64).reshape(-1)
        self.args = (skip, max_steps, float(sticky), int(noop_max), int(bool(maxpool)), frame_stack)
        self.obs = np.zeros((n, frame_stack, 84, 84), np.uint8)
        self.fin = np.zeros_like(self.obs)
        self.rew = np.zeros(n, np.float32)
        self.term = np.zeros(n, np.uint8)
        self.trunc = np.zeros(n, np.uint8)
        self.info = np.zeros((n, 10), np.int64)
        self.ep_ret = np.zeros(n, np.float64)
        self.ep_len = np.zeros(n, np.int64)

    def _bufs(self):
        return [_ptr(x) for x in (self.obs, self.fin, self.rew, self.term, self.trunc, self.info, self.ep_ret,
                                  self.ep_len)]


class OracleVec(_VecBase):
    def __init__(self, rom, levels, n, **kw):
        super().__init__(rom, levels, n, **kw)
        L = self.L = oracle()
        self.h = L.or_create(_ptr(self._rom), len(self._rom), n, _ptr(self._lv), _ptr(self._lut), *self.args,
                             _ptr(self._rng))
        if not self.h:
            raise RuntimeError("or_create failed")
        L.or_set_buffers(self.h, *self._bufs())

    def reset(self):
        self.L.or_reset(self.h)
        return self.obs

    def step(self, actions):
        a = np.ascontiguousarray(actions, np.int64)
        self.L.or_step(self.h, _ptr(a))
        return self.obs, self.rew, self.term.astype(bool), self.trunc.astype(bool), self.info

    def ram(self, i):
        out = np.zeros(0x800, np.uint8)
        self.L.or_env_ram(self.h, int(i), _ptr(out))
        return out

    def canon(self, i):
        out = np.zeros(CANON_BYTES, np.uint8)
        self.L.or_env_canon(self.h, int(i), _ptr(out))
        return out

    def level_canon(self, lv):
        out = np.zeros(CANON_BYTES, np.uint8)
        self.L.or_level_canon(self.h, int(lv), _ptr(out))
        return out

    def level_obs(self, lv):
        out = np.zeros(OBS, np.uint8)
        self.L.or_level_obs(self.h, int(lv), _ptr(out))
        return out.reshape(84, 84)

    def frames(self):
        return int(self.L.or_frames(self.h))

    def bad_ops(self):
        return int(self.L.or_bad_ops(self.h))

    def instructions(self):
        return int(self.L.or_instructions(self.h))

    def reemulations(self):
        out = np.zeros(3, np.int64)
        self.L.or_reemulations(self.h, _ptr(out))
        return dict(zip(("one", "pair", "k2"), out.tolist()))

    def close(self):
        if getattr(self, "h", None):
            self.L.or_destroy(self.h)
            self.h = None

    __del__ = close


class RefVec(_VecBase):
    def __init__(self, rom, levels, n, n_threads=0, prof=False, **kw):
        super().__init__(rom, levels, n, **kw)
        L = self.L = reference(prof)
        self.h = L.fm_create(_ptr(self._rom), len(self._rom), n, _ptr(self._lv), _ptr(self._lut), *self.args,
                             _ptr(self._rng), int(n_threads))
        if not self.h:
            raise RuntimeError("fm_create failed")
        L.fm_set_buffers(self.h, *self._bufs())

    def reset(self):
        self.L.fm_reset(self.h)
        return self.obs

    def step(self, actions):
        a = np.ascontiguousarray(actions, np.int64)
        self.L.fm_step_async(self.h, _ptr(a))
        self.L.fm_step_wait(self.h)
        return self.obs, self.rew, self.term.astype(bool), self.trunc.astype(bool), self.info

    def ram(self, i):
        out = np.zeros(0x800, np.uint8)
        self.L.fm_env_ram(self.h, int(i), _ptr(out))
        return out

    def frames(self):
        return int(self.L.fm_frames(self.h))

    def bad_ops(self):
        return int(self.L.fm_bad_ops(self.h))

    def close(self):
        if getattr(self, "h", None):
            self.L.fm_destroy(self.h)
            self.h = None

    __del__ = close
