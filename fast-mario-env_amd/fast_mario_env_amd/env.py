"""Batched Super Mario Bros envs on one MI355X, behind the reference's Python API.

    from fast_mario_env_amd import HipVecEnv            # CudaVecEnv-compatible (torch tensors on the GPU)
    env = HipVecEnv("1-1", n_envs=32768, seed=0, sticky=0.25, noop_max=30, maxpool=True)
    obs = env.reset()                                    # (N, 4, 84, 84) uint8, internal buffer
    obs, rew, term, trunc, info = env.step(actions)      # actions: (N,) int64 on the GPU

    from fast_mario_env_amd import FastVecEnv           # FastVecEnv-compatible (numpy in, numpy out)

Semantics are those of the reference's FastVecEnv (csrc/fastmario.cpp, tests/reference_env.py):
SIMPLE_MOVEMENT, frame-level sticky actions from one numpy PCG64 stream per env (seed*1000 +
env_offset + i), frame skip with optional 2-frame gray max-pool, life loss and flag end the episode,
random no-op starts, cv2 RGB2GRAY + INTER_AREA 84x84, time limit, frame stack, auto-reset with
final_obs. Every step runs as gfx950 kernels (libmario_hip.so) on torch's current stream.
"""
from __future__ import annotations

import csv
import json
import os
import time

import numpy as np

from . import _native
from ._native import check, lib
from .rom import check_rom, decode_level, load_rom

OBS_HW = 84
N_ACTIONS = 7
SIMPLE_MOVEMENT = [["NOOP"], ["right"], ["right", "A"], ["right", "B"], ["right", "A", "B"], ["A"], ["left"]]
INFO_FIELDS = ("x_pos", "flag_get", "life", "score", "time", "world", "stage", "coins", "y_pos", "status")
INFO_KEYS = ("x_pos", "flag_get", "life", "score", "time", "world", "stage")
CANON_BYTES = 4464

# nes-py master palette, 0xRRGGBB (the data table of the reference's fastmario.cpp:26-34)
PALETTE = np.array([
    0x7C7C7C, 0x0000FC, 0x0000BC, 0x4428BC, 0x940084, 0xA80020, 0xA81000, 0x881400,
    0x503000, 0x007800, 0x006800, 0x005800, 0x004058, 0x000000, 0x000000, 0x000000,
    0xBCBCBC, 0x0078F8, 0x0058F8, 0x6844FC, 0xD800CC, 0xE40058, 0xF83800, 0xE45C10,
    0xAC7C00, 0x00B800, 0x00A800, 0x00A844, 0x008888, 0x000000, 0x000000, 0x000000,
    0xF8F8F8, 0x3CBCFC, 0x6888FC, 0x9878F8, 0xF878F8, 0xF85898, 0xF87858, 0xFCA044,
    0xF8B800, 0xB8F818, 0x58D854, 0x58F898, 0x00E8D8, 0x787878, 0x000000, 0x000000,
    0xFCFCFC, 0xA4E4FC, 0xB8B8F8, 0xD8B8F8, 0xF8B8F8, 0xF8A4C0, 0xF0D0B0, 0xFCE0A8,
    0xF8D878, 0xD8F878, 0xB8F8B8, 0xB8F8D8, 0x00FCFC, 0xF8D8F8, 0x000000, 0x000000], np.uint32)


def palette_rgb() -> np.ndarray:
    """nes-py master palette as (64, 3) uint8 RGB."""
    p = PALETTE
    return np.stack([(p >> 16) & 255, (p >> 8) & 255, p & 255], -1).astype(np.uint8)


def gray_lut() -> np.ndarray:
    """palette value (0-255, taken & 63) -> gray, as cv2.cvtColor(RGB2GRAY): 14-bit fixed-point BT.601
    weights with round-half-up (env.py:42-47 of the reference)."""
    rgb = palette_rgb().astype(np.int64)
    g = (rgb[:, 0] * 4899 + rgb[:, 1] * 9617 + rgb[:, 2] * 1868 + (1 << 13)) >> 14
    return np.ascontiguousarray(g[np.arange(256) & 63], np.uint8)


def rng_state(seed: int) -> list[int]:
    """numpy PCG64 state of np.random.default_rng(seed) as the 6 words the library takes
    (state_hi, state_lo, inc_hi, inc_lo, has_uint32, uinteger); env.py:50-55 of the reference."""
    st = np.random.default_rng(seed).bit_generator.state
    s, inc = st["state"]["state"], st["state"]["inc"]
    m = (1 << 64) - 1
    return [s >> 64, s & m, inc >> 64, inc & m, st["has_uint32"], st["uinteger"]]


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("fast_mario_env_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch


def _ptr(t) -> int:
    return int(t.data_ptr())


def _stream(torch, dev):
    return torch.cuda.current_stream(dev).cuda_stream


class MonitorCSV:
    """Episode log in the monitor.csv format that Stable-Baselines3's VecMonitor / load_results read: a
    ``#``-prefixed JSON line with the start time, a header, then one row per finished episode with the return,
    length, wall time since the start and the final x_pos / flag_get (the columns of the reference's
    env.py:93-110).

    `path` may name the file itself (ending in ``.monitor.csv``), an existing directory (the file is then
    ``monitor.monitor.csv`` inside it), or a prefix to which ``.monitor.csv`` is appended."""

    COLUMNS = ("r", "l", "t", "x_pos", "flag_get")
    SUFFIX = ".monitor.csv"

    @classmethod
    def resolve(cls, path) -> str:
        path = os.fspath(path)
        if path.endswith(cls.SUFFIX):
            return path
        if os.path.isdir(path):
            return os.path.join(path, "monitor" + cls.SUFFIX)
        return path + cls.SUFFIX

    def __init__(self, path):
        self.path = self.resolve(path)
        parent = os.path.dirname(os.path.abspath(self.path))
        os.makedirs(parent, exist_ok=True)
        self._fh = open(self.path, "w", newline="")
        meta = {"t_start": time.time(), "env_id": "None"}
        self._fh.write("#" + json.dumps(meta) + "\n")
        self._rows = csv.writer(self._fh, lineterminator="\n")
        self._rows.writerow(self.COLUMNS)
        self._fh.flush()

    def write(self, episode: dict):
        """Append one finished episode (a dict with the COLUMNS keys) and flush it to disk."""
        self._rows.writerow([episode[c] for c in self.COLUMNS])
        self._fh.flush()

    def close(self):
        if not self._fh.closed:
            self._fh.close()


class HipVecEnv:
    """N Super Mario Bros envs stepped on one AMD GPU, one lane per env (drop-in for CudaVecEnv,
    src/fast_mario_env/cuda/vec_env.py:238-393).

    Args mirror CudaVecEnv: level ("w-s" or a list of N levels), n_envs, seed, sticky, noop_max,
    max_steps, skip, frame_stack, device, rom_path, rom_mode, env_offset (env i uses the PCG64 stream
    seed*1000 + env_offset + i). Beyond CudaVecEnv: maxpool, any frame_stack in 1..16, every rom_mode,
    and a rom_mode per env (a list of N modes; the variants share PRG, so one workgroup holds them all).
    `rom` gives ROM bytes directly: bytes for every env, or a dict mode -> bytes. `block`, `extra_opts`,
    `kernel` and `render_kernel` select CUDA kernel variants in the reference; they are accepted for
    compatibility and have no effect here.

    reset() -> obs; step(actions) -> (obs, rew f32, term bool, trunc bool, info). info maps
    INFO_FIELDS to int32 (N,) views of info_t, plus ep_ret f64 / ep_len i32 / final_obs, valid where
    term | trunc. Every returned tensor is an internal buffer overwritten by the next call.
    """

    def __init__(self, level="1-1", n_envs=1024, seed=0, sticky=0.0, noop_max=0, max_steps=2000, skip=4,
                 frame_stack=4, device="cuda", block=64, rom_path=None, rom_mode="vanilla", extra_opts=(),
                 kernel="v2", env_offset=0, render_kernel="k_render2", maxpool=False, rom=None):
        # arguments first (ValueError), then the device (RuntimeError without a ROCm GPU)
        if not 1 <= skip <= 16:
            raise ValueError("skip must be in 1..16")
        if not 1 <= frame_stack <= 16:
            raise ValueError("frame_stack must be in 1..16")
        if not 0.0 <= float(sticky) <= 1.0:
            raise ValueError("sticky must be in [0, 1]")
        self.n = n = int(n_envs)
        self.num_envs = n
        self.k = frame_stack
        levels = [level] * n if isinstance(level, (str, tuple)) else list(level)
        if len(levels) != n:
            raise ValueError(f"got {len(levels)} levels for {n} envs")
        self.levels = levels
        lv = np.array([decode_level(x) for x in levels], np.int32).reshape(-1)
        modes = [rom_mode] * n if isinstance(rom_mode, str) else list(rom_mode)
        if len(modes) != n:
            raise ValueError(f"got {len(modes)} rom modes for {n} envs")
        distinct = list(dict.fromkeys(modes))           # ROM index = order of first appearance
        if len(distinct) > 4:
            raise ValueError(f"at most 4 rom modes per instance, got {len(distinct)}")
        torch = self._torch = _torch()
        self.dev = torch.device(device)
        if self.dev.index is None:
            self.dev = torch.device("cuda", torch.cuda.current_device())
        roms = []
        for m in distinct:
            if isinstance(rom, dict):
                b = bytes(rom[m])
            elif rom is not None:
                b = bytes(rom)
            else:
                b = load_rom(rom_path, m)
            check_rom(b)
            roms.append(b)
        self.rom_modes = modes
        self._rom = np.frombuffer(b"".join(roms), np.uint8).copy()
        self._rom_lens = np.array([len(b) for b in roms], np.int64)
        self._env_rom = np.array([distinct.index(m) for m in modes], np.int32)
        self._lut = gray_lut()
        rng = np.array([rng_state(seed * 1000 + env_offset + i) for i in range(n)], np.uint64).reshape(-1)
        L = lib()
        with torch.cuda.device(self.dev):
            self.h = L.mh_create_roms(self._rom.ctypes.data, self._rom_lens.ctypes.data, len(roms),
                                      self._env_rom.ctypes.data, n, lv.ctypes.data, self._lut.ctypes.data,
                                      skip, max_steps, float(sticky), int(noop_max), int(bool(maxpool)), frame_stack,
                                      rng.ctypes.data, self.dev.index)
        if not self.h:
            raise RuntimeError(f"mh_create_roms failed: {_native.last_error()}")
        z = lambda *s, dt: torch.zeros(*s, dtype=dt, device=self.dev)  # noqa: E731
        self.actions = z(n, dt=torch.int64)
        self.obs = z(n, frame_stack, OBS_HW, OBS_HW, dt=torch.uint8)
        self.final_obs = z(n, frame_stack, OBS_HW, OBS_HW, dt=torch.uint8)
        self.rew = z(n, dt=torch.float32)
        self.term = z(n, dt=torch.bool)
        self.trunc = z(n, dt=torch.bool)
        self.info_t = z(n, len(INFO_FIELDS), dt=torch.int32)
        self.ep_ret = z(n, dt=torch.float64)
        self.ep_len = z(n, dt=torch.int32)
        check(L.mh_set_buffers(self.h, _ptr(self.obs), _ptr(self.final_obs), _ptr(self.rew), _ptr(self.term),
                               _ptr(self.trunc), _ptr(self.info_t), _ptr(self.ep_ret), _ptr(self.ep_len)),
              "mh_set_buffers")
        self.info = {k: self.info_t[:, i] for i, k in enumerate(INFO_FIELDS)}
        self.info["ep_ret"] = self.ep_ret
        self.info["ep_len"] = self.ep_len
        self.info["final_obs"] = self.final_obs

    # ---------------------------------------------------------------- API
    def reset(self):
        check(lib().mh_reset(self.h, _stream(self._torch, self.dev)), "mh_reset")
        return self.obs

    def step_async(self, actions):
        torch = self._torch
        if not isinstance(actions, torch.Tensor):
            actions = torch.as_tensor(np.asarray(actions))
        if actions.numel() != self.n:
            raise ValueError(f"expected {self.n} actions, got {actions.numel()}")
        if actions.data_ptr() != self.actions.data_ptr():
            self.actions.copy_(actions.reshape(-1).to(self.dev, torch.int64, non_blocking=True))
        check(lib().mh_step_async(self.h, _ptr(self.actions), _stream(torch, self.dev)), "mh_step_async")

    def step(self, actions):
        self.step_async(actions)
        return self.obs, self.rew, self.term, self.trunc, self.info

    def ram(self):
        """(N, 2048) uint8 RAM of every env (a copy)."""
        out = self._torch.empty(self.n, 0x800, dtype=self._torch.uint8, device=self.dev)
        check(lib().mh_env_ram(self.h, _ptr(out), _stream(self._torch, self.dev)), "mh_env_ram")
        return out

    def canon(self):
        """(N, 4464) uint8 canonical console states (layout in include/mario_hip.h)."""
        out = self._torch.empty(self.n, CANON_BYTES, dtype=self._torch.uint8, device=self.dev)
        check(lib().mh_env_canon(self.h, _ptr(out), _stream(self._torch, self.dev)), "mh_env_canon")
        return out

    def level_canon(self):
        nl = lib().mh_num_levels(self.h)
        out = self._torch.empty(nl, CANON_BYTES, dtype=self._torch.uint8, device=self.dev)
        check(lib().mh_level_canon(self.h, _ptr(out), _stream(self._torch, self.dev)), "mh_level_canon")
        return out

    def level_obs(self):
        nl = lib().mh_num_levels(self.h)
        out = self._torch.empty(nl, OBS_HW, OBS_HW, dtype=self._torch.uint8, device=self.dev)
        check(lib().mh_level_obs(self.h, _ptr(out), _stream(self._torch, self.dev)), "mh_level_obs")
        return out

    @property
    def frames(self) -> int:
        """Emulated NES frames, counted like the reference CPU path (hack frames and re-renders included)."""
        return int(lib().mh_frames(self.h))

    def bad_ops(self) -> int:
        return int(lib().mh_bad_ops(self.h))

    def instructions(self) -> int:
        """6502 instructions retired so far (poll-loop fast-forwards included, as the reference counts them)."""
        return int(lib().mh_instructions(self.h))

    def ff_instructions(self) -> int:
        """Of instructions(), those the exact sprite-0 poll-loop fast-forward retired without executing."""
        return int(lib().mh_ff_instructions(self.h))

    def hack_redraws(self) -> int:
        """Hack frames of drawn agent frames run a second time to be drawn: the busy run's last frame (the others
        run undrawn; frames and instructions count it once)."""
        return int(lib().mh_hack_redraws(self.h))

    REEMU_KINDS = ("one", "pair", "k2")

    def reemulations(self) -> dict:
        """Early-termination re-emulations so far: 'one' (frame last re-run alone), 'pair' (its max-pool
        partner re-run too), and 'k2' (of both, the episode ends at frame K-2 under max-pool)."""
        out = np.zeros(3, np.int64)
        check(lib().mh_reemulations(self.h, out.ctypes.data), "mh_reemulations")
        return dict(zip(self.REEMU_KINDS, out.tolist()))

    def bytes_per_env(self) -> int:
        return int(lib().mh_env_bytes(self.h))

    STAGES = ("k_step", "k_obs_late", "k_reset", "k_stack")

    def timing(self, enable: bool = True):
        """Start (or stop) per-stage HIP-event timing of step(); read it with timing_read()."""
        check(lib().mh_timing(self.h, int(bool(enable))), "mh_timing")

    def timing_read(self) -> tuple[dict, int]:
        """-> ({stage: summed ms}, timed steps); synchronizes."""
        ms = np.zeros(len(self.STAGES), np.float64)
        n = np.zeros(1, np.int64)
        check(lib().mh_timing_read(self.h, ms.ctypes.data, n.ctypes.data), "mh_timing_read")
        return dict(zip(self.STAGES, ms.tolist())), int(n[0])

    def synchronize(self):
        check(lib().mh_step_wait(self.h, _stream(self._torch, self.dev)), "mh_step_wait")

    def close(self):
        h, self.h = getattr(self, "h", None), None
        if h:
            lib().mh_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


CudaVecEnv = HipVecEnv   # the reference's name for the GPU flavour


class FastVecEnv:
    """The reference's FastVecEnv API (src/fast_mario_env/env.py:113-266) with numpy in and out; the
    envs step on the GPU. step_async() queues the step and returns; step_wait() synchronizes and
    builds the per-env info dicts (final_obs, TimeLimit.truncated and episode on episode ends).
    `n_threads` sizes the reference's CPU thread pool and has no effect here."""

    def __init__(self, level="1-1", n_envs=8, seed=0, frame_stack=4, sticky=0.0, noop_max=0, max_steps=2000,
                 maxpool=False, skip=4, n_threads=None, copy_obs=True, rom_path=None, rom_mode="vanilla",
                 monitor_path=None, env_offset=0, device="cuda", rom=None):
        if frame_stack < 1:
            raise ValueError("frame_stack must be >= 1")
        self.venv = HipVecEnv(level, n_envs, seed=seed, sticky=sticky, noop_max=noop_max, max_steps=max_steps,
                              skip=skip, frame_stack=frame_stack, device=device, rom_path=rom_path,
                              rom_mode=rom_mode, env_offset=env_offset, maxpool=maxpool, rom=rom)
        self.n = self.num_envs = n_envs
        self.k = frame_stack
        self.copy_obs = copy_obs
        self.levels = self.venv.levels
        self.n_threads = n_threads
        self.monitor = MonitorCSV(monitor_path) if monitor_path else None
        self.t0 = time.time()
        self._closed = False

    def set_buffers(self, obs, fin, rew, term, trunc, info, ep_ret, ep_len):
        """Have every step write its outputs into caller-owned buffers (env.py:183-188 of the reference).

        * numpy arrays (the reference's form): obs / fin (N, k, 84, 84) uint8, rew (N,) float32, term / trunc
          (N,) uint8 or bool, info (N, 10) int64 (int32 accepted), ep_ret (N,) float64, ep_len (N,) int64 (int32
          accepted). reset() and step_wait() copy the results into them; fin / ep_ret / ep_len rows change only
          for envs whose episode ended, as in the reference.
        * torch tensors on the env's GPU or raw device addresses: the kernels write them directly (info and
          ep_len int32). The library refuses pageable host memory, memory of another GPU and misaligned
          buffers; step_wait() keeps returning copies of the env's own buffers, so read yours.
        The caller keeps the buffers alive."""
        bufs = (obs, fin, rew, term, trunc, info, ep_ret, ep_len)
        if all(isinstance(b, np.ndarray) for b in bufs):
            n, k = self.n, self.k
            want = (((n, k, OBS_HW, OBS_HW), (np.uint8,)), ((n, k, OBS_HW, OBS_HW), (np.uint8,)),
                    ((n,), (np.float32,)), ((n,), (np.uint8, np.bool_)), ((n,), (np.uint8, np.bool_)),
                    ((n, len(INFO_FIELDS)), (np.int64, np.int32)), ((n,), (np.float64,)), ((n,), (np.int64, np.int32)))
            names = ("obs", "fin", "rew", "term", "trunc", "info", "ep_ret", "ep_len")
            for b, (shape, dts), nm in zip(bufs, want, names):
                if b.shape != shape or b.dtype.type not in dts:
                    raise ValueError(f"set_buffers: {nm} must be {shape} of {[d.__name__ for d in dts]}, "
                                     f"got {b.shape} {b.dtype}")
            self._host_bufs = dict(zip(names, bufs))
            return
        if any(isinstance(b, np.ndarray) for b in bufs):
            raise ValueError("set_buffers: pass all eight buffers as numpy arrays or all as device buffers")
        addr = [x if isinstance(x, int) else _ptr(x) for x in bufs]
        check(lib().mh_set_buffers(self.venv.h, *addr), "mh_set_buffers")
        self._host_bufs = None

    def _fill_host(self, obs, rew=None, term=None, trunc=None, info=None, done=None, fin=None, epr=None, epl=None):
        hb = getattr(self, "_host_bufs", None)
        if not hb:
            return
        hb["obs"][...] = obs
        if rew is None:
            return
        hb["rew"][...] = rew
        hb["term"][...] = term
        hb["trunc"][...] = trunc
        hb["info"][...] = info
        if done is not None and done.size:
            hb["fin"][done] = fin
            hb["ep_ret"][done] = epr[done]
            hb["ep_len"][done] = epl[done]

    @property
    def frames(self) -> int:
        return self.venv.frames

    def bad_ops(self) -> int:
        return self.venv.bad_ops()

    def bytes_per_env(self) -> int:
        return self.venv.bytes_per_env()

    def reset(self):
        obs = self.venv.reset().cpu().numpy()
        self._fill_host(obs)
        return obs.copy() if self.copy_obs else obs

    def step_async(self, actions):
        a = np.ascontiguousarray(np.asarray(actions).reshape(-1), np.int64)
        if a.shape[0] != self.n:
            raise ValueError(f"expected {self.n} actions, got {a.shape[0]}")
        self.venv.step_async(a)

    def step_wait(self):
        v = self.venv
        v.synchronize()
        obs = v.obs.cpu().numpy()
        term = v.term.cpu().numpy().astype(bool)
        trunc = v.trunc.cpu().numpy().astype(bool)
        rew = v.rew.cpu().numpy().copy()
        info_arr = v.info_t.cpu().numpy().astype(np.int64)
        inf = info_arr.tolist()
        done = np.flatnonzero(term | trunc)
        fin = v.final_obs[done].cpu().numpy() if done.size else None
        epr = v.ep_ret.cpu().numpy() if done.size else None
        epl = v.ep_len.cpu().numpy() if done.size else None
        self._fill_host(obs, rew, term, trunc, info_arr, done, fin, epr, epl)
        infos = []
        for i in range(self.n):
            r = inf[i]
            infos.append({"x_pos": r[0], "flag_get": bool(r[1]), "life": r[2], "score": r[3], "time": r[4],
                          "world": r[5], "stage": r[6]})
        for j, i in enumerate(done):
            info = infos[i]
            info["final_obs"] = fin[j]
            info["TimeLimit.truncated"] = bool(trunc[i] and not term[i])
            e = dict(r=round(float(epr[i]), 6), l=int(epl[i]), t=round(time.time() - self.t0, 6),
                     x_pos=info["x_pos"], flag_get=info["flag_get"])
            info["episode"] = e
            if self.monitor:
                self.monitor.write(e)
        return obs, rew, term, trunc, infos

    def step(self, actions):
        self.step_async(actions)
        return self.step_wait()

    def ram(self, i: int) -> np.ndarray:
        """Copy of env i's 2 KB work RAM."""
        return self.venv.ram()[int(i)].cpu().numpy()

    def close(self):
        if getattr(self, "_closed", True):
            return
        self._closed = True
        self.venv.close()
        if self.monitor:
            self.monitor.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipRawNES:
    """N raw consoles stepped one frame at a time without the env layer (the batched form of the
    reference's RawNES, env.py:58-90). frame(buttons, render) steps all of them; ram / screen return
    (N, 2048) / (N, 240, 256) uint8 device tensors (screen holds palette values, as nes-py's)."""

    def __init__(self, rom_bytes: bytes, n: int = 1, device="cuda"):
        torch = self._torch = _torch()
        check_rom(rom_bytes)
        self.dev = torch.device(device)
        if self.dev.index is None:
            self.dev = torch.device("cuda", torch.cuda.current_device())
        self.n = n
        self._rom = np.frombuffer(rom_bytes, np.uint8).copy()
        with torch.cuda.device(self.dev):
            self.h = lib().mh_raw_create(self._rom.ctypes.data, len(self._rom), n, self.dev.index)
        if not self.h:
            raise ValueError(f"mh_raw_create failed: {_native.last_error()}")
        self._buttons = torch.zeros(n, dtype=torch.uint8, device=self.dev)

    def frame(self, buttons, render: bool = True):
        torch = self._torch
        b = torch.as_tensor(buttons).to(self.dev, torch.uint8).reshape(-1)
        if b.numel() == 1 and self.n > 1:
            b = b.expand(self.n)
        self._buttons.copy_(b)
        check(lib().mh_raw_frame(self.h, _ptr(self._buttons), int(bool(render)), _stream(torch, self.dev)),
              "mh_raw_frame")

    def _out(self, fn, shape):
        out = self._torch.empty(*shape, dtype=self._torch.uint8, device=self.dev)
        check(fn(self.h, _ptr(out), _stream(self._torch, self.dev)), fn.__name__)
        return out

    @property
    def ram(self):
        return self._out(lib().mh_raw_ram, (self.n, 0x800))

    @property
    def screen(self):
        return self._out(lib().mh_raw_screen, (self.n, 240, 256))

    @property
    def screen_rgb(self):
        """(N, 240, 256, 3) uint8 RGB24 device tensor: the screen through nes-py's palette, as nes-py's own
        screen array."""
        torch = self._torch
        if getattr(self, "_rgb64", None) is None:
            self._rgb64 = torch.from_numpy(palette_rgb().reshape(-1).copy()).to(self.dev)
        out = torch.empty(self.n, 240, 256, 3, dtype=torch.uint8, device=self.dev)
        check(lib().mh_raw_screen_rgb(self.h, _ptr(self._rgb64), _ptr(out), _stream(torch, self.dev)),
              "mh_raw_screen_rgb")
        return out

    def canon(self):
        return self._out(lib().mh_raw_canon, (self.n, CANON_BYTES))

    def backup(self):
        check(lib().mh_raw_backup(self.h, _stream(self._torch, self.dev)), "mh_raw_backup")

    def restore(self):
        check(lib().mh_raw_restore(self.h, _stream(self._torch, self.dev)), "mh_raw_restore")

    def bad_ops(self) -> int:
        return int(lib().mh_raw_bad_ops(self.h))

    def instructions(self) -> int:
        return int(lib().mh_raw_instructions(self.h))

    def ff_instructions(self) -> int:
        return int(lib().mh_raw_ff_instructions(self.h))

    def __del__(self):
        h, self.h = getattr(self, "h", None), None
        if h:
            try:
                lib().mh_raw_destroy(h)
            except Exception:
                pass


class RawNES(HipRawNES):
    """Single raw console with the reference RawNES interface (ram (2048,), screen (240, 256) as numpy)."""

    def __init__(self, rom_bytes: bytes, device="cuda"):
        super().__init__(rom_bytes, 1, device)

    def frame(self, buttons: int, render: bool = True):
        super().frame(int(buttons), render)

    @property
    def ram(self):
        return super().ram[0].cpu().numpy()

    @property
    def screen(self):
        return super().screen[0].cpu().numpy()


def resize_area(gray, fast: bool = True):
    """240x256 uint8 -> 84x84 with the INTER_AREA float path, computed on the GPU. Accepts a numpy
    array (returns numpy) or a (..., 240, 256) uint8 device tensor (returns a device tensor)."""
    torch = _torch()
    is_np = isinstance(gray, np.ndarray)
    g = torch.as_tensor(np.ascontiguousarray(gray, np.uint8)).cuda() if is_np else gray.contiguous()
    if tuple(g.shape[-2:]) != (240, 256) or g.dtype != torch.uint8:
        raise ValueError("expected (..., 240, 256) uint8 images")
    lead = g.shape[:-2]
    flat = g.reshape(-1, 240, 256)
    out = torch.empty(flat.shape[0], OBS_HW, OBS_HW, dtype=torch.uint8, device=g.device)
    check(lib().mh_resize(_ptr(flat), _ptr(out), flat.shape[0], torch.cuda.current_stream(g.device).cuda_stream),
          "mh_resize")
    out = out.reshape(*lead, OBS_HW, OBS_HW)
    return out.cpu().numpy() if is_np else out
