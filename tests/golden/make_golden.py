"""Writes the golden traces under tests/golden/ from the reference C++ (oracle/_ref, built by
`make -C oracle` from /root/reference/csrc/fastmario.cpp) on this repository's synthetic ROMs.

    python tests/golden/make_golden.py

Each trace is a list of 8-byte blake2b digests, one per frame / step, of exactly the arrays the
reference exposes through its own C ABI (fm_raw_ram / fm_raw_screen, and the FastVecEnv output
buffers + fm_env_ram). The schedules (buttons, render flags, backup/restore, actions) are derived from
fixed seeds, so a test can regenerate them and compare any implementation against these digests.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(HERE, "roms"))
import fuzz  # noqa: E402
from build_roms import MODES, rom_path  # noqa: E402

GOLDEN = os.path.join(HERE, "golden_traces.json")
CONFIG1 = os.path.join(HERE, "config1_trace.npz")


def digest(*arrays) -> str:
    h = hashlib.blake2b(digest_size=8)
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ---------------------------------------------------------------- schedules
RAW_CASES = ([("mini_smb", 0, 300)] + [(f"program_{s}", s, 240) for s in range(8)] +
             [(f"random_{s}", s, 120) for s in range(8)] + [(f"screenoff_{s}", s, 240) for s in range(4)])


def raw_rom(name: str) -> bytes:
    if name == "mini_smb":
        return open(rom_path("vanilla"), "rb").read()
    kind, seed = name.split("_")
    if kind == "screenoff":
        return fuzz.program_rom(int(seed), screen_off=True)
    return fuzz.program_rom(int(seed)) if kind == "program" else fuzz.random_rom(int(seed))


def raw_schedule(seed: int, frames: int):
    """(buttons, render, op) per frame; op 1 = backup before the frame, 2 = restore before it."""
    rng = np.random.default_rng(1000 + seed)
    btn, out, have = 0, [], False
    for _ in range(frames):
        if rng.random() < 0.2:
            btn = int(rng.integers(0, 256))
        u = rng.random()
        op = 0
        if u < 0.01:
            op, have = 1, True
        elif u < 0.02 and have:
            op = 2
        out.append((btn, bool(rng.random() < 0.5), op))
    return out


def run_raw(console, schedule):
    """console: object with frame(buttons, render), backup(), restore(), ram, screen."""
    trace = []
    for btn, render, op in schedule:
        if op == 1:
            console.backup()
        elif op == 2:
            console.restore()
        console.frame(btn, render)
        trace.append(digest(console.ram, console.screen) if render else digest(console.ram))
    return trace


ENV_CASES = {
    "default": dict(),
    "sticky_noop": dict(sticky=0.25, noop_max=30),
    "maxpool_sticky": dict(maxpool=True, sticky=0.25),
    "short_timelimit": dict(max_steps=60, noop_max=5),
    "headline": dict(sticky=0.25, noop_max=30, maxpool=True),
    "skip1_stack2": dict(skip=1, frame_stack=2, noop_max=3),
    "skip6_maxpool": dict(skip=6, maxpool=True, noop_max=4, sticky=0.5),
}
ENV_LEVELS = ["1-1", "1-2", "4-1", "8-4", "2-3", "1-1"]
ENV_STEPS = 200
ACTION_P = [.05, .2, .25, .15, .25, .05, .05]


def env_actions(n, steps, seed=130):
    rng = np.random.default_rng(seed)
    return [rng.choice(7, n, p=ACTION_P) for _ in range(steps)]


def run_env(venv, actions):
    """venv: cpu_libs-style vector env (reset() / step() with numpy outputs, ram(i), fin, ep_ret, ep_len)."""
    n = venv.n
    trace = [digest(venv.reset())]
    for a in actions:
        obs, rew, term, trunc, info = venv.step(a)
        ram = np.stack([venv.ram(i) for i in range(n)])
        parts = [obs, rew, term, trunc, np.asarray(info, np.int64), ram]
        done = term | trunc
        if done.any():
            idx = np.flatnonzero(done)
            parts += [venv.fin[idx], np.asarray(venv.ep_ret[idx], np.float64), np.asarray(venv.ep_len[idx], np.int64)]
        trace.append(digest(*parts))
    return trace


def config1_actions(steps=1000, n=32):
    """Golden-trace workload: actions uniform in {0..6} from default_rng(0), shape (32,), one draw per step."""
    rng = np.random.default_rng(0)
    return [rng.integers(0, 7, n) for _ in range(steps)]


CONFIG1_KEEP = (0, 1, 10, 100, 999)


def main():
    from cpu_libs import RefRaw, RefVec, have_ref, reference

    if not have_ref():
        sys.exit("oracle/_ref/libfastmario_ref.so is missing: run `make -C oracle` where /root/reference exists")
    out = {"raw": {}, "env": {}, "meta": {}}
    for name, seed, frames in RAW_CASES:
        rom = raw_rom(name)
        ref = RefRaw(rom)
        out["raw"][name] = {"seed": seed, "frames": frames, "trace": run_raw(ref, raw_schedule(seed, frames)),
                            "bad_ops": ref.bad_ops(), "rom": digest(np.frombuffer(rom, np.uint8))}
        print("raw", name, out["raw"][name]["bad_ops"], flush=True)
    from fast_mario_env_amd.rom import decode_level  # pure-Python level table
    mini = open(rom_path("vanilla"), "rb").read()
    levels = [decode_level(x) for x in ENV_LEVELS]
    for cname, kw in ENV_CASES.items():
        ref = RefVec(mini, levels, len(levels), seed=7, **kw)
        tr = run_env(ref, env_actions(len(levels), ENV_STEPS))
        out["env"][cname] = {"kw": kw, "trace": tr, "frames": ref.frames(), "bad_ops": ref.bad_ops()}
        print("env", cname, ref.frames(), flush=True)
        ref.close()
    # rom_mode variants: boot + a short run on each CHR variant
    for mode in MODES:
        rom = open(rom_path(mode), "rb").read()
        ref = RefVec(rom, levels[:3], 3, seed=1, sticky=0.25, noop_max=8, maxpool=True)
        out["env"][f"mode_{mode}"] = {"kw": dict(sticky=0.25, noop_max=8, maxpool=True), "mode": mode,
                                      "levels": ENV_LEVELS[:3], "seed": 1,
                                      "trace": run_env(ref, env_actions(3, 60, seed=5)), "frames": ref.frames()}
        ref.close()
    # palette and resize known answers straight from the reference ABI
    L = reference()
    pal = np.zeros(64, np.uint32)
    L.fm_palette(pal.ctypes.data)
    out["meta"]["palette"] = pal.tolist()
    rng = np.random.default_rng(0)
    imgs, res = [], []
    for t in range(40):
        img = rng.integers(0, 256, (240, 256), np.uint8) if t % 2 else \
            np.roll(rng.integers(0, 256, (30, 32)).astype(np.uint8).repeat(8, 0).repeat(8, 1), rng.integers(0, 8, 2), (0, 1)).copy()
        dst = np.zeros((84, 84), np.uint8)
        L.fm_resize_ref(img.ctypes.data, 256, 240, dst.ctypes.data, 84, 84)
        dst2 = np.zeros((84, 84), np.uint8)
        L.fm_resize_fast(img.ctypes.data, dst2.ctypes.data)
        assert np.array_equal(dst, dst2)
        res.append(digest(dst))
    out["meta"]["resize_seed0_40"] = res
    # the golden-trace workload on the synthetic ROM: 32 envs of 1-1, 1000 steps
    n = 32
    ref = RefVec(mini, [decode_level("1-1")] * n, n, seed=0, frame_stack=4, skip=4, sticky=0.0, noop_max=0,
                 maxpool=False, max_steps=2000)
    keep = {}
    trace = [digest(ref.reset())]
    for t, a in enumerate(config1_actions()):
        obs, rew, term, trunc, info = ref.step(a)
        ram = np.stack([ref.ram(i) for i in range(n)])
        trace.append(digest(obs, rew, term, trunc, np.asarray(info, np.int64), ram))
        if t in CONFIG1_KEEP:
            keep[f"obs_{t}"] = obs.copy(); keep[f"ram_{t}"] = ram
            keep[f"rew_{t}"] = rew.copy(); keep[f"term_{t}"] = term.copy(); keep[f"trunc_{t}"] = trunc.copy()
            keep[f"info_{t}"] = np.asarray(info, np.int64).copy()
    out["config1"] = {"trace": trace, "frames": ref.frames(), "bad_ops": ref.bad_ops()}
    ref.close()
    np.savez_compressed(CONFIG1, **keep)
    with open(GOLDEN, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", GOLDEN, os.path.getsize(GOLDEN), CONFIG1, os.path.getsize(CONFIG1))


if __name__ == "__main__":
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "fast-mario-env_amd"))
    main()
