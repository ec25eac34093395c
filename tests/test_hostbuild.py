"""The device code on the CPU under AddressSanitizer and UndefinedBehaviorSanitizer, against the golden traces.

tests/hostbuild compiles the GPU kernels' device headers (nes_device.hpp, env_device.hpp, lane_kernels.hpp)
as x86 C++ with one lane per env (its hip/hip_runtime.h stands in for HIP's) and drives the same lane bodies
the kernels call (host_driver.cpp), every buffer sized exactly. Any out-of-bounds access or undefined behaviour
in the device code aborts the run; the outputs must equal the digests the reference C++ wrote
(tests/golden/golden_traces.json). Test infrastructure only: the product is the GPU build.
"""
import os
import struct
import subprocess

import numpy as np
import pytest
from conftest import ROOT

import make_golden as G
from build_roms import rom_path
from cpu_libs import gray_lut, rng_state

HB = os.path.join(ROOT, "tests", "hostbuild")
EXE = os.path.join(HB, "host_driver_san")
GOLD = __import__("json").load(open(G.GOLDEN))
MINI = open(rom_path("vanilla"), "rb").read()
SAN_ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")


@pytest.fixture(scope="module")
def exe():
    if not os.path.isfile(os.path.join(HB, "Makefile")):
        pytest.skip("tests/hostbuild is not in this tree")
    r = subprocess.run(["make", "-s", "-C", HB], capture_output=True, text=True)
    if r.returncode != 0:
        if "not found" in r.stderr or "No such file" in r.stderr:
            pytest.skip("no clang++ for the host build")
        raise AssertionError(r.stderr[-3000:])
    return EXE


class _Proc:
    def __init__(self, exe, mode, path):
        self.p = subprocess.Popen([exe, mode, path], stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                                  stderr=subprocess.PIPE, env=SAN_ENV)

    def send(self, data: bytes):
        self.p.stdin.write(data)
        self.p.stdin.flush()

    def recv(self, n: int) -> bytes:
        out = self.p.stdout.read(n)
        if len(out) != n:
            err = self.p.stderr.read().decode(errors="replace")
            raise AssertionError(f"host build ended early (sanitizer report?):\n{err[-6000:]}")
        return out

    def quit(self, nbytes):
        self.send(b"Q")
        vals = struct.unpack(f"<{nbytes // 8}q", self.recv(nbytes))
        self.p.wait(timeout=60)
        assert self.p.returncode == 0, self.p.stderr.read().decode(errors="replace")[-6000:]
        return vals


class HostRaw:
    """One raw console of the host build (the interface G.run_raw drives)."""

    def __init__(self, exe, rom: bytes, tmp):
        path = os.path.join(tmp, "rom.nes")
        open(path, "wb").write(rom)
        self.proc = _Proc(exe, "raw", path)
        self.ram = np.zeros(2048, np.uint8)
        self.screen = np.zeros((240, 256), np.uint8)

    def frame(self, buttons, render):
        self.proc.send(b"F" + bytes([int(buttons) & 255, int(bool(render))]))
        self.ram = np.frombuffer(self.proc.recv(2048), np.uint8)
        self.screen = np.frombuffer(self.proc.recv(240 * 256), np.uint8).reshape(240, 256)

    def backup(self):
        self.proc.send(b"B")

    def restore(self):
        self.proc.send(b"S")

    def finish(self):
        return self.proc.quit(24)        # bad ops, instructions, fast-forwarded instructions


class HostVec:
    """A vector env of the host build (the interface G.run_env drives)."""

    def __init__(self, exe, rom, levels, n, tmp, seed=0, frame_stack=4, sticky=0.0, noop_max=0, max_steps=2000,
                 maxpool=False, skip=4):
        self.n, self.k = n, frame_stack
        cfg = bytearray()
        cfg += struct.pack("<q", len(rom)) + rom + struct.pack("<i", n)
        cfg += np.asarray(levels, np.int32).reshape(-1).tobytes() + gray_lut().tobytes()
        cfg += struct.pack("<iidiii", skip, max_steps, float(sticky), noop_max, int(bool(maxpool)), frame_stack)
        cfg += np.array([rng_state(seed * 1000 + i) for i in range(n)], np.uint64).reshape(-1).tobytes()
        path = os.path.join(tmp, "env.cfg")
        open(path, "wb").write(bytes(cfg))
        self.proc = _Proc(exe, "env", path)
        self.sz = n * frame_stack * 84 * 84

    def reset(self):
        self.proc.send(b"R")
        self.obs = np.frombuffer(self.proc.recv(self.sz), np.uint8).reshape(self.n, self.k, 84, 84)
        return self.obs

    def step(self, actions):
        n, r = self.n, self.proc.recv
        self.proc.send(b"T" + np.ascontiguousarray(actions, np.int64).tobytes())
        self.obs = np.frombuffer(r(self.sz), np.uint8).reshape(n, self.k, 84, 84)
        rew = np.frombuffer(r(4 * n), np.float32)
        term = np.frombuffer(r(n), np.uint8).astype(bool)
        trunc = np.frombuffer(r(n), np.uint8).astype(bool)
        info = np.frombuffer(r(80 * n), np.int64).reshape(n, 10)
        self._ram = np.frombuffer(r(2048 * n), np.uint8).reshape(n, 2048)
        self.fin = np.frombuffer(r(self.sz), np.uint8).reshape(n, self.k, 84, 84)
        self.ep_ret = np.frombuffer(r(8 * n), np.float64)
        self.ep_len = np.frombuffer(r(8 * n), np.int64)
        return self.obs, rew, term, trunc, info

    def ram(self, i):
        return self._ram[i]

    def finish(self):
        return self.proc.quit(40)        # frames, bad ops, instructions, fast-forwarded instructions, hack redraws


def test_hostbuild_sanitizer_catches_a_planted_overrun(exe):
    """The checker is live: a one-byte read past a buffer aborts the sanitizer build."""
    r = subprocess.run([exe, "plant", "4384"], capture_output=True, text=True, env=SAN_ENV, timeout=60)
    assert r.returncode != 0 and "AddressSanitizer" in r.stderr


RAW = [c[0] for c in G.RAW_CASES]


@pytest.mark.parametrize("case", RAW)
def test_hostbuild_raw_golden(exe, tmp_path, case):
    g = GOLD["raw"][case]
    con = HostRaw(exe, G.raw_rom(case), str(tmp_path))
    tr = G.run_raw(con, G.raw_schedule(g["seed"], g["frames"]))
    bad = [i for i, (a, b) in enumerate(zip(tr, g["trace"])) if a != b]
    assert not bad, f"first mismatching frame {bad[0]}"
    bad_ops, instr, ff = con.finish()
    assert bad_ops == g["bad_ops"] and 0 <= ff <= instr


ENV = list(G.ENV_CASES)


@pytest.mark.parametrize("config", ENV)
def test_hostbuild_env_golden(exe, tmp_path, config):
    from fast_mario_env_amd.rom import decode_level
    g = GOLD["env"][config]
    names = G.ENV_LEVELS
    venv = HostVec(exe, MINI, [decode_level(x) for x in names], len(names), str(tmp_path), seed=7, **g["kw"])
    tr = G.run_env(venv, G.env_actions(len(names), G.ENV_STEPS))
    bad = [i for i, (a, b) in enumerate(zip(tr, g["trace"])) if a != b]
    assert not bad, f"first mismatching step {bad[0] - 1}"
    frames, bad_ops, instr, ff, redraws = venv.finish()
    assert frames == g["frames"] and bad_ops == 0 and 0 <= ff <= instr and redraws >= 0
