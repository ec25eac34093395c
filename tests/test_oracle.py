"""Pins the CPU oracle (oracle/liboracle.so), which the GPU path is checked against.

* golden traces written by the reference C++ (tests/golden/make_golden.py) on the synthetic ROMs:
  per-frame RAM/screen digests of raw consoles and per-step env digests;
* a live differential against oracle/_ref (the reference compiled from its own sources) on more
  fuzz seeds, when that library is present;
* numpy's own PCG64 Generator for random() / integers();
* closed forms: the palette table, cv2's RGB2GRAY fixed-point weights, the INTER_AREA tables;
* textbook 8-bit arithmetic (ALU test ROMs), independent of the reference's formulas.
"""
import ctypes
import json
import os

import numpy as np
import pytest
from conftest import scaled

import alu_rom
import fuzz
import make_golden as G
from build_roms import MODES, build, rom_path
from cpu_libs import OracleRaw, OracleVec, RefRaw, RefVec, gray_lut, have_ref, have_ref_prof, oracle, prof_counter

GOLD = json.load(open(G.GOLDEN))
MINI = open(rom_path("vanilla"), "rb").read()
requires_ref = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (no reference tree)")
requires_ref_prof = pytest.mark.skipif(not have_ref_prof(), reason="oracle/_ref prof build absent (no reference tree)")


def _levels(names):
    from fast_mario_env_amd.rom import decode_level
    return [decode_level(x) for x in names]


# ---------------------------------------------------------------- fixtures are what they claim to be
@pytest.mark.parametrize("mode", MODES)
def test_roms_rebuild_identically(mode):
    assert build(mode) == open(rom_path(mode), "rb").read()


# ---------------------------------------------------------------- golden traces (reference C++)
@pytest.mark.parametrize("case", [c[0] for c in G.RAW_CASES])
def test_raw_golden(case):
    g = GOLD["raw"][case]
    rom = G.raw_rom(case)
    assert G.digest(np.frombuffer(rom, np.uint8)) == g["rom"]
    con = OracleRaw(rom)
    tr = G.run_raw(con, G.raw_schedule(g["seed"], g["frames"]))
    bad = [i for i, (a, b) in enumerate(zip(tr, g["trace"])) if a != b]
    assert not bad, f"first mismatching frame {bad[0]}"
    assert con.bad_ops() == g["bad_ops"]


@pytest.mark.parametrize("config", list(G.ENV_CASES))
def test_env_golden(config):
    g = GOLD["env"][config]
    names = G.ENV_LEVELS
    venv = OracleVec(MINI, _levels(names), len(names), seed=7, **g["kw"])
    tr = G.run_env(venv, G.env_actions(len(names), G.ENV_STEPS))
    bad = [i for i, (a, b) in enumerate(zip(tr, g["trace"])) if a != b]
    assert not bad, f"first mismatching step {bad[0] - 1}"
    assert venv.frames() == g["frames"] and venv.bad_ops() == 0


@pytest.mark.parametrize("mode", MODES)
def test_rom_mode_golden(mode):
    g = GOLD["env"][f"mode_{mode}"]
    rom = open(rom_path(mode), "rb").read()
    venv = OracleVec(rom, _levels(g["levels"]), len(g["levels"]), seed=g["seed"], **g["kw"])
    tr = G.run_env(venv, G.env_actions(len(g["levels"]), 60, seed=5))
    assert tr == g["trace"]
    assert venv.frames() == g["frames"]


def test_config1_golden():
    """The CPU golden-trace workload (32 envs of 1-1, seed 0, no sticky / no-op / max-pool) on the synthetic ROM;
    the first 250 steps by default, all 1000 with FME_TEST_SCALE >= 4."""
    g = GOLD["config1"]
    steps = min(1000, scaled(250))
    n = 32
    venv = OracleVec(MINI, _levels(["1-1"]) * n, n, seed=0)
    keep = np.load(G.CONFIG1)
    assert G.digest(venv.reset()) == g["trace"][0]
    for t, a in enumerate(G.config1_actions()[:steps]):
        obs, rew, term, trunc, info = venv.step(a)
        ram = np.stack([venv.ram(i) for i in range(n)])
        assert G.digest(obs, rew, term, trunc, np.asarray(info, np.int64), ram) == g["trace"][t + 1], t
        if t in G.CONFIG1_KEEP:
            assert np.array_equal(obs, keep[f"obs_{t}"]) and np.array_equal(ram, keep[f"ram_{t}"])
            assert np.array_equal(info, keep[f"info_{t}"]) and np.array_equal(rew, keep[f"rew_{t}"])


# ---------------------------------------------------------------- live differential vs the reference
@requires_ref
@pytest.mark.parametrize("seed", range(100, 112))
def test_raw_vs_reference(seed):
    rom = fuzz.program_rom(seed) if seed % 2 else fuzz.random_rom(seed)
    sched = G.raw_schedule(seed, scaled(150))
    a, b = OracleRaw(rom), RefRaw(rom)
    assert G.run_raw(a, sched) == G.run_raw(b, sched)
    assert a.bad_ops() == b.bad_ops()


@requires_ref
@pytest.mark.parametrize("kw", [dict(sticky=0.5, noop_max=12, maxpool=True), dict(skip=3, max_steps=40, sticky=0.1),
                                dict(skip=16, frame_stack=1, noop_max=2), dict(skip=2, maxpool=True, frame_stack=3)])
def test_env_vs_reference(kw):
    names = ["1-1", "3-3", "7-2", "1-1"]
    acts = G.env_actions(4, scaled(100), seed=11)
    a = OracleVec(MINI, _levels(names), 4, seed=9, **kw)
    b = RefVec(MINI, _levels(names), 4, seed=9, **kw)
    assert G.run_env(a, acts) == G.run_env(b, acts)
    assert a.frames() == b.frames()


@requires_ref
def test_env_offset_and_threads_vs_reference():
    """env_offset reproduces a slice of a larger batch; the reference's thread count changes nothing."""
    from cpu_libs import RefVec as R
    names = ["1-1"] * 4
    acts = G.env_actions(4, 40, seed=2)
    full = OracleVec(MINI, _levels(names), 4, seed=2, sticky=0.25, noop_max=10)
    part = OracleVec(MINI, _levels(names[:2]), 2, seed=2, sticky=0.25, noop_max=10, env_offset=2)
    thr = R(MINI, _levels(names), 4, n_threads=3, seed=2, sticky=0.25, noop_max=10)
    assert np.array_equal(full.reset()[2:], part.reset())
    assert np.array_equal(full.obs, thr.reset())
    for x in acts:
        assert np.array_equal(full.step(x)[0][2:], part.step(x[2:])[0])
        assert np.array_equal(full.obs, thr.step(x)[0])


# ---------------------------------------------------------------- the instruction counter
@requires_ref_prof
@pytest.mark.parametrize("case", ["mini_smb", "program_1", "program_4", "random_2"])
def test_raw_instruction_count_vs_reference_prof(case):
    """The oracle's retired-instruction count equals the reference's own FM_PROF counter prof_cpu_instr
    (nes_core.hpp:1195), which counts every executed instruction and no idle-skipped JMP * iteration."""
    rom = G.raw_rom(case)
    sched = G.raw_schedule(7, scaled(120))
    ref = RefRaw(rom, prof=True)
    ctr = prof_counter()
    ctr.value = 0
    con = OracleRaw(rom)
    G.run_raw(ref, sched)
    G.run_raw(con, sched)
    assert con.instructions() == ctr.value > 0


@requires_ref_prof
@pytest.mark.parametrize("kw", [dict(sticky=0.25, noop_max=30, maxpool=True), dict(skip=3, max_steps=40)])
def test_env_instruction_count_vs_reference_prof(kw):
    """Same for the env path from reset on (no-op starts, hack frames and early-termination re-emulations
    included), with the reference stepping inline (n_threads=0) so the global counter is not raced."""
    names = ["1-1", "4-1", "8-4", "1-2"]
    ctr = prof_counter()
    ref = RefVec(MINI, _levels(names), 4, n_threads=0, prof=True, seed=3, **kw)
    ctr.value = 0                              # level boot happened in the constructor: not counted
    con = OracleVec(MINI, _levels(names), 4, seed=3, **kw)
    ref.reset(); con.reset()
    for a in G.env_actions(4, scaled(80), seed=4):
        ref.step(a); con.step(a)
    assert con.instructions() == ctr.value > 0
    assert con.frames() == ref.frames()


# ---------------------------------------------------------------- numpy PCG64
@pytest.mark.parametrize("seed", [0, 1, 7, 12345, 2**40 + 3])
def test_pcg64_matches_numpy(seed):
    from cpu_libs import rng_state
    rng = np.random.default_rng(seed)
    ops = np.random.default_rng(seed + 1).choice([0, 0, 0, 31, 2, 7, 100000, 2**32], 400).astype(np.int64)
    want = []
    for o in ops:
        want.append(np.float64(rng.random()).view(np.uint64) if o == 0 else np.uint64(rng.integers(0, o)))
    st = np.array(rng_state(seed), np.uint64)
    out = np.zeros(len(ops), np.uint64)
    st_out = np.zeros(6, np.uint64)
    oracle().or_pcg_run(st.ctypes.data, ops.ctypes.data, len(ops), out.ctypes.data, st_out.ctypes.data)
    assert np.array_equal(out, np.array(want, np.uint64))
    s = rng.bit_generator.state
    m = (1 << 64) - 1
    assert [int(x) for x in st_out] == [s["state"]["state"] >> 64, s["state"]["state"] & m, s["state"]["inc"] >> 64,
                                        s["state"]["inc"] & m, s["has_uint32"], s["uinteger"]]


# ---------------------------------------------------------------- closed forms
def test_palette_and_gray_lut():
    from fast_mario_env_amd import PALETTE
    from fast_mario_env_amd import gray_lut as product_lut
    p = np.zeros(64, np.uint32)
    oracle().or_palette(p.ctypes.data)
    assert p.tolist() == GOLD["meta"]["palette"] == PALETTE.tolist()
    lut = gray_lut()
    assert np.array_equal(lut, product_lut())
    assert 4899 + 9617 + 1868 == 1 << 14          # the fixed-point weights sum to one
    rgb = np.stack([(p >> 16) & 255, (p >> 8) & 255, p & 255], -1).astype(np.float64)
    exact = rgb @ np.array([0.299, 0.587, 0.114])
    assert np.all(np.abs(lut[:64] - exact) <= 0.5 + 1e-9)   # rounding of BT.601 luma
    assert np.array_equal(lut[64:], np.tile(lut[:64], 3))   # values are taken & 63
    for i in range(64):
        if rgb[i, 0] == rgb[i, 1] == rgb[i, 2]:
            assert lut[i] == rgb[i, 0]                        # neutral colours keep their level


@pytest.mark.parametrize("ssize,count", [(256, 336), (240, 312)])
def test_area_tables(ssize, count):
    di = np.zeros(1024, np.int32); si = np.zeros(1024, np.int32); w = np.zeros(1024, np.float32)
    k = oracle().or_area_tab(ssize, 84, di.ctypes.data, si.ctypes.data, w.ctypes.data)
    assert k == count
    di, si, w = di[:k], si[:k], w[:k]
    assert np.all(np.diff(di) >= 0) and di[0] == 0 and di[-1] == 83
    for d in range(84):
        s = si[di == d]
        assert 1 <= len(s) <= 4 and np.array_equal(s, np.arange(s[0], s[0] + len(s)))
        assert abs(float(w[di == d].astype(np.float64).sum()) - 1.0) < 1e-5
    counts = np.bincount(si, minlength=ssize)
    assert counts.min() >= 1 and counts.max() <= 2         # every source row/column feeds 1 or 2 outputs


def test_resize_known_answers():
    rng = np.random.default_rng(0)
    got = []
    for t in range(40):
        img = rng.integers(0, 256, (240, 256), np.uint8) if t % 2 else \
            np.roll(rng.integers(0, 256, (30, 32)).astype(np.uint8).repeat(8, 0).repeat(8, 1), rng.integers(0, 8, 2), (0, 1)).copy()
        dst = np.zeros((84, 84), np.uint8)
        oracle().or_resize(img.ctypes.data, dst.ctypes.data)
        got.append(G.digest(dst))
    assert got == GOLD["meta"]["resize_seed0_40"]
    for v in (0, 1, 77, 128, 254, 255):                        # constant images stay constant
        img = np.full((240, 256), v, np.uint8)
        dst = np.zeros((84, 84), np.uint8)
        oracle().or_resize(img.ctypes.data, dst.ctypes.data)
        assert np.all(dst == v)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_alu_textbook(seed):
    rom, expect = alu_rom.build(seed)
    con = OracleRaw(rom)
    con.frame(0, False)
    con.frame(0, False)
    got = con.ram[0x200:0x200 + len(expect)]
    bad = np.flatnonzero(got != expect)
    if bad.size:
        i = bad[0] // 2
        pytest.fail(f"case {i} {alu_rom.cases(seed)[i]}: got {got[2*i:2*i+2]} want {expect[2*i:2*i+2]}")
    assert con.bad_ops() == 0


# ---------------------------------------------------------------- committed GPU fidelity records
def test_fidelity_records():
    """The committed fidelity records (tests/fidelity/*.jsonl, written on the GPU by the scripts beside them) hold
    the runs they claim, with no mismatch: 512 envs over the 32 levels x 1,500 steps in each of 5 configurations
    (every env every step against the oracle), and 512 raw consoles x 20,040 frames (RAM and machine state every
    frame, the screen every 4th), once with the library's launch shape and once with 16 consoles per wave."""
    import json
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fidelity")
    env = [json.loads(l) for l in open(os.path.join(d, "env_fidelity.jsonl"))]
    assert [r["config"] for r in env] == ["default", "sticky_noop", "short_timelimit", "headline", "runner"]
    for r in env:
        assert r["n"] == 512 and r["steps"] == 1500 and r["ok"] and not r["mismatches"], r["config"]
        assert r["bad_ops"] == 0 and r["oracle_bad_ops"] == 0 and r["episodes"] > 1000
    assert sum(r["flags"] for r in env) > 0          # the runner reaches the flagpole
    assert env[3]["reemulations"]["pair"] > 0 and env[3]["reemulations"]["k2"] > 0
    raw = [json.loads(l) for l in open(os.path.join(d, "raw_fidelity.jsonl"))]
    assert [r["consoles_per_wave"] for r in raw] == ["auto", "16"]     # k_raw's launch shapes: 1 and 16 per wave
    for r in raw:
        assert r["ok"] and not r["mismatches"] and r["consoles"] == 512 and r["frames"] == 20040
        assert r["bad_ops"] == 0 and r["instructions"] == raw[0]["instructions"]
