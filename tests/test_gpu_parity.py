"""GPU parity: the HIP path (libmario_hip.so through the C ABI) against the CPU oracle, bit for bit.

Raw consoles: RAM, rendered screen and the full canonical machine state after every frame, on the
synthetic workload ROM and on generated fuzz ROMs. Env level: stacked obs, rewards, terminated,
truncated, info, RAM, final_obs, episode return/length and frame counts every step, across the
wrapper configurations of the reference's fidelity tests (tests/test_fidelity_env.py:17-22) plus
max-pool.
"""
import numpy as np
import pytest
from conftest import scaled

import fuzz
from build_roms import rom_path
from cpu_libs import OracleRaw, OracleVec

pytestmark = pytest.mark.gpu

MINI = open(rom_path("vanilla"), "rb").read()
# k_raw's consoles per wave: "auto" lets the library choose (few consoles: one per wave, every SIMD busy), 16 fills
# every wave, so that lanes of one wave run different consoles and force catch-ups on each other
CPW = ["auto", "16"]


def _first_diff(a, b):
    d = np.flatnonzero(np.asarray(a).reshape(-1) != np.asarray(b).reshape(-1))
    return d[:8].tolist()


def _raw_run(rom, n, frames, seed, render_p=0.5, backup_p=0.0, rgb=False, cpw="auto", monkeypatch=None):
    import torch

    from fast_mario_env_amd import HipRawNES, palette_rgb
    pal = palette_rgb()
    if cpw != "auto":
        monkeypatch.setenv("MH_RAW_CONSOLES_PER_WAVE", cpw)
    gpu = HipRawNES(rom, n)
    cpu = [OracleRaw(rom) for _ in range(n)]
    rng = np.random.default_rng(seed)
    buttons = np.zeros(n, np.uint8)
    have = False
    for f in range(frames):
        ch = rng.random(n) < 0.15
        buttons[ch] = rng.integers(0, 256, int(ch.sum()))
        render = bool(rng.random() < render_p)
        u = rng.random()
        if u < backup_p:
            gpu.backup(); [c.backup() for c in cpu]; have = True
        elif u < 2 * backup_p and have:
            gpu.restore(); [c.restore() for c in cpu]
        gpu.frame(torch.from_numpy(buttons), render)
        for i, c in enumerate(cpu):
            c.frame(int(buttons[i]), render)
        ram = gpu.ram.cpu().numpy()
        canon = gpu.canon().cpu().numpy()
        scr = gpu.screen.cpu().numpy() if render else None
        for i, c in enumerate(cpu):
            assert np.array_equal(ram[i], c.ram), (f, i, "ram", _first_diff(ram[i], c.ram))
            assert np.array_equal(canon[i], c.canon()), (f, i, "canon", _first_diff(canon[i], c.canon()))
            if render:
                assert np.array_equal(scr[i], c.screen), (f, i, "screen", _first_diff(scr[i], c.screen))
        if render and rgb:   # RGB24 screen (the raw-emulator workload's output): nes-py's palette of the oracle's
            rgb_gpu = gpu.screen_rgb.cpu().numpy()
            for i, c in enumerate(cpu):
                assert np.array_equal(rgb_gpu[i], pal[c.screen & 63]), (f, i, "rgb screen")
    assert gpu.bad_ops() == sum(c.bad_ops() for c in cpu)
    assert gpu.instructions() == sum(c.instructions() for c in cpu)


@pytest.mark.parametrize("cpw", CPW)
def test_raw_mini_smb(cpw, monkeypatch):
    _raw_run(MINI, 8, scaled(120), seed=1, rgb=True, cpw=cpw, monkeypatch=monkeypatch)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_raw_program_fuzz(seed):
    _raw_run(fuzz.program_rom(seed), 4, scaled(80), seed=seed, backup_p=0.05)


@pytest.mark.parametrize("cpw", CPW + ["4"])
def test_raw_program_fuzz_two_waves(cpw, monkeypatch):
    # 40 consoles; with 16 per wave two full waves and a partial one, so catch-ups that one lane forces on the
    # others of its wave (PPU register accesses at different points) are compared across many lanes
    _raw_run(fuzz.program_rom(3), 40, scaled(40), seed=3, backup_p=0.05, cpw=cpw, monkeypatch=monkeypatch)


@pytest.mark.parametrize("cpw", CPW)
@pytest.mark.parametrize("seed", [0, 1, 3])
def test_raw_screen_off_fuzz(seed, cpw, monkeypatch):
    # an NMI handler that makes its VRAM, scroll and address writes with rendering off (a bulk $2007 loop among
    # them) and turns rendering on at its end; 40 consoles: a console often runs alone in its wave (always, with
    # one console per wave) and its lone runs make those writes themselves
    _raw_run(fuzz.program_rom(seed, screen_off=True), 40, scaled(60), seed=seed, backup_p=0.05, cpw=cpw,
             monkeypatch=monkeypatch)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_raw_random_fuzz(seed):
    _raw_run(fuzz.random_rom(seed), 4, scaled(40), seed=seed, render_p=0.5, backup_p=0.05)


CONFIGS = {
    "default": dict(),
    "sticky_noop": dict(sticky=0.25, noop_max=30),
    "maxpool_sticky": dict(maxpool=True, sticky=0.25),
    "short_timelimit": dict(max_steps=60, noop_max=5),
    "headline": dict(sticky=0.25, noop_max=30, maxpool=True),
    # frame-skip edges of the early-termination re-emulation: which frames are snapshotted depends on K and
    # max-pool (K=1: none; K=2 max-pool: frame 0 only; K=3 without max-pool: frames 0 and 1; K=6: 0..3)
    "skip1_stack2": dict(skip=1, frame_stack=2, noop_max=3),
    "skip2_maxpool": dict(skip=2, maxpool=True, sticky=0.25, noop_max=3),
    "skip3_short": dict(skip=3, sticky=0.25, max_steps=80),
    "skip6_maxpool": dict(skip=6, maxpool=True, noop_max=4, sticky=0.5),
}
ACTION_P = [.05, .2, .25, .15, .25, .05, .05]
# Early-termination re-emulation kinds each configuration must exercise in _env_run (counted on the GPU and
# by the oracle, which must agree): "one" re-runs the last frame alone, "pair" its max-pool partner too, "k2"
# ends at frame K-2 under max-pool. K = 1 has no early termination; K = 2 has no pair.
EXPECT_REEMU = {
    "default": ("one",), "sticky_noop": ("one",), "maxpool_sticky": ("one", "pair", "k2"),
    "short_timelimit": ("one",), "headline": ("one", "pair"), "skip1_stack2": (),
    "skip2_maxpool": ("one", "k2"), "skip3_short": ("one",), "skip6_maxpool": ("one", "pair", "k2"),
}


def _levels(names):
    from fast_mario_env_amd import decode_level
    return [decode_level(x) for x in names]


@pytest.mark.parametrize("config", list(CONFIGS))
def test_env_vs_oracle(config):
    _env_run(["1-1", "1-1", "4-1", "8-4", "2-3", "1-2", "1-1", "5-2"], config, scaled(150))


def test_env_rom_modes_per_env():
    """A rom_mode per env (the divergence-stress workload's cycling over the four variants): every env against
    its own one-env oracle on its mode's ROM, with its own PCG64 stream (env_offset = its index)."""
    import torch

    from build_roms import MODES
    from fast_mario_env_amd import HipVecEnv
    kw = CONFIGS["headline"]
    names = ["1-1", "4-1", "1-1", "8-4", "2-3", "1-1", "1-2", "5-2"]
    n = len(names)
    modes = [MODES[i % len(MODES)] for i in range(n)]
    roms = {m: open(rom_path(m), "rb").read() for m in MODES}
    gpu = HipVecEnv(names, n, seed=7, rom=roms, rom_mode=modes, **kw)
    cpu = [OracleVec(roms[modes[i]], _levels([names[i]]), 1, seed=7, env_offset=i, **kw) for i in range(n)]
    o2 = gpu.reset().cpu().numpy()
    for i in range(n):
        assert np.array_equal(cpu[i].reset()[0], o2[i]), (i, "reset obs")
    rng = np.random.default_rng(131)
    for t in range(scaled(60)):
        a = rng.choice(7, n, p=ACTION_P)
        gpu.step(torch.from_numpy(a).cuda())
        o2, r2, te2, tr2, i2 = (x.cpu().numpy() for x in (gpu.obs, gpu.rew, gpu.term, gpu.trunc, gpu.info_t))
        ram = gpu.ram().cpu().numpy()
        for i in range(n):
            o1, r1, te1, tr1, i1 = cpu[i].step(a[i:i + 1])
            assert r1[0] == r2[i] and te1[0] == te2[i] and tr1[0] == tr2[i], (t, i, modes[i], "reward/done")
            assert np.array_equal(i1[0], i2[i]), (t, i, modes[i], "info")
            assert np.array_equal(cpu[i].ram(0), ram[i]), (t, i, modes[i], "ram")
            assert np.array_equal(o1[0], o2[i]), (t, i, modes[i], "obs")
    assert gpu.bad_ops() == 0


def test_env_vs_oracle_two_waves():
    # 40 envs (two full 16-env waves and a partial one) with the headline wrappers
    names = ["1-1", "4-1", "8-4", "2-3", "1-2", "5-2", "3-3", "7-1"] * 5
    _env_run(names, "headline", scaled(60))


def _env_run(names, config, steps):
    import torch

    from fast_mario_env_amd import HipVecEnv
    kw = CONFIGS[config]
    n = len(names)
    cpu = OracleVec(MINI, _levels(names), n, seed=7, **kw)
    gpu = HipVecEnv(names, n, seed=7, rom=MINI, **kw)
    o1 = cpu.reset().copy()
    o2 = gpu.reset().cpu().numpy()
    assert np.array_equal(o1, o2), "reset obs"
    assert np.array_equal(gpu.canon().cpu().numpy(), np.stack([cpu.canon(i) for i in range(n)])), "reset state"
    rng = np.random.default_rng(130)
    eps = 0
    for t in range(steps):
        a = rng.choice(7, n, p=ACTION_P)
        o1, r1, te1, tr1, i1 = cpu.step(a)
        o2, r2, te2, tr2, i2 = gpu.step(torch.from_numpy(a).cuda())
        o2, r2, te2, tr2, i2 = (x.cpu().numpy() for x in (o2, r2, te2, tr2, gpu.info_t))
        assert np.array_equal(r1, r2), (t, "reward", r1, r2)
        assert np.array_equal(te1, te2) and np.array_equal(tr1, tr2), (t, "done", te1, te2, tr1, tr2)
        assert np.array_equal(i1, i2), (t, "info", i1, i2)
        ram = gpu.ram().cpu().numpy()
        for i in range(n):
            assert np.array_equal(cpu.ram(i), ram[i]), (t, i, "ram", _first_diff(cpu.ram(i), ram[i]))
        assert np.array_equal(o1, o2), (t, "obs", np.argwhere(o1 != o2)[:5].tolist())
        done = te1 | tr1
        if done.any():
            fo = gpu.final_obs.cpu().numpy()
            epr, epl = gpu.ep_ret.cpu().numpy(), gpu.ep_len.cpu().numpy()
            for i in np.flatnonzero(done):
                eps += 1
                assert np.array_equal(cpu.fin[i], fo[i]), (t, i, "final_obs")
                assert cpu.ep_ret[i] == epr[i] and cpu.ep_len[i] == epl[i], (t, i, "episode")
    canon = gpu.canon().cpu().numpy()
    for i in range(n):
        assert np.array_equal(canon[i], cpu.canon(i)), (i, "final state", _first_diff(canon[i], cpu.canon(i)))
    assert gpu.frames == cpu.frames()
    assert gpu.bad_ops() == 0 and cpu.bad_ops() == 0
    assert gpu.instructions() == cpu.instructions()
    # the sprite-0 poll fast-forward (state-identical, so the counts above cannot show it) must have fired: the
    # synthetic game polls sprite 0 every frame of a level
    assert 0 < gpu.ff_instructions() < gpu.instructions()
    re_gpu, re_cpu = gpu.reemulations(), cpu.reemulations()
    assert re_gpu == re_cpu, (re_gpu, re_cpu)
    if steps >= 150:
        for kind in EXPECT_REEMU.get(config, ()):
            assert re_cpu[kind] > 0, (config, kind, re_cpu)
        if CONFIGS[config].get("skip") == 1:
            assert sum(re_cpu.values()) == 0
    if config == "short_timelimit":
        assert eps > 0


def test_hack_frames_redrawn_vs_oracle():
    """Busy runs after drawn agent frames (the player in a pipe / area transition while frames K-2 and K-1 are
    drawn): the HIP path runs such hack frames undrawn from a snapshot and runs the last one again drawn; the
    oracle draws every one, as the reference does. 512 envs of levels whose busy runs are common, right+jump
    with p = 0.5 (as in the divergence-stress workload), headline wrappers, every output every step. The
    oracle runs as 16 instances of 32 envs (their own PCG64 streams by env_offset) on a thread pool."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    import torch

    from fast_mario_env_amd import HipVecEnv
    kw = CONFIGS["headline"]
    names = ["4-4", "5-1"] * 256
    n, m = len(names), 32
    cpu = [OracleVec(MINI, _levels(names[k:k + m]), m, seed=3, env_offset=k, **kw) for k in range(0, n, m)]
    gpu = HipVecEnv(names, n, seed=3, rom=MINI, **kw)
    pool = ThreadPoolExecutor(min(16, os.cpu_count() or 1))
    o1 = np.concatenate([c.reset() for c in cpu])
    assert np.array_equal(o1, gpu.reset().cpu().numpy()), "reset obs"
    rng = np.random.default_rng(17)
    for t in range(scaled(240)):
        a = np.where(rng.random(n) < 0.5, 2, rng.integers(0, 7, n))
        outs = list(pool.map(lambda kc: [x.copy() for x in kc[1].step(a[kc[0]:kc[0] + m])], zip(range(0, n, m), cpu)))
        o1, r1, te1, tr1, i1 = (np.concatenate(z) for z in zip(*outs))
        o2, r2, te2, tr2, _ = gpu.step(torch.from_numpy(a).cuda())
        o2, r2, te2, tr2, i2 = (x.cpu().numpy() for x in (o2, r2, te2, tr2, gpu.info_t))
        assert np.array_equal(r1, r2) and np.array_equal(te1, te2) and np.array_equal(tr1, tr2), (t, "reward/done")
        assert np.array_equal(i1, i2), (t, "info")
        assert np.array_equal(o1, o2), (t, "obs", np.argwhere(o1 != o2)[:5].tolist())
    pool.shutdown()
    ram = gpu.ram().cpu().numpy()
    for i in range(n):
        assert np.array_equal(cpu[i // m].ram(i % m), ram[i]), (i, "ram")
    assert gpu.frames == sum(c.frames() for c in cpu)
    assert gpu.instructions() == sum(c.instructions() for c in cpu)
    assert gpu.bad_ops() == 0
    assert gpu.hack_redraws() > 0, "no busy run after a drawn frame: the redraw path was not exercised"


def test_env_2048_in_kernel_observations():
    """2,048 envs (128 waves) with the headline wrappers, every env every step against the oracle. k_step's waves
    take tickets in the order they finish their frame loops; the first 64 compute their envs' observations inside
    k_step (obs_tail after the frame loop, behind its release / acquire fences) and only the last 64 leave them
    to k_obs_late. With 64 waves or fewer every wave defers, so the smaller parity tests cover k_obs_late alone.
    The oracle runs as 16 instances of 128 envs (their own PCG64 streams by env_offset) on a thread pool."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    import torch

    from fast_mario_env_amd import HipVecEnv
    kw = CONFIGS["headline"]
    names = ["1-1", "4-1", "8-4", "2-3", "1-2", "5-2", "3-3", "7-1"] * 256
    n, m = len(names), 128
    assert n // 16 > 64      # waves of 16 envs beyond the 64 that defer
    pool = ThreadPoolExecutor(min(16, os.cpu_count() or 1))
    cpu = list(pool.map(lambda k: OracleVec(MINI, _levels(names[k:k + m]), m, seed=3, env_offset=k, **kw),
                        range(0, n, m)))
    gpu = HipVecEnv(names, n, seed=3, rom=MINI, **kw)
    o1 = np.concatenate(list(pool.map(lambda c: c.reset().copy(), cpu)))
    assert np.array_equal(o1, gpu.reset().cpu().numpy()), "reset obs"
    rng = np.random.default_rng(23)
    for t in range(scaled(60)):
        a = rng.integers(0, 7, n)
        outs = list(pool.map(lambda kc: [x.copy() for x in kc[1].step(a[kc[0]:kc[0] + m])], zip(range(0, n, m), cpu)))
        o1, r1, te1, tr1, i1 = (np.concatenate(z) for z in zip(*outs))
        o2, r2, te2, tr2, _ = gpu.step(torch.from_numpy(a).cuda())
        o2, r2, te2, tr2, i2 = (x.cpu().numpy() for x in (o2, r2, te2, tr2, gpu.info_t))
        assert np.array_equal(r1, r2) and np.array_equal(te1, te2) and np.array_equal(tr1, tr2), (t, "reward/done")
        assert np.array_equal(i1, i2), (t, "info")
        bad = np.flatnonzero((o1 != o2).reshape(n, -1).any(1))
        assert bad.size == 0, (t, "obs of envs", bad[:8].tolist())
    pool.shutdown()
    ram = gpu.ram().cpu().numpy()
    for i in range(n):
        assert np.array_equal(cpu[i // m].ram(i % m), ram[i]), (i, "ram")
    assert gpu.frames == sum(c.frames() for c in cpu)
    assert gpu.instructions() == sum(c.instructions() for c in cpu)
    assert gpu.bad_ops() == 0


def test_config1_golden_trace_on_gpu():
    """The CPU golden-trace workload (32 envs of 1-1, seed 0, no sticky / no-op / max-pool, actions from
    default_rng(0)) through the HIP path, against the digests the reference C++ wrote for all 1,000 steps
    (obs, reward, terminated, truncated, int64 info and every env's RAM) and the full arrays kept at steps
    0, 1, 10, 100 and 999."""
    import json

    import torch

    import make_golden as G
    from fast_mario_env_amd import HipVecEnv
    g = json.load(open(G.GOLDEN))["config1"]
    keep = np.load(G.CONFIG1)
    n = 32
    env = HipVecEnv("1-1", n, seed=0, rom=MINI)
    assert G.digest(env.reset().cpu().numpy()) == g["trace"][0]
    for t, a in enumerate(G.config1_actions()):
        obs, rew, term, trunc, _ = env.step(torch.from_numpy(np.asarray(a, np.int64)).cuda())
        obs, rew, term, trunc = (x.cpu().numpy() for x in (obs, rew, term, trunc))
        info = env.info_t.cpu().numpy().astype(np.int64)
        ram = env.ram().cpu().numpy()
        assert G.digest(obs, rew, term, trunc, info, ram) == g["trace"][t + 1], t
        if t in G.CONFIG1_KEEP:
            assert np.array_equal(obs, keep[f"obs_{t}"]) and np.array_equal(ram, keep[f"ram_{t}"]), t
            assert np.array_equal(info, keep[f"info_{t}"]) and np.array_equal(rew, keep[f"rew_{t}"]), t
    assert env.frames == g["frames"] and env.bad_ops() == g["bad_ops"] == 0
