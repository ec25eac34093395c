"""GPU parity at the benchmark workloads' real sizes.

The small parity tests fit in one workgroup (128 env slots). These run many:
- the headline configuration exactly as bench.py measures it: 32,768 envs of 1-1 (2,048 waves in 256 workgroups of
  8 waves, the benchmark's launch shape), max-pool, bench.py's own action stream over its 300 preroll steps and its
  default warm-up and timed window (405 steps);
- 4,096 envs of mixed levels with the headline wrappers (the launch shrinks to 256 one-wave workgroups, one per CU);
- the 65,536-env divergence-stress instance (512 workgroups of 8 waves; its second frame buffer starts 4.03e9
  bytes in and ends past 2^33);
- 4,096 raw consoles over 800 frames, past the point where the consoles run out of phase.
The outputs are recorded on the device; a sample of envs (a fixed stride, the last env, and envs whose episodes
ended, which take the reset, final_obs and re-emulation paths) is then replayed by one-env CPU oracles on the
sampled env's own PCG64 stream (env_offset = its index, as the reference's env_offset equivalence allows,
env.py:155-156), bit for bit, on a thread pool. Every env is also checked against size-independent properties: the
frame-stack shift and reset stack of k_stack, final_obs, and zero bad ops.
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from build_roms import MODES, rom_path
from cpu_libs import OracleRaw, OracleVec

pytestmark = pytest.mark.gpu

ROMS = {m: open(rom_path(m), "rb").read() for m in MODES}
HEADLINE = dict(sticky=0.25, noop_max=30, skip=4, maxpool=True, frame_stack=4, max_steps=2000)
STRESS = dict(sticky=0.25, noop_max=30, skip=4, maxpool=False, frame_stack=4, max_steps=2000)


def _levels(names):
    from fast_mario_env_amd import decode_level
    return [decode_level(x) for x in names]


def _first_diff(a, b):
    d = np.flatnonzero(np.asarray(a).reshape(-1) != np.asarray(b).reshape(-1))
    return d[:8].tolist()


def _record(env, actions, keep=None):
    """Reset, then step every row of `actions` (T, N) on the device. Checks k_stack's invariants on every env as
    it goes (the stack shifts by one frame; a finished episode's final_obs is the shifted stack plus the last
    frame, and its new stack is [0, ..., 0, reset frame]) and keeps the outputs of the envs `keep` (all if
    None) on the device, plus every env's done flags."""
    idx = None if keep is None else torch.as_tensor(keep, dtype=torch.long, device=env.dev)
    rows = (lambda x: x) if idx is None else (lambda x: x[idx])
    prev = env.reset().clone()
    rec = {"obs0": rows(prev).clone(), "canon0": rows(env.canon()), "done": []}
    keys = ("obs", "rew", "term", "trunc", "info", "ram", "fin", "ep_ret", "ep_len")
    for k in keys:
        rec[k] = []
    for t, a in enumerate(actions):
        obs, rew, term, trunc, _ = env.step(a)
        done = term | trunc
        live = ~done
        assert torch.equal(obs[live][:, :-1], prev[live][:, 1:]), (t, "stack shift")
        if done.any():
            assert torch.equal(env.final_obs[done][:, :-1], prev[done][:, 1:]), (t, "final_obs shift")
            assert not obs[done][:, :-1].any(), (t, "reset stack")
        prev.copy_(obs)
        rec["done"].append(done.clone())
        rec["obs"].append(rows(obs).clone())
        rec["rew"].append(rows(rew).clone())
        rec["term"].append(rows(term).clone())
        rec["trunc"].append(rows(trunc).clone())
        rec["info"].append(rows(env.info_t).clone())
        rec["ram"].append(rows(env.ram()))
        # final_obs / episode stats are valid only where the episode ended
        d = rows(done)
        rec["fin"].append(torch.where(d[:, None, None, None], rows(env.final_obs), 0))
        rec["ep_ret"].append(torch.where(d, rows(env.ep_ret), 0))
        rec["ep_len"].append(torch.where(d, rows(env.ep_len), 0))
    torch.cuda.synchronize()
    return rec


def _sample(n, stride, done_steps, extra):
    done_any = torch.stack(done_steps).any(0).cpu().numpy()
    picks = set(range(0, n, stride)) | {n - 1}
    done_idx = np.flatnonzero(done_any)
    picks |= set(done_idx[np.linspace(0, len(done_idx) - 1, min(extra, len(done_idx))).astype(int)].tolist()) \
        if len(done_idx) else set()
    return sorted(picks), int(done_any.sum())


def _replay_one(j, i, host, obs0, canon0, names, modes, kw, seed, acts):
    """Env i (row j of the recorded outputs) against a one-env oracle on its own PCG64 stream; returns the number
    of episodes it ended."""
    eps = 0
    cpu = OracleVec(ROMS[modes[i]], _levels([names[i]]), 1, seed=seed, env_offset=i, **kw)
    assert np.array_equal(cpu.reset()[0], obs0[j]), (i, "reset obs")
    assert np.array_equal(cpu.canon(0), canon0[j]), (i, "reset state", _first_diff(cpu.canon(0), canon0[j]))
    for t in range(len(acts)):
        o, r, te, tr, inf = cpu.step(acts[t, i:i + 1])
        assert r[0] == host["rew"][t][j] and te[0] == host["term"][t][j] and tr[0] == host["trunc"][t][j], \
            (t, i, "reward/done", r[0], host["rew"][t][j])
        assert np.array_equal(inf[0], host["info"][t][j]), (t, i, "info", inf[0], host["info"][t][j])
        assert np.array_equal(cpu.ram(0), host["ram"][t][j]), (t, i, "ram", _first_diff(cpu.ram(0), host["ram"][t][j]))
        assert np.array_equal(o[0], host["obs"][t][j]), (t, i, "obs", _first_diff(o[0], host["obs"][t][j]))
        if te[0] or tr[0]:
            eps += 1
            assert np.array_equal(cpu.fin[0], host["fin"][t][j]), (t, i, "final_obs")
            assert cpu.ep_ret[0] == host["ep_ret"][t][j] and cpu.ep_len[0] == host["ep_len"][t][j], (t, i, "episode")
    assert cpu.bad_ops() == 0
    cpu.close()
    return eps


def _replay_samples(rec, samples, names, modes, kw, seed, actions):
    """rec holds the outputs of exactly the envs `samples`, in that order. The one-env oracles run on a thread
    pool (ctypes releases the GIL inside each step)."""
    acts = actions.cpu().numpy()
    host = {k: [x.cpu().numpy() for x in rec[k]] for k in
            ("obs", "rew", "term", "trunc", "info", "ram", "fin", "ep_ret", "ep_len")}
    obs0 = rec["obs0"].cpu().numpy()
    canon0 = rec["canon0"].cpu().numpy()
    with ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as pool:
        futs = [pool.submit(_replay_one, j, i, host, obs0, canon0, names, modes, kw, seed, acts)
                for j, i in enumerate(samples)]
        return sum(f.result() for f in futs)


def _run(names, modes, kw, seed, actions, stride, extra, two_pass=False, counters=False):
    """Run the GPU instance, pick the samples (a stride, the last env, envs whose episodes ended) and replay them
    on the CPU. With two_pass, a first run only finds the samples and a second, identical instance records
    just their outputs (the device then holds a few envs' outputs per step instead of every env's)."""
    from fast_mario_env_amd import HipVecEnv
    n = len(names)
    rom = {m: ROMS[m] for m in set(modes)}

    def make():
        return HipVecEnv(names, n, seed=seed, rom=rom, rom_mode=modes, device="cuda:0", **kw)
    env = make()
    print(f"scale run: {n} envs, {len(actions)} steps", flush=True)
    rec = _record(env, actions, keep=[] if two_pass else None)
    assert env.bad_ops() == 0
    samples, n_done = _sample(n, stride, rec["done"], extra)
    if two_pass:
        env.close()
        del rec
        env = make()
        rec = _record(env, actions, keep=samples)
        assert env.bad_ops() == 0
    else:
        idx = torch.as_tensor(samples, device="cuda:0")
        rec = {k: (v[idx] if k in ("obs0", "canon0") else [x[idx] for x in v]) if k != "done" else v
               for k, v in rec.items()}
    print(f"  {n_done} envs ended an episode; replaying {len(samples)} sampled envs on the CPU", flush=True)
    eps = _replay_samples(rec, samples, names, modes, kw, seed, actions)
    re = env.reemulations()
    counts = {"instructions": env.instructions(), "ff_instructions": env.ff_instructions()}
    env.close()
    return (n_done, eps, re, counts) if counters else (n_done, eps, re)


def test_headline_4096_envs_mixed_levels():
    """Headline wrappers (sticky 0.25, no-op 30, skip 4, max-pool) at 4,096 envs, levels mixed: the launch shrinks to
    256 one-wave workgroups (one per CU), and the last 64 waves leave their observations to k_obs_late."""
    from fast_mario_env_amd import ALL_LEVELS
    n, T = 4096, 50
    lv = np.random.default_rng(11).integers(0, 32, n)
    names = [ALL_LEVELS[k] for k in lv]
    g = torch.Generator(device="cuda:0").manual_seed(5)
    actions = torch.randint(0, 7, (T, n), generator=g, device="cuda:0")
    n_done, eps, re = _run(names, ["vanilla"] * n, HEADLINE, 0, actions, stride=61, extra=24)
    assert n_done > 0 and eps > 0
    assert re["one"] > 0 and re["pair"] > 0 and re["k2"] > 0, re


def test_divergence_stress_65536_envs():
    """The divergence-stress instance at its full size: 65,536 envs, levels drawn from default_rng(7) over the 32
    world-stage pairs, rom_mode cycled over the four variants per env, sticky 0.25, no-op 30, skip 4, no
    max-pool; per env, action 2 (right + A) with p = 0.5, else uniform over 0..6. 330 steps: as far as bench.py's
    stress line (300 preroll steps, then its warm-up and timed window), where busy runs in one env of a wave set the
    kernel's time."""
    from fast_mario_env_amd import ALL_LEVELS
    n, T = 65536, 330
    lv = np.random.default_rng(7).integers(0, 32, n)
    names = [ALL_LEVELS[k] for k in lv]
    modes = [MODES[i % 4] for i in range(n)]
    rng = np.random.default_rng(3)
    acts = np.where(rng.random((T, n)) < 0.5, 2, rng.integers(0, 7, (T, n)))
    actions = torch.from_numpy(acts).to("cuda:0")
    n_done, eps, re = _run(names, modes, STRESS, 0, actions, stride=1021, extra=24, two_pass=True)
    assert n_done > 1000 and eps >= 24, (n_done, eps)
    assert re["one"] > 0, re


def test_ordered_launch_40960_envs_every_env_vs_oracle():
    """Past 32,768 envs on 256 CUs k_step has more blocks than CUs, and each step launches its block groups in the
    order k_work and k_order derive from the last step's work (k_step_ordered): 40,960 envs (320 groups) of mixed
    levels, every env's observation, reward, done flags and info against 16 oracle instances each step, so a group
    that ran twice or not at all in a step would show."""
    from fast_mario_env_amd import ALL_LEVELS, HipVecEnv
    n, T, m = 40960, 6, 2560
    lv = np.random.default_rng(13).integers(0, 32, n)
    names = [ALL_LEVELS[k] for k in lv]
    gpu = HipVecEnv(names, n, seed=2, rom=ROMS["vanilla"], device="cuda:0", **HEADLINE)
    pool = ThreadPoolExecutor(min(16, os.cpu_count() or 1))
    cpu = list(pool.map(lambda k: OracleVec(ROMS["vanilla"], _levels(names[k:k + m]), m, seed=2, env_offset=k,
                                            **HEADLINE), range(0, n, m)))
    o1 = np.concatenate(list(pool.map(lambda c: c.reset().copy(), cpu)))
    assert np.array_equal(o1, gpu.reset().cpu().numpy()), "reset obs"
    rng = np.random.default_rng(29)
    for t in range(T):
        a = np.where(rng.random(n) < 0.5, 2, rng.integers(0, 7, n))
        outs = list(pool.map(lambda kc: [x.copy() for x in kc[1].step(a[kc[0]:kc[0] + m])], zip(range(0, n, m), cpu)))
        o1, r1, te1, tr1, i1 = (np.concatenate(z) for z in zip(*outs))
        o2, r2, te2, tr2, _ = gpu.step(torch.from_numpy(a).to("cuda:0"))
        o2, r2, te2, tr2, i2 = (x.cpu().numpy() for x in (o2, r2, te2, tr2, gpu.info_t))
        assert np.array_equal(r1, r2) and np.array_equal(te1, te2) and np.array_equal(tr1, tr2), (t, "reward/done")
        assert np.array_equal(i1, i2), (t, "info", np.flatnonzero((i1 != i2).any(1))[:8].tolist())
        bad = np.flatnonzero((o1 != o2).reshape(n, -1).any(1))
        assert bad.size == 0, (t, "obs of envs", bad[:8].tolist())
    pool.shutdown()
    assert gpu.frames == sum(c.frames() for c in cpu)
    assert gpu.instructions() == sum(c.instructions() for c in cpu)
    assert gpu.bad_ops() == 0
    gpu.close()


def test_headline_32768_envs_bench_stream():
    """The measured configuration itself: 32,768 envs of 1-1 with the headline wrappers (sticky 0.25, no-op 30,
    skip 4, max-pool, stack 4, seed 0), launched as bench.py launches it (2,048 waves in 256 workgroups of 8 waves,
    two waves per SIMD), driven by bench.py's own action stream for its 300 preroll steps and its default warm-up
    and timed window (5 + 100 steps), so the steady state that the benchmark times is compared too. Two passes:
    the first finds the envs whose episodes ended, the second records a sample (every 1,021st env, the last one,
    24 envs with episode ends), replayed by one-env oracles."""
    from bench import headline_actions
    n, preroll, timed = 32768, 300, 105
    pre, acts = headline_actions(n, preroll, timed)
    actions = torch.cat([pre, acts])
    del pre, acts
    n_done, eps, re, counts = _run(["1-1"] * n, ["vanilla"] * n, HEADLINE, 0, actions, stride=1021, extra=24,
                                   two_pass=True, counters=True)
    assert n_done > 1000 and eps >= 24, (n_done, eps)
    assert re["one"] > 0 and re["pair"] > 0 and re["k2"] > 0, re
    # the sprite-0 poll fast-forward carries a large share of the retired instructions at this workload
    assert 0.2 * counts["instructions"] < counts["ff_instructions"] < counts["instructions"], counts


def _raw_frames(n, prologue, frames):
    """The raw-emulator workload's button bytes per frame: a Start/none prologue that enters 1-1, then
    SIMPLE_MOVEMENT buttons drawn per console and frame from default_rng(1) as one (frames, n) draw, as bench.py
    draws them (its warm-up and timed frames are the first rows)."""
    buttons_tab = np.array([0x00, 0x80, 0x81, 0x82, 0x83, 0x01, 0x40], np.uint8)
    sched = [np.full(n, 8 if f % 2 == 0 else 0, np.uint8) for f in range(prologue)]
    draws = np.random.default_rng(1).integers(0, 7, (frames, n))
    return sched + [buttons_tab[d] for d in draws]


def test_raw_4096_consoles():
    """Raw consoles at 4,096 (the raw-emulator workload's size), every frame rendered, over 800 frames: past
    frame ~200 the consoles run out of phase (deaths, level reloads and game-over screens at different points of
    a frame), which is where long single-console instruction runs set the launch's length. Sampled consoles
    against one CPU console each, every frame: RAM, palette screen and the whole machine state; the RGB24 screen
    every 10th frame."""
    from fast_mario_env_amd import HipRawNES, palette_rgb
    n, prologue, frames = 4096, 40, 760
    sched = _raw_frames(n, prologue, frames)
    gpu = HipRawNES(ROMS["vanilla"], n)
    samples = sorted(set(range(0, n, 61)) | {n - 1})
    cpu = [OracleRaw(ROMS["vanilla"]) for _ in samples]
    pal = palette_rgb()
    idx = torch.tensor(samples, device="cuda:0")
    sel = np.array(samples)
    pool = ThreadPoolExecutor(min(16, os.cpu_count() or 1))
    print(f"raw run: {n} consoles, {len(sched)} frames, {len(samples)} sampled", flush=True)
    for f, b in enumerate(sched):
        gpu.frame(torch.from_numpy(b), True)
        list(pool.map(lambda jc: jc[1].frame(int(b[sel[jc[0]]]), True), enumerate(cpu)))
        ram = gpu.ram[idx].cpu().numpy()
        scr = gpu.screen[idx].cpu().numpy()
        canon = gpu.canon()[idx].cpu().numpy()
        c_ram = np.stack([c.ram for c in cpu])
        c_scr = np.stack([c.screen for c in cpu])
        c_canon = np.stack([c.canon() for c in cpu])
        for what, g_, c_ in (("ram", ram, c_ram), ("screen", scr, c_scr), ("state", canon, c_canon)):
            if not np.array_equal(g_, c_):
                j = int(np.flatnonzero((g_ != c_).reshape(len(samples), -1).any(1))[0])
                raise AssertionError((f, samples[j], what, _first_diff(g_[j], c_[j])))
        if f % 10 == 9:
            rgb = gpu.screen_rgb[idx].cpu().numpy()
            assert np.array_equal(rgb, pal[c_scr & 63]), (f, "rgb screen")
        if f % 200 == 199:
            print(f"  frame {f + 1}/{len(sched)}", flush=True)
    pool.shutdown()
    assert gpu.bad_ops() == 0
    assert sum(c.instructions() for c in cpu) > 0
