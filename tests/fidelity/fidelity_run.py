"""GPU-vs-oracle fidelity record at the reference's own scale: all 32 levels x 16 envs (512 envs), 1,500 steps per
configuration, every env compared at every step (test infrastructure; the product path is the HIP library).

    python tests/fidelity/fidelity_run.py [--steps 1500] [--out tests/fidelity/env_fidelity.jsonl]

The reference publishes the same shape for its CUDA backend against its CPU one (512 envs x 1,500 steps x 3
configurations, benchmarks/results/cuda_fidelity.jsonl:1-3). Here HipVecEnv runs the 512 envs on the GPU and the
CPU checker (oracle/liboracle.so, the restatement pinned against the reference's golden traces) runs them as 16
instances of 32 envs on their own PCG64 streams (env_offset), on a thread pool. Per step and env: observation
stack, reward, terminated, truncated, the ten info values and the 2 KB of RAM; at every episode end the final
observation stack and the episode return and length; at the end the whole console state, the frame,
instruction and bad-opcode counts and the early-termination re-emulations. One JSON line per configuration:
episodes, flag clears, the largest x_pos, mismatches (the first ones, with step and env) and the run time.
Actions: over the 7 SIMPLE_MOVEMENT actions from default_rng(2024 + configuration index), uniform except for the
"runner" configuration (POLICY), which reaches the flagpole; the ROM is the repository's synthetic stand-in
(tests/golden/roms), the only one this environment has.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "fast-mario-env_amd"), os.path.join(ROOT, "tests"),
          os.path.join(ROOT, "tests", "golden", "roms")):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

from build_roms import rom_path  # noqa: E402
from cpu_libs import OracleVec  # noqa: E402

# the reference's three CUDA-fidelity configurations (cuda_fidelity.jsonl) and the headline wrappers
CONFIGS = {
    "default": dict(),
    "sticky_noop": dict(sticky=0.25, noop_max=30),
    "short_timelimit": dict(max_steps=60, noop_max=5),
    "headline": dict(sticky=0.25, noop_max=30, maxpool=True),
    "runner": dict(sticky=0.25, noop_max=30, maxpool=True),
}
# Action probabilities per configuration (default: uniform). The runner mostly runs right and jumps, which reaches
# the flagpole at the level end (random play never does, as in the reference's random-action runs).
POLICY = {"runner": [0.02, 0.13, 0.25, 0.2, 0.35, 0.03, 0.02]}
I_X, I_FLAG = 0, 1     # info columns: x_pos, flag_get
M = 32                 # envs per oracle instance


def run(config, steps, seed, log):
    import torch

    from fast_mario_env_amd import ALL_LEVELS, HipVecEnv, decode_level
    kw = CONFIGS[config]
    names = [lv for lv in ALL_LEVELS for _ in range(16)]
    n = len(names)
    rom = open(rom_path("vanilla"), "rb").read()
    pool = ThreadPoolExecutor(16)
    cpu = list(pool.map(lambda k: OracleVec(rom, [decode_level(x) for x in names[k:k + M]], M, seed=seed,
                                            env_offset=k, **kw), range(0, n, M)))
    gpu = HipVecEnv(names, n, seed=seed, rom=rom, **kw)
    t0 = time.perf_counter()
    mism = []

    def miss(t, what, envs):
        if len(mism) < 20:
            mism.append({"step": t, "what": what, "envs": [int(e) for e in np.asarray(envs).reshape(-1)[:8]]})

    o1 = np.concatenate(list(pool.map(lambda c: c.reset().copy(), cpu)))
    o2 = gpu.reset().cpu().numpy()
    if not np.array_equal(o1, o2):
        miss(-1, "reset obs", np.flatnonzero((o1 != o2).reshape(n, -1).any(1)))
    rng = np.random.default_rng(2024 + list(CONFIGS).index(config))
    episodes = flags = 0
    max_x = 0

    def cpu_step(kc):
        k, c = kc
        o, r, te, tr, inf = c.step(a[k:k + M])
        ram = np.stack([c.ram(i) for i in range(M)])
        return o.copy(), r.copy(), te.copy(), tr.copy(), inf.copy(), ram, c.fin.copy(), c.ep_ret.copy(), c.ep_len.copy()

    for t in range(steps):
        a = rng.choice(7, n, p=POLICY[config]) if config in POLICY else rng.integers(0, 7, n)
        outs = list(pool.map(cpu_step, zip(range(0, n, M), cpu)))
        o1, r1, te1, tr1, i1, ram1, fin1, epr1, epl1 = (np.concatenate(z) for z in zip(*outs))
        o2, r2, te2, tr2, _ = gpu.step(torch.from_numpy(a).cuda())
        o2, r2, te2, tr2, i2, ram2 = (x.cpu().numpy() for x in (o2, r2, te2, tr2, gpu.info_t, gpu.ram()))
        for what, x, y in (("reward", r1, r2), ("terminated", te1, te2), ("truncated", tr1, tr2)):
            if not np.array_equal(x, y):
                miss(t, what, np.flatnonzero(x != y))
        if not np.array_equal(i1, i2):
            miss(t, "info", np.flatnonzero((i1 != i2).any(1)))
        if not np.array_equal(ram1, ram2):
            miss(t, "ram", np.flatnonzero((ram1 != ram2).any(1)))
        if not np.array_equal(o1, o2):
            miss(t, "obs", np.flatnonzero((o1 != o2).reshape(n, -1).any(1)))
        done = np.flatnonzero(te1.astype(bool) | tr1.astype(bool))
        if done.size:
            fo, epr, epl = (x.cpu().numpy() for x in (gpu.final_obs, gpu.ep_ret, gpu.ep_len))
            if not np.array_equal(fin1[done], fo[done]):
                miss(t, "final_obs", done)
            if not (np.array_equal(epr1[done], epr[done]) and np.array_equal(epl1[done], epl[done])):
                miss(t, "episode return / length", done)
            episodes += int(done.size)
            flags += int((i1[done, I_FLAG] != 0).sum())
        max_x = max(max_x, int(i1[:, I_X].max()))
        if (t + 1) % 100 == 0:
            log(f"[fidelity] {config} step {t + 1}/{steps}: {episodes} episodes, {len(mism)} mismatches, "
                f"{time.perf_counter() - t0:.0f} s")
    canon = gpu.canon().cpu().numpy()
    bad_state = [i for i in range(n) if not np.array_equal(canon[i], cpu[i // M].canon(i % M))]
    if bad_state:
        miss(steps, "final console state", bad_state)
    frames_c = sum(c.frames() for c in cpu)
    instr_c = sum(c.instructions() for c in cpu)
    bad_c = sum(c.bad_ops() for c in cpu)
    re_c = {}
    for c in cpu:
        for k, v in c.reemulations().items():
            re_c[k] = re_c.get(k, 0) + v
    if gpu.frames != frames_c:
        miss(steps, "frames", [])
    if gpu.instructions() != instr_c:
        miss(steps, "instructions", [])
    if gpu.reemulations() != re_c:
        miss(steps, "re-emulations", [])
    rec = {"config": config, "wrappers": kw, "policy": POLICY.get(config, "uniform"),
           "level": "32 levels x 16 envs: " + ",".join(ALL_LEVELS), "n": n,
           "steps": steps, "seed": seed, "episodes": episodes, "flags": flags, "max_x": max_x,
           "frames": int(gpu.frames), "instructions": int(gpu.instructions()),
           "ff_instructions": int(gpu.ff_instructions()), "reemulations": re_c,
           "bad_ops": int(gpu.bad_ops()), "oracle_bad_ops": int(bad_c), "mismatches": mism, "ok": not mism,
           "rom": "synthetic stand-in (tests/golden/roms, vanilla)", "secs": round(time.perf_counter() - t0, 1)}
    pool.shutdown()
    for c in cpu:
        c.close()
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=1500)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--configs", default=",".join(CONFIGS))
    ap.add_argument("--out", default=os.path.join(HERE, "env_fidelity.jsonl"))
    args = ap.parse_args()
    log = lambda m: print(m, flush=True)  # noqa: E731
    recs = []
    for config in args.configs.split(","):
        rec = run(config, args.steps, args.seed, log)
        log(json.dumps({k: v for k, v in rec.items() if k != "level"}))
        recs.append(rec)
    with open(args.out, "w") as f:
        for rec in recs:
            f.write(json.dumps(rec) + "\n")
    sys.exit(0 if all(r["ok"] for r in recs) else 1)


if __name__ == "__main__":
    main()
