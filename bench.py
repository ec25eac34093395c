#!/usr/bin/env python
"""Headline benchmark: batched Super Mario Bros agent steps on one MI355X (the full wrapper stack at 32768 envs).

    python bench.py [--steps K] [--warmup W] [--envs N] [--gpus 1]

Workload: N = 32768 envs on level 1-1, sticky 0.25, no-op starts up to 30, skip 4, 2-frame max-pool,
gray + INTER_AREA 84x84, frame stack 4, time limit 2000, auto-reset, seed 0 (env i: PCG64 stream i);
actions uniform in {0..6}, pre-generated on the device from torch.Generator seed 0. The ROM is the
real one when the reference's lookup finds it, else this repository's synthetic NROM stand-in
(tests/golden/roms/mini_smb_vanilla.nes); the JSON line names which.

One step = mh_step_async (k_step, k_obs, k_reset, k_stack) on torch's current stream;
inputs are resident in HBM. K steps are timed between two device synchronizations after W warm-up
steps. Stage times come from HIP events recorded on the same stream. The reference C++ FastVecEnv
(oracle/_ref, the checker build of the reference) is timed on the host cores on a bounded sample of
the same workload and reported beside the GPU number.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "fast-mario-env_amd"), os.path.join(ROOT, "tests"),
           os.path.join(ROOT, "tests", "golden", "roms")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "agent env-steps/sec (skip=4) at 32768 envs on 1 MI355X; % HBM/VALU roofline"
HBM_PEAK_GBS = 8000.0
# bytes k_step must move per env and agent step: console state read + write,
# env words read + write, action, reward / term / trunc / info out; ep stats on episode end.
STATE_BYTES = 4384 + 4 * 41
ENV_WORD_BYTES = 4 * 30
K_STEP_BYTES = 2 * STATE_BYTES + 2 * ENV_WORD_BYTES + 8 + 4 + 1 + 1 + 40
K_STEP_DONE_BYTES = 12
OBS = 84 * 84


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def pick_rom():
    from fast_mario_env_amd import RomNotFoundError, load_rom
    try:
        data = load_rom()
        return data, "super-mario-bros.nes (real ROM)"
    except (RomNotFoundError, ValueError):
        from build_roms import rom_path
        path = rom_path("vanilla")
        return open(path, "rb").read(), "mini_smb_vanilla.nes (synthetic NROM stand-in; no SMB ROM on this machine)"


def profile_values(name, workload_key):
    """`- key: value` lines of a committed rocprofv3 summary under profiles/, if it covers this workload."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.isfile(path):
        return {}
    vals = {}
    for line in open(path):
        if ":" in line and line.strip().startswith("-"):
            k, v = line.strip("- \n").split(":", 1)
            vals[k.strip()] = v.strip()
    wl = vals.get("workload", "").split(";")[0].strip()
    return vals if wl == workload_key else {}


def traffic_from_profiles(workload_key):
    """HBM bytes per k_step launch from the committed rocprofv3 --pmc summary, if one exists for this workload."""
    try:
        return float(profile_values("k_step_pmc_traffic.md", workload_key)["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def valu_issue_from_profiles(workload_key):
    """k_step's VALU issue fraction from the committed rocprofv3 SQ-counter summary, if one exists."""
    try:
        return float(profile_values("k_step_sq_counters_headline.md", workload_key)["valu_issue_fraction"])
    except (KeyError, ValueError):
        return None


def cpu_baseline(rom, seconds):
    """The reference C++ thread pool (oracle/_ref) on the host cores, headline settings, bounded sample."""
    import numpy as np

    from cpu_libs import OracleVec, RefVec, have_ref
    from fast_mario_env_amd import decode_level
    cores = os.cpu_count() or 1
    n = max(256, 32 * cores)
    kw = dict(seed=0, sticky=0.25, noop_max=30, skip=4, maxpool=True, frame_stack=4, max_steps=2000)
    lv = [decode_level("1-1")] * n
    if have_ref():
        env, kind, threads = RefVec(rom, lv, n, n_threads=cores, **kw), "reference", cores
    else:
        n = 64
        env, kind, threads = OracleVec(rom, [decode_level("1-1")] * n, n, **kw), "port", 1
    env.reset()
    rng = np.random.default_rng(0)
    for _ in range(3):
        env.step(rng.integers(0, 7, n))
    steps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        env.step(rng.integers(0, 7, n))
        steps += 1
    dt = time.perf_counter() - t0
    env.close()
    try:
        load1 = os.getloadavg()[0]
    except OSError:
        load1 = None
    model = ""
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {"value": round(n * steps / dt, 1), "unit": "agent-steps/s", "cores": threads, "kind": kind,
            "sample": f"{n} envs x {steps} timed steps after 3 warm-up steps ({dt:.1f} s), level 1-1, headline "
                      f"wrapper settings; {model}; load1 {load1}"}


def run_ppo(args, rom, rom_name, rom_sha):
    """PPO rollout workload (config 5): the headline envs feeding a random-init bf16 Nature CNN, Gumbel-max
    actions from seed 3, 128-step rollouts with frame-deduplicated storage and GAE (0.99, 0.95)."""
    import torch

    from fast_mario_env_amd import HipVecEnv
    from fast_mario_env_amd.rollout import Rollout, make_net
    n, T = args.envs, args.ppo_steps
    env = HipVecEnv("1-1", n, seed=0, sticky=0.25, noop_max=30, max_steps=2000, skip=4, frame_stack=4,
                    maxpool=True, rom=rom, device="cuda:0")
    env.reset()
    net = make_net(seed=0)
    warm = Rollout(env, net, T=4, seed=3)
    warm.collect()
    warm.advantages()
    del warm
    ro = Rollout(env, net, T=T, seed=3)
    torch.cuda.synchronize()
    log(f"PPO rollout: {n} envs x {T} steps")
    t0 = time.perf_counter()
    env_ms = ro.collect()
    adv, ret = ro.advantages()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    out = {
        "metric": "end-to-end env-steps/sec of a PPO rollout (bf16 Nature CNN policy) at 32768 envs on 1 MI355X",
        "value": round(n * T / dt, 1), "unit": "env-steps/s", "n_gpus": 1, "steps": T, "warmup": 4,
        "ms_per_step": round(dt * 1e3 / T, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8 env / bf16 policy", "data": "synthetic",
        "config": {"workload": "ppo rollout: headline envs + Nature CNN, 128-step rollouts", "envs": n,
                   "rollout_steps": T, "rom": rom_name, "rom_sha1": rom_sha, "policy": "Nature CNN, random init, bf16",
                   "sampling": "Gumbel-max, torch.Generator seed 3", "gae": [0.99, 0.95],
                   "storage": "newest frame per step (frame-deduplicated)"},
        "env_share": round(env_ms / (dt * 1e3), 4), "env_ms_per_step": round(env_ms / T, 3),
        "rollout_storage_gb": round(ro.frames.numel() / 1e9, 2),
    }
    env.close()
    print(json.dumps(out), flush=True)


def run_replay(args, rom, rom_name, rom_sha):
    """Replay workload (the GPU FrameReplay): the headline envs' transitions added to a 64-slot ring per env,
    then batches of 4096 3-step transitions sampled. Kernel times come from HIP events on the stream the
    kernels run on; the rooflines count the bytes each kernel must move."""
    import torch

    from fast_mario_env_amd import HipVecEnv
    from fast_mario_env_amd.replay import FrameReplay
    n, C, B, ns, reps = args.envs, 64, 4096, 3, 20
    env = HipVecEnv("1-1", n, seed=0, sticky=0.25, noop_max=30, max_steps=2000, skip=4, frame_stack=4,
                    maxpool=True, rom=rom, device="cuda:0")
    rb = FrameReplay(C, n, 4, device="cuda:0", seed=0)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0)
    obs = env.reset().clone()
    add_ms, news = [], 0
    log(f"replay: {n} envs, ring of {C} slots per env ({rb.nbytes() / 1e9:.1f} GB)")
    for t in range(C + reps):                      # fill past one wrap of the ring, time the last `reps` adds
        a = torch.randint(0, 7, (n,), generator=g, device="cuda:0")
        o2, r, te, tr, _ = env.step(a)
        d = te | tr
        nxt = torch.where(d[:, None, None, None], env.final_obs, o2)
        if t >= C:
            news += int(rb._new_ep.sum())
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        rb.add(obs, nxt, a, r, d, tr & ~te)
        if t >= C:
            e1.record()
            add_ms.append((e0, e1))
        obs = o2.clone()
    torch.cuda.synchronize()
    add_t = sum(x.elapsed_time(y) for x, y in add_ms) / reps
    env.close()
    rb.sample(B, ns, 0.99)                         # warm-up
    torch.cuda.synchronize()
    gat, draw_t = [], 0.0
    t0 = time.perf_counter()
    for _ in range(reps):
        d0 = time.perf_counter()
        e, p = rb.draw(B, ns)
        torch.cuda.synchronize()
        draw_t += time.perf_counter() - d0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        rb.gather(e, p, ns, 0.99)
        e1.record()
        gat.append((e0, e1))
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    gat_t = sum(x.elapsed_time(y) for x, y in gat) / reps
    rb.check_errors()
    fb = 84 * 84
    # add: the newest next_obs frame read and written per env, the obs frame too for envs starting an
    # episode, and 16 B of slot metadata; gather: 2k frames read and written per sample plus its metadata
    add_bytes = n * (2 * fb + 16) + (news / reps) * 2 * fb
    gat_bytes = B * (2 * 4 * 2 * fb + ns * 6 + 2 + 40)
    out = {
        "metric": "replay: sampled 3-step transitions/sec (batch 4096) from a 64-slot-per-env ring at 32768 envs on 1 MI355X",
        "value": round(B * reps / dt, 1), "unit": "transitions/s", "n_gpus": 1, "steps": reps, "warmup": C,
        "ms_per_step": round(dt * 1e3 / reps, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": "replay: headline env transitions into FrameReplay, batch 4096, n_step 3", "envs": n,
                   "capacity_per_env": C, "batch": B, "n_step": ns, "rom": rom_name, "rom_sha1": rom_sha},
        "roofline": {"bound": "hbm", "kernel": "k_replay_gather", "achieved": round(gat_bytes / gat_t / 1e6, 1),
                     "peak": 8000.0, "unit": "GB/s", "frac": round(gat_bytes / gat_t / 1e6 / 8000.0, 4),
                     "traffic": None, "algorithmic_bytes_per_launch": int(gat_bytes)},
        "add": {"kernel": "k_replay_add", "ms": round(add_t, 4), "achieved_GBps": round(add_bytes / add_t / 1e6, 1),
                "frac": round(add_bytes / add_t / 1e6 / 8000.0, 4), "algorithmic_bytes_per_launch": int(add_bytes),
                "transitions_per_s": round(n / add_t * 1e3, 1)},
        "gather_ms": round(gat_t, 4), "draw_ms": round(draw_t * 1e3 / reps, 3),
        "ring_gb": round(rb.nbytes() / 1e9, 2),
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--envs", type=int, default=32768)
    ap.add_argument("--probe-copy-mib", type=int, default=0,
                    help="before the steps, copy a buffer of this many MiB once (a kernel of known traffic "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=["headline", "ppo", "replay"], default="headline",
                    help="headline: the env step (default); ppo: a PPO rollout feeding a Nature CNN (config 5); "
                         "replay: env transitions into the GPU FrameReplay and sampled batches")
    ap.add_argument("--ppo-steps", type=int, default=128, help="rollout length of --workload ppo")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: every GPU box in this build has one GPU and the env step "
              f"needs no collectives (envs shard by env_offset with zero exchange). Got --gpus {args.gpus}, "
              f"WORLD_SIZE {world}.", file=sys.stderr)
        sys.exit(2)

    import torch

    from fast_mario_env_amd import HipVecEnv
    rom, rom_name = pick_rom()
    rom_sha = hashlib.sha1(rom).hexdigest()[:12]
    if args.workload == "ppo":
        run_ppo(args, rom, rom_name, rom_sha)
        return
    if args.workload == "replay":
        run_replay(args, rom, rom_name, rom_sha)
        return
    n = args.envs
    log(f"creating {n} envs on {torch.cuda.get_device_name(0)} ({rom_name})")
    t0 = time.perf_counter()
    env = HipVecEnv("1-1", n, seed=0, sticky=0.25, noop_max=30, max_steps=2000, skip=4, frame_stack=4,
                    maxpool=True, rom=rom, device="cuda:0")
    env.reset()
    torch.cuda.synchronize()
    log(f"boot + reset cache + reset: {time.perf_counter() - t0:.1f} s")
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(0)
    acts = torch.randint(0, 7, (args.warmup + args.steps, n), generator=gen, device="cuda:0", dtype=torch.int64)
    done_acc = torch.zeros(n, dtype=torch.int32, device="cuda:0")     # episodes ended per env (no per-step allocation)
    done_tmp = torch.zeros(n, dtype=torch.bool, device="cuda:0")
    if args.probe_copy_mib:
        src = torch.ones(args.probe_copy_mib << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {args.probe_copy_mib} MiB device-to-device")
        del src, dst
    for i in range(args.warmup):
        _, _, term, trunc, _ = env.step(acts[i])
        # the timed loop's own bookkeeping ops run here first: torch loads a kernel's code on its first
        # use, ~0.1 s that would otherwise land inside the timed steps
        torch.logical_or(term, trunc, out=done_tmp)
        done_acc.add_(done_tmp)
    done_acc.zero_()
    torch.cuda.synchronize()
    log(f"{args.warmup} warm-up steps done")
    f0, i0 = env.frames, env.instructions()
    env.timing(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    # progress lines need a device sync, which idles the GPU between steps: long runs only
    every = args.steps // 4 if args.steps >= 400 else 0
    for i in range(args.steps):
        _, _, term, trunc, _ = env.step(acts[args.warmup + i])
        torch.logical_or(term, trunc, out=done_tmp)
        done_acc.add_(done_tmp)
        if every and (i + 1) % every == 0:
            torch.cuda.synchronize()
            log(f"step {i + 1}/{args.steps}")
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    stages, timed = env.timing_read()
    env.timing(False)
    frames = env.frames - f0
    instr = env.instructions() - i0
    bad = env.bad_ops()
    p_done = float(done_acc.sum().item()) / (n * args.steps)
    value = n * args.steps / dt
    k_step_ms = stages["k_step"] / max(1, timed)
    workload = f"headline/{n}envs/1-1/rom:{rom_sha}"
    k_bytes = n * (K_STEP_BYTES + K_STEP_DONE_BYTES * p_done)
    achieved = k_bytes / (k_step_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles(workload)
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "agent-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {"workload": "headline: full wrapper stack, 32768 envs of 1-1", "envs": n, "level": "1-1",
                   "rom": rom_name, "rom_sha1": rom_sha, "sticky": 0.25, "noop_max": 30, "skip": 4, "maxpool": True,
                   "frame_stack": 4, "max_steps": 2000, "seed": 0, "actions": "uniform {0..6}, torch.Generator seed 0"},
        "roofline": {"bound": "hbm", "kernel": "k_step", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 6),
                     "traffic": traffic,
                     "algorithmic_bytes_per_launch": round(k_bytes),
                     "valu_issue_frac": valu_issue_from_profiles(workload),
                     "note": "k_step is bound by dependent VALU/LDS/memory latency per lane, not by HBM; "
                             "valu_issue_frac is SQ_INSTS_VALU x 4 cycles over 1024 SIMDs x duration x 2.4 GHz "
                             "from the committed rocprofv3 SQ-counter summary in profiles/"},
        "stages_ms_per_step": {k: round(v / max(1, timed), 3) for k, v in stages.items()},
        "p_done": round(p_done, 5),
        "frames_per_step": round(frames / (n * args.steps), 3),
        "instructions_per_step": round(instr / (n * args.steps), 1),
        "emulated_instructions_per_s": round(instr / dt, 1),
        "bad_ops": bad,
    }
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        out["cpu_baseline"] = cpu_baseline(rom, args.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    env.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
