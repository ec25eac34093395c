#!/usr/bin/env python
"""Benchmarks of batched Super Mario Bros stepping on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload headline|stress|raw|ppo|replay] [--gpus 1]

headline (default; the metric's configuration): 32,768 envs of 1-1, sticky 0.25, no-op starts up to 30,
    skip 4, 2-frame max-pool, gray + INTER_AREA 84x84, frame stack 4, time limit 2000, auto-reset, seed 0
    (env i: PCG64 stream i); actions uniform in {0..6} from torch.Generator seed 0 on the device.
stress: the divergence-stress configuration: 65,536 envs, level of env i drawn from default_rng(7) over the
    32 world-stage pairs, rom_mode cycled over the four variants per env, sticky 0.25, no-op 30, skip 4, no
    max-pool; per env and step, action 2 (right + A) with p = 0.5, else uniform (torch.Generator seed 0).
raw: the raw-emulator configuration: 4,096 consoles, skip 1, no wrappers, every frame rendered and delivered
    as an RGB24 screen plus the 2 KB RAM; a Start/none prologue enters 1-1, then SIMPLE_MOVEMENT buttons
    drawn per console and frame from default_rng(1); K timed frames.
ppo / replay: the PPO rollout feeding a Nature CNN, and the GPU FrameReplay.

The ROM is the real one when the reference's lookup finds it, else this repository's synthetic NROM stand-in
(tests/golden/roms/mini_smb_*.nes); the JSON line names which. One step is one mh_step_async (k_step,
k_obs_late, k_reset, k_stack) or, for raw, one frame and its outputs, on torch's current stream with inputs resident in
HBM. Before the W warm-up steps, --preroll untimed steps carry the envs past their first episodes so that the
timed window has episode ends, resets and early-termination re-emulations in it (the first steps after a
reset are the cheapest ones). K steps are timed between two device synchronizations; per-kernel times come
from HIP events recorded on the launch stream. The reference C++ (oracle/_ref, the checker build of the
reference) is timed on the host cores on a bounded sample of the same workload and reported beside the GPU
number.
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
# env words read + write, action, reward / term / trunc / info out, the new 84x84 observation out;
# ep stats on episode end.
STATE_BYTES = 4384 + 4 * 41
ENV_WORD_BYTES = 4 * 30
OBS = 84 * 84
K_STEP_BYTES = 2 * STATE_BYTES + 2 * ENV_WORD_BYTES + 8 + 4 + 1 + 1 + 40 + OBS
K_STEP_DONE_BYTES = 12
SIMPLE_BUTTONS = (0x00, 0x80, 0x81, 0x82, 0x83, 0x01, 0x40)


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def pick_rom(mode="vanilla"):
    """(bytes, description) of the ROM for a rom_mode: the real one if found, else the synthetic stand-in."""
    from fast_mario_env_amd import RomNotFoundError, load_rom
    try:
        return load_rom(rom_mode=mode), f"{mode}: real ROM"
    except (RomNotFoundError, ValueError):
        from build_roms import rom_path
        path = rom_path(mode)
        return open(path, "rb").read(), f"{mode}: {os.path.basename(path)} (synthetic NROM stand-in; no SMB ROM here)"


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


def traffic_from_profiles(profile, workload_key):
    """HBM bytes per launch from a committed rocprofv3 --pmc summary, if one exists for this workload."""
    try:
        return float(profile_values(profile, workload_key)["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


# Peak wave64 VALU issue of the chip: 256 CUs x 4 SIMDs, one wave64 VALU instruction per SIMD every 4 cycles
# (16 lanes wide), at the 2.4 GHz peak engine clock: 614.4 G wave-instructions/s.
VALU_PEAK_G = 1024 * 2.4 / 4


def valu_profile(profile, workload_key):
    """The committed rocprofv3 SQ-counter summary of a kernel on this workload (profiles/<profile>): VALU
    instructions per launch, its counter-based issue fraction, the window and the kernel build it measured.
    Counters cannot be read inside this run; the summary names its command."""
    v = profile_values(profile, workload_key)
    try:
        valu = float(v["valu_per_launch"])
        frac = float(v["valu_issue_fraction"])
    except (KeyError, ValueError):
        return None
    v["_valu"], v["_frac"] = valu, frac
    return v


def valu_roofline(kernel, profile, workload_key, kernel_ms, executed_per_launch, traffic, hbm):
    """The binding roofline of an interpreter kernel: VALU issue. achieved = the VALU wave-instructions of one
    launch (the committed SQ profile of this workload, same window) / this run's average launch time from HIP
    events on the launch stream, against VALU_PEAK_G. Falls back to the HBM figure when no profile exists."""
    v = valu_profile(profile, workload_key)
    if v is None:
        return dict(hbm, note=f"no SQ-counter profile for this workload in profiles/{profile}: HBM figure only")
    achieved = v["_valu"] / (kernel_ms * 1e-3) / 1e9
    sha = v.get("kernel_source_sha1", "").split(" ")[0]
    out = {"bound": "valu_issue", "kernel": kernel, "achieved": round(achieved, 2), "peak": VALU_PEAK_G,
           "unit": "G VALU wave-instructions/s (wave64; 1024 SIMDs x 2.4 GHz / 4 cycles)",
           "frac": round(achieved / VALU_PEAK_G, 4), "traffic": traffic,
           "valu_per_launch": v["_valu"],
           "valu_per_executed_instruction": round(v["_valu"] / max(1.0, executed_per_launch), 2),
           "frac_counters": v["_frac"], "source": f"profiles/{profile}",
           "profile_kernel_source_sha1": sha, "profile_matches_build": sha == kernel_source_sha1()}
    for k in ("window", "active_lane_fraction", "occupancy_waves_per_simd", "lds_bank_conflict_per_lds_instr"):
        if k in v:
            out[k] = v[k]
    return out


def kernel_source_sha1():
    """sha1 of the HIP sources the library is built from and of its build script (compiler flags): names the
    kernel build a profile measured."""
    h = hashlib.sha1()
    d = os.path.join(ROOT, "fast-mario-env_amd", "csrc")
    for f in sorted(os.listdir(d)):
        if f.endswith((".hip", ".hpp")):
            h.update(open(os.path.join(d, f), "rb").read())
    h.update(open(os.path.join(ROOT, "fast-mario-env_amd", "build_native.py"), "rb").read())
    return h.hexdigest()[:12]


def host_info():
    try:
        load1 = round(os.getloadavg()[0], 2)
    except OSError:
        load1 = None
    model = ""
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return model, load1


def host_threads():
    """Worker threads for the CPU baselines: the host's cores, capped by OMP_NUM_THREADS where it is set (the
    GPU boxes set it to their CPU share, whatever os.cpu_count() shows)."""
    cores = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(cores, int(cap))) if cap.isdigit() else cores


def mem_available_gb():
    try:
        for line in open("/proc/meminfo"):
            if line.startswith("MemAvailable:"):
                return int(line.split()[1]) / 2**20
    except OSError:
        pass
    return 0.0


def _timed_cpu_steps(envs_actions, seconds, min_steps=1):
    """Steps every (env, action-fn) pair once per step until `seconds` passed (at least min_steps)."""
    steps, t0 = 0, time.perf_counter()
    while steps < min_steps or time.perf_counter() - t0 < seconds:
        for env, act in envs_actions:
            env.step(act(env.n))
        steps += 1
    return steps, time.perf_counter() - t0


def cpu_baseline_env(rom_by_mode, kw, levels, modes, seconds, n_req, action_fn, what, preroll):
    """The reference C++ thread pool (oracle/_ref) on the host cores: one FastVecEnv per rom_mode (the reference
    takes one rom_mode per instance), envs split by their mode, stepped one after the other each step. Like the
    GPU run, the envs first take `preroll` untimed steps (the steps right after a reset are the cheapest), then 3
    warm-up steps; then steps are timed for `seconds`."""
    from cpu_libs import OracleVec, RefVec, have_ref
    from fast_mario_env_amd import decode_level
    cores = host_threads()
    n, why = n_req, ""
    need_gb = 0.4 * n / 1024                   # ~0.36 MB per env (state, snapshots, frames, stacks)
    if mem_available_gb() < need_gb + 4:
        n = max(1024, 8 * cores)
        why = f"; {n_req} envs would need ~{need_gb:.0f} GB of host RAM, {mem_available_gb():.0f} GB available"
    by_mode = {}
    for i in range(n):
        by_mode.setdefault(modes[i], []).append(i)
    t_build = time.perf_counter()
    if have_ref():
        kind, threads = "reference", cores
        envs = [RefVec(rom_by_mode[m], [decode_level(levels[i]) for i in idx], len(idx), n_threads=cores, **kw)
                for m, idx in by_mode.items()]
    else:
        kind, threads, n = "port", 1, 64
        envs = [OracleVec(rom_by_mode[modes[0]], [decode_level(levels[0])] * n, n, **kw)]
    for e in envs:
        e.reset()
    build_s = time.perf_counter() - t_build
    pairs = [(e, action_fn) for e in envs]
    t_pre = time.perf_counter()
    _timed_cpu_steps(pairs, 0.0, min_steps=preroll) if preroll else None
    pre_s = time.perf_counter() - t_pre
    _timed_cpu_steps(pairs, 0.0, min_steps=3)
    steps, dt = _timed_cpu_steps(pairs, seconds)
    for e in envs:
        e.close()
    model, load1 = host_info()
    return {"value": round(n * steps / dt, 1), "unit": "agent-steps/s", "cores": threads, "kind": kind,
            "sample": f"{n} envs ({what}) x {steps} timed steps (steps {preroll + 4}..{preroll + 3 + steps} after the "
                      f"reset: {preroll} untimed preroll steps and 3 warm-up steps first, as the GPU's window starts "
                      f"after its preroll) in {dt:.1f} s; construction + reset {build_s:.1f} s, preroll {pre_s:.1f} s; "
                      f"{len(envs)} instance(s) by rom_mode; {model}; load1 {load1}{why}"}


def cpu_baseline_raw(rom, n, prologue, button_rows, seconds_cap):
    """The reference's raw console (fm_raw_*, oracle/_ref): n consoles split over one Python thread per host
    core (ctypes releases the GIL during each frame call), the GPU run's prologue, then the GPU run's own button
    rows for its first n consoles (its warm-up frames untimed, then its timed frames), every frame rendered
    (palette screen + RAM in place; no RGB24 conversion). Stops early after seconds_cap."""
    import concurrent.futures as cf

    import numpy as np

    from cpu_libs import OracleRaw, RefRaw, have_ref
    cores = host_threads()
    kind = "reference" if have_ref() else "port"
    mk = RefRaw if have_ref() else OracleRaw
    if kind == "port":
        n, cores = 64, 1
    warm, rows = button_rows
    cons = [mk(rom) for _ in range(n)]
    parts = [cons[t::cores] for t in range(cores)]

    def run(part, buttons):
        for c, b in zip(part, buttons):
            c.frame(int(b), True)

    with cf.ThreadPoolExecutor(cores) as pool:
        for f in range(prologue):
            b = np.full(n, 8 if f % 2 == 0 else 0, np.uint8)
            list(pool.map(run, parts, [b[t::cores] for t in range(cores)]))
        for b in warm:
            list(pool.map(run, parts, [b[:n][t::cores] for t in range(cores)]))
        frames, t0 = 0, time.perf_counter()
        for b in rows:
            list(pool.map(run, parts, [b[:n][t::cores] for t in range(cores)]))
            frames += 1
            if time.perf_counter() - t0 > seconds_cap:
                break
        dt = time.perf_counter() - t0
    model, load1 = host_info()
    first = prologue + len(warm)
    return {"value": round(n * frames / dt, 1), "unit": "env-frames/s", "cores": cores, "kind": kind,
            "sample": f"{n} consoles x {frames} timed frames ({frames} of the GPU's {len(rows)} timed frames: frames "
                      f"{first + 1}..{first + frames} after power-on, the GPU's first {n} consoles' buttons) in "
                      f"{dt:.1f} s, after the {prologue}-frame prologue and {len(warm)} warm-up frames; {cores} "
                      f"threads; {model}; load1 {load1}"}


def run_ppo(args):
    """PPO rollout workload (config 5): the headline envs feeding a random-init bf16 Nature CNN, Gumbel-max
    actions from seed 3, 128-step rollouts with frame-deduplicated storage and GAE (0.99, 0.95)."""
    import torch

    from fast_mario_env_amd import HipVecEnv
    from fast_mario_env_amd.rollout import Rollout, make_net
    rom, rom_name = pick_rom()
    rom_sha = hashlib.sha1(rom).hexdigest()[:12]
    n, T = args.envs or 32768, args.ppo_steps
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


def run_replay(args):
    """Replay workload (the GPU FrameReplay): the headline envs' transitions added to a 64-slot ring per env,
    then batches of 4096 3-step transitions sampled. Kernel times come from HIP events on the stream the
    kernels run on; the rooflines count the bytes each kernel must move."""
    import torch

    from fast_mario_env_amd import HipVecEnv
    from fast_mario_env_amd.replay import FrameReplay
    rom, rom_name = pick_rom()
    rom_sha = hashlib.sha1(rom).hexdigest()[:12]
    n, C, B, ns, reps = args.envs or 32768, 64, 4096, 3, 20
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


def headline_actions(n, preroll, timed, device="cuda:0"):
    """The headline workload's actions on the device: `preroll` rows drawn one step at a time from a seed-0
    torch.Generator (the untimed preroll), then `timed` rows drawn at once from a second seed-0 generator (the
    warm-up and timed steps), each uniform in {0..6}, int64 (rows, n). The GPU parity test of the headline
    shape replays exactly this stream."""
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    pre = [torch.randint(0, 7, (n,), generator=gen, device=device, dtype=torch.int64) for _ in range(preroll)]
    gen_t = torch.Generator(device=device)
    gen_t.manual_seed(0)
    acts = torch.randint(0, 7, (timed, n), generator=gen_t, device=device, dtype=torch.int64)
    return (torch.stack(pre) if pre else acts[:0]), acts


def step_loop(env, args, next_actions, timed_actions):
    """--preroll untimed steps (fresh actions from next_actions()), W warm-up and K timed steps over the rows of
    timed_actions (pre-generated on the device). Returns the measurements of the K timed steps."""
    import torch
    n = env.n
    done_acc = torch.zeros(n, dtype=torch.int32, device=env.dev)   # episodes ended per env (no per-step allocation)
    done_tmp = torch.zeros(n, dtype=torch.bool, device=env.dev)
    t0 = time.perf_counter()
    for i in range(args.preroll):
        env.step(next_actions())
        if (i + 1) % 100 == 0:
            torch.cuda.synchronize()
            log(f"preroll {i + 1}/{args.preroll}")
    torch.cuda.synchronize()
    log(f"{args.preroll} preroll steps: {time.perf_counter() - t0:.1f} s")
    for i in range(args.warmup):
        _, _, term, trunc, _ = env.step(timed_actions[i])
        # the timed loop's own bookkeeping ops run here first: torch loads a kernel's code on its first
        # use, ~0.1 s that would otherwise land inside the timed steps
        torch.logical_or(term, trunc, out=done_tmp)
        done_acc.add_(done_tmp)
    done_acc.zero_()
    torch.cuda.synchronize()
    f0, i0, ff0 = env.frames, env.instructions(), env.ff_instructions()
    re0 = env.reemulations()
    env.timing(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    every = args.steps // 4 if args.steps >= 400 else 0   # progress lines sync the device: long runs only
    for i in range(args.steps):
        _, _, term, trunc, _ = env.step(timed_actions[args.warmup + i])
        torch.logical_or(term, trunc, out=done_tmp)
        done_acc.add_(done_tmp)
        if every and (i + 1) % every == 0:
            torch.cuda.synchronize()
            log(f"step {i + 1}/{args.steps}")
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    stages, timed = env.timing_read()
    env.timing(False)
    re1 = env.reemulations()
    steps = args.steps
    return dict(dt=dt, stages={k: v / max(1, timed) for k, v in stages.items()},
                p_done=float(done_acc.sum().item()) / (n * steps),
                frames=(env.frames - f0) / (n * steps),
                instr=(env.instructions() - i0) / (n * steps),
                ff=(env.ff_instructions() - ff0) / (n * steps),
                instr_total=env.instructions() - i0,
                reemu={k: re1[k] - re0[k] for k in re1}, bad=env.bad_ops())


def env_line(args, metric, n, m, workload_key, config, sq_profile, dtype="u8"):
    """The JSON line of an env workload from the step_loop measurements."""
    value = n * args.steps / m["dt"]
    k_step_ms = m["stages"]["k_step"]
    k_bytes = n * (K_STEP_BYTES + K_STEP_DONE_BYTES * m["p_done"])
    achieved = k_bytes / (k_step_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles("k_step_pmc_traffic.md", workload_key)
    hbm = {"bound": "hbm", "kernel": "k_step", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 6), "traffic": traffic,
           "algorithmic_bytes_per_launch": round(k_bytes),
           "note": "k_step's algorithmic bytes (console state, env words, action, outputs, new observation) over its "
                   "live launch time; traffic: rocprofv3 FETCH_SIZE + WRITE_SIZE per launch"}
    executed = (m["instr"] - m["ff"]) * n
    return {
        "metric": metric, "value": round(value, 1), "unit": "agent-steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(m["dt"] * 1e3 / args.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": config,
        "roofline": valu_roofline("k_step", sq_profile, workload_key, k_step_ms, executed, traffic, hbm),
        "hbm_roofline": hbm,
        "stages_ms_per_step": {k: round(v, 3) for k, v in m["stages"].items()},
        "p_done": round(m["p_done"], 5),
        "preroll_steps": args.preroll,
        "frames_per_step": round(m["frames"], 4),
        "instructions_per_step": round(m["instr"], 1),
        "executed_instructions_per_step": round(m["instr"] - m["ff"], 1),
        "fast_forwarded_instructions_per_step": round(m["ff"], 1),
        "emulated_instructions_per_s": round(m["instr_total"] / m["dt"], 1),
        "reemulations_in_window": m["reemu"],
        "bad_ops": m["bad"],
        "kernel_source_sha1": kernel_source_sha1(),
    }


def run_headline(args):
    import torch

    from fast_mario_env_amd import HipVecEnv
    rom, rom_name = pick_rom()
    rom_sha = hashlib.sha1(rom).hexdigest()[:12]
    n = args.envs or 32768
    kw = dict(sticky=0.25, noop_max=30, max_steps=2000, skip=4, frame_stack=4, maxpool=True)
    log(f"creating {n} envs on {torch.cuda.get_device_name(0)} ({rom_name})")
    t0 = time.perf_counter()
    env = HipVecEnv("1-1", n, seed=0, rom=rom, device="cuda:0", **kw)
    env.reset()
    torch.cuda.synchronize()
    log(f"boot + reset cache + reset: {time.perf_counter() - t0:.1f} s")
    pre_rows, acts = headline_actions(n, args.preroll, args.warmup + args.steps)
    pre_it = iter(pre_rows)
    pre = lambda: next(pre_it)  # noqa: E731
    if args.probe_copy_mib:
        src = torch.ones(args.probe_copy_mib << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: {args.probe_copy_mib} MiB device-to-device")
        del src, dst
    m = step_loop(env, args, pre, acts)
    env.close()
    config = {"workload": f"headline: full wrapper stack, {n} envs of 1-1", "envs": n, "level": "1-1",
              "rom": rom_name, "rom_sha1": rom_sha, "seed": 0, **kw,
              "actions": "uniform {0..6}, torch.Generator seed 0 (preroll: its own seed-0 generator)"}
    out = env_line(args, METRIC, n, m, f"headline/{n}envs/1-1/rom:{rom_sha}", config,
                   "k_step_sq_counters_headline.md")
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        import numpy as np
        rng = np.random.default_rng(0)
        out["cpu_baseline"] = cpu_baseline_env({"vanilla": rom}, dict(seed=0, **kw), ["1-1"] * args.cpu_envs,
                                               ["vanilla"] * args.cpu_envs, args.cpu_seconds, args.cpu_envs,
                                               lambda k: rng.integers(0, 7, k), "headline settings, 1-1",
                                               args.preroll)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


def stress_actions(gen, n):
    import torch
    u = torch.rand(n, generator=gen, device="cuda:0")
    r = torch.randint(0, 7, (n,), generator=gen, device="cuda:0", dtype=torch.int64)
    return torch.where(u < 0.5, torch.full_like(r, 2), r)


def run_stress(args):
    import numpy as np
    import torch

    from build_roms import MODES
    from fast_mario_env_amd import ALL_LEVELS, HipVecEnv
    n = args.envs or 65536
    roms, names = {}, []
    for m in MODES:
        roms[m], nm = pick_rom(m)
        names.append(nm)
    rom_sha = hashlib.sha1(b"".join(roms[m] for m in MODES)).hexdigest()[:12]
    levels = [ALL_LEVELS[k] for k in np.random.default_rng(7).integers(0, 32, n)]
    modes = [MODES[i % 4] for i in range(n)]
    kw = dict(sticky=0.25, noop_max=30, max_steps=2000, skip=4, frame_stack=4, maxpool=False)
    log(f"creating {n} envs ({len(set(levels))} levels x 4 rom modes) on {torch.cuda.get_device_name(0)}")
    t0 = time.perf_counter()
    env = HipVecEnv(levels, n, seed=0, rom=roms, rom_mode=modes, device="cuda:0", **kw)
    env.reset()
    torch.cuda.synchronize()
    log(f"boot + reset cache + reset: {time.perf_counter() - t0:.1f} s")
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(0)
    acts = torch.stack([stress_actions(gen, n) for _ in range(args.warmup + args.steps)])
    m = step_loop(env, args, lambda: stress_actions(gen, n), acts)
    env.close()
    config = {"workload": f"stress: {n} envs, 32 levels x 4 rom modes, biased actions", "envs": n,
              "levels": "ALL_LEVELS[default_rng(7).integers(0, 32, n)]", "rom_mode": "MODES[i % 4]",
              "roms": names, "rom_sha1": rom_sha, "seed": 0, **kw,
              "actions": "per env and step: 2 with p=0.5 else uniform {0..6}; torch.Generator seed 0"}
    metric = f"agent env-steps/sec (skip=4) at {n} envs, divergence stress (32 levels x 4 rom modes) on 1 MI355X"
    out = env_line(args, metric, n, m, f"stress/{n}envs/rom:{rom_sha}", config, "k_step_sq_counters_stress.md")
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        rng = np.random.default_rng(0)
        ncpu = args.cpu_envs

        def act(k):
            return np.where(rng.random(k) < 0.5, 2, rng.integers(0, 7, k))
        out["cpu_baseline"] = cpu_baseline_env(roms, dict(seed=0, **kw), levels, modes, args.cpu_seconds, ncpu, act,
                                               "the first envs of the stress configuration", args.preroll)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


def run_raw(args):
    import numpy as np
    import torch

    from fast_mario_env_amd import HipRawNES, palette_rgb
    from fast_mario_env_amd._native import check, lib
    rom, rom_name = pick_rom()
    rom_sha = hashlib.sha1(rom).hexdigest()[:12]
    n, prologue = args.envs or 4096, 40
    frames = args.steps
    dev = "cuda:0"
    log(f"creating {n} raw consoles ({rom_name})")
    con = HipRawNES(rom, n, device=dev)
    L = lib()
    s = torch.cuda.current_stream(0).cuda_stream
    rgb = torch.empty(n, 240, 256, 3, dtype=torch.uint8, device=dev)
    ram = torch.empty(n, 2048, dtype=torch.uint8, device=dev)
    rgb64 = torch.from_numpy(palette_rgb().reshape(-1).copy()).to(dev)
    tab = torch.tensor(SIMPLE_BUTTONS, dtype=torch.uint8, device=dev)
    rng = np.random.default_rng(1)
    sched = [torch.full((n,), 8 if f % 2 == 0 else 0, dtype=torch.uint8, device=dev) for f in range(prologue)]
    draws_np = rng.integers(0, 7, (args.warmup + frames, n))
    draws = torch.from_numpy(draws_np).to(dev)
    buttons = tab[draws]                                          # (W + K, n) button bytes on the device

    def one(b):
        check(L.mh_raw_frame(con.h, b.data_ptr(), 1, s), "mh_raw_frame")
        check(L.mh_raw_screen_rgb(con.h, rgb64.data_ptr(), rgb.data_ptr(), s), "mh_raw_screen_rgb")
        check(L.mh_raw_ram(con.h, ram.data_ptr(), s), "mh_raw_ram")

    for b in sched:
        one(b)
    for f in range(args.warmup):
        one(buttons[f])
    torch.cuda.synchronize()
    i0, ff0 = con.instructions(), con.ff_instructions()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2 * frames)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for f in range(frames):
        ev[2 * f].record()
        check(L.mh_raw_frame(con.h, buttons[args.warmup + f].data_ptr(), 1, s), "mh_raw_frame")
        ev[2 * f + 1].record()
        check(L.mh_raw_screen_rgb(con.h, rgb64.data_ptr(), rgb.data_ptr(), s), "mh_raw_screen_rgb")
        check(L.mh_raw_ram(con.h, ram.data_ptr(), s), "mh_raw_ram")
        if frames >= 1000 and (f + 1) % (frames // 4) == 0:
            torch.cuda.synchronize()
            log(f"frame {f + 1}/{frames}")
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    k_raw_ms = sum(ev[2 * f].elapsed_time(ev[2 * f + 1]) for f in range(frames)) / frames
    instr = con.instructions() - i0
    ff = con.ff_instructions() - ff0
    bad = con.bad_ops()
    # k_raw's algorithmic bytes per console and frame: console state read + written, the button byte, the
    # rendered palette screen written
    k_bytes = n * (2 * STATE_BYTES + 1 + 240 * 256)
    achieved = k_bytes / (k_raw_ms * 1e-3) / 1e9
    hbm = {"bound": "hbm", "kernel": "k_raw", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 6), "traffic": None,
           "algorithmic_bytes_per_launch": k_bytes,
           "note": "console state read + written, buttons, palette screen written, over k_raw's live launch time"}
    workload_key = f"raw/{n}consoles/rom:{rom_sha}"
    out = {
        "metric": f"raw emulator env-frames/sec (skip=1, every frame rendered, RGB24 + RAM out) at {n} consoles on 1 MI355X",
        "value": round(n * frames / dt, 1), "unit": "env-frames/s", "n_gpus": 1, "steps": frames, "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / frames, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": f"raw: {n} consoles, 1-1 via a {prologue}-frame Start/none prologue, then SIMPLE_MOVEMENT "
                               f"buttons from default_rng(1) per console and frame", "envs": n, "rom": rom_name,
                   "rom_sha1": rom_sha, "outputs_per_frame": "RGB24 screen (184,320 B) + RAM (2,048 B) per console"},
        "roofline": valu_roofline("k_raw", "k_raw_sq_counters_raw.md", workload_key, k_raw_ms, (instr - ff) / frames,
                                  None, hbm),
        "hbm_roofline": hbm,
        "k_raw_ms": round(k_raw_ms, 4),
        "instructions_per_frame": round(instr / (n * frames), 1),
        "executed_instructions_per_frame": round((instr - ff) / (n * frames), 1),
        "fast_forwarded_instructions_per_frame": round(ff / (n * frames), 1),
        "bad_ops": bad, "kernel_source_sha1": kernel_source_sha1(),
    }
    del con
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        host_rows = np.array(SIMPLE_BUTTONS, np.uint8)[draws_np]
        out["cpu_baseline"] = cpu_baseline_raw(rom, min(n, args.cpu_raw_consoles), prologue,
                                               (host_rows[:args.warmup], host_rows[args.warmup:]), 4 * args.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (frames for raw); default 100 (raw 5000)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--preroll", type=int, default=None,
                    help="untimed steps before the warm-up so the timed window has episode ends (default 300 for "
                         "headline and stress, 0 otherwise)")
    ap.add_argument("--envs", type=int, default=0, help="env count (default: the workload's configuration)")
    ap.add_argument("--probe-copy-mib", type=int, default=0,
                    help="before the steps, copy a buffer of this many MiB once (a kernel of known traffic "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--cpu-envs", type=int, default=4096,
                    help="envs of the CPU baseline sample (host RAM allowing); it takes the GPU run's preroll first")
    ap.add_argument("--cpu-raw-consoles", type=int, default=256,
                    help="consoles of the raw workload's CPU baseline (it runs the GPU run's own frames)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", choices=["headline", "stress", "raw", "ppo", "replay"], default="headline")
    ap.add_argument("--ppo-steps", type=int, default=128, help="rollout length of --workload ppo")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: every GPU box in this build has one GPU and the env step "
              f"needs no collectives (envs shard by env_offset with zero exchange). Got --gpus {args.gpus}, "
              f"WORLD_SIZE {world}.", file=sys.stderr)
        sys.exit(2)
    if args.steps is None:
        args.steps = 5000 if args.workload == "raw" else 100
    if args.preroll is None:
        args.preroll = 300 if args.workload in ("headline", "stress") else 0
    {"headline": run_headline, "stress": run_stress, "raw": run_raw, "ppo": run_ppo,
     "replay": run_replay}[args.workload](args)


if __name__ == "__main__":
    main()
