"""GPU-vs-oracle fidelity record of the raw consoles over a long horizon (test infrastructure; the product path is the
HIP library).

    python tests/fidelity/raw_fidelity_run.py [--consoles 512] [--frames 5000] [--cpw auto|1|2|4|8|16]
        [--out tests/fidelity/raw_fidelity.jsonl]

The reference publishes a 100k-frame raw run with RAM every frame (README.md:166-170). Here HipRawNES runs the
consoles on the GPU and the CPU checker (oracle/liboracle.so) runs one console each on a thread pool, with the
raw-emulator workload's schedule: a Start/none prologue that enters 1-1, then SIMPLE_MOVEMENT buttons drawn per
console and frame from default_rng(1), every frame rendered. Every console every frame: the 2 KB of RAM and the
whole machine state (the canonical dump); the palette screen every 4th frame; at the end the bad-opcode and
retired-instruction counts. Past frame ~200 the consoles are out of phase (deaths, level reloads and game-over
screens at different points of a frame), the regime whose long single-console instruction runs set the raw
kernel's time. --cpw sets k_raw's consoles per wave (MH_RAW_CONSOLES_PER_WAVE; "auto": the library's choice, one
per wave at 512 consoles). One JSON line per ROM.
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
from cpu_libs import OracleRaw  # noqa: E402

PROLOGUE = 40
BUTTONS = np.array([0x00, 0x80, 0x81, 0x82, 0x83, 0x01, 0x40], np.uint8)   # SIMPLE_MOVEMENT as joypad bytes


def run(mode, n, frames, cpw, log):
    import torch

    from fast_mario_env_amd import HipRawNES
    rom = open(rom_path(mode), "rb").read()
    gpu = HipRawNES(rom, n)
    cpu = [OracleRaw(rom) for _ in range(n)]
    pool = ThreadPoolExecutor(16)
    parts = [list(range(t, n, 16)) for t in range(16)]
    draws = np.random.default_rng(1).integers(0, 7, (frames, n))
    sched = [np.full(n, 8 if f % 2 == 0 else 0, np.uint8) for f in range(PROLOGUE)] + [BUTTONS[d] for d in draws]
    mism = []
    t0 = time.perf_counter()
    screens = 0

    def cpu_frame(idx, b):
        for i in idx:
            cpu[i].frame(int(b[i]), True)

    for f, b in enumerate(sched):
        gpu.frame(torch.from_numpy(b), True)
        list(pool.map(cpu_frame, parts, [b] * len(parts)))
        ram = gpu.ram.cpu().numpy()
        canon = gpu.canon().cpu().numpy()
        bad = [i for i in range(n) if not (np.array_equal(ram[i], cpu[i].ram) and np.array_equal(canon[i], cpu[i].canon()))]
        if f % 4 == 3:
            scr = gpu.screen.cpu().numpy()
            bad += [i for i in range(n) if not np.array_equal(scr[i], cpu[i].screen)]
            screens += n
        if bad and len(mism) < 20:
            mism.append({"frame": f, "consoles": sorted(set(bad))[:8]})
        if (f + 1) % 500 == 0:
            log(f"[raw fidelity] {mode} frame {f + 1}/{len(sched)}: {len(mism)} mismatching frames, "
                f"{time.perf_counter() - t0:.0f} s")
    bad_c = sum(c.bad_ops() for c in cpu)
    instr_c = sum(c.instructions() for c in cpu)
    if gpu.instructions() != instr_c:
        mism.append({"frame": len(sched), "what": "instructions"})
    rec = {"rom": f"synthetic stand-in (tests/golden/roms, {mode})", "consoles": n, "consoles_per_wave": cpw,
           "frames": len(sched),
           "prologue": PROLOGUE, "console_frames": n * len(sched), "screens_compared": screens,
           "instructions": int(gpu.instructions()), "ff_instructions": int(gpu.ff_instructions()),
           "bad_ops": int(gpu.bad_ops()), "oracle_bad_ops": int(bad_c), "mismatches": mism, "ok": not mism,
           "secs": round(time.perf_counter() - t0, 1)}
    pool.shutdown()
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--consoles", type=int, default=512)
    ap.add_argument("--frames", type=int, default=5000)
    ap.add_argument("--modes", default="vanilla")
    ap.add_argument("--cpw", default="auto")
    ap.add_argument("--out", default=os.path.join(HERE, "raw_fidelity.jsonl"))
    args = ap.parse_args()
    log = lambda m: print(m, flush=True)  # noqa: E731
    if args.cpw != "auto":
        os.environ["MH_RAW_CONSOLES_PER_WAVE"] = args.cpw
    recs = []
    for mode in args.modes.split(","):
        rec = run(mode, args.consoles, args.frames, args.cpw, log)
        log(json.dumps(rec))
        recs.append(rec)
    with open(args.out, "w") as f:
        for rec in recs:
            f.write(json.dumps(rec) + "\n")
    sys.exit(0 if all(r["ok"] for r in recs) else 1)


if __name__ == "__main__":
    main()
