"""Builds the synthetic workload ROMs: `python tests/golden/roms/build_roms.py` writes
mini_smb_{vanilla,downsample,pixel,rectangle}.nes beside this file.

The four images share the same program (mini_smb.s) and differ only in their CHR art, the way the
gym-super-mario-bros ROM modes differ only in graphics:
  vanilla     detailed procedural tile art
  downsample  each 2x2 pixel block repeats its top-left pixel
  pixel       each tile is one colour (its most frequent one)
  rectangle   each tile is a filled rectangle with a one-pixel border in another colour
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
from asm6502 import assemble, ines  # noqa: E402

MODES = ("vanilla", "downsample", "pixel", "rectangle")

_DIGITS = [
    "01110 10001 10011 10101 11001 10001 01110",
    "00100 01100 00100 00100 00100 00100 01110",
    "01110 10001 00001 00010 00100 01000 11111",
    "11111 00010 00100 00010 00001 10001 01110",
    "00010 00110 01010 10010 11111 00010 00010",
    "11111 10000 11110 00001 00001 10001 01110",
    "00110 01000 10000 11110 10001 10001 01110",
    "11111 00001 00010 00100 01000 01000 01000",
    "01110 10001 10001 01110 10001 10001 01110",
    "01110 10001 10001 01111 00001 00010 01100",
]


def _tiles_vanilla() -> np.ndarray:
    """(256, 8, 8) 2-bit pixel values."""
    rng = np.random.default_rng(1985)
    t = np.zeros((256, 8, 8), np.uint8)
    t[0x01] = 3
    for d, rows in enumerate(_DIGITS):
        for y, r in enumerate(rows.split()):
            for x, c in enumerate(r):
                t[0x30 + d, y, x + 1] = 3 if c == "1" else 0
    for k in range(0x3A, 0x40):                      # letters: blocky glyphs
        t[k] = (rng.integers(0, 2, (8, 8)) * 3).astype(np.uint8)
        t[k, 7] = 0
    yy, xx = np.mgrid[0:8, 0:8]
    for q in range(4):                              # ground: bricks with mortar lines
        g = np.full((8, 8), 2, np.uint8)
        g[(yy + 4 * (q >> 1)) % 8 == 0] = 1
        g[(xx + 4 * ((yy // 4 + q) & 1)) % 8 == 0] = 1
        t[0x40 + q] = g
    for q in range(4):                              # brick
        g = np.full((8, 8), 2, np.uint8)
        g[yy % 4 == 3] = 3
        g[((xx + 4 * ((yy // 4) & 1)) % 8 == 0) & (yy % 4 != 3)] = 3
        t[0x44 + q] = g
    for q in range(4):                              # question block
        g = np.full((8, 8), 2, np.uint8)
        g[0, :] = 3; g[:, 0] = 3
        if q == 0:
            g[3:6, 4:7] = 1
        if q == 3:
            g[7, :] = 1; g[:, 7] = 1
        t[0x48 + q] = g
    for q in range(4):                              # pipe columns
        g = np.full((8, 8), 1, np.uint8)
        g[:, (q * 3) % 8] = 3
        g[:, (q * 3 + 1) % 8] = 2
        t[0x4C + q] = g
    for q in range(4):                              # used block
        g = np.full((8, 8), 1, np.uint8)
        g[(xx + yy) % 5 == 0] = 3
        t[0x50 + q] = g
    for q in range(4):                              # flag base
        t[0x54 + q] = np.where((xx ^ yy) & 2, 2, 3)
    mario = rng.integers(0, 4, (16, 16)).astype(np.uint8)
    mario[:2, :] = 0; mario[:, :3] = 0; mario[:, 13:] = 0
    mario[2:5, 4:12] = 1; mario[11:16, 3:7] = 2; mario[11:16, 9:13] = 2
    for k in range(4):
        t[0x10 + k] = mario[(k >> 1) * 8:(k >> 1) * 8 + 8, (k & 1) * 8:(k & 1) * 8 + 8]
    goomba = np.zeros((16, 16), np.uint8)
    r2 = (np.mgrid[0:16, 0:16] - 7.5) ** 2
    goomba[(r2[0] / 64 + r2[1] / 49) < 1] = 1
    goomba[5:8, 4:6] = 3; goomba[5:8, 10:12] = 3; goomba[13:16, 2:7] = 2; goomba[13:16, 9:14] = 2
    flat = np.zeros((16, 16), np.uint8)
    flat[11:16, 1:15] = 1; flat[12:14, 4:12] = 3
    for k in range(4):
        sl = (slice((k >> 1) * 8, (k >> 1) * 8 + 8), slice((k & 1) * 8, (k & 1) * 8 + 8))
        t[0x20 + k] = goomba[sl]
        t[0x24 + k] = flat[sl]
    t[0x28] = 0; t[0x28][:, 3:5] = 3
    for k in range(0x60, 0x100):                    # filler: random art, exercises every colour
        t[k] = rng.integers(0, 4, (8, 8)).astype(np.uint8)
    return t


def _transform(t: np.ndarray, mode: str) -> np.ndarray:
    if mode == "vanilla":
        return t
    out = t.copy()
    if mode == "downsample":
        out = t[:, ::2, ::2].repeat(2, 1).repeat(2, 2)
    elif mode == "pixel":
        for k in range(256):
            out[k] = np.bincount(t[k].ravel(), minlength=4).argmax()
    elif mode == "rectangle":
        for k in range(256):
            c = np.bincount(t[k].ravel(), minlength=4).argmax()
            out[k] = c
            if c:
                out[k, 0, :] = out[k, 7, :] = out[k, :, 0] = out[k, :, 7] = (c % 3) + 1
    else:
        raise ValueError(mode)
    out[0x01] = 3   # the sprite-0 tile stays solid in every mode
    out[0x00] = 0
    return out


def chr_bytes(mode: str) -> bytes:
    t = _transform(_tiles_vanilla(), mode)
    planes = np.zeros((256, 16), np.uint8)
    w = (1 << (7 - np.arange(8))).astype(np.uint8)
    planes[:, :8] = ((t & 1) * w).sum(2)
    planes[:, 8:] = (((t >> 1) & 1) * w).sum(2)
    half = planes.tobytes()
    return half + half                                # same art in both pattern tables


def build(mode: str = "vanilla") -> bytes:
    with open(os.path.join(HERE, "mini_smb.s")) as f:
        prg = assemble(f.read())
    return ines(prg, chr_bytes(mode), mirroring=1)


def rom_path(mode: str = "vanilla") -> str:
    return os.path.join(HERE, f"mini_smb_{mode}.nes")


if __name__ == "__main__":
    for m in MODES:
        data = build(m)
        with open(rom_path(m), "wb") as f:
            f.write(data)
        print(rom_path(m), len(data))
