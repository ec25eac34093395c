"""ALU test ROMs with a textbook model of the expected results.

Each ROM runs a straight-line list of cases from its reset routine:
    CLV; CLC|SEC; LDA #a; <op>; STA $0200+2i; PHP; PLA; STA $0201+2i
then idles in `JMP *`. The expected (result, pushed status byte) of every case is computed here from
the 6502's arithmetic definitions (signed overflow as an out-of-range signed sum, borrow as a
negative difference, ...) and mapped to nes-py's status byte layout (N=0x01, V=0x02, bit2=0x04,
B=0x08, D=0x10, I=0x20, Z=0x40, C=0x80; the reset value 0x34 with D cleared by CLD gives 0x24).
"""
from __future__ import annotations

import numpy as np

try:
    from .asm6502 import ines
except ImportError:
    from asm6502 import ines

OPS = ("ADC", "SBC", "CMP", "AND", "ORA", "EOR", "BIT", "ASL", "ROL", "LSR", "ROR", "INC", "DEC", "CPX", "CPY")
_IMM = {"ADC": 0x69, "SBC": 0xE9, "CMP": 0xC9, "AND": 0x29, "ORA": 0x09, "EOR": 0x49, "CPX": 0xE0, "CPY": 0xC0}
_ACC = {"ASL": 0x0A, "ROL": 0x2A, "LSR": 0x4A, "ROR": 0x6A}
N_CASES = 760
BASE_P = 0x24


def _s8(v):
    return v - 256 if v >= 128 else v


def textbook(op, a, m, c):
    """-> (result byte stored, N, V, Z, C) with V/C None when the op leaves them unchanged (V is 0 after CLV)."""
    if op == "ADC":
        s = a + m + c
        r = s & 0xFF
        return r, r >> 7, int(not -128 <= _s8(a) + _s8(m) + c <= 127), int(r == 0), int(s > 255)
    if op == "SBC":
        d = a - m - (1 - c)
        r = d & 0xFF
        return r, r >> 7, int(not -128 <= _s8(a) - _s8(m) - (1 - c) <= 127), int(r == 0), int(d >= 0)
    if op in ("CMP", "CPX", "CPY"):
        d = (a - m) & 0xFF
        return a, d >> 7, 0, int(a == m), int(a >= m)
    if op in ("AND", "ORA", "EOR"):
        r = {"AND": a & m, "ORA": a | m, "EOR": a ^ m}[op]
        return r, r >> 7, 0, int(r == 0), c
    if op == "BIT":
        return a, m >> 7, (m >> 6) & 1, int((a & m) == 0), c
    if op in ("ASL", "ROL"):
        r = ((a << 1) | (c if op == "ROL" else 0)) & 0xFF
        return r, r >> 7, 0, int(r == 0), a >> 7
    if op in ("LSR", "ROR"):
        r = (a >> 1) | ((c << 7) if op == "ROR" else 0)
        return r, r >> 7, 0, int(r == 0), a & 1
    if op in ("INC", "DEC"):
        r = (m + (1 if op == "INC" else -1)) & 0xFF
        return r, r >> 7, 0, int(r == 0), c
    raise ValueError(op)


def status_byte(n, v, z, c):
    return BASE_P | (0x01 if n else 0) | (0x02 if v else 0) | (0x40 if z else 0) | (0x80 if c else 0)


def cases(seed):
    rng = np.random.default_rng(seed)
    edge = np.array([0x00, 0x01, 0x7F, 0x80, 0x81, 0xFE, 0xFF, 0x40, 0x3F, 0xC0])
    out = []
    for i in range(N_CASES):
        op = OPS[int(rng.integers(0, len(OPS)))]
        pick = lambda: int(edge[rng.integers(0, len(edge))]) if rng.random() < 0.3 else int(rng.integers(0, 256))  # noqa: E731
        out.append((op, pick(), pick(), int(rng.integers(0, 2))))
    return out


def build(seed) -> tuple[bytes, np.ndarray]:
    """-> (iNES image, expected RAM bytes $0200..$0200+2*N_CASES)."""
    code = bytearray([0x78, 0xD8, 0xA2, 0xFF, 0x9A])            # SEI CLD LDX #$FF TXS
    expect = np.zeros(2 * N_CASES, np.uint8)
    for i, (op, a, m, c) in enumerate(cases(seed)):
        code += bytes([0xB8, 0x38 if c else 0x18])               # CLV; SEC / CLC
        if op in _IMM and op not in ("CPX", "CPY"):
            code += bytes([0xA9, a, _IMM[op], m])                # LDA #a; op #m
        elif op == "CPX":
            code += bytes([0xA2, a, 0xE0, m, 0x8A])              # LDX #a; CPX #m; TXA
        elif op == "CPY":
            code += bytes([0xA0, a, 0xC0, m, 0x98])              # LDY #a; CPY #m; TYA
        elif op == "BIT":
            code += bytes([0xA2, m, 0x86, 0x10, 0xA9, a, 0x24, 0x10])   # LDX #m; STX $10; LDA #a; BIT $10
        elif op in _ACC:
            code += bytes([0xA9, a, _ACC[op]])                   # LDA #a; op A
        else:                                                    # INC / DEC zero page, then LDA it
            code += bytes([0xA2, m, 0x86, 0x10, 0xE6 if op == "INC" else 0xC6, 0x10, 0xA5, 0x10])
        # LDA/TXA/TYA above set N/Z before the op except for INC/DEC (whose LDA sets them again) and
        # CPX/CPY/BIT (whose TXA/TYA/none keep them): capture the flags right after the op instead.
        addr = 0x0200 + 2 * i
        if op in ("CPX", "CPY"):
            code = code[:-1]                                     # drop TXA/TYA: A := a via LDA below
            code += bytes([0x08])                                # PHP (flags of the compare)
            code += bytes([0xA9, a, 0x8D, addr & 0xFF, addr >> 8, 0x68, 0x8D, (addr + 1) & 0xFF, (addr + 1) >> 8])
        elif op in ("INC", "DEC"):
            code = code[:-2]                                     # drop LDA $10
            code += bytes([0x08, 0xA5, 0x10, 0x8D, addr & 0xFF, addr >> 8, 0x68, 0x8D, (addr + 1) & 0xFF, (addr + 1) >> 8])
        else:
            code += bytes([0x08, 0x8D, addr & 0xFF, addr >> 8, 0x68, 0x8D, (addr + 1) & 0xFF, (addr + 1) >> 8])
        r, n, v, z, cc = textbook(op, a, m, c)
        expect[2 * i] = r
        expect[2 * i + 1] = status_byte(n, v, z, cc)
    here = 0x8000 + len(code)
    code += bytes([0x4C, here & 0xFF, here >> 8])                # JMP *
    prg = bytearray([0xEA]) * 0x8000
    prg[:len(code)] = code
    prg[0x7FFA:0x8000] = bytes([here & 0xFF, here >> 8, 0x00, 0x80, here & 0xFF, here >> 8])
    return ines(bytes(prg), bytes(0x2000), 1), expect
