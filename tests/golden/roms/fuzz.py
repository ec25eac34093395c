"""Generated NROM images for differential testing of the emulator core.

Two families, both fully determined by a seed:

* ``random_rom(seed)``: random PRG and CHR bytes with random vectors. The CPU executes noise: every
  opcode (official and not), every addressing mode, PPU/APU/joypad registers as operands and even
  as code addresses, BRK/RTI/JMP (ind) chains, stack wrap.
* ``program_rom(seed)``: a structured random program. A reset routine sets up PPU memory so a sprite-0
  hit happens on a known line; the main loop runs random official instructions over a pool of
  interesting addresses (RAM mirrors, PPU registers and their mirrors, OAM DMA, joypad ports),
  balanced stack traffic, subroutine calls, the SMB-shaped sprite-0 poll loop
  (`LDA $2002 / AND #$40 / BEQ`), and ends each pass with either `JMP *` (the idle loop the emulators
  fast-forward) or a jump back. The NMI handler does OAM DMA, VRAM / palette / scroll / control writes.
  With ``screen_off`` the NMI handler turns rendering off first (as Super Mario Bros.' does), makes its
  VRAM, scroll and address writes in that state (some with +32 increments, one a bulk $2007 loop) and
  turns rendering back on at its end, so the next frame draws with the fine x, v and name tables written
  while the screen was off.
"""
from __future__ import annotations

import numpy as np

try:
    from .asm6502 import _OPS, _SIZE, ines
except ImportError:  # loaded as a plain module
    from asm6502 import _OPS, _SIZE, ines

_MNEMONICS = sorted(_OPS)
_UNSAFE = {"JMP", "JSR", "RTS", "RTI", "BRK", "PHA", "PLA", "PHP", "PLP", "TXS", "SEI", "CLI",
           "BPL", "BMI", "BVC", "BVS", "BCC", "BCS", "BNE", "BEQ"}


def random_rom(seed: int) -> bytes:
    rng = np.random.default_rng(seed)
    banks = int(rng.integers(1, 3))
    prg = rng.integers(0, 256, 0x4000 * banks, dtype=np.uint8)
    chr_ = rng.integers(0, 256, 0x2000, dtype=np.uint8)
    # keep the vectors inside PRG most of the time so the noise runs from ROM
    for off in (0x3FFA, 0x3FFC, 0x3FFE):
        off += 0x4000 * (banks - 1)
        if rng.random() < 0.9:
            prg[off + 1] = rng.integers(0x80, 0x100)
    return ines(prg.tobytes(), chr_.tobytes(), int(rng.integers(0, 2)))


class _Gen:
    """Emits machine code into a 32 KB PRG image at $8000."""

    def __init__(self, rng):
        self.rng = rng
        self.img = bytearray([0xEA]) * 0x8000
        self.pc = 0x8000

    def emit(self, *bs):
        for b in bs:
            self.img[self.pc - 0x8000] = b & 0xFF
            self.pc += 1

    def op(self, mn, mode, val=0):
        code = _OPS[mn][mode]
        n = _SIZE[mode]
        if n == 1:
            self.emit(code)
        elif n == 2:
            self.emit(code, val)
        else:
            self.emit(code, val & 0xFF, val >> 8)

    def addr(self, write):
        r = self.rng.random()
        if r < 0.45:
            return int(self.rng.integers(0x0200, 0x0800)) + 0x800 * int(self.rng.integers(0, 4))
        if r < 0.60:
            reg = int(self.rng.choice([0, 1, 3, 4, 5, 6, 7, 2, 7, 5, 6]))
            return 0x2000 + reg + 8 * int(self.rng.integers(0, 2) * self.rng.integers(0, 1024))
        if r < 0.65:
            return int(self.rng.choice([0x4016, 0x4017, 0x4015, 0x4000, 0x5000, 0x6000]))
        if r < 0.70 and write:
            return 0x4014
        return int(self.rng.integers(0x8000, 0x10000))

    def random_insn(self, allow_io=True):
        rng = self.rng
        while True:
            mn = _MNEMONICS[int(rng.integers(0, len(_MNEMONICS)))]
            if mn not in _UNSAFE:
                break
        modes = sorted(_OPS[mn])
        mode = modes[int(rng.integers(0, len(modes)))]
        write = mn in ("STA", "STX", "STY", "INC", "DEC", "ASL", "LSR", "ROL", "ROR")
        if mode in ("imp", "acc"):
            self.op(mn, mode)
        elif mode == "imm":
            self.op(mn, mode, int(rng.integers(0, 256)))
        elif mode in ("zp", "zpx", "zpy"):
            self.op(mn, mode, int(rng.integers(0x10, 0x100)))
        elif mode in ("indx", "indy"):
            self.op(mn, mode, int(rng.choice([0x00, 0x02, 0x04, 0x06, 0xFE, 0xFF])))
        else:
            a = self.addr(write) if allow_io else int(rng.integers(0x0200, 0x0800))
            if a == 0x4014 and not write:
                a = 0x0300
            if a == 0x4014 and mn != "STA":
                a = 0x0300
            self.op(mn, mode, a)


def program_rom(seed: int, length: int = 400, screen_off: bool = False) -> bytes:
    rng = np.random.default_rng(seed)
    g = _Gen(rng)
    # ---- CHR: tile 1 is solid, the rest random
    chr_ = bytearray(rng.integers(0, 256, 0x2000, dtype=np.uint8).tobytes())
    for page in (0, 0x1000):
        for i in range(16):
            chr_[page + 16 + i] = 0xFF
    # ---- reset routine at $8000
    g.pc = 0x8000
    reset = g.pc
    g.emit(0x78, 0xD8, 0xA2, 0xFF, 0x9A)                        # SEI CLD LDX #$FF TXS
    g.emit(0xA9, 0x00, 0x8D, 0x00, 0x20, 0x8D, 0x01, 0x20)      # PPU off
    # zero-page pointers used by (zp,X) / (zp),Y point into RAM
    for zp in (0x00, 0x02, 0x04, 0x06, 0xFE):
        lo = int(rng.integers(0, 256)); hi = int(rng.integers(0x02, 0x08))
        g.emit(0xA9, lo, 0x85, zp, 0xA9, hi, 0x85, zp + 1 if zp < 0xFF else 0x00)
    # fill the first nametable with the solid tile on a band of rows (sprite-0 hits there)
    g.emit(0xA9, 0x20, 0x8D, 0x06, 0x20, 0xA9, 0x00, 0x8D, 0x06, 0x20)   # $2006 = $2000
    g.emit(0xA2, 0x00)                                                     # LDX #0
    loop = g.pc
    g.emit(0xA9, 0x01, 0x8D, 0x07, 0x20, 0xE8, 0xD0, (loop - (loop + 8)) & 0xFF)
    # palette
    g.emit(0xA9, 0x3F, 0x8D, 0x06, 0x20, 0xA9, 0x00, 0x8D, 0x06, 0x20)
    for i in range(32):
        g.emit(0xA9, int(rng.integers(0, 64)), 0x8D, 0x07, 0x20)
    # sprite 0 in OAM shadow page $0200 on a solid row
    g.emit(0xA9, int(rng.integers(8, 60)), 0x8D, 0x00, 0x02, 0xA9, 0x01, 0x8D, 0x01, 0x02,
           0xA9, int(rng.integers(0, 4)), 0x8D, 0x02, 0x02, 0xA9, int(rng.integers(8, 240)), 0x8D, 0x03, 0x02)
    g.emit(0xA9, 0x90 | int(rng.integers(0, 2)) << 5, 0x8D, 0x00, 0x20)   # NMI on, maybe 8x16
    g.emit(0xA9, 0x1E, 0x8D, 0x01, 0x20)                                   # BG + sprites on
    main = g.pc
    subs = []
    # ---- main body
    for _ in range(length):
        r = rng.random()
        if r < 0.70:
            g.random_insn()
        elif r < 0.75:                                       # balanced stack traffic
            push = 0x48 if rng.random() < 0.5 else 0x08
            g.emit(push)
            g.random_insn(allow_io=False)
            g.emit(0x68 if push == 0x48 else 0x28)
        elif r < 0.80:                                       # forward branch over one 3-byte insn
            g.emit(int(rng.choice([0x10, 0x30, 0x50, 0x70, 0x90, 0xB0, 0xD0, 0xF0])), 3)
            g.op("LDA", "abs", int(rng.integers(0x0200, 0x0800)))
        elif r < 0.83:                                       # subroutine call (fixed up later)
            g.emit(0x20, 0, 0)
            subs.append(g.pc - 2)
        elif r < 0.85:                                       # SMB-shaped poll: wait for sprite-0 clear
            top = g.pc
            g.emit(0xAD, 0x02, 0x20, 0x29, 0x40, 0xD0, (top - (top + 7)) & 0xFF)
        elif r < 0.86:                                       # wait for set (hits on the solid band)
            top = g.pc
            g.emit(0xAD, 0x02, 0x20, 0x29, 0x40, 0xF0, (top - (top + 7)) & 0xFF)
        elif r < 0.88:                                       # rare unofficial opcode, then re-sync
            g.emit(int(rng.choice([0x02, 0x04, 0x0B, 0x1A, 0x44, 0x80, 0x89, 0x9C, 0xA3, 0xC2, 0xE2, 0xFF])),
                   0xEA, 0xEA)
        else:
            g.random_insn()
    if rng.random() < 0.6:
        g.emit(0x4C, g.pc & 0xFF, g.pc >> 8)                  # JMP * (idle until NMI)
    else:
        g.emit(0x4C, main & 0xFF, main >> 8)
    # ---- subroutines
    sub_addrs = []
    for _ in range(4):
        sub_addrs.append(g.pc)
        for _ in range(int(rng.integers(3, 20))):
            g.random_insn()
        g.emit(0x60)
    for at in subs:
        a = sub_addrs[int(rng.integers(0, len(sub_addrs)))]
        g.img[at - 0x8000] = a & 0xFF
        g.img[at - 0x8000 + 1] = a >> 8
    # ---- NMI handler: DMA, VRAM / palette / scroll / control writes, then RTI
    nmi = g.pc
    g.emit(0x48, 0x8A, 0x48, 0x98, 0x48)                      # PHA TXA PHA TYA PHA
    g.emit(0xA9, 0x00, 0x8D, 0x03, 0x20)
    g.emit(0xA9, int(rng.choice([0x02, 0x02, 0x03, 0x07])), 0x8D, 0x14, 0x40)
    if screen_off:
        g.emit(0xA9, 0x00, 0x8D, 0x01, 0x20)                  # rendering off
        g.emit(0xA9, 0x90 | int(rng.integers(0, 2)) << 2, 0x8D, 0x00, 0x20)   # NMI on, +1 or +32 increments
        a = int(rng.integers(0x2000, 0x3000))                 # bulk $2007 run: LDX #n / STA $2007 / DEX / BNE
        g.emit(0xA9, a >> 8, 0x8D, 0x06, 0x20, 0xA9, a & 0xFF, 0x8D, 0x06, 0x20,
               0xA9, int(rng.integers(0, 256)), 0xA2, int(rng.integers(1, 256)))
        top = g.pc
        g.emit(0x8D, 0x07, 0x20, 0xCA, 0xD0, (top - (top + 6)) & 0xFF)
    for _ in range(int(rng.integers(2, 12))):
        k = rng.random()
        if screen_off and k < 0.15:                           # scroll pair (fine x) or a lone $2006 write
            if rng.random() < 0.5:
                g.emit(0xA9, int(rng.integers(0, 256)), 0x8D, 0x05, 0x20, 0xA9, int(rng.integers(0, 256)), 0x8D, 0x05, 0x20)
            else:
                g.emit(0xA9, int(rng.integers(0, 256)), 0x8D, 0x06, 0x20)
        elif k < 0.4:                                           # VRAM byte at a random nametable address
            a = int(rng.integers(0x2000, 0x3000))
            g.emit(0xAD, 0x02, 0x20, 0xA9, a >> 8, 0x8D, 0x06, 0x20, 0xA9, a & 0xFF, 0x8D, 0x06, 0x20,
                   0xA9, int(rng.integers(0, 256)), 0x8D, 0x07, 0x20)
        elif k < 0.55:                                        # palette entry
            a = 0x3F00 + int(rng.integers(0, 32))
            g.emit(0xA9, 0x3F, 0x8D, 0x06, 0x20, 0xA9, a & 0xFF, 0x8D, 0x06, 0x20,
                   0xA9, int(rng.integers(0, 64)), 0x8D, 0x07, 0x20)
        elif k < 0.7:                                         # $2007 read
            g.emit(0xAD, 0x07, 0x20)
        else:
            g.random_insn()
    g.emit(0xAD, 0x02, 0x20)                                 # reset the write toggle
    g.emit(0xA9, int(rng.integers(0, 256)), 0x8D, 0x05, 0x20, 0xA9, int(rng.integers(0, 240)), 0x8D, 0x05, 0x20)
    g.emit(0xA9, 0x90 | (int(rng.integers(0, 8)) << 3 & 0x38) | int(rng.integers(0, 4)), 0x8D, 0x00, 0x20)
    g.emit(0xA9, int(rng.choice([0x1E, 0x18, 0x1E, 0x08, 0x10, 0x1A, 0x1C])), 0x8D, 0x01, 0x20)
    g.emit(0x68, 0xA8, 0x68, 0xAA, 0x68, 0x40)                # PLA TAY PLA TAX PLA RTI
    irq = g.pc
    g.emit(0x40)
    assert g.pc < 0xFFF0, "program too long"
    g.img[0x7FFA:0x8000] = bytes([nmi & 0xFF, nmi >> 8, reset & 0xFF, reset >> 8, irq & 0xFF, irq >> 8])
    return ines(bytes(g.img), bytes(chr_), int(rng.integers(0, 2)))
