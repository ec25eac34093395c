"""A small two-pass 6502 assembler for the synthetic NROM test ROMs.

No Super Mario Bros ROM is available to this build, so the emulator is exercised on NROM images
assembled here from this repository's own sources (`*.s` beside this file) plus generated fuzz images.

Syntax (one statement per line, `;` starts a comment):
    label:                      define a label at the current address
    NAME = expr                 define a constant
    .org expr                   set the current address (inside $8000-$FFFF)
    .byte e, e, "text"          raw bytes
    .word e, e                  little-endian 16-bit words
    .fill count, value          `count` copies of a byte
    .align n[, value]           pad to a multiple of n
    LDA #imm / zp / zp,X / abs / abs,X / abs,Y / (zp,X) / (zp),Y ; JMP (abs) ; ASL [A] ; BNE label
Expressions: decimal, $hex, %binary, 'c', symbols, `*` (current address), + - * / % & | ^ << >> ~,
unary `<` (low byte) and `>` (high byte), parentheses. A forward reference assembles as absolute.
"""
from __future__ import annotations

import re
import struct

# ---------------------------------------------------------------- opcode table (official opcodes)
# mode keys: imp acc imm zp zpx zpy abs absx absy ind indx indy rel
_OPS = {
    "ADC": dict(imm=0x69, zp=0x65, zpx=0x75, abs=0x6D, absx=0x7D, absy=0x79, indx=0x61, indy=0x71),
    "AND": dict(imm=0x29, zp=0x25, zpx=0x35, abs=0x2D, absx=0x3D, absy=0x39, indx=0x21, indy=0x31),
    "ASL": dict(acc=0x0A, zp=0x06, zpx=0x16, abs=0x0E, absx=0x1E),
    "BIT": dict(zp=0x24, abs=0x2C),
    "BPL": dict(rel=0x10), "BMI": dict(rel=0x30), "BVC": dict(rel=0x50), "BVS": dict(rel=0x70),
    "BCC": dict(rel=0x90), "BCS": dict(rel=0xB0), "BNE": dict(rel=0xD0), "BEQ": dict(rel=0xF0),
    "BRK": dict(imp=0x00),
    "CMP": dict(imm=0xC9, zp=0xC5, zpx=0xD5, abs=0xCD, absx=0xDD, absy=0xD9, indx=0xC1, indy=0xD1),
    "CPX": dict(imm=0xE0, zp=0xE4, abs=0xEC),
    "CPY": dict(imm=0xC0, zp=0xC4, abs=0xCC),
    "DEC": dict(zp=0xC6, zpx=0xD6, abs=0xCE, absx=0xDE),
    "EOR": dict(imm=0x49, zp=0x45, zpx=0x55, abs=0x4D, absx=0x5D, absy=0x59, indx=0x41, indy=0x51),
    "CLC": dict(imp=0x18), "SEC": dict(imp=0x38), "CLI": dict(imp=0x58), "SEI": dict(imp=0x78),
    "CLV": dict(imp=0xB8), "CLD": dict(imp=0xD8), "SED": dict(imp=0xF8),
    "INC": dict(zp=0xE6, zpx=0xF6, abs=0xEE, absx=0xFE),
    "JMP": dict(abs=0x4C, ind=0x6C),
    "JSR": dict(abs=0x20),
    "LDA": dict(imm=0xA9, zp=0xA5, zpx=0xB5, abs=0xAD, absx=0xBD, absy=0xB9, indx=0xA1, indy=0xB1),
    "LDX": dict(imm=0xA2, zp=0xA6, zpy=0xB6, abs=0xAE, absy=0xBE),
    "LDY": dict(imm=0xA0, zp=0xA4, zpx=0xB4, abs=0xAC, absx=0xBC),
    "LSR": dict(acc=0x4A, zp=0x46, zpx=0x56, abs=0x4E, absx=0x5E),
    "NOP": dict(imp=0xEA),
    "ORA": dict(imm=0x09, zp=0x05, zpx=0x15, abs=0x0D, absx=0x1D, absy=0x19, indx=0x01, indy=0x11),
    "TAX": dict(imp=0xAA), "TXA": dict(imp=0x8A), "DEX": dict(imp=0xCA), "INX": dict(imp=0xE8),
    "TAY": dict(imp=0xA8), "TYA": dict(imp=0x98), "DEY": dict(imp=0x88), "INY": dict(imp=0xC8),
    "ROL": dict(acc=0x2A, zp=0x26, zpx=0x36, abs=0x2E, absx=0x3E),
    "ROR": dict(acc=0x6A, zp=0x66, zpx=0x76, abs=0x6E, absx=0x7E),
    "RTI": dict(imp=0x40), "RTS": dict(imp=0x60),
    "SBC": dict(imm=0xE9, zp=0xE5, zpx=0xF5, abs=0xED, absx=0xFD, absy=0xF9, indx=0xE1, indy=0xF1),
    "STA": dict(zp=0x85, zpx=0x95, abs=0x8D, absx=0x9D, absy=0x99, indx=0x81, indy=0x91),
    "STX": dict(zp=0x86, zpy=0x96, abs=0x8E),
    "STY": dict(zp=0x84, zpx=0x94, abs=0x8C),
    "TXS": dict(imp=0x9A), "TSX": dict(imp=0xBA),
    "PHA": dict(imp=0x48), "PLA": dict(imp=0x68), "PHP": dict(imp=0x08), "PLP": dict(imp=0x28),
}
_SIZE = dict(imp=1, acc=1, imm=2, zp=2, zpx=2, zpy=2, abs=3, absx=3, absy=3, ind=3, indx=2, indy=2, rel=2)
OFFICIAL_OPCODES = sorted({op for modes in _OPS.values() for op in modes.values()})
assert len(OFFICIAL_OPCODES) == 151


class AsmError(Exception):
    pass


# ---------------------------------------------------------------- expressions
_TOK = re.compile(r"\s*(?:(\$[0-9A-Fa-f]+)|(%[01]+)|(\d+)|('.')|([A-Za-z_.@][A-Za-z0-9_.@]*)|(<<|>>|[-+*/%&|^~()<>]))")


class _Expr:
    def __init__(self, text, syms, pc):
        self.toks, pos = [], 0
        text = text.strip()
        while pos < len(text):
            m = _TOK.match(text, pos)
            if not m or m.end() == pos:
                raise AsmError(f"bad expression {text!r}")
            pos = m.end()
            self.toks.append(m.groups())
        self.i, self.syms, self.pc, self.unknown = 0, syms, pc, False

    def peek(self):
        return self.toks[self.i] if self.i < len(self.toks) else None

    def op(self):
        t = self.peek()
        return t[5] if t else None

    def eval(self):
        v = self.binary(0)
        if self.i != len(self.toks):
            raise AsmError("trailing tokens in expression")
        return v

    _PREC = [("|",), ("^",), ("&",), ("<<", ">>"), ("+", "-"), ("*", "/", "%")]

    def binary(self, lvl):
        if lvl == len(self._PREC):
            return self.unary()
        v = self.binary(lvl + 1)
        while self.op() in self._PREC[lvl]:
            o = self.op()
            self.i += 1
            w = self.binary(lvl + 1)
            v = {"|": lambda: v | w, "^": lambda: v ^ w, "&": lambda: v & w, "<<": lambda: v << w,
                 ">>": lambda: v >> w, "+": lambda: v + w, "-": lambda: v - w, "*": lambda: v * w,
                 "/": lambda: v // w if w else 0, "%": lambda: v % w if w else 0}[o]()
        return v

    def unary(self):
        o = self.op()
        if o in ("<", ">", "-", "~"):
            self.i += 1
            v = self.unary()
            return {"<": v & 0xFF, ">": (v >> 8) & 0xFF, "-": -v, "~": ~v}[o]
        if o == "*":
            self.i += 1
            return self.pc
        if o == "(":
            self.i += 1
            v = self.binary(0)
            if self.op() != ")":
                raise AsmError("missing )")
            self.i += 1
            return v
        t = self.peek()
        if t is None:
            raise AsmError("unexpected end of expression")
        self.i += 1
        hx, bn, dec, ch, name, _ = t
        if hx:
            return int(hx[1:], 16)
        if bn:
            return int(bn[1:], 2)
        if dec:
            return int(dec)
        if ch:
            return ord(ch[1])
        if name:
            if name in self.syms:
                return self.syms[name]
            self.unknown = True
            return 0
        raise AsmError(f"unexpected token {t}")


def _split_args(s):
    out, depth, cur, q = [], 0, "", False
    for c in s:
        if c == '"':
            q = not q
        if not q and c == "(":
            depth += 1
        if not q and c == ")":
            depth -= 1
        if c == "," and depth == 0 and not q:
            out.append(cur.strip())
            cur = ""
        else:
            cur += c
    if cur.strip():
        out.append(cur.strip())
    return out


class Assembler:
    def __init__(self, base=0x8000, size=0x8000):
        self.base, self.size = base, size

    def _parse_operand(self, mn, arg):
        """-> (mode candidates, expression text)."""
        modes = _OPS[mn]
        a = arg.strip()
        if not a or a.upper() == "A":
            return (["acc"] if "acc" in modes else ["imp"]), None
        if a.startswith("#"):
            return ["imm"], a[1:]
        if "rel" in modes:
            return ["rel"], a
        m = re.fullmatch(r"\((.*),\s*[Xx]\s*\)", a)
        if m:
            return ["indx"], m.group(1)
        m = re.fullmatch(r"\((.*)\)\s*,\s*[Yy]", a)
        if m:
            return ["indy"], m.group(1)
        forced_abs = a.lower().startswith("a:")
        if forced_abs:
            a = a[2:]
        m = re.fullmatch(r"(.*),\s*([XxYy])", a)
        if m:
            r = m.group(2).lower()
            cands = [f"abs{r}"] if forced_abs else [f"zp{r}", f"abs{r}"]
            return cands, m.group(1)
        if mn == "JMP" and a.startswith("(") and a.endswith(")"):
            return ["ind"], a[1:-1]
        return (["abs"] if forced_abs else ["zp", "abs"]), a

    def assemble(self, src: str) -> bytearray:
        lines = []
        for ln, raw in enumerate(src.splitlines(), 1):
            line = re.sub(r";.*$", "", raw.replace("\t", " ")).strip()
            if line:
                lines.append((ln, line))
        syms: dict[str, int] = {}
        sizes: dict[int, str] = {}
        for pass_no in range(8):
            img = bytearray([0xFF]) * self.size
            pc = self.base
            changed = False
            for ln, line in lines:
                try:
                    pc, ch = self._line(line, ln, pc, syms, sizes, img, pass_no)
                except AsmError as e:
                    raise AsmError(f"line {ln}: {e}: {line}") from None
                changed |= ch
            if pass_no >= 1 and not changed:
                return img
        raise AsmError("symbols did not converge")

    def _ev(self, text, syms, pc, final):
        e = _Expr(text, syms, pc)
        v = e.eval()
        if final and e.unknown:
            raise AsmError(f"undefined symbol in {text!r}")
        return v, e.unknown

    def _emit(self, img, pc, bs):
        for b in bs:
            off = pc - self.base
            if not 0 <= off < self.size:
                raise AsmError(f"address ${pc:04X} outside the PRG image")
            img[off] = b & 0xFF
            pc += 1
        return pc

    def _define(self, syms, name, v):
        changed = syms.get(name) != v
        syms[name] = v
        return changed

    def _line(self, line, ln, pc, syms, sizes, img, pass_no):
        changed = False
        final = pass_no >= 1
        m = re.match(r"^([A-Za-z_.@][A-Za-z0-9_.@]*):\s*(.*)$", line)
        if m:
            changed |= self._define(syms, m.group(1), pc)
            line = m.group(2).strip()
            if not line:
                return pc, changed
        m = re.match(r"^([A-Za-z_][A-Za-z0-9_]*)\s*(?:=|\.equ\b)\s*(.+)$", line)
        if m:
            v, unk = self._ev(m.group(2), syms, pc, False)
            if not unk:
                changed |= self._define(syms, m.group(1), v)
            elif final:
                raise AsmError("constant uses an undefined symbol")
            return pc, changed
        parts = line.split(None, 1)
        word, rest = parts[0], (parts[1] if len(parts) > 1 else "")
        wl = word.lower()
        if wl == ".org":
            return self._ev(rest, syms, pc, True)[0], changed
        if wl == ".byte":
            out = []
            for a in _split_args(rest):
                if a.startswith('"'):
                    out += list(a[1:-1].encode())
                else:
                    out.append(self._ev(a, syms, pc, final)[0])
            return self._emit(img, pc, out), changed
        if wl == ".word":
            out = []
            for a in _split_args(rest):
                v = self._ev(a, syms, pc, final)[0]
                out += [v & 0xFF, (v >> 8) & 0xFF]
            return self._emit(img, pc, out), changed
        if wl == ".fill":
            args = _split_args(rest)
            n = self._ev(args[0], syms, pc, True)[0]
            v = self._ev(args[1], syms, pc, final)[0] if len(args) > 1 else 0
            return self._emit(img, pc, [v] * n), changed
        if wl == ".align":
            args = _split_args(rest)
            n = self._ev(args[0], syms, pc, True)[0]
            v = self._ev(args[1], syms, pc, True)[0] if len(args) > 1 else 0xFF
            return self._emit(img, pc, [v] * ((-pc) % n)), changed
        mn = word.upper()
        if mn not in _OPS:
            raise AsmError(f"unknown mnemonic {word}")
        cands, expr = self._parse_operand(mn, rest)
        modes = _OPS[mn]
        cands = [c for c in cands if c in modes]
        if not cands:
            raise AsmError(f"addressing mode not available for {mn}")
        v, unk = (0, False) if expr is None else self._ev(expr, syms, pc, final)
        key = ln
        if key in sizes and sizes[key] in cands:
            mode = sizes[key]
            if mode.startswith("zp") and (unk or not 0 <= v < 256) and len(cands) > 1:
                mode = cands[-1]
        else:
            mode = cands[0] if (len(cands) == 1 or (not unk and 0 <= v < 256)) else cands[-1]
        if sizes.get(key) != mode:
            changed = True
        sizes[key] = mode
        op = modes[mode]
        n = _SIZE[mode]
        if mode == "rel":
            off = v - (pc + 2)
            if final and not -128 <= off <= 127:
                raise AsmError(f"branch out of range ({off})")
            out = [op, off & 0xFF]
        elif n == 1:
            out = [op]
        elif n == 2:
            if final and not (mode == "imm" and -128 <= v <= 255) and not 0 <= v <= 255:
                raise AsmError(f"operand ${v:X} does not fit in a byte")
            out = [op, v & 0xFF]
        else:
            out = [op, v & 0xFF, (v >> 8) & 0xFF]
        return self._emit(img, pc, out), changed


def ines(prg: bytes, chr_: bytes, mirroring: int = 1) -> bytes:
    """iNES image: mapper 0, 16/32 KB PRG, 8 KB CHR-ROM; mirroring 0 = horizontal, 1 = vertical."""
    if len(prg) not in (0x4000, 0x8000) or len(chr_) != 0x2000:
        raise ValueError("NROM needs 16 or 32 KB PRG and 8 KB CHR")
    hdr = b"NES\x1a" + struct.pack("BBBB", len(prg) // 0x4000, 1, mirroring & 1, 0) + bytes(8)
    return hdr + bytes(prg) + bytes(chr_)


def assemble(src: str, base: int = 0x8000) -> bytes:
    return bytes(Assembler(base, 0x10000 - base).assemble(src))
