// Device-side NES console for gfx950: one env per lane.
//
// Layout in HBM (all lane-interleaved, NP = env count rounded up to a multiple of 64):
//   MEM[row * NP + e]  one byte per row: RAM 0..2047, VRAM 2048..4095, OAM 4096..4351, PAL 4352..4383.
//                      Lanes that touch the same emulated address touch one contiguous 64-byte run.
//   SC[word * NP + e]  32-bit scalar registers of the CPU / PPU / joypads (enum Scalar).
// PRG (32 KB) and CHR (8 KB) are read-only and shared by every env: each workgroup stages them in LDS.
//
// The machine follows the reference's nes-py-exact model (csrc/nes_core.hpp): instruction-atomic CPU
// with skip cycles, catch-up PPU advanced only at PPU register accesses / the NMI point / frame end,
// exact sprite-0 hit, nes-py's flag layout and bus quirks. Counters are kept relative to the current
// frame start (32-bit) instead of the reference's absolute int64 values; the 64-bit iteration count at
// the frame start is only needed for the OAM-DMA odd/even cycle (nes_core.hpp:194).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// an empty asm that makes the compiler hold x in a vector register at this point (the host build of this
// code, tests/hostbuild, defines it with a host register constraint)
#ifndef MH_REG_BARRIER
#define MH_REG_BARRIER(x) asm volatile("" : "+v"(x))
#endif

namespace mh {

constexpr int ROW_RAM = 0, ROW_VRAM = 2048, ROW_OAM = 4096, ROW_PAL = 4352, MEM_ROWS = 4384;
// Most envs (consoles) of one instance: the padded count np (a multiple of 64) keeps MEM_ROWS * np below
// 2^32, so every byte of the console memory has a 32-bit offset from its base.
constexpr uint32_t MAX_ENVS = (uint32_t)((0xffffffffull / MEM_ROWS) & ~63ull);
static_assert(MAX_ENVS == 979648 && (uint64_t)MEM_ROWS * MAX_ENVS <= 0xffffffffull, "32-bit console memory offsets");
// Emulator launch shape. Each env runs on LANES_PER_ENV lanes of a 64-lane wave (its parts: lanes
// s, s + ENVS_PER_WAVE, ...), so a wave carries ENVS_PER_WAVE = 64 / LANES_PER_ENV envs, and a block of
// WAVES_PER_BLOCK waves holds LDS_LANES = 128 env slots sharing one LDS copy of the cartridge. The parts run
// the same console in lockstep, which costs the wave nothing (an instruction issues once for all its lanes),
// and split the renderer's pixel groups and the sprite evaluation between them. Fewer envs per wave means
// fewer divergent instruction streams per wave; with 2 parts, 32768 envs are 1024 waves, one per SIMD; with
// 4 parts they are 2048 waves in blocks of 8, two per SIMD, so one wave issues while the other waits.
#ifndef MH_LANES_PER_ENV
#define MH_LANES_PER_ENV 4
#endif
constexpr int LANES_PER_ENV = MH_LANES_PER_ENV;
// (1 lane per env is the host build of this code, tests/hostbuild: one lane plays the whole wave of an env)
static_assert(LANES_PER_ENV == 1 || LANES_PER_ENV == 2 || LANES_PER_ENV == 4, "an env runs on 1, 2 or 4 lanes");
constexpr int ENVS_PER_WAVE = 64 / LANES_PER_ENV;
constexpr int LDS_LANES = 128;                                  // env slots sharing one block's per-lane LDS buffers
constexpr int WAVES_PER_BLOCK = LDS_LANES / ENVS_PER_WAVE;
constexpr int EMU_WAVES_PER_SIMD = WAVES_PER_BLOCK / 4;        // one block per CU (its LDS), 4 SIMDs per CU
// a wave's ballot bit of every part of the env in its lane 0 (shifted by the env's slot in the wave)
constexpr uint64_t PART_LANES = LANES_PER_ENV == 1 ? 1ull : LANES_PER_ENV == 2 ? 0x0000000100000001ull
                                                                            : 0x0001000100010001ull;
constexpr int LDS_SP_WORDS = 64, LDS_GP_WORDS = 8; // words per lane: sprite line (256 B), gray palette (32 B)
constexpr int LDS_BG_WORDS = 20;                   // words per lane: two name-table rows (64 tiles) + their attributes
constexpr int LDS_BG_ATTR = 64;                    // byte offset of the attribute bytes in the tile row
constexpr int LDS_OAM_WORDS = 64;                  // words per lane: OAM (sprite i = word i: y, tile, attr, x)
constexpr int LDS_XCHG_WORDS = LANES_PER_ENV;     // words per env slot: the parts' pieces of the sprite-range mask
constexpr int LDS_GP_REGION = LDS_GP_WORDS + LDS_BG_WORDS + LDS_OAM_WORDS + LDS_XCHG_WORDS;   // palette, tile row, OAM, exchange
constexpr int FRAME_ITERS = 29781;                 // CPU iterations per nes-py Emulator::step
#ifndef MH_LONE_MAX_ENVS
#define MH_LONE_MAX_ENVS 6
#endif
// Lone runs (Console::lone_run) take over a wave's instructions once at most this many of its consoles have any
// left in the current stretch: those consoles' runs follow one another.
constexpr int LONE_MAX_ENVS = MH_LONE_MAX_ENVS;
// Render lines per frame slice (a power of two). A wave runs its lanes' CPUs to the end of a group of
// this many lines and then catches their PPUs up together; a wave iteration costs the slowest lane's
// instruction, so longer slices let the lanes' per-line instruction counts average out, while a lane
// that must catch up inside a slice (a PPU register access) renders those lines alone. 8 measured best.
constexpr int SLICE_LINES = 8;
constexpr int LINE_END = 341;
constexpr int GRAY_PIX = 256 * 240;
// Byte offset of VRAM word w (bytes 4w .. 4w+3) of console e in a memory block of np consoles. The VRAM
// span of the block (rows ROW_VRAM .. ROW_VRAM + 2047 of the byte-row layout) holds 32-bit words, word w of
// console e at index w np + e: one load fetches four consecutive VRAM bytes of a console.
__device__ __forceinline__ size_t vram_word_offset(uint32_t np, uint32_t e, uint32_t w) {
    return (size_t)ROW_VRAM * np + ((size_t)w * np + e) * 4;
}
// Console::ppu_flags bits: PPUMASK (show / hide-edge, bits 0-3) and PPUCTRL (bits 4-8) settings
enum : uint32_t { PF_SHOW_BG = 1, PF_SHOW_SPR = 2, PF_HIDE_EDGE_BG = 4, PF_HIDE_EDGE_SPR = 8, PF_LONG_SPR = 16,
                  PF_NMI_EN = 32, PF_BG_PAGE = 64, PF_SPR_PAGE = 128, PF_INC32 = 256 };
enum : uint8_t { FN = 0x01, FV = 0x02, FONE = 0x04, FB = 0x08, FD = 0x10, FI = 0x20, FZ = 0x40, FC = 0x80 };
// Error flags or-ed into a console's bad-op counter (every parity check requires a zero count):
// ERR_HACK_LIMIT  the env layer's busy-state loop hit its frame limit;
// ERR_TWIN        a sprite evaluation ran on some of an env's lanes without the others, so the pieces of the
//                 sprite-range mask it read from their exchange words were stale.
constexpr uint32_t ERR_HACK_LIMIT = 1u << 24, ERR_TWIN = 1u << 25, ERR_FLAGS = ERR_HACK_LIMIT | ERR_TWIN;
enum : uint8_t { ST_PRE = 0, ST_RENDER = 1, ST_POST = 2, ST_VBLANK = 3 };

// Scalar words of one console, interleaved as SC[w * NP + e].
enum Scalar : int {
    S_ITER_LO = 0, S_ITER_HI, S_EXEC_REL, S_PC, S_SP, S_A, S_X, S_Y, S_P, S_ZERO_SKIP,
    S_JOY_STROBE0, S_JOY_STROBE1, S_JOY_BUTTONS0, S_JOY_BUTTONS1, S_JOY_BITS0, S_JOY_BITS1,
    S_PSTATE, S_EVEN, S_VBLANK, S_S0HIT, S_FIRST_WRITE, S_DATA_BUFFER, S_OAM_ADDR, S_FINE_X,
    S_SHOW_BG, S_SHOW_SPR, S_HIDE_EDGE_BG, S_HIDE_EDGE_SPR, S_LONG_SPR, S_NMI_EN, S_BG_PAGE, S_SPR_PAGE,
    S_NSL, S_SL_LO, S_SL_HI, S_PCYC, S_SCANLINE, S_V, S_T, S_INC, S_COUNT
};

// Base cycles per opcode (data table of nes_core.hpp:42-51; 0 = not an official opcode).
constexpr uint8_t kCycleData[256] = {
    7, 6, 0, 0, 0, 3, 5, 0, 3, 2, 2, 0, 0, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    6, 6, 0, 0, 3, 3, 5, 0, 4, 2, 2, 0, 4, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    6, 6, 0, 0, 0, 3, 5, 0, 3, 2, 2, 0, 3, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    6, 6, 0, 0, 0, 3, 5, 0, 4, 2, 2, 0, 5, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    0, 6, 0, 0, 3, 3, 3, 0, 2, 0, 2, 0, 4, 4, 4, 0, 2, 6, 0, 0, 4, 4, 4, 0, 2, 5, 2, 0, 0, 5, 0, 0,
    2, 6, 2, 0, 3, 3, 3, 0, 2, 2, 2, 0, 4, 4, 4, 0, 2, 5, 0, 0, 4, 4, 4, 0, 2, 4, 2, 0, 4, 4, 4, 0,
    2, 6, 0, 0, 3, 3, 5, 0, 2, 2, 2, 0, 4, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    2, 6, 0, 0, 3, 3, 5, 0, 2, 2, 2, 2, 4, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
};

// ---------------------------------------------------------------- decode table
// One word per opcode with everything the fast instruction path needs, generated from the
// reference's decode cascade (implied, branch, type 1, type 2, type 0; nes_core.hpp:619-1163):
// addressing mode, page-cross rule, data read, ALU operation, source and destination register,
// stack / control-flow operation, flag class and base cycles. Invalid opcodes keep their addressing
// (type 0 with an invalid operation still consumes its operand bytes and page-cross cycle).
namespace dec {
enum : uint32_t { M_NONE = 0, M_IMM, M_ZP, M_ZPX, M_ZPY, M_ABS, M_ABSX, M_ABSY, M_INDX, M_INDY };
enum : uint32_t { OP_PASS = 0, OP_ORA, OP_AND, OP_EOR, OP_ADC, OP_SBC, OP_CMP, OP_BIT, OP_ASL, OP_ROL, OP_LSR,
                  OP_ROR, OP_INC, OP_DEC, OP_FLAG, OP_NOP };
enum : uint32_t { R_M = 0, R_A, R_X, R_Y, R_SP };                       // R_M: the data operand
enum : uint32_t { D_NONE = 0, D_A, D_X, D_Y, D_SP, D_MEM };
enum : uint32_t { X_NONE = 0, X_BRK, X_JSR, X_RTS, X_RTI, X_PHA, X_PHP, X_PLA, X_PLP, X_JMP, X_JMPI, X_BRANCH };
enum : uint32_t { FL_NONE = 0, FL_NZ, FL_NZC, FL_NZCV, FL_BIT, FL_OP };
constexpr uint32_t PEN = 1u << 4, RD = 1u << 5, OK = 1u << 7;
constexpr int ALU_SH = 8, SRC_SH = 12, DST_SH = 15, X_SH = 18, FL_SH = 22, FOP_SH = 25, CYC_SH = 28;

constexpr uint32_t mk(uint32_t am, bool pen, bool rd, bool ok, uint32_t alu, uint32_t src, uint32_t dst,
                      uint32_t x, uint32_t fl, uint32_t fop = 0) {
    return am | (pen ? PEN : 0u) | (rd ? RD : 0u) | (ok ? OK : 0u) | alu << ALU_SH | src << SRC_SH |
           dst << DST_SH | x << X_SH | fl << FL_SH | fop << FOP_SH;
}
constexpr uint32_t entry(int op) {
    const int cc = op & 3, bbb = (op >> 2) & 7, fn = op >> 5;
    const uint32_t cyc = (uint32_t)kCycleData[op] << CYC_SH;
    switch (op) {   // the implied table (nes_core.hpp:630-690); flag ops: fop 0 CLC 1 SEC 2 CLI 3 SEI 4 CLV 5 CLD 6 SED
        case 0x00: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_BRK, FL_NONE) | cyc;
        case 0x08: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_PHP, FL_NONE) | cyc;
        case 0x18: return mk(M_NONE, false, false, true, OP_FLAG, R_M, D_NONE, X_NONE, FL_OP, 0) | cyc;
        case 0x20: return mk(M_ABS, false, false, true, OP_NOP, R_M, D_NONE, X_JSR, FL_NONE) | cyc;
        case 0x28: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_PLP, FL_NONE) | cyc;
        case 0x38: return mk(M_NONE, false, false, true, OP_FLAG, R_M, D_NONE, X_NONE, FL_OP, 1) | cyc;
        case 0x40: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_RTI, FL_NONE) | cyc;
        case 0x48: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_PHA, FL_NONE) | cyc;
        case 0x4c: return mk(M_ABS, false, false, true, OP_NOP, R_M, D_NONE, X_JMP, FL_NONE) | cyc;
        case 0x58: return mk(M_NONE, false, false, true, OP_FLAG, R_M, D_NONE, X_NONE, FL_OP, 2) | cyc;
        case 0x60: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_RTS, FL_NONE) | cyc;
        case 0x68: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_PLA, FL_NONE) | cyc;
        case 0x6c: return mk(M_ABS, false, false, true, OP_NOP, R_M, D_NONE, X_JMPI, FL_NONE) | cyc;
        case 0x78: return mk(M_NONE, false, false, true, OP_FLAG, R_M, D_NONE, X_NONE, FL_OP, 3) | cyc;
        case 0x88: return mk(M_NONE, false, false, true, OP_DEC, R_Y, D_Y, X_NONE, FL_NZ) | cyc;
        case 0x8a: return mk(M_NONE, false, false, true, OP_PASS, R_X, D_A, X_NONE, FL_NZ) | cyc;
        case 0x98: return mk(M_NONE, false, false, true, OP_PASS, R_Y, D_A, X_NONE, FL_NZ) | cyc;
        case 0x9a: return mk(M_NONE, false, false, true, OP_PASS, R_X, D_SP, X_NONE, FL_NONE) | cyc;
        case 0xa8: return mk(M_NONE, false, false, true, OP_PASS, R_A, D_Y, X_NONE, FL_NZ) | cyc;
        case 0xaa: return mk(M_NONE, false, false, true, OP_PASS, R_A, D_X, X_NONE, FL_NZ) | cyc;
        case 0xb8: return mk(M_NONE, false, false, true, OP_FLAG, R_M, D_NONE, X_NONE, FL_OP, 4) | cyc;
        case 0xba: return mk(M_NONE, false, false, true, OP_PASS, R_SP, D_X, X_NONE, FL_NZ) | cyc;
        case 0xc8: return mk(M_NONE, false, false, true, OP_INC, R_Y, D_Y, X_NONE, FL_NZ) | cyc;
        case 0xca: return mk(M_NONE, false, false, true, OP_DEC, R_X, D_X, X_NONE, FL_NZ) | cyc;
        case 0xd8: return mk(M_NONE, false, false, true, OP_FLAG, R_M, D_NONE, X_NONE, FL_OP, 5) | cyc;
        case 0xe8: return mk(M_NONE, false, false, true, OP_INC, R_X, D_X, X_NONE, FL_NZ) | cyc;
        case 0xea: return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_NONE, FL_NONE) | cyc;
        case 0xf8: return mk(M_NONE, false, false, true, OP_FLAG, R_M, D_NONE, X_NONE, FL_OP, 6) | cyc;
        default: break;
    }
    if ((op & 0x1f) == 0x10) return mk(M_NONE, false, false, true, OP_NOP, R_M, D_NONE, X_BRANCH, FL_NONE) | cyc;
    if (cc == 1) {
        const uint32_t am = bbb == 0 ? M_INDX : bbb == 1 ? M_ZP : bbb == 2 ? M_IMM : bbb == 3 ? M_ABS
                          : bbb == 4 ? M_INDY : bbb == 5 ? M_ZPX : bbb == 6 ? M_ABSY : M_ABSX;
        const bool pen = fn != 4 && (bbb == 4 || bbb == 6 || bbb == 7);
        switch (fn) {
            case 0: return mk(am, pen, true, true, OP_ORA, R_A, D_A, X_NONE, FL_NZ) | cyc;
            case 1: return mk(am, pen, true, true, OP_AND, R_A, D_A, X_NONE, FL_NZ) | cyc;
            case 2: return mk(am, pen, true, true, OP_EOR, R_A, D_A, X_NONE, FL_NZ) | cyc;
            case 3: return mk(am, pen, true, true, OP_ADC, R_A, D_A, X_NONE, FL_NZCV) | cyc;
            case 4: return mk(am, pen, false, true, OP_PASS, R_A, D_MEM, X_NONE, FL_NONE) | cyc;
            case 5: return mk(am, pen, true, true, OP_PASS, R_M, D_A, X_NONE, FL_NZ) | cyc;
            case 6: return mk(am, pen, true, true, OP_CMP, R_A, D_NONE, X_NONE, FL_NZC) | cyc;
            default: return mk(am, pen, true, true, OP_SBC, R_A, D_A, X_NONE, FL_NZCV) | cyc;
        }
    }
    if (cc == 2 && bbb != 4 && bbb != 6) {
        const bool xy = fn == 4 || fn == 5;
        const uint32_t am = bbb == 0 ? M_IMM : bbb == 1 ? M_ZP : bbb == 2 ? M_NONE : bbb == 3 ? M_ABS
                          : bbb == 5 ? (xy ? M_ZPY : M_ZPX) : (xy ? M_ABSY : M_ABSX);
        const bool pen = bbb == 7, acc = bbb == 2;
        if (fn < 4) {
            const uint32_t alu = fn == 0 ? OP_ASL : fn == 1 ? OP_ROL : fn == 2 ? OP_LSR : OP_ROR;
            return (acc ? mk(am, pen, false, true, alu, R_A, D_A, X_NONE, FL_NZC)
                        : mk(am, pen, true, true, alu, R_M, D_MEM, X_NONE, FL_NZC)) | cyc;
        }
        switch (fn) {
            case 4: return mk(am, pen, false, true, OP_PASS, R_X, D_MEM, X_NONE, FL_NONE) | cyc;
            case 5: return mk(am, pen, true, true, OP_PASS, R_M, D_X, X_NONE, FL_NZ) | cyc;
            case 6: return mk(am, pen, true, true, OP_DEC, R_M, D_MEM, X_NONE, FL_NZ) | cyc;
            default: return mk(am, pen, true, true, OP_INC, R_M, D_MEM, X_NONE, FL_NZ) | cyc;
        }
    }
    if (cc == 0 && (bbb & 1 || bbb == 0)) {
        const uint32_t am = bbb == 0 ? M_IMM : bbb == 1 ? M_ZP : bbb == 3 ? M_ABS : bbb == 5 ? M_ZPX : M_ABSX;
        const bool pen = bbb == 7;
        switch (fn) {
            case 1: return mk(am, pen, true, true, OP_BIT, R_A, D_NONE, X_NONE, FL_BIT) | cyc;
            case 4: return mk(am, pen, false, true, OP_PASS, R_Y, D_MEM, X_NONE, FL_NONE) | cyc;
            case 5: return mk(am, pen, true, true, OP_PASS, R_M, D_Y, X_NONE, FL_NZ) | cyc;
            case 6: return mk(am, pen, true, true, OP_CMP, R_Y, D_NONE, X_NONE, FL_NZC) | cyc;
            case 7: return mk(am, pen, true, true, OP_CMP, R_X, D_NONE, X_NONE, FL_NZC) | cyc;
            default: return mk(am, pen, false, false, OP_NOP, R_M, D_NONE, X_NONE, FL_NONE) | cyc;
        }
    }
    return mk(M_NONE, false, false, false, OP_NOP, R_M, D_NONE, X_NONE, FL_NONE) | cyc;
}
struct Table {
    uint32_t w[256];
    constexpr Table() : w() {
        for (int i = 0; i < 256; i++) w[i] = entry(i);
    }
};
}  // namespace dec

__device__ __constant__ static const dec::Table kDecode{};

// Read-only cartridge view: PRG/CHR in LDS, name-table offsets in registers (uniform).
// Pointers through which wave-uniform addresses of read-only data are loaded with scalar loads (the constant
// address space): the PRG image in device memory, which no kernel writes.
#ifndef MH_SCALAR_CONST
#define MH_SCALAR_CONST __attribute__((address_space(4)))
#endif
// Device memory addressed as such (global loads and stores: no flat-address aperture check, and their waits
// count only vector memory, not the scalar loads in flight beside them)
#ifndef MH_GLOBAL
#define MH_GLOBAL __attribute__((address_space(1)))
#endif

// ---------------------------------------------------------------- long lone runs
// A console that is one of the last few of its wave with instructions to run (at most LONE_MAX_ENVS; the frame
// loop calls Console::lone_run() for each of them in turn, under its own lanes) runs them in lone_long(): out of
// line, in registers of its own (not the frame loop's), wave-uniform, with one body per opcode whose decode word
// is known at compile time, so that the addressing, the operation, its flags and its control flow fold to the
// few scalar instructions the opcode needs. Measured on one console running a loop of register instructions:
// 0.18 us per instruction (built with the structurizer skipping uniform regions, which leaves the opcode switch a
// plain compare tree; 0.37 us without), against 0.67 us for a body that takes the decode word's fields at run
// time (inline, as a switch per field).
// The registers of a lone run, wave-uniform: pc, a, x, y, sp, p, exec_at (ex), zero_skip (zs), the PPU's v and t
// (vt: v | t << 16), fine x and write toggle (px: fine_x | first_write << 8; outputs: bit 16, the run wrote the
// name tables through $2007, and bit 17, it wrote a PPU register), and n, the instructions run (an output).
struct LoneRegs { uint32_t pc, a, x, y, sp, p; int32_t ex; uint32_t zs, vt, px, n; };
// LoneCore::pflags: the PPU register writes a lone run may make ($2005, $2006, $2007 to the pattern and name
// tables) while rendering is off, and the PPUCTRL bits they need
constexpr uint32_t LP_WRITES = 1u, LP_INC32 = 2u, LP_NT_SHIFT = 4;
struct LoneCore {
    LoneRegs r;
    MH_GLOBAL uint8_t* mem;                    // the console's RAM row 0 (row stride np), the same in every active lane
    MH_GLOBAL uint8_t* vmem;                   // its VRAM word 0 (word stride 4 np)
    uint32_t np, pflags;
    const MH_SCALAR_CONST uint32_t* gprg;      // PRG image (read only): scalar loads
    __device__ __forceinline__ uint32_t ram(uint32_t ad) const {
        return __builtin_amdgcn_readfirstlane(mem[(size_t)((ad & 0x7ffu) * np)]);
    }
    __device__ __forceinline__ void set_ram(uint32_t ad, uint32_t v) { mem[(size_t)((ad & 0x7ffu) * np)] = (uint8_t)v; }
    __device__ __forceinline__ uint32_t prg(uint32_t ad) const {
        ad &= 0x7fffu;
        return (gprg[ad >> 2] >> (8u * (ad & 3u))) & 0xffu;
    }
    // the bus reads and writes a lone run may make: RAM, PRG, and $4000-$7FFF but the joypads (reads) or OAM
    // DMA and the joypad strobe (writes), which read 0 and ignore writes; anything else (the PPU registers above
    // all) is left to frame()
    __device__ __forceinline__ static bool reads_ok(uint32_t ad) { return (ad - 0x2000u) >= 0x2000u && (ad | 1u) != 0x4017u; }
    __device__ __forceinline__ static bool writes_ok(uint32_t ad) { return (ad - 0x2000u) >= 0x2000u && (ad & ~2u) != 0x4014u; }
    __device__ __forceinline__ uint32_t read(uint32_t ad) const { return ad < 0x2000u ? ram(ad) : ad >= 0x8000u ? prg(ad) : 0u; }
    // While rendering is off (both PPUMASK show bits clear), the catch-up PPU neither moves v nor draws anything
    // but the universal background colour, so the scroll and address writes and the $2007 writes to the pattern
    // or name tables do not depend on where the PPU has been caught up to, and a lone run makes them without the
    // catch-up that frame() takes before a PPU register access (a lone run stops before the NMI point, and before
    // any other PPU register access, $2001 included). $2007 writes to the palette ($3EFF-$3FFE) change that
    // colour: left to frame().
    __device__ __forceinline__ bool ppu_write_ok(uint32_t ad) const {
        if (!(pflags & LP_WRITES) || (ad - 0x2000u) >= 0x2000u) return false;
        const uint32_t reg = ad & 7u, v = r.vt & 0xffffu;
        return reg == 5u || reg == 6u || (reg == 7u && (v - 0x3effu) >= 0x100u);
    }
    // scroll_write, addr_write and data_write (+ its sp_line reset), as Console does them
    __device__ __forceinline__ void ppu_write(uint32_t reg, uint32_t d) {
        uint32_t v = r.vt & 0xffffu, t = r.vt >> 16, fx = r.px & 0xffu, fw = (r.px >> 8) & 1u, dirty = r.px >> 16;
        if (reg == 5u) {
            if (fw) { t = (t & ~0x1fu) | (d >> 3); fx = d & 7u; fw = 0; }
            else { t = (t & ~0x73e0u) | ((d & 7u) << 12) | ((d & 0xf8u) << 2); fw = 1; }
        } else if (reg == 6u) {
            if (fw) { t = (t & 0x00ffu) | ((d & 0x3fu) << 8); fw = 0; }
            else { t = (t & 0xff00u) | d; v = t; fw = 1; }
        } else {
            if (v >= 0x2000u && v < 0x3effu) {   // name table (nt_row()): below $2000 the CHR ROM ignores writes
                const uint32_t k = v < 0x2400u ? 0u : v < 0x2800u ? 1u : v < 0x2c00u ? 2u : 3u;
                const uint32_t i = ((((pflags >> LP_NT_SHIFT) >> k) & 1u) << 10) | (v & 0x3ffu);
                vmem[(size_t)((i >> 2) * 4u * np) + (i & 3u)] = (uint8_t)d;
            }
            v = (v + ((pflags & LP_INC32) ? 32u : 1u)) & 0xffffu;
            dirty = 1;
        }
        r.vt = v | t << 16;
        r.px = fx | fw << 8 | dirty << 16 | 1u << 17;
    }
};

// One instruction of opcode OP (operand bytes b1, b2) on a lone console; false, with no effect, if it needs
// frame() (an invalid opcode, a bus access lone runs do not make). instruction()'s rules and the reference's
// results (nes_core.hpp:619-1163), with every choice on the decode word resolved at compile time.
template <uint32_t OP>
__device__ __forceinline__ bool lone_op(LoneCore& c, uint32_t b1, uint32_t b2) {
    using namespace dec;
    constexpr uint32_t D = entry((int)OP);
    constexpr uint32_t am = D & 15u, alu = (D >> ALU_SH) & 15u, src = (D >> SRC_SH) & 7u, dst = (D >> DST_SH) & 7u;
    constexpr uint32_t xop = (D >> X_SH) & 15u, fl = (D >> FL_SH) & 7u, fop = (D >> FOP_SH) & 7u;
    constexpr bool rd = (D & RD) != 0, wr = dst == D_MEM, pen = (D & PEN) != 0;
    constexpr bool zpm = am == M_ZP || am == M_ZPX || am == M_ZPY;   // zero-page modes touch RAM only
    if constexpr (!(D & OK)) {
        return false;
    } else {
        LoneRegs& r = c.r;
        if constexpr (OP == 0x4cu)
            if ((b1 | b2 << 8) == r.pc) return false;   // JMP *: frame()'s idle fast-forward
        const uint32_t absv = b1 | b2 << 8;
        const uint32_t p2 = (absv & 0xff00u) | ((absv + 1u) & 0xffu);   // JMP (ind): high byte, page wrap
        uint32_t ea = 0, base = absv;
        int32_t sk = 0;
        if constexpr (am == M_IMM) ea = (r.pc + 1u) & 0xffffu;
        if constexpr (am == M_ZP) ea = b1;
        if constexpr (am == M_ZPX) ea = (b1 + r.x) & 0xffu;
        if constexpr (am == M_ZPY) ea = (b1 + r.y) & 0xffu;
        if constexpr (am == M_ABS) ea = absv;
        if constexpr (am == M_ABSX) ea = (absv + r.x) & 0xffffu;
        if constexpr (am == M_ABSY) ea = (absv + r.y) & 0xffffu;
        if constexpr (am == M_INDX) { const uint32_t z = (b1 + r.x) & 0xffu; ea = c.ram(z) | c.ram((z + 1u) & 0xffu) << 8; }
        if constexpr (am == M_INDY) { base = c.ram(b1) | c.ram((b1 + 1u) & 0xffu) << 8; ea = (base + r.y) & 0xffffu; }
        if constexpr (xop == X_JMPI) {
            if (!LoneCore::reads_ok(absv) || !LoneCore::reads_ok(p2)) return false;
        } else {
            if constexpr (rd && am != M_IMM && !zpm) if (!LoneCore::reads_ok(ea)) return false;
            if constexpr (wr && !zpm) if (!LoneCore::writes_ok(ea) && !c.ppu_write_ok(ea)) return false;
        }
        if constexpr (pen && (am == M_ABSX || am == M_ABSY || am == M_INDY)) sk = ((base ^ ea) & 0xff00u) ? 1 : 0;
        uint32_t m = b1;
        if constexpr (rd && am != M_IMM) m = zpm ? c.ram(ea) : c.read(ea);
        // the operation (alu_op()'s results): result, carry out, overflow
        const uint32_t rv = src == R_A ? r.a : src == R_X ? r.x : src == R_Y ? r.y : src == R_SP ? r.sp : m;
        const uint32_t sv = rd ? m : rv, cin = (r.p >> 7) & 1u;   // FC is bit 7
        uint32_t res = sv, c_out = 0, v_out = 0;
        if constexpr (alu == OP_ORA) res = r.a | m;
        if constexpr (alu == OP_AND) res = r.a & m;
        if constexpr (alu == OP_EOR) res = r.a ^ m;
        if constexpr (alu == OP_ADC || alu == OP_SBC || alu == OP_CMP) {
            const uint32_t ax = alu == OP_CMP ? rv : r.a, m2 = alu == OP_ADC ? m : m ^ 0xffu;
            const uint32_t t = ax + m2 + (alu == OP_CMP ? 1u : cin);
            res = t & 0xffu; c_out = t >> 8; v_out = (ax ^ t) & (m2 ^ t) & 0x80u;
        }
        if constexpr (alu == OP_ASL) { res = (sv << 1) & 0xffu; c_out = sv >> 7; }
        if constexpr (alu == OP_ROL) { res = ((sv << 1) | cin) & 0xffu; c_out = sv >> 7; }
        if constexpr (alu == OP_LSR) { res = sv >> 1; c_out = sv & 1u; }
        if constexpr (alu == OP_ROR) { res = (sv >> 1) | cin << 7; c_out = sv & 1u; }
        if constexpr (alu == OP_INC) res = (sv + 1u) & 0xffu;
        if constexpr (alu == OP_DEC) res = (sv - 1u) & 0xffu;
        const uint32_t nz = (res ? 0u : (uint32_t)FZ) | (res >> 7);   // FN is bit 0
        if constexpr (fl == FL_NZ) r.p = (r.p & ~(uint32_t)(FZ | FN)) | nz;
        if constexpr (fl == FL_NZC) r.p = (r.p & ~(uint32_t)(FZ | FN | FC)) | nz | (c_out ? (uint32_t)FC : 0u);
        if constexpr (fl == FL_NZCV)
            r.p = (r.p & ~(uint32_t)(FZ | FN | FC | FV)) | nz | (c_out ? (uint32_t)FC : 0u) | (v_out ? (uint32_t)FV : 0u);
        if constexpr (fl == FL_BIT)
            r.p = (r.p & ~(uint32_t)(FZ | FV | FN)) | ((r.a & m) ? 0u : (uint32_t)FZ) | ((m & 0x40u) ? (uint32_t)FV : 0u) | (m >> 7);
        if constexpr (fl == FL_OP) {   // CLC SEC CLI SEI CLV CLD SED
            constexpr uint32_t fm = fop < 2 ? FC : fop < 4 ? FI : fop == 4 ? FV : FD;
            constexpr uint32_t fset = (fop == 1 || fop == 3 || fop == 6) ? fm : 0u;
            r.p = (r.p & ~fm) | fset;
        }
        if constexpr (dst == D_A) r.a = res;
        if constexpr (dst == D_X) r.x = res;
        if constexpr (dst == D_Y) r.y = res;
        if constexpr (dst == D_SP) r.sp = res;
        if constexpr (wr) {
            if (zpm || ea < 0x2000u) c.set_ram(ea, res);
            else if ((ea - 0x2000u) < 0x2000u) c.ppu_write(ea & 7u, res);   // admitted above (ppu_write_ok)
            // writes elsewhere are ignored
        }
        // control flow
        const uint32_t ret = (r.pc + 2u) & 0xffffu;
        uint32_t npc = (r.pc + (am == M_NONE ? 1u : (am == M_ABS || am == M_ABSX || am == M_ABSY) ? 3u : 2u)) & 0xffffu;
        if constexpr (xop == X_BRANCH) {   // on N, V, C, Z (op bits 6-7) equal to op bit 5
            constexpr uint32_t fbit = (0x40800201u >> (8 * (OP >> 6))) & 0xffu;   // FN FV FC FZ
            if (((r.p & fbit) != 0) == ((OP & 0x20u) != 0)) {
                npc = (ret + (uint32_t)(int32_t)(int8_t)b1) & 0xffffu;
                sk += ((ret ^ npc) & 0xff00u) ? 3 : 1;
            } else {
                npc = ret;
            }
        }
        if constexpr (xop == X_JMP) npc = absv;
        if constexpr (xop == X_JMPI) npc = c.read(absv) | c.read(p2) << 8;
        if constexpr (xop == X_JSR) {
            c.set_ram(0x100u | r.sp, ret >> 8);
            c.set_ram(0x100u | ((r.sp - 1u) & 0xffu), ret & 0xffu);
            r.sp = (r.sp - 2u) & 0xffu;
            npc = absv;
        }
        if constexpr (xop == X_BRK) {
            c.set_ram(0x100u | r.sp, ret >> 8);
            c.set_ram(0x100u | ((r.sp - 1u) & 0xffu), ret & 0xffu);
            c.set_ram(0x100u | ((r.sp - 2u) & 0xffu), r.p | 0x30u);
            r.sp = (r.sp - 3u) & 0xffu;
            r.p |= FI;
            npc = c.prg(0xfffe) | c.prg(0xffff) << 8;
            sk += 7;
        }
        if constexpr (xop == X_PHA || xop == X_PHP) {
            c.set_ram(0x100u | r.sp, xop == X_PHA ? r.a : r.p);
            r.sp = (r.sp - 1u) & 0xffu;
        }
        if constexpr (xop == X_PLA || xop == X_PLP) {
            const uint32_t u = c.ram(0x100u | ((r.sp + 1u) & 0xffu));
            r.sp = (r.sp + 1u) & 0xffu;
            if constexpr (xop == X_PLA) { r.a = u; r.p = (r.p & ~(uint32_t)(FZ | FN)) | (u ? 0u : (uint32_t)FZ) | (u >> 7); }
            else r.p = u;
        }
        if constexpr (xop == X_RTS) {
            const uint32_t lo = c.ram(0x100u | ((r.sp + 1u) & 0xffu)), hi = c.ram(0x100u | ((r.sp + 2u) & 0xffu));
            r.sp = (r.sp + 2u) & 0xffu;
            npc = ((lo | hi << 8) + 1u) & 0xffffu;
        }
        if constexpr (xop == X_RTI) {
            const uint32_t f = c.ram(0x100u | ((r.sp + 1u) & 0xffu)), lo = c.ram(0x100u | ((r.sp + 2u) & 0xffu)),
                           hi = c.ram(0x100u | ((r.sp + 3u) & 0xffu));
            r.sp = (r.sp + 3u) & 0xffu;
            r.p = f; npc = lo | hi << 8;
        }
        r.pc = npc;
        sk += (int32_t)((D >> CYC_SH) & 7u);
        r.ex += sk >= 1 ? sk : 1;
        r.zs = sk <= 0 ? 1u : 0u;   // opcodes the cycle table gives 0 cycles (and no penalty)
        return true;
    }
}

// A wave-uniform 64-bit value (a pointer): the builtin returns a signed int, so each half is taken as unsigned
// before it is widened (else the low half's bit 31 would spread into the high half).
__device__ __forceinline__ uint64_t lone_uniform64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (uint64_t)lo | (uint64_t)hi << 32;
}

// Runs lone instructions from r until one needs frame(): its catch-up point 3 (ex + 1) past lim, its opcode or
// operands outside PRG, the idle `JMP *`, or what lone_op() refuses. Returns the registers after the last one
// run and, in n, how many ran. Not inlined: its registers are its own, not the frame loop's.
__device__ __attribute__((noinline)) LoneRegs lone_long(LoneRegs in, int32_t lim, uint8_t* mem, uint8_t* vmem,
                                                        uint32_t np, uint32_t pflags, const uint8_t* gprg) {
    LoneCore c;
    c.r.pc = __builtin_amdgcn_readfirstlane(in.pc); c.r.a = __builtin_amdgcn_readfirstlane(in.a);
    c.r.x = __builtin_amdgcn_readfirstlane(in.x); c.r.y = __builtin_amdgcn_readfirstlane(in.y);
    c.r.sp = __builtin_amdgcn_readfirstlane(in.sp); c.r.p = __builtin_amdgcn_readfirstlane(in.p);
    c.r.ex = (int32_t)__builtin_amdgcn_readfirstlane((uint32_t)in.ex);
    c.r.zs = __builtin_amdgcn_readfirstlane(in.zs);
    c.r.vt = __builtin_amdgcn_readfirstlane(in.vt); c.r.px = __builtin_amdgcn_readfirstlane(in.px);
    lim = (int32_t)__builtin_amdgcn_readfirstlane((uint32_t)lim);
    c.mem = (MH_GLOBAL uint8_t*)(void*)lone_uniform64((uint64_t)mem);
    c.vmem = (MH_GLOBAL uint8_t*)(void*)lone_uniform64((uint64_t)vmem);
    c.np = __builtin_amdgcn_readfirstlane(np);
    c.pflags = __builtin_amdgcn_readfirstlane(pflags);
    c.gprg = (const MH_SCALAR_CONST uint32_t*)(const void*)lone_uniform64((uint64_t)gprg);
    // the catch-up test 3 (ex + 1) > lim as ex > exlim, exlim = floor((lim - 3) / 3)
    const int32_t l3 = lim - 3;
    const int32_t exlim = l3 / 3 - (l3 % 3 < 0 ? 1 : 0);
    uint32_t n = 0;
    for (;;) {
        if (c.r.ex > exlim) break;                         // parks or catches up in frame()
        if (c.r.pc - 0x8000u > 0x7ffdu) break;             // opcode or operands through the bus
        const uint32_t pa = c.r.pc & 0x7fffu;
        const uint64_t w = (uint64_t)c.gprg[(pa >> 2) + 1] << 32 | c.gprg[pa >> 2];
        const uint32_t b0 = (uint32_t)(w >> (8 * (pa & 3u)));   // bytes pc .. pc + 3
        const uint32_t op = b0 & 0xffu, b1 = (b0 >> 8) & 0xffu, b2 = (b0 >> 16) & 0xffu;
        switch (op) {   // an opcode that needs frame() (lone_op() false) ends the run
#define MH_LONE_CASE(i) case i: if (!lone_op<i>(c, b1, b2)) goto done; break;
#define MH_LONE_CASE4(i) MH_LONE_CASE(i) MH_LONE_CASE(i + 1) MH_LONE_CASE(i + 2) MH_LONE_CASE(i + 3)
#define MH_LONE_CASE16(i) MH_LONE_CASE4(i) MH_LONE_CASE4(i + 4) MH_LONE_CASE4(i + 8) MH_LONE_CASE4(i + 12)
#define MH_LONE_CASE64(i) MH_LONE_CASE16(i) MH_LONE_CASE16(i + 16) MH_LONE_CASE16(i + 32) MH_LONE_CASE16(i + 48)
            MH_LONE_CASE64(0) MH_LONE_CASE64(64) MH_LONE_CASE64(128) MH_LONE_CASE64(192)
#undef MH_LONE_CASE64
#undef MH_LONE_CASE16
#undef MH_LONE_CASE4
#undef MH_LONE_CASE
            default: goto done;
        }
        n++;
    }
done:
    c.r.n = n;
    return c.r;
}

struct Cart {
    const uint8_t* prg;      // 0x8000 bytes (16 KB images mirrored)
    const uint8_t* gprg;     // the same PRG image in device memory (scalar loads of wave-uniform addresses)
    const uint8_t* chr;      // 0x2000 bytes
    const uint32_t* dec;     // decode words (LDS copy of kDecode)
    uint32_t nt_bits;        // bit k set: name table k ($2000 + k * $400) maps to VRAM $400, else to $000
};

struct Console {
    // ---- memory views
    // Addresses are a wave-uniform base and a 32-bit per-lane byte offset (the MEM array is below 4 GiB:
    // MAX_ENVS), so a load or store is one address add into the offset and the base stays in scalar registers.
    uint8_t* mbase;          // MEM: row r of env e at byte r * np + e
    uint32_t eo;             // e
    uint32_t vo;             // byte offset of this env's VRAM word 0 (word w at vo + 4 w np)
    uint32_t np;
    Cart cart;
    uint8_t* gray;           // GRAY slot + 4 e: pixels 4i..4i+3 in the 32-bit word at gray + 4 i np
    const uint8_t* lut;      // palette value -> gray (LDS, 256 entries)
    bool render;
    uint8_t part;            // which of the env's LANES_PER_ENV lanes this is (all run the console; the
                             // renderer and the sprite evaluation split their work between them)
    // Small fields share 32-bit words as bitfields (8 or 16 bits wide, so they wrap as the byte and
    // half-word types they stand for): the compiler keeps a word in one register instead of one per
    // field. Fewer live registers mean fewer spills, and fewer register copies where the paths of
    // the frame loop join.
    // ---- CPU
    uint16_t pc;
    uint32_t a : 8, x : 8, y : 8, sp : 8;
    uint8_t p;
    int32_t exec_at, ppu_calls, nmi_thresh;  // relative to the current frame start
    uint32_t iter_lo;                        // low word of the iteration count at the frame start
    uint32_t iter_hi;
    int32_t cur, skip;
    // ---- joypads
    // both ports in one word (buttons 0 | buttons 1 << 8 | shift register 0 << 16 | shift register 1 << 24);
    // their strobes are bits 0 and 1 of joy_strobe (below)
    uint32_t joy;
    // ---- PPU
    uint32_t pstate : 8, even : 8, vblank : 8, s0hit : 8;
    uint32_t first_write : 8, joy_strobe : 8, zero_skip : 8, pal_dirty : 8;   // zero_skip: CPU, pal_dirty: derived
    uint32_t fine_x : 8, oam_addr : 8, data_buffer : 8, nsl : 8;
    // ppu_flags: the PPUCTRL / PPUMASK settings as PF_* bits; bg_key: name table and coarse y (v bits 5-11)
    // of the tile row held in LDS (-1: none)
    uint32_t ppu_flags : 16;
    int32_t bg_key : 16;
    uint32_t sl_lo, sl_hi;                   // sprite list: 8 indices packed in two words
    int32_t pcyc, scanline;
    uint32_t v : 16, t : 16;
    // ---- counters
    uint32_t bad_ops, instructions;          // instructions: retired, poll-loop fast-forwards included
    uint32_t ff_instructions;                // of those, the ones poll_skip fast-forwarded without executing
    uint32_t nframe;                         // frame() calls since load(): the wave's issue priority in frame()
    // ---- derived state (not part of the machine state)
    // pend_line: scanline of a sprite evaluation not yet materialized (-1: the list is current);
    // sp_line: scanline the LDS sprite line buffer holds (-1: invalid); pal_dirty (above): the LDS gray
    // palette must be rebuilt
    int32_t pend_line : 16, sp_line : 16;
    uint32_t* lds_sp;        // per-lane sprite line buffer: word (x / 4) of this lane at lds_sp[(x / 4) * LDS_LANES]
    uint32_t* lds_gp;        // per-lane gray palette: word (i / 4) at lds_gp[(i / 4) * LDS_LANES]
    uint32_t* lds_bg;        // per-lane background tile row (same word stride), valid for v's bits 5-11 == bg_key
    uint32_t* lds_oam;       // per-lane OAM (same word stride): the live copy between load()/power_on() and store()

    // ------------------------------------------------------------ interleaved memory
    __device__ __forceinline__ uint8_t ld(uint32_t row) const { return mbase[(uint32_t)__umul24(row, np) + eo]; }
    __device__ __forceinline__ void st(uint32_t row, uint8_t val) { mbase[(uint32_t)__umul24(row, np) + eo] = val; }
    __device__ __forceinline__ uint8_t ram(uint32_t a) const { return ld(ROW_RAM + (a & 0x7ff)); }
    __device__ __forceinline__ uint8_t oam(uint32_t i) const {
        i &= 0xff;
        return ((const uint8_t*)lds_oam)[(i >> 2) * LDS_LANES * 4 + (i & 3)];
    }
    __device__ __forceinline__ void set_oam(uint32_t i, uint8_t val) {
        i &= 0xff;
        ((uint8_t*)lds_oam)[(i >> 2) * LDS_LANES * 4 + (i & 3)] = val;
    }
    // sprite k's four OAM bytes: y | tile << 8 | attr << 16 | x << 24
    __device__ __forceinline__ uint32_t oam_sprite(int k) const { return lds_oam[k * LDS_LANES]; }
    __device__ __forceinline__ uint8_t pal(uint32_t i) const { return ld(ROW_PAL + (i & 0x1f)); }
    // VRAM is word-interleaved: byte i of this env is byte i % 4 of 32-bit word i / 4, and word w sits at
    // byte vo + 4 w np of MEM, so a name-table row is 8 word loads
    __device__ __forceinline__ uint8_t vram(uint32_t i) const {
        i &= 0x7ff;
        return mbase[vo + (uint32_t)__umul24(i >> 2, 4 * np) + (i & 3)];
    }
    __device__ __forceinline__ void set_vram(uint32_t i, uint8_t d) {
        i &= 0x7ff;
        mbase[vo + (uint32_t)__umul24(i >> 2, 4 * np) + (i & 3)] = d;
    }
    __device__ __forceinline__ uint32_t vram_word(uint32_t w) const {
        return *(const uint32_t*)(mbase + (vo + (uint32_t)__umul24(w & 0x1ff, 4 * np)));
    }
    __device__ __forceinline__ uint8_t sl(int k) const {
        return (uint8_t)((k < 4 ? sl_lo >> (8 * k) : sl_hi >> (8 * (k - 4))) & 0xff);
    }
    __device__ __forceinline__ void set_sl(int k, uint8_t i) {
        if (k < 4) sl_lo = (sl_lo & ~(0xffu << (8 * k))) | ((uint32_t)i << (8 * k));
        else sl_hi = (sl_hi & ~(0xffu << (8 * (k - 4)))) | ((uint32_t)i << (8 * (k - 4)));
    }
    __device__ __forceinline__ uint8_t prg(uint16_t a) const { return cart.prg[a & 0x7fff]; }
    // PPUCTRL / PPUMASK settings (0 or 1; inc(): the VRAM address increment, 1 or 32)
    __device__ __forceinline__ uint32_t show_bg() const { return ppu_flags & 1u; }
    __device__ __forceinline__ uint32_t show_spr() const { return (ppu_flags >> 1) & 1u; }
    __device__ __forceinline__ uint32_t hide_edge_bg() const { return (ppu_flags >> 2) & 1u; }
    __device__ __forceinline__ uint32_t hide_edge_spr() const { return (ppu_flags >> 3) & 1u; }
    __device__ __forceinline__ uint32_t long_spr() const { return (ppu_flags >> 4) & 1u; }
    __device__ __forceinline__ uint32_t nmi_en() const { return (ppu_flags >> 5) & 1u; }
    __device__ __forceinline__ uint32_t bg_page() const { return (ppu_flags >> 6) & 1u; }
    __device__ __forceinline__ uint32_t spr_page() const { return (ppu_flags >> 7) & 1u; }
    __device__ __forceinline__ uint16_t inc() const { return (ppu_flags & PF_INC32) ? 32 : 1; }
    // joypad port 0's buttons for the next frames (the env layer's action)
    __device__ __forceinline__ void set_buttons0(uint8_t b) { joy = (joy & ~0xffu) | b; }

    // ------------------------------------------------------------ state in / out
    __device__ void load(const uint32_t* sc, uint32_t e) {
        auto w = [&](int k) { return sc[(size_t)k * np + e]; };
        iter_lo = w(S_ITER_LO); iter_hi = w(S_ITER_HI);
        exec_at = (int32_t)w(S_EXEC_REL);
        ppu_calls = 0;
        pc = (uint16_t)w(S_PC); sp = (uint8_t)w(S_SP); a = (uint8_t)w(S_A); x = (uint8_t)w(S_X);
        y = (uint8_t)w(S_Y); p = (uint8_t)w(S_P); zero_skip = (uint8_t)w(S_ZERO_SKIP);
        joy_strobe = (uint8_t)((w(S_JOY_STROBE0) & 1u) | (w(S_JOY_STROBE1) & 1u) << 1);
        joy = (w(S_JOY_BUTTONS0) & 0xffu) | (w(S_JOY_BUTTONS1) & 0xffu) << 8 | (w(S_JOY_BITS0) & 0xffu) << 16 |
              (w(S_JOY_BITS1) & 0xffu) << 24;
        pstate = (uint8_t)w(S_PSTATE); even = (uint8_t)w(S_EVEN); vblank = (uint8_t)w(S_VBLANK);
        s0hit = (uint8_t)w(S_S0HIT); first_write = (uint8_t)w(S_FIRST_WRITE);
        data_buffer = (uint8_t)w(S_DATA_BUFFER); oam_addr = (uint8_t)w(S_OAM_ADDR); fine_x = (uint8_t)w(S_FINE_X);
        ppu_flags = (w(S_SHOW_BG) ? PF_SHOW_BG : 0u) | (w(S_SHOW_SPR) ? PF_SHOW_SPR : 0u) |
                    (w(S_HIDE_EDGE_BG) ? PF_HIDE_EDGE_BG : 0u) | (w(S_HIDE_EDGE_SPR) ? PF_HIDE_EDGE_SPR : 0u) |
                    (w(S_LONG_SPR) ? PF_LONG_SPR : 0u) | (w(S_NMI_EN) ? PF_NMI_EN : 0u) |
                    (w(S_BG_PAGE) ? PF_BG_PAGE : 0u) | (w(S_SPR_PAGE) ? PF_SPR_PAGE : 0u) |
                    (w(S_INC) == 32 ? PF_INC32 : 0u);
        nsl = (uint8_t)w(S_NSL); sl_lo = w(S_SL_LO); sl_hi = w(S_SL_HI);
        pcyc = (int32_t)w(S_PCYC); scanline = (int32_t)w(S_SCANLINE);
        v = (uint16_t)w(S_V); t = (uint16_t)w(S_T);
        pend_line = -1; sp_line = -1; pal_dirty = true; bg_key = -1;
        for (int k = 0; k < LDS_OAM_WORDS; k++) {
            const uint32_t r = ROW_OAM + 4 * k;
            lds_oam[k * LDS_LANES] = (uint32_t)ld(r) | (uint32_t)ld(r + 1) << 8 | (uint32_t)ld(r + 2) << 16 |
                                     (uint32_t)ld(r + 3) << 24;
        }
        nmi_threshold();
        nframe = 0;
    }
    __device__ void store(uint32_t* sc, uint32_t e) {
        materialize_sprites();
        for (int k = 0; k < LDS_OAM_WORDS; k++) {
            const uint32_t w = oam_sprite(k), r = ROW_OAM + 4 * k;
            st(r, (uint8_t)w); st(r + 1, (uint8_t)(w >> 8)); st(r + 2, (uint8_t)(w >> 16)); st(r + 3, (uint8_t)(w >> 24));
        }
        auto w = [&](int k, uint32_t val) { sc[(size_t)k * np + e] = val; };
        w(S_ITER_LO, iter_lo); w(S_ITER_HI, iter_hi); w(S_EXEC_REL, (uint32_t)exec_at);
        w(S_PC, pc); w(S_SP, sp); w(S_A, a); w(S_X, x); w(S_Y, y); w(S_P, p); w(S_ZERO_SKIP, zero_skip);
        w(S_JOY_STROBE0, joy_strobe & 1u); w(S_JOY_STROBE1, (joy_strobe >> 1) & 1u);
        w(S_JOY_BUTTONS0, joy & 0xffu); w(S_JOY_BUTTONS1, (joy >> 8) & 0xffu);
        w(S_JOY_BITS0, (joy >> 16) & 0xffu); w(S_JOY_BITS1, joy >> 24);
        w(S_PSTATE, pstate); w(S_EVEN, even); w(S_VBLANK, vblank); w(S_S0HIT, s0hit);
        w(S_FIRST_WRITE, first_write); w(S_DATA_BUFFER, data_buffer); w(S_OAM_ADDR, oam_addr);
        w(S_FINE_X, fine_x); w(S_SHOW_BG, show_bg()); w(S_SHOW_SPR, show_spr());
        w(S_HIDE_EDGE_BG, hide_edge_bg()); w(S_HIDE_EDGE_SPR, hide_edge_spr()); w(S_LONG_SPR, long_spr());
        w(S_NMI_EN, nmi_en()); w(S_BG_PAGE, bg_page()); w(S_SPR_PAGE, spr_page());
        w(S_NSL, nsl); w(S_SL_LO, sl_lo); w(S_SL_HI, sl_hi); w(S_PCYC, (uint32_t)pcyc);
        w(S_SCANLINE, (uint32_t)scanline); w(S_V, v); w(S_T, t); w(S_INC, inc());
    }

    // power-on: zeroed machine, then CPU and PPU reset (nes_core.hpp:123-147)
    __device__ void power_on() {
        for (uint32_t r = 0; r < MEM_ROWS; r++)
            if (r < ROW_VRAM || r >= ROW_VRAM + 2048) st(r, 0);
        for (uint32_t w = 0; w < 512; w++) *(uint32_t*)(mbase + (vo + (uint32_t)__umul24(w, 4 * np))) = 0;
        iter_lo = iter_hi = 0; exec_at = 0; ppu_calls = 0;
        joy_strobe = 3; joy = 0;
        zero_skip = 0; a = x = y = 0; p = 0x34;
        pc = (uint16_t)(prg(0xfffc) | prg(0xfffd) << 8);
        sp = 0xfd;
        s0hit = 0; data_buffer = 0; vblank = 0; even = 1; ppu_flags = PF_SHOW_BG | PF_SHOW_SPR;
        first_write = 1; v = 0; pcyc = 0; scanline = 0;
        oam_addr = 0; fine_x = 0; t = 0; pstate = ST_PRE; nsl = 0; sl_lo = sl_hi = 0;
        pend_line = -1; sp_line = -1; pal_dirty = true; bg_key = -1;
        for (int k = 0; k < LDS_OAM_WORDS; k++) lds_oam[k * LDS_LANES] = 0;
        nmi_threshold();
    }

    // ------------------------------------------------------------ CPU bus (nes_core.hpp:150-208)
    // Accesses for which needs_sync() holds see the PPU caught up to 3 * (cur + 1): frame() syncs
    // before it issues them (the reference catches up inside the access; the target is the same).
    __device__ __forceinline__ static bool needs_sync(uint16_t ad, bool wr) {
        const bool ppu = (ad & 0xe000) == 0x2000, r2 = (ad & 7) == 2, r7 = (ad & 7) == 7;
        return (ppu & (wr | r2 | r7)) | (wr & (ad == 0x4014));
    }
    __device__ __forceinline__ uint8_t read(uint16_t ad) {
        if (ad >= 0x8000) return prg(ad);
        if (ad < 0x2000) return ram(ad);
        if (ad < 0x4000) {
            const uint16_t r = ad & 0x2007;
            if (r == 0x2002) return status_read();
            if (r == 0x2007) return data_read();
            if (r == 0x2004) return oam(oam_addr);
            return 0;
        }
        if (ad == 0x4016) return pad_read(0);
        if (ad == 0x4017) return pad_read(1);
        return 0;
    }
    __device__ __forceinline__ void write(uint16_t ad, uint8_t val) {
        if (ad < 0x2000) { st(ROW_RAM + (ad & 0x7ff), val); return; }
        if (ad < 0x4000) {
            // a pending sprite evaluation is materialized before its inputs (OAM, oam_addr, sprite
            // size) change; the sprite line buffer is rebuilt after any write that can change it
            const uint16_t r = ad & 0x2007;
            if (r == 0x2000 || r == 0x2003 || r == 0x2004) materialize_sprites();
            switch (r) {
                case 0x2000: ctrl_write(val); sp_line = -1; break;
                case 0x2001: mask_write(val); break;
                case 0x2003: oam_addr = val; break;
                case 0x2004: set_oam(oam_addr, val); oam_addr++; sp_line = -1; break;
                case 0x2005: scroll_write(val); break;
                case 0x2006: addr_write(val); break;
                case 0x2007: data_write(val); sp_line = -1; break;
                default: break;
            }
            return;
        }
        if (ad == 0x4014) {  // OAM DMA: 513 cycles, +1 on an odd absolute cycle; copies from RAM pages only
            materialize_sprites();
            skip += 513 + (int)((iter_lo + (uint32_t)cur + 1u) & 1u);
            const uint16_t src = (uint16_t)(val << 8);
            if (src < 0x2000) {
                if (!(oam_addr & 3)) {
                    // word-aligned: sprite words straight from four RAM bytes each
                    for (int k = 0; k < LDS_OAM_WORDS; k++) {
                        const uint32_t a0 = src + 4 * k;
                        lds_oam[((k + (oam_addr >> 2)) & 63) * LDS_LANES] =
                            (uint32_t)ram(a0) | (uint32_t)ram(a0 + 1) << 8 | (uint32_t)ram(a0 + 2) << 16 |
                            (uint32_t)ram(a0 + 3) << 24;
                    }
                } else {
                    for (int i = 0; i < 256; i++) set_oam(oam_addr + i, ram(src + i));
                }
            }
            sp_line = -1;
            return;
        }
        if (ad == 0x4016) {   // strobe both ports; its falling edge latches the buttons into the shift registers
            joy_strobe = (val & 1) ? 3 : 0;
            if (!(val & 1)) joy = (joy & 0xffffu) | (joy << 16);
        }
    }
    // port i: while strobed, button A; else the next bit of its shift register, which then shifts
    __device__ __forceinline__ uint8_t pad_read(int i) {
        const uint32_t sh = 16 + 8 * i;
        const uint8_t bit = (joy_strobe >> i) & 1 ? (uint8_t)((joy >> (8 * i)) & 1u) : (uint8_t)((joy >> sh) & 1u);
        if (!((joy_strobe >> i) & 1)) joy = (joy & ~(0xffu << sh)) | ((((joy >> sh) & 0xffu) >> 1) << sh);
        return bit | 0x40;
    }

    // ------------------------------------------------------------ PPU registers (nes_core.hpp:211-260)
    __device__ void ctrl_write(uint8_t c) {
        ppu_flags = (ppu_flags & (PF_SHOW_BG | PF_SHOW_SPR | PF_HIDE_EDGE_BG | PF_HIDE_EDGE_SPR)) |
                    ((c >> 7) & 1 ? PF_NMI_EN : 0u) | ((c >> 5) & 1 ? PF_LONG_SPR : 0u) |
                    ((c >> 4) & 1 ? PF_BG_PAGE : 0u) | ((c >> 3) & 1 ? PF_SPR_PAGE : 0u) | ((c & 4) ? PF_INC32 : 0u);
        t = (uint16_t)((t & 0xf3ff) | ((c & 3) << 10));
    }
    __device__ void mask_write(uint8_t k) {
        ppu_flags = (ppu_flags & ~(PF_SHOW_BG | PF_SHOW_SPR | PF_HIDE_EDGE_BG | PF_HIDE_EDGE_SPR)) |
                    (!(k & 2) ? PF_HIDE_EDGE_BG : 0u) | (!(k & 4) ? PF_HIDE_EDGE_SPR : 0u) |
                    ((k >> 3) & 1 ? PF_SHOW_BG : 0u) | ((k >> 4) & 1 ? PF_SHOW_SPR : 0u);
    }
    __device__ uint8_t status_read() {
        uint8_t r = (uint8_t)((s0hit << 6) | (vblank << 7));
        vblank = 0; first_write = 1;
        return r;
    }
    __device__ void addr_write(uint8_t d) {
        if (first_write) { t = (uint16_t)((t & 0x00ff) | ((d & 0x3f) << 8)); first_write = 0; }
        else { t = (uint16_t)((t & 0xff00) | d); v = t; first_write = 1; }
    }
    __device__ uint8_t data_read() {
        uint8_t d = vbus_read(v);
        v = (uint16_t)(v + inc());
        if (v < 0x3f00) { uint8_t b = data_buffer; data_buffer = d; d = b; }
        return d;
    }
    __device__ void data_write(uint8_t d) { vbus_write(v, d); v = (uint16_t)(v + inc()); }
    __device__ void scroll_write(uint8_t d) {
        if (first_write) { t = (uint16_t)((t & ~0x1f) | (d >> 3)); fine_x = d & 7; first_write = 0; }
        else { t = (uint16_t)((t & ~0x73e0) | ((d & 7) << 12) | ((d & 0xf8) << 2)); first_write = 1; }
    }

    // ------------------------------------------------------------ picture bus (nes_core.hpp:263-285)
    __device__ __forceinline__ uint32_t nt_row(uint16_t ad) const {
        const uint32_t k = ad < 0x2400 ? 0 : ad < 0x2800 ? 1 : ad < 0x2c00 ? 2 : 3;
        return (((cart.nt_bits >> k) & 1u) << 10) | (ad & 0x3ffu);
    }
    __device__ uint8_t vbus_read(uint16_t ad) const {
        if (ad < 0x2000) return cart.chr[ad];
        if (ad < 0x3eff) return vram(nt_row(ad));
        if (ad < 0x3fff) return pal(ad);
        return 0;
    }
    __device__ void vbus_write(uint16_t ad, uint8_t d) {
        if (ad < 0x2000) return;
        if (ad < 0x3eff) { set_vram(nt_row(ad), d); bg_key = -1; }
        else if (ad < 0x3fff) { st(ROW_PAL + (ad == 0x3f10 ? 0 : (ad & 0x1f)), d); pal_dirty = true; }
    }
    __device__ __forceinline__ uint8_t nametable(uint16_t ad) const {
        return vram((((cart.nt_bits >> ((ad >> 10) & 3u)) & 1u) << 10) | (ad & 0x3ffu));
    }

    // ------------------------------------------------------------ PPU timing (nes_core.hpp:289-308)
    __device__ void nmi_threshold() {
        int line = pstate == ST_PRE ? -1 : pstate == ST_POST ? 240 : scanline;
        int32_t pos = (line + 1) * 341 + (pcyc - 1);
        const int32_t vbl = 242 * 341;
        int32_t d = pos <= vbl ? vbl - pos + 1 : (262 * 341 - pos) + vbl + 1;
        nmi_thresh = ppu_calls + d - 8;
    }
    __device__ void advance_to(int32_t target) {
        if (target > ppu_calls) { ppu_run(target - ppu_calls); nmi_threshold(); }
    }

    __device__ void coarse_x_add(int n) {
        int tot = (v & 0x1f) + n;
        v = (uint16_t)((v & ~0x1f) | (tot & 31));
        if ((tot >> 5) & 1) v ^= 0x400;
    }
    __device__ void fine_y_step() {
        if ((v & 0x7000) != 0x7000) { v += 0x1000; return; }
        v &= ~0x7000;
        int yy = (v >> 5) & 31;
        if (yy == 29) { yy = 0; v ^= 0x800; }
        else if (yy == 31) yy = 0;
        else yy++;
        v = (uint16_t)((v & ~0x3e0) | (yy << 5));
    }
    __device__ void copy_h() { v = (uint16_t)((v & ~0x41f) | (t & 0x41f)); }
    __device__ void copy_v() { v = (uint16_t)((v & ~0x7be0) | (t & 0x7be0)); }

    // Per-line sprite list from oam_addr/4 (nes_core.hpp:336-349). The PPU only records the scanline
    // of an evaluation; the list is computed from OAM when something needs it (rendering, a change
    // of OAM / oam_addr / sprite size, or the end of the kernel). Until then its inputs are unchanged,
    // so the late evaluation gives the same list.
    __device__ void materialize_sprites() {
        if (pend_line < 0) return;
        // in-range sprites as a 64-bit mask (bit i: pend_line - y_i in [0, h)), from index oam_addr / 4 on;
        // the list is its first (at most 8) set bits, entries past the count keep their old values
        const uint32_t h = long_spr() ? 16u : 8u;
        // The env's parts each test 64 / LANES_PER_ENV sprites (part q: sprites NS q .. NS q + NS - 1) into
        // exchange word q of the env, then every part reads every word. The wave barrier is a convergence
        // point: every lane active here has stored its word before any lane loads (a wave's LDS accesses
        // complete in order). All parts must be here together, or a part would read a stale word: a part
        // missing from the wave's active lanes sets ERR_TWIN.
        constexpr int NS = 64 / LANES_PER_ENV;
        const uint32_t in_wave = __lane_id() & (ENVS_PER_WAVE - 1);
        if (((__ballot(1) >> in_wave) & PART_LANES) != PART_LANES) bad_ops |= ERR_TWIN;
        auto in_range = [&](int i) { return ((uint32_t)(pend_line - (int)(oam_sprite(i) & 0xffu)) < h ? 1u : 0u); };
        uint32_t mlo = 0, mhi = 0;
        if constexpr (LANES_PER_ENV == 1) {
#pragma unroll
            for (int i = 0; i < 32; i++) { mlo |= in_range(i) << i; mhi |= in_range(32 + i) << i; }
        } else {
            uint32_t piece = 0;
#pragma unroll
            for (int i = 0; i < NS; i++) piece |= in_range(NS * part + i) << i;
            uint32_t* const xw = lds_oam + LDS_OAM_WORDS * LDS_LANES;
            xw[part * LDS_LANES] = piece;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (LANES_PER_ENV == 2) {
                mlo = xw[0]; mhi = xw[LDS_LANES];
            } else {
                mlo = xw[0] | xw[LDS_LANES] << 16; mhi = xw[2 * LDS_LANES] | xw[3 * LDS_LANES] << 16;
            }
        }
        const int i0 = oam_addr >> 2;
        if (i0 < 32) mlo &= ~0u << i0;
        else { mlo = 0; mhi &= ~0u << (i0 - 32); }
        int n = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const bool has = (mlo | mhi) != 0;
            const uint32_t i = mlo ? (uint32_t)__builtin_ctz(mlo) : 32u + (uint32_t)__builtin_ctz(mhi | 0x80000000u);
            if (has) set_sl(k, (uint8_t)i);
            n += has;
            if (mlo) mlo &= mlo - 1; else mhi &= mhi - 1;
        }
        nsl = (uint8_t)n;
        pend_line = -1;
    }
    // "nsl > 0 && sl[0] == 0" without materializing: sprite 0 heads the list exactly when the
    // evaluation starts at index 0 and sprite 0 is in range.
    __device__ __forceinline__ bool sprite0_first() const {
        if (pend_line < 0) return nsl > 0 && sl(0) == 0;
        if (oam_addr >= 4) return false;
        int d = pend_line - (int)(oam_sprite(0) & 0xffu);
        return d >= 0 && d < (long_spr() ? 16 : 8);
    }
    __device__ uint8_t bg_colour(int px, uint8_t* pattern) const {
        int xf = (fine_x + px) % 8;
        uint8_t tile = nametable((uint16_t)(0x2000 | (v & 0x0fff)));
        uint16_t pa = (uint16_t)(((tile * 16) + ((v >> 12) & 7)) | (bg_page() << 12));
        uint8_t c = (uint8_t)(((cart.chr[pa] >> (7 ^ xf)) & 1) | (((cart.chr[pa + 8] >> (7 ^ xf)) & 1) << 1));
        *pattern = c;
        uint16_t aa = (uint16_t)(0x23c0 | (v & 0x0c00) | ((v >> 4) & 0x38) | ((v >> 2) & 7));
        int sh = ((v >> 4) & 4) | (v & 2);
        return (uint8_t)(c | (((nametable(aa) >> sh) & 3) << 2));
    }
    // sprite i's 2-bit pattern at (px, py), with C++ int semantics for stale lists (nes_core.hpp:369-391)
    __device__ uint8_t sprite_pattern(int i, int px, int py) const {
        const uint32_t ow = oam_sprite(i);
        uint8_t sx = (uint8_t)(ow >> 24);
        uint8_t sy = (uint8_t)((ow & 0xffu) + 1), tile = (uint8_t)(ow >> 8), attr = (uint8_t)(ow >> 16);
        int h = long_spr() ? 16 : 8;
        int xs = (px - sx) % 8, yo = (py - sy) % h;
        if (!(attr & 0x40)) xs ^= 7;
        if (attr & 0x80) yo ^= (h - 1);
        uint16_t ad;
        if (!long_spr()) {
            ad = (uint16_t)(tile * 16 + yo);
            if (spr_page()) ad += 0x1000;
        } else {
            yo = (yo & 7) | ((yo & 8) << 1);
            ad = (uint16_t)((tile >> 1) * 32 + yo);
            ad |= (tile & 1) << 12;
        }
        return (uint8_t)(((vbus_read(ad) >> xs) & 1) | (((vbus_read((uint16_t)(ad + 8)) >> xs) & 1) << 1));
    }

    // Visible dots [x0, x1): sprite-0 hit and the coarse-x increments of v (nes_core.hpp:394-413).
    // Rendered and unrendered frames both take the hit from here; dots_drawn only adds pixels.
    __device__ __forceinline__ void dots_hit_scroll(int x0, int x1) {
        if (!show_bg()) return;
        if (!s0hit && show_spr() && sprite0_first()) {
            int sx = (int)(oam_sprite(0) >> 24);
            int lo = x0 > sx ? x0 : sx;
            int hi = x1 < sx + 8 ? x1 : sx + 8;
            if (hide_edge_spr() && lo < 8) lo = 8;
            if (lo < hi) {
                coarse_x_add(inc_count(x0, lo));
                for (int px = lo; px < hi; px++) {
                    if (!s0hit && (!hide_edge_bg() || px >= 8)) {
                        uint8_t pat;
                        bg_colour(px, &pat);
                        if (pat && sprite_pattern(0, px, scanline)) s0hit = 1;
                    }
                    if ((fine_x + px) % 8 == 7) coarse_x_add(1);
                }
                coarse_x_add(inc_count(hi, x1));
                return;
            }
        }
        coarse_x_add(inc_count(x0, x1));
    }
    __device__ __forceinline__ int inc_count(int lo, int hi) const {   // x in [lo, hi) with (fine_x + x) % 8 == 7
        int r = (7 - fine_x) & 7;
        return (hi - r + 7) / 8 - (lo - r + 7) / 8;
    }

    // an optimization barrier: the value is materialized in a register here
    __device__ __forceinline__ static void in_register(uint32_t& x) { MH_REG_BARRIER(x); }
    // bytes of the 8-byte value hi:lo picked by the selector bytes of sel (each 0..7)
    __device__ __forceinline__ static uint32_t byte_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
        return __builtin_amdgcn_perm(hi, lo, sel);
    }

    // ---- per-lane LDS buffers of the renderer
    __device__ __forceinline__ uint8_t lds_byte(const uint32_t* base, int i) const {
        return (uint8_t)(base[(i >> 2) * LDS_LANES] >> (8 * (i & 3)));
    }
    // gray value of every palette address, lut[pal[i]]; rebuilt after palette writes
    __device__ void build_gray_palette() {
        for (int w = 0; w < LDS_GP_WORDS; w++) {
            uint32_t word = 0;
            for (int b = 0; b < 4; b++) word |= (uint32_t)lut[pal(4 * w + b)] << (8 * b);
            lds_gp[w * LDS_LANES] = word;
        }
        pal_dirty = false;
    }
    // First opaque listed sprite per x of line py (nes_core.hpp:427-441), one byte per x: bits 0-3 the
    // sprite palette entry (attr << 2 | pattern, palette address 0x10 + it), bit 6 in front of the
    // background, bit 7 set (a sprite pixel is here; 0: none). The pattern row of each listed sprite is
    // fetched once, with the addressing of sprite_pattern().
    __device__ void build_sprite_line(int py) {
        for (int w = 0; w < LDS_SP_WORDS; w++) lds_sp[w * LDS_LANES] = 0;
        const int h = long_spr() ? 16 : 8;
        for (int k = 0; k < nsl; k++) {
            const int i = sl(k);
            const uint32_t ow = oam_sprite(i);
            const uint8_t sx = (uint8_t)(ow >> 24), sy = (uint8_t)((ow & 0xffu) + 1), tile = (uint8_t)(ow >> 8),
                          attr = (uint8_t)(ow >> 16);
            int yo = (py - sy) % h;
            if (attr & 0x80) yo ^= (h - 1);
            uint16_t ad;
            if (!long_spr()) {
                ad = (uint16_t)(tile * 16 + yo);
                if (spr_page()) ad += 0x1000;
            } else {
                yo = (yo & 7) | ((yo & 8) << 1);
                ad = (uint16_t)((tile >> 1) * 32 + yo);
                ad |= (tile & 1) << 12;
            }
            const uint8_t lo = vbus_read(ad), hi = vbus_read((uint16_t)(ad + 8));
            const uint32_t tag = 0x80u | ((attr & 3u) << 2) | (attr & 0x20 ? 0u : 0x40u);
            // The sprite's 8 pixels as 8 bytes (pixel sx + j in byte j: pattern | tag, or 0 where transparent),
            // merged into the (at most 3) line words they cover: a byte takes the sprite only where no
            // earlier listed sprite is opaque (a written byte always has bit 7 set). Pixels past x = 255 fall
            // in words past the line and are dropped.
            const uint32_t rlo = (attr & 0x40) ? (uint32_t)lo : __builtin_bitreverse32((uint32_t)lo) >> 24;
            const uint32_t rhi = (attr & 0x40) ? (uint32_t)hi : __builtin_bitreverse32((uint32_t)hi) >> 24;
            uint32_t cw[2];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const uint32_t pat = (__umul24((rlo >> (4 * q)) & 0xfu, 0x204081u) & 0x01010101u) |
                                     ((__umul24((rhi >> (4 * q)) & 0xfu, 0x204081u) & 0x01010101u) << 1);
                const uint32_t nz = (pat + 0x7f7f7f7fu) & 0x80808080u;
                cw[q] = (pat | tag * 0x01010101u) & (nz | (nz - (nz >> 7)));
            }
            const uint64_t span = ((uint64_t)cw[1] << 32 | cw[0]) ;
            const int w0 = sx >> 2, sh = 8 * (sx & 3);
            const uint64_t lo64 = span << sh;
            const uint32_t cv[3] = {(uint32_t)lo64, (uint32_t)(lo64 >> 32), sh ? (uint32_t)(span >> (64 - sh)) : 0u};
#pragma unroll
            for (int i = 0; i < 3; i++) {
                if (w0 + i < LDS_SP_WORDS) {
                    uint32_t* wp = &lds_sp[(w0 + i) * LDS_LANES];
                    const uint32_t old = *wp, occ = old & 0x80808080u;
                    *wp = old | (cv[i] & ~(occ | (occ - (occ >> 7))));
                }
            }
        }
        sp_line = py;
    }

    // Background tiles of a line into the per-lane LDS cache: the 32-tile name-table row at coarse y of
    // v0's name table A (words 0-7) and of its horizontal neighbour B (words 8-15, where coarse x wraps
    // to; nes_core.hpp:394-413), and the two attribute rows (words 16-19: bytes 0-7 A, 8-15 B). The row
    // depends on v0's bits 5-11 only: lines of one coarse y share it whatever their scroll. 20 word
    // loads, independent of each other.
    __device__ __forceinline__ void fill_bg_row(uint16_t v0) {
        const uint32_t na = (v0 >> 10) & 3u, cy = (v0 >> 5) & 31u;
        const uint32_t pa = ((cart.nt_bits >> na) & 1u) << 8, pb = ((cart.nt_bits >> (na ^ 1u)) & 1u) << 8;  // words
        uint32_t w[LDS_BG_WORDS];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            w[i] = vram_word(pa + cy * 8 + i);
            w[8 + i] = vram_word(pb + cy * 8 + i);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            w[16 + i] = vram_word(pa + 0xf0 + (cy >> 2) * 2 + i);
            w[18 + i] = vram_word(pb + 0xf0 + (cy >> 2) * 2 + i);
        }
#pragma unroll
        for (int i = 0; i < LDS_BG_WORDS; i++) lds_bg[i * LDS_LANES] = w[i];
    }
    // Tile k (0..32) of the line whose row is cached (c0: the line's starting coarse x, cy: its coarse
    // y): index | attribute byte << 8 | the attribute's shift in it << 16, unpacked by bg_planes (the
    // loads are not waited for here). Column c0 + k is in name table A below 32, else in B.
    __device__ __forceinline__ uint32_t bg_tile_of(int k, uint32_t c0, uint32_t cy) const {
        const uint8_t* row = (const uint8_t*)lds_bg;
        const uint32_t col = c0 + (uint32_t)k;                                   // 0 .. 63
        const uint32_t tile = row[(col >> 2) * LDS_LANES * 4 + (col & 3)];
        const uint32_t ab = LDS_BG_ATTR + (col >> 5) * 8 + ((col & 31) >> 2);   // attribute byte
        const uint32_t at = row[(ab >> 2) * LDS_LANES * 4 + (ab & 3)];
        const uint32_t sh = ((cy & 2u) << 1) | (col & 2u);
        return tile | at << 8 | sh << 16;
    }
    // Pattern planes of row fy of tile ta (bg_tile_of) and its gray table: byte p is the gray value of
    // background pattern p (p = 0: the universal background, palette address 0; else palette address
    // 4 at + p). pal[w]: gray values of palette addresses 4w .. 4w+3.
    __device__ __forceinline__ void bg_planes(uint32_t ta, int fy, const uint32_t (&pal)[4], uint32_t& lo, uint32_t& hi,
                                              uint32_t& gt) const {
        const uint16_t pa = (uint16_t)((((ta & 0xffu) * 16) + fy) | (bg_page() << 12));
        lo = cart.chr[pa];
        hi = cart.chr[pa + 8];
        const uint32_t at = (ta >> (8 + (ta >> 16))) & 3u;
        const uint32_t w01 = (at & 1u) ? pal[1] : pal[0], w23 = (at & 1u) ? pal[3] : pal[2];
        gt = (((at & 2u) ? w23 : w01) & 0xffffff00u) | (pal[0] & 0xffu);
    }

    // Pixels of visible dots [x0, x1): gray values into the frame buffer (nes_core.hpp:467-513), with
    // v as it is at x0 (dots_hit_scroll advances it afterwards). Pixels go in screen-aligned groups
    // of 8, so every lane of a wave runs the same code whatever its fine scroll: a group spans two
    // background tiles, kept as a 16-bit window per pattern plane (a PPU's shift registers), and the
    // tile after them is fetched one group ahead from the LDS tile row. Sprites come from the LDS line
    // buffer, where the first opaque listed sprite of each x sits.
    //
    // Four pixels are one 32-bit word, a byte each, and are computed together without branches: the
    // pattern bits of the four pixels are spread to the four bytes by a multiply, the background gray
    // value is a byte permute of the two tiles' gray tables, a sprite pixel's gray value is a byte
    // permute of the sprite palette's 16 gray values, and priority is a per-byte mask.
    __device__ __forceinline__ void dots_drawn(int x0, int x1) {
        const int py = scanline;
        materialize_sprites();
        if (pal_dirty) build_gray_palette();
        const bool spr = show_spr() && nsl;
        if (spr && sp_line != py) build_sprite_line(py);
        const int f = fine_x, fy = (v >> 12) & 7;
        const int g0 = x0 >> 3, g1 = (x1 + 7) >> 3;
        uint32_t bc0 = 0, bcy = 0;             // line-start coarse x and coarse y
        if (show_bg()) {
            // line-start address: v addresses the tile of pixel x0, (f + x0) / 8 tiles into the line
            const int kb = (f + x0) >> 3;
            int c0 = (v & 0x1f) - kb;
            uint16_t v0 = v;
            if (c0 < 0) { c0 += 32; v0 ^= 0x400; }
            v0 = (uint16_t)((v0 & ~0x1f) | c0);
            if ((int32_t)((v0 >> 5) & 0x7f) != bg_key) { fill_bg_row(v0); bg_key = (v0 >> 5) & 0x7f; }
            bc0 = v0 & 31u; bcy = (v0 >> 5) & 31u;
        }
        // gray values of the background palettes (addresses 0..15) and the sprite palettes (0x10 + 0..15)
        uint32_t bp0 = lds_gp[0], bp1 = lds_gp[LDS_LANES], bp2 = lds_gp[2 * LDS_LANES], bp3 = lds_gp[3 * LDS_LANES];
        // keep them in registers: a select of these loads must not become a load from a selected address
        in_register(bp0); in_register(bp1); in_register(bp2); in_register(bp3);
        uint32_t sp0 = 0, sp1 = 0, sp2 = 0, sp3 = 0;
        if (spr) {
            sp0 = lds_gp[4 * LDS_LANES]; sp1 = lds_gp[5 * LDS_LANES];
            sp2 = lds_gp[6 * LDS_LANES]; sp3 = lds_gp[7 * LDS_LANES];
        }
        const bool any_spr = __any(spr);
        const uint32_t bgpal[4] = {bp0, bp1, bp2, bp3};
        // pixel bb of a group takes the second tile's attribute when f + bb >= 8: bytes bb >= 8 - f
        const uint64_t second = f ? (~0ull << (8 * (8 - f))) : 0ull;
        const uint32_t tsel0 = (uint32_t)second & 0x04040404u, tsel1 = (uint32_t)(second >> 32) & 0x04040404u;
        // The env's parts split the groups in pairs: part q draws groups S m + 2 q and S m + 2 q + 1, S = 2 x
        // LANES_PER_ENV (a fixed owner per group, so a group cut by a catch-up boundary is finished by the
        // lane that started it). One iteration draws one pair (p, p + 1) from tiles p, p + 1 and p + 2, and
        // fetches the planes of the next pair's three tiles, the indices of the pair after it and the next
        // pair's sprite bytes, which are used one iteration later, so no LDS round trip sits between two
        // pairs. The fetches are unconditional (indices clamped to the buffers; a layer that is off masks
        // its values afterwards), so every iteration issues the same LDS operations. A group of a pair that
        // lies outside [x0, x1) gets an empty pixel mask and is not written.
        constexpr int S = 2 * LANES_PER_ENV;   // groups between two pairs of one part
        auto tile_of = [&](int k) { return bg_tile_of(k < 32 ? k : 32, bc0, bcy); };
        int pg = (g0 & ~(S - 1)) + 2 * (int)part;
        if (pg + 1 < g0) pg += S;
        uint32_t alo, ahi, agt, blo, bhi, bgt, clo, chi, cgt;
        bg_planes(tile_of(pg), fy, bgpal, alo, ahi, agt);
        bg_planes(tile_of(pg + 1), fy, bgpal, blo, bhi, bgt);
        bg_planes(tile_of(pg + 2), fy, bgpal, clo, chi, cgt);
        uint32_t nxa = tile_of(pg + S), nxb = tile_of(pg + S + 1), nxc = tile_of(pg + S + 2);
        const int ws0 = 2 * pg < 60 ? 2 * pg : 60;
        uint32_t s0 = lds_sp[ws0 * LDS_LANES], s1 = lds_sp[(ws0 + 1) * LDS_LANES];   // the pair's sprite bytes
        uint32_t s2 = lds_sp[(ws0 + 2) * LDS_LANES], s3 = lds_sp[(ws0 + 3) * LDS_LANES];
        // A layer that is off is masked out of every pixel rather than zeroed at its fetch: with the background
        // pattern masked to 0 a pixel takes byte 0 of its tile's gray table, the universal background, as it
        // does with the background off; with the sprite bytes masked no sprite pixel is taken.
        const uint32_t keep_bg = show_bg() ? ~0u : 0u, keep_sp = spr ? ~0u : 0u;
        uint32_t* wp = (uint32_t*)gray + ((size_t)py * 64 + 2 * pg) * np;   // word of pixels 8pg .. 8pg+3
        // the two words of the group drawn from tiles (lo0, hi0, gt0) and (lo1, hi1, gt1) with sprite bytes ca, cb
        auto group_words = [&](uint32_t lo0, uint32_t hi0, uint32_t gt0, uint32_t lo1, uint32_t hi1, uint32_t gt1,
                               uint32_t ca, uint32_t cb, uint32_t keep_bg, uint32_t keep_sp, uint32_t (&out)[2]) {
            // pixel 8g + bb is bit 15 - bb of the window after the fine-scroll shift; reversed: bit 16 + bb
            const uint32_t rlo = __builtin_bitreverse32(((lo0 << 8) | lo1) << f);
            const uint32_t rhi = __builtin_bitreverse32(((hi0 << 8) | hi1) << f);
#pragma unroll
            for (int q = 0; q < 2; q++) {
                // background pattern of the four pixels, one per byte (0..3)
                const uint32_t nlo = (rlo >> (16 + 4 * q)) & 0xfu, nhi = (rhi >> (16 + 4 * q)) & 0xfu;
                const uint32_t bgp = (((__umul24(nlo, 0x204081u) & 0x01010101u) |
                                       ((__umul24(nhi, 0x204081u) & 0x01010101u) << 1))) & keep_bg;
                uint32_t word = byte_perm(gt1, gt0, bgp | (q ? tsel1 : tsel0));
                if (any_spr) {
                    const uint32_t c = q ? cb : ca;
                    const uint32_t opaque = (bgp + 0x7f7f7f7fu) & 0x80808080u;       // background pattern != 0
                    const uint32_t take = c & (~opaque | (c << 1)) & 0x80808080u & keep_sp;
                    const uint32_t tmask = take | (take - (take >> 7));
                    const uint32_t sel = c & 0x07070707u;
                    const uint32_t hi8 = (c << 4) & 0x80808080u;                    // entry 8..15
                    const uint32_t hmask = hi8 | (hi8 - (hi8 >> 7));
                    const uint32_t sg = (byte_perm(sp3, sp2, sel) & hmask) | (byte_perm(sp1, sp0, sel) & ~hmask);
                    word = (sg & tmask) | (word & ~tmask);
                }
                out[q] = word;
            }
        };
        // the group's two words at w (pixels xg .. xg + 7): streaming stores when all 8 pixels are in [x0, x1)
        // (the frame buffers are read by the next kernel only, so they should not evict the console state from
        // the L2), else a read-modify-write of the pixels in [x0, x1)
        auto store_group = [&](int xg, uint32_t* w, const uint32_t (&out)[2]) {
            if (xg >= x0 && xg + 8 <= x1) { __builtin_nontemporal_store(out[0], w); __builtin_nontemporal_store(out[1], w + np); }
            else {
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int xq = xg + 4 * q;
                    const int lo = x0 > xq ? x0 - xq : 0, hi = x1 < xq + 4 ? x1 - xq : 4;
                    if (lo < hi) {
                        const uint32_t in = (uint32_t)((((1ull << (8 * hi)) - 1) >> (8 * lo)) << (8 * lo));
                        uint32_t* wq = w + q * np;
                        *wq = (*wq & ~in) | (out[q] & in);
                    }
                }
            }
        };
        for (; pg < g1; pg += S) {
            uint32_t dlo, dhi, dgt, elo, ehi, egt, flo, fhi, fgt;
            bg_planes(nxa, fy, bgpal, dlo, dhi, dgt);
            bg_planes(nxb, fy, bgpal, elo, ehi, egt);
            bg_planes(nxc, fy, bgpal, flo, fhi, fgt);
            const uint32_t na = tile_of(pg + 2 * S), nb = tile_of(pg + 2 * S + 1), nc = tile_of(pg + 2 * S + 2);
            const int ws = 2 * pg + 2 * S < 60 ? 2 * pg + 2 * S : 60;
            const uint32_t t0 = lds_sp[ws * LDS_LANES], t1 = lds_sp[(ws + 1) * LDS_LANES];
            const uint32_t t2 = lds_sp[(ws + 2) * LDS_LANES], t3 = lds_sp[(ws + 3) * LDS_LANES];
            uint32_t out0[2], out1[2];
            // pixels 0-7 may hide either layer
            group_words(alo, ahi, agt, blo, bhi, bgt, s0, s1, (pg == 0 && hide_edge_bg()) ? 0u : keep_bg,
                        (pg == 0 && hide_edge_spr()) ? 0u : keep_sp, out0);
            group_words(blo, bhi, bgt, clo, chi, cgt, s2, s3, keep_bg, keep_sp, out1);
            store_group(8 * pg, wp, out0);
            store_group(8 * pg + 8, wp + 2 * np, out1);
            wp += 2 * S * np;
            alo = dlo; ahi = dhi; agt = dgt;
            blo = elo; bhi = ehi; bgt = egt;
            clo = flo; chi = fhi; cgt = fgt;
            nxa = na; nxb = nb; nxc = nc;
            s0 = t0; s1 = t1; s2 = t2; s3 = t3;
        }
    }

    // NMI raised by PPU call `call` (1-based, frame-relative); nes_core.hpp:520-531
    __device__ void nmi(int32_t call) {
        int32_t it = (call - 1) / 3;
        push((uint8_t)(pc >> 8)); push((uint8_t)pc); push((uint8_t)(p | 0x20));
        p |= FI;
        pc = (uint16_t)(prg(0xfffa) | prg(0xfffb) << 8);
        int32_t d = (zero_skip && it == exec_at) ? 0 : (exec_at - it + 1);
        exec_at = it + d + 6;
        zero_skip = 0;
    }

    // advance the PPU by n calls (nes_core.hpp:539-616)
    __device__ void ppu_run(int32_t n) {
        while (n > 0) {
            int c = pcyc;
            if (pstate == ST_PRE) {
                bool on = show_bg() && show_spr();
                int end = LINE_END - (!even && on);
                int k = c >= end ? 1 : (n < end - c ? n : end - c);
                int lo = c, hi = c + k;
                if (lo <= 1 && 1 < hi) vblank = s0hit = 0;
                if (on) {
                    if (lo <= 258 && 258 < hi) copy_h();
                    if (lo <= 304 && 281 < hi) copy_v();
                }
                ppu_calls += k; n -= k;
                if (hi - 1 >= end) { pstate = ST_RENDER; scanline = 0; pcyc = 1; }
                else pcyc = hi;
            } else if (pstate == ST_RENDER) {
                if (c >= 1 && c <= 256) {
                    int k = n < 257 - c ? n : 257 - c;
                    if (render) dots_drawn(c - 1, c - 1 + k);
                    dots_hit_scroll(c - 1, c - 1 + k);
                    pcyc += k; ppu_calls += k; n -= k;
                    c = pcyc;
                }
                if (n <= 0) {
                    // the calls ran out inside the visible dots
                } else if (c == 257 && n >= LINE_END - 256) {
                    // the rest of the line in one step when all of it is due: dot 257 (fine y), dot 258
                    // (copy_h), dots 259..340, and the line end (85 calls), as the cases below would
                    if (show_bg()) fine_y_step();
                    if (show_bg() && show_spr()) copy_h();
                    pend_line = scanline;   // sprite evaluation for the next line (materialized lazily)
                    sp_line = -1;
                    scanline++;
                    pcyc = 1; ppu_calls += LINE_END - 256; n -= LINE_END - 256;
                    if (scanline >= 240) pstate = ST_POST;
                } else if (c == 257) {
                    if (show_bg()) fine_y_step();
                    pcyc++; ppu_calls++; n--;
                } else if (c == 258) {
                    if (show_bg() && show_spr()) copy_h();
                    pcyc++; ppu_calls++; n--;
                } else if (c > 258 && c < LINE_END) {
                    int k = n < LINE_END - c ? n : LINE_END - c;
                    pcyc += k; ppu_calls += k; n -= k;
                } else if (c >= LINE_END) {
                    pend_line = scanline;   // sprite evaluation for the next line (materialized lazily)
                    sp_line = -1;
                    scanline++;
                    pcyc = 1; ppu_calls++; n--;
                    if (scanline >= 240) pstate = ST_POST;
                } else {
                    pcyc++; ppu_calls++; n--;
                }
            } else if (pstate == ST_POST) {
                if (c >= LINE_END) { scanline++; pcyc = 1; pstate = ST_VBLANK; ppu_calls++; n--; }
                else { int k = n < LINE_END - c ? n : LINE_END - c; pcyc += k; ppu_calls += k; n -= k; }
            } else {
                if (c >= LINE_END) {
                    scanline++; pcyc = 1;
                    if (scanline >= 261) { pstate = ST_PRE; scanline = 0; even = !even; }
                    ppu_calls++; n--;
                } else if (c == 1 && scanline == 241) {
                    vblank = 1; ppu_calls++; n--; pcyc = 2;
                    if (nmi_en()) nmi(ppu_calls);
                } else {
                    int lim = LINE_END - c;
                    if (scanline == 241 && c < 1) lim = 1 - c;
                    int k = n < lim ? n : lim;
                    pcyc += k; ppu_calls += k; n -= k;
                }
            }
        }
    }

    // ------------------------------------------------------------ CPU (nes_core.hpp:619-899)
    __device__ __forceinline__ void set_nz(uint8_t r) { p = (uint8_t)((p & ~(FZ | FN)) | (r ? 0 : FZ) | (r & 0x80 ? FN : 0)); }
    __device__ __forceinline__ void flag(uint8_t f, bool on) { p = on ? (uint8_t)(p | f) : (uint8_t)(p & ~f); }
    __device__ __forceinline__ bool has(uint8_t f) const { return (p & f) != 0; }
    __device__ __forceinline__ void push(uint8_t d) { st(ROW_RAM + ((0x100 | sp) & 0x7ff), d); sp--; }
    __device__ __forceinline__ uint8_t pull() { sp++; return ram(0x100 | sp); }
    __device__ __forceinline__ void cross_penalty(uint16_t u, uint16_t w, int k) { if ((u & 0xff00) != (w & 0xff00)) skip += k; }

    // End of the next frame slice: the PPU call after which dots 1..256 of the last line of the next
    // group of SLICE_LINES render lines are done (the current group's if its last line is still ahead),
    // capped at the frame end `cap`.
    __device__ __forceinline__ int32_t next_slice(int32_t cap) const {
        int line = 0;
        if (pstate == ST_RENDER) line = pcyc < 257 ? scanline : scanline + 1;
        const int last = (line | (SLICE_LINES - 1)) < 239 ? (line | (SLICE_LINES - 1)) : 239;
        int32_t d = line <= 239 ? calls_until(last, 257) : calls_until(SLICE_LINES - 1, 257);
        if (d < 1) d = 1;
        const int32_t s = ppu_calls + d;
        return s < cap ? s : cap;
    }

    // The data operation of decode word D: the result byte and the new flags, from the packed registers regs
    // (a | x << 8 | y << 16 | sp << 24), the data operand m (the first operand byte when nothing was read), the
    // flags p and whether a data operand was read. Every choice is a select on bits of the decode word: chains of
    // equality tests on one small field would be lowered to a branch tree, i.e. exec-mask branches on every
    // instruction of a divergent wave.
    struct AluOut { uint32_t r8, p; };
    __device__ __forceinline__ static AluOut alu_op(uint32_t D, uint32_t regs, uint32_t m, uint32_t p, bool rd) {
        using namespace dec;
        const uint32_t alu = (D >> ALU_SH) & 15u, src = (D >> SRC_SH) & 7u, fl = (D >> FL_SH) & 7u;
        const uint32_t a = regs & 0xffu;
        const uint32_t rv = src ? (regs >> (8 * (src - 1))) & 0xffu : (uint32_t)m;   // R_A, R_X, R_Y, R_SP, or M
        const uint32_t sv = rd ? (uint32_t)m : rv;                // operand of the unary operations
        const uint32_t cin = (p & FC) ? 1u : 0u;
        const uint32_t sum = a + m + cin;                         // ADC
        const uint32_t dif = a - m - (1u - cin);                  // SBC
        const uint32_t cmp = rv - m;                              // CMP / CPX / CPY
        const bool u0 = alu & 1u, u1 = alu & 2u, u2 = alu & 4u, u3 = alu & 8u;
        const uint32_t rc = u0 ? cin : 0u;                        // ROL / ROR carry in
        // OP_ results by the bits of alu: PASS ORA AND EOR ADC SBC CMP BIT ASL ROL LSR ROR INC DEC FLAG NOP
        const uint32_t g0 = u0 ? (uint32_t)(a | m) : sv, g1 = u0 ? (uint32_t)(a ^ m) : (uint32_t)(a & m);
        const uint32_t g2 = u0 ? dif : sum, g3 = u0 ? sv : cmp;
        const uint32_t g4 = (sv << 1) | rc, g5 = (sv >> 1) | (rc << 7), g6 = u0 ? sv - 1 : sv + 1, g7 = sv;
        const uint32_t h0 = u1 ? g1 : g0, h1 = u1 ? g3 : g2, h2 = u1 ? g5 : g4, h3 = u1 ? g7 : g6;
        const uint32_t res = u3 ? (u2 ? h3 : h2) : (u2 ? h1 : h0);
        const uint32_t r8 = res & 0xffu;
        // carry: ADC bit 8 of the sum; SBC / CMP no borrow; ASL / ROL bit 7; LSR / ROR bit 0
        const uint32_t c_sub = ((res >> 8) & 1u) ^ 1u, c_adc = (sum >> 8) & 1u;
        const uint32_t carry = u3 ? (u1 ? (sv & 1u) : ((sv >> 7) & 1u)) : ((u0 | u1) ? c_sub : c_adc);
        const uint32_t ovf = u0 ? ((a ^ dif) & (~(uint32_t)m ^ dif) & 0x80u) : ((a ^ sum) & (m ^ sum) & 0x80u);
        // flag groups NONE NZ NZC NZCV BIT OP as masks of the bits they replace
        const uint32_t nzv = (r8 ? 0u : FZ) | (r8 >> 7);          // FN is bit 0
        const uint32_t fz = (a & m) ? 0u : FZ;
        const uint32_t bitv = fz | (m & 0x40 ? FV : 0u) | (m >> 7);
        const uint32_t fop = (D >> FOP_SH) & 7u;
        const uint32_t fm = fop < 2 ? FC : fop < 4 ? FI : fop == 4 ? FV : FD;   // CLC SEC CLI SEI CLV CLD SED
        const uint32_t fset = (fop == 1 || fop == 3 || fop == 6) ? fm : 0u;
        uint32_t keep = 0xffu, set = 0u;
        if ((0xeu >> fl) & 1u) { keep &= ~(uint32_t)(FZ | FN); set |= nzv; }             // NZ, NZC, NZCV
        if ((0xcu >> fl) & 1u) { keep &= ~(uint32_t)FC; set |= carry ? FC : 0u; }        // NZC, NZCV
        if (fl == FL_NZCV) { keep &= ~(uint32_t)FV; set |= ovf ? FV : 0u; }
        if (fl == FL_BIT) { keep &= ~(uint32_t)(FZ | FV | FN); set |= bitv; }
        if (fl == FL_OP) { keep &= ~fm; set |= fset; }
        return AluOut{r8, (p & keep) | set};
    }

    // One whole instruction from its decode word: addressing, at most one data read and one data
    // write through the bus, the ALU as register selects, and one small switch for the stack /
    // control-flow operations, in the reference's bus order (operand bytes, pointer, data read, data
    // write; JSR pushes before reading its operand, a branch reads its offset only when taken).
    // `pf`: the opcode and both following bytes are in PRG (pc <= 0xfffd) and were read as op, q1, q2,
    // which has no side effects; otherwise they are fetched through the bus, with the PPU caught up
    // first because a fetch may hit a PPU register. Returns false, with no effect, when the PPU must be
    // caught up to `tgt` first; the caller does that and starts the instruction again.
    __device__ __forceinline__ bool instruction(int32_t j, int32_t tgt, bool pf, uint8_t op, uint8_t q1, uint8_t q2) {
        using namespace dec;
        if (!pf && ppu_calls < tgt) return false;
        uint8_t b1 = q1, b2 = q2;
        uint32_t D;
        if (!pf) {
            // Opcode and operand bytes through the bus. Their loads are waited for inside this branch: a wait
            // where the paths join would also wait for every store still in flight from earlier instructions.
            uint32_t o = read(pc);
            in_register(o);
            op = (uint8_t)o;
            D = cart.dec[op];
            const uint32_t xop0 = (D >> X_SH) & 15u;
            if (xop0 != X_JSR && xop0 != X_BRANCH) {   // JSR and branches fetch below, in their order
                const uint32_t am0 = D & 15u;
                uint32_t t1 = b1, t2 = b2;
                if (am0 != M_NONE) t1 = read((uint16_t)(pc + 1));
                if (am0 == M_ABS || am0 == M_ABSX || am0 == M_ABSY) t2 = read((uint16_t)(pc + 2));
                in_register(t1); in_register(t2);
                b1 = (uint8_t)t1; b2 = (uint8_t)t2;
            }
        } else {
            D = cart.dec[op];
        }
        const uint32_t am = D & 15u, xop = (D >> X_SH) & 15u, dst = (D >> DST_SH) & 7u;
        const bool rd = (D & RD) != 0, wr = dst == D_MEM;
        // addressing as selects on mode-set bits (no branch except for the zero-page pointer loads)
        const uint32_t mb = 1u << am;
        constexpr uint32_t X_IDX = 1u << M_ZPX | 1u << M_ABSX, Y_IDX = 1u << M_ZPY | 1u << M_ABSY | 1u << M_INDY;
        constexpr uint32_t ZP_EA = 1u << M_ZP | 1u << M_ZPX | 1u << M_ZPY, IND = 1u << M_INDX | 1u << M_INDY;
        const uint16_t absv = (uint16_t)(b1 | b2 << 8);
        uint16_t base = absv;
        if (mb & IND) {   // pointer from the zero page
            const uint8_t z = am == M_INDX ? (uint8_t)(b1 + x) : b1;
            base = (uint16_t)(ram(z) | ram((uint8_t)(z + 1)) << 8);
        }
        const uint32_t idx = (mb & X_IDX) ? (uint32_t)x : (mb & Y_IDX) ? (uint32_t)y : 0u;
        const uint16_t ea = (mb & ZP_EA) ? (uint16_t)((b1 + idx) & 0xffu)
                          : am == M_IMM ? (uint16_t)(pc + 1) : (uint16_t)(base + idx);
        const uint16_t p2 = (uint16_t)((absv & 0xff00) | ((absv + 1) & 0xff));   // JMP (ind): high byte, page wrap
        const bool sync = xop == X_JMPI ? (needs_sync(absv, false) | needs_sync(p2, false))
                                        : ((rd & needs_sync(ea, false)) | (wr & needs_sync(ea, true)));
        if (sync && ppu_calls < tgt) return false;   // only when pf: no bus access has happened yet
        cur = j;
        skip = 0;
        instructions++;
        if (D & PEN) cross_penalty(base, (uint16_t)(base + idx), 1);
        // data operand and ALU
        const uint8_t m = rd && am != M_IMM ? read(ea) : b1;
        const uint32_t regs = (uint32_t)a | (uint32_t)x << 8 | (uint32_t)y << 16 | (uint32_t)sp << 24;
        const AluOut ao = alu_op(D, regs, m, p, rd);
        p = (uint8_t)ao.p;
        const uint8_t r8 = (uint8_t)ao.r8;
        // the destination register as a byte insert into the packed a | x << 8 | y << 16 | sp << 24 (D_A .. D_SP
        // are 1 .. 4): the four fields share one word, so writing all four from it is one register write
        const uint32_t dsh = (8u * (dst - D_A)) & 31u, dmask = 0xffu << dsh;   // masked: no register for D_NONE / D_MEM
        const uint32_t nregs = (dst - D_A) < 4u ? (regs & ~dmask) | ((uint32_t)r8 << dsh) : regs;
        a = nregs; x = nregs >> 8; y = nregs >> 16; sp = nregs >> 24;
        if (wr) write(ea, r8);
        // control flow: the next pc by instruction length, branches and JMP as selects
        constexpr uint32_t ABS3 = 1u << M_ABS | 1u << M_ABSX | 1u << M_ABSY;
        uint16_t npc = (uint16_t)(pc + (am == M_NONE ? 1 : (mb & ABS3) ? 3 : 2));
        const uint16_t ret = (uint16_t)(pc + 2);
        {   // branch on N, V, C, Z (op bits 6-7) equal to op bit 5; 2 bytes; the offset is read only when taken
            const uint32_t fbit = (0x40800201u >> (8 * (op >> 6))) & 0xffu;   // FN FV FC FZ
            const bool taken = (xop == X_BRANCH) & (((p & fbit) != 0) == ((op & 0x20) != 0));
            uint8_t off = b1;
            if (taken && !pf) off = read((uint16_t)(pc + 1));
            const uint16_t to = (uint16_t)(ret + (int8_t)off);
            npc = xop == X_BRANCH ? (taken ? to : ret) : xop == X_JMP ? absv : npc;
            skip += taken ? (((ret ^ to) & 0xff00) ? 3 : 1) : 0;
        }
        // Stack operations as at most three pushes or three pulls with predicated accesses (the pulls are
        // in flight together), then their results as selects: BRK, JSR, PHA, PHP push; RTI, RTS, PLA, PLP pull.
        if (xop >= X_BRK && xop <= X_PLP) {
            const uint32_t npush = xop == X_BRK ? 3u : xop == X_JSR ? 2u : (xop == X_PHA || xop == X_PHP) ? 1u : 0u;
            const uint32_t npull = xop == X_RTI ? 3u : xop == X_RTS ? 2u : (xop == X_PLA || xop == X_PLP) ? 1u : 0u;
            const uint8_t v0 = (xop == X_BRK || xop == X_JSR) ? (uint8_t)(ret >> 8) : xop == X_PHA ? a : p;
            if (npush > 0) st(ROW_RAM + (0x100 | sp), v0);
            if (npush > 1) st(ROW_RAM + (0x100 | (uint8_t)(sp - 1)), (uint8_t)ret);
            if (npush > 2) st(ROW_RAM + (0x100 | (uint8_t)(sp - 2)), (uint8_t)(p | 0x30));
            uint8_t u0 = 0, u1 = 0, u2 = 0;
            if (npull > 0) u0 = ram(0x100 | (uint8_t)(sp + 1));
            if (npull > 1) u1 = ram(0x100 | (uint8_t)(sp + 2));
            if (npull > 2) u2 = ram(0x100 | (uint8_t)(sp + 3));
            sp = (uint8_t)(sp - npush + npull);
            if (xop == X_BRK) { p |= FI; npc = (uint16_t)(prg(0xfffe) | prg(0xffff) << 8); skip += 7; }
            if (xop == X_JSR) npc = pf ? absv : (uint16_t)(read((uint16_t)(pc + 1)) | read((uint16_t)(pc + 2)) << 8);
            if (xop == X_RTS) npc = (uint16_t)((u0 | u1 << 8) + 1);
            if (xop == X_RTI) { p = u0; npc = (uint16_t)(u1 | u2 << 8); }
            if (xop == X_PLA) { a = u0; set_nz(a); }
            if (xop == X_PLP) p = u0;
        }
        if (xop == X_JMPI) { const uint8_t lo = read(absv); const uint8_t hi = read(p2); npc = (uint16_t)(lo | hi << 8); }
        pc = npc;
        if (D & OK) skip += (int)((D >> CYC_SH) & 7u);
        else bad_ops++;
        exec_at = j + (skip >= 1 ? skip : 1);
        zero_skip = skip <= 0;
        return true;
    }

    // ------------------------------------------------------------ a lone console's instruction run
    // While a console is one of the last few of its wave with an instruction to run (at most LONE_MAX_ENVS; the
    // others parked at their slice end, or out of the frame loop), an iteration of frame()'s loop costs about
    // what it costs a full wave: every opcode's work as selects, the wave votes and the catch-up checks.
    // lone_run() runs that console's instructions back to back instead (the frame loop calls it for those
    // consoles one after the other, each under its own lanes' exec mask), in lone_long(), with its registers
    // wave-uniform and one body per opcode.
    // It runs the instructions whose opcode and operands are in PRG and whose bus accesses touch only RAM, PRG,
    // or addresses that read as 0 or ignore writes ($4000-$7FFF but the joypads and OAM DMA), as instruction()
    // would; it stops before any other instruction (PPU register, joypad or DMA access, invalid opcode), before
    // the idle loop `JMP *` (fast-forwarded by frame()), before an instruction at the NMI check, and at the
    // slice or frame end, leaving that instruction to frame()'s own iteration. Returns the number of instructions
    // run. Called by this console's lanes only (its parts, with identical values), while no lane of the wave
    // waits for a catch-up.
    __device__ __forceinline__ static uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
    __device__ __forceinline__ uint32_t lone_run(int32_t end, int32_t slice) {
        // frame()'s stopping rules as one limit on the catch-up point 3 (j + 1) of instruction j: at most the slice
        // end, at most 3 end (j < end), and no NMI check that needs a catch-up first (below nmi_thresh, or
        // already caught up to it)
        const int32_t calls = (int32_t)uniform((uint32_t)ppu_calls), nmi = (int32_t)uniform((uint32_t)nmi_thresh);
        const int32_t last = (int32_t)uniform((uint32_t)slice);
        int32_t lim = nmi - 1 > calls ? nmi - 1 : calls;
        lim = lim < last ? lim : last;
        lim = lim < 3 * end ? lim : 3 * end;
        const uint32_t pflags = ((ppu_flags & (PF_SHOW_BG | PF_SHOW_SPR)) ? 0u : LP_WRITES) |
                                ((ppu_flags & PF_INC32) ? LP_INC32 : 0u) | cart.nt_bits << LP_NT_SHIFT;
        const LoneRegs o = lone_long(LoneRegs{pc, a, x, y, sp, p, exec_at, zero_skip, (uint32_t)v | (uint32_t)t << 16,
                                              (uint32_t)fine_x | (uint32_t)first_write << 8, 0u},
                                     lim, mbase + eo, mbase + vo, np, pflags, cart.gprg);
        if (o.n) {
            pc = (uint16_t)o.pc;
            a = o.a; x = o.x; y = o.y; sp = o.sp;
            p = (uint8_t)o.p;
            exec_at = o.ex;
            zero_skip = o.zs;
            if (o.px >> 17) {   // the run wrote a PPU register
                v = o.vt & 0xffffu; t = o.vt >> 16;
                fine_x = o.px & 0xffu; first_write = (o.px >> 8) & 1u;
                if (o.px & 0x10000u) { bg_key = -1; sp_line = -1; }   // name tables written: the tile-row and sprite-line caches
            }
            instructions += o.n;
        }
        return o.n;
    }

    // PPU calls from the current PPU position to (line, dot) on the frame timeline of
    // nmi_threshold() (pre-render line = -1, 262 x 341 calls); the one-dot-shorter odd pre-render
    // line is not modelled, so callers keep a margin. 0 means the very next call processes that dot.
    __device__ __forceinline__ int32_t calls_until(int line, int dot) const {
        const int now_line = pstate == ST_PRE ? -1 : pstate == ST_POST ? 240 : scanline;
        int32_t d = ((line + 1) * 341 + (dot - 1)) - ((now_line + 1) * 341 + (pcyc - 1));
        if (d < 0) d += 262 * 341;
        return d;
    }

    // Exact fast-forward of the sprite-0 wait loops `LDA $2002 / AND #$40 / BEQ|BNE *-5` at pc (BEQ:
    // wait for the hit, BNE: wait for the clear at the pre-render line), with the PPU caught up to the
    // read of the first iteration (at j). Iterations whose $2002 reads provably return the same value
    // are not executed: they would only re-read an unchanged s0hit, clear an already clear vblank flag
    // and set first_write, and the PPU is caught up lazily anyway. The span ends before the first dot
    // where s0hit could change (sprite 0's first line, or the pre-render clear), before the NMI sync
    // point and inside the frame. Returns true if it advanced.
    __device__ __forceinline__ bool poll_skip(int32_t j, int32_t end, bool wait_hit) {
        if (wait_hit == (s0hit != 0)) return false;   // this read ends the loop: run it normally
        int32_t limit;                           // first PPU call count at which s0hit may differ
        if (wait_hit) {
            // A hit needs sprite 0 at the head of the list of the line being drawn. The list already
            // evaluated serves the current line (in RENDER) or line 0 of the next frame (elsewhere).
            // The lists still to come are evaluated at the ends of render lines m (the current one
            // onwards in RENDER, 0 onwards elsewhere) and serve line m + 1 (240: line 0 of the next
            // frame); with OAM, oam_addr and sprite size fixed (the loop writes nothing) sprite 0 can
            // head one only for y0 <= m < y0 + h.
            if (sprite0_first() && pstate == ST_RENDER) return false;
            const int y0 = (int)(oam_sprite(0) & 0xffu), h = long_spr() ? 16 : 8;
            const int m = pstate == ST_RENDER && scanline > y0 ? scanline : y0;
            if (m <= 239 && m < y0 + h) limit = ppu_calls + calls_until(m + 1, 1) - 2;
            else if (y0 <= 238) limit = ppu_calls + calls_until(y0 + 1, 1) - 2;   // next frame
            else limit = 0x7fffffff;
            if (pstate != ST_RENDER && sprite0_first()) {
                const int32_t l0 = ppu_calls + calls_until(0, 1) - 2;
                if (l0 < limit) limit = l0;
            }
        } else {
            limit = ppu_calls + calls_until(-1, 1) - 2;
        }
        const int32_t c = 9 + ((((pc + 7) ^ pc) & 0xff00) ? 2 : 0);   // LDA 4 + AND 2 + taken branch 3 (+2)
        // start jl of the last skipped iteration: its three instructions start before the frame end
        // and below the NMI check, and its read precedes `limit`
        int32_t jl = end - 7;
        const int32_t by_nmi = (nmi_thresh - 1) / 3 - 7;
        const int32_t by_limit = (limit - 1) / 3 - 1;
        if (by_nmi < jl) jl = by_nmi;
        if (by_limit < jl) jl = by_limit;
        if (jl < j) return false;
        const int32_t k = (jl - j) / c + 1;
        vblank = 0;
        first_write = 1;
        a = s0hit ? 0x40 : 0x00;
        set_nz(a);
        exec_at = j + k * c;
        zero_skip = 0;
        instructions += 3 * (uint32_t)k;
        ff_instructions += 3 * (uint32_t)k;
        return true;
    }

    // One nes-py Emulator::step (nes_core.hpp:1166-1204) with the exact `JMP *` idle fast-forward.
    //
    // Every lane runs the same loop body: one whole instruction per iteration, and one PPU catch-up
    // site (`want`) for the NMI point, PPU-register accesses, the poll fast-forward and the frame
    // slices. Branching per opcode is confined to register arithmetic, so a wave whose lanes run
    // different instructions stays converged on the memory accesses.
    //
    // The frame is cut into slices that end right after the visible dots of every SLICE_LINES-th render
    // line (and at the frame end). A lane only starts an instruction j whose catch-up point 3 (j + 1) is
    // at most its slice end; once every lane of the wave is parked at its slice end, all of them catch
    // their PPU up to it together, so the slice's lines are rendered with the whole wave active. This is the
    // reference's catch-up PPU cut at more points (the PPU result does not depend on where it is
    // caught up), and never past a parked lane's next catch-up point 3 (j + 1), so an NMI raised
    // inside the slice catch-up sees exactly the CPU state of the reference's catch-up at the start
    // of j.
    __device__ __forceinline__ void frame() {
        // The kernel ends with its slowest wave (at steady state ~1.35x the mean wave), and the two waves of a
        // SIMD compete for its issue slots: a wave at an earlier frame of its agent step issues first (frames
        // 0 and 1 of the step at priority 3, frame 2 at 2, later frames, hack frames and re-emulations at 1; the
        // observation tails after the frame loop run at 0), so a wave that falls behind takes the slots of a
        // SIMD-mate that is ahead. Measured on 32,768 envs of 1-1: k_step 17.27 -> 16.57 ms (frame-index
        // mappings 3/2/1/1 16.86, 3/2/2/1 16.76, 3/3/3/2 16.69, 3/3/2/2 16.93 ms; priorities from a global count
        // of the frames the waves have started 17.17 ms).
        {
            const uint32_t f = __builtin_amdgcn_readfirstlane(nframe);
            nframe++;
            if (f < 2) __builtin_amdgcn_s_setprio(3);
            else if (f < 3) __builtin_amdgcn_s_setprio(2);
            else __builtin_amdgcn_s_setprio(1);
        }
        const int32_t end = FRAME_ITERS, last_call = 3 * FRAME_ITERS;
        int32_t want = -1;
        int32_t slice = next_slice(last_call);   // end of this lane's current slice, in PPU calls
        bool parked = false, synced = false;
        for (;;) {
            if (__any(want >= 0)) {
                // Every lane catches up with the one that must, each to its own next catch-up point
                // 3 (j + 1) (the reference's point before its instruction j; an NMI due by then is raised
                // exactly as in the lane's own catch-up), at most its slice end: the lines pending in
                // the wave are rendered together instead of by one lane at a time.
                int32_t t = want;
                if (t < 0) { const int32_t nx = 3 * (exec_at + 1); t = nx < slice ? nx : slice; }
                advance_to(t);
                want = -1;
            }
            if (__all(parked)) {
                // The whole wave is at the slice boundary: catch up together (next iteration), then
                // open the next slice. `slice` and `synced` are wave-uniform, so every lane takes
                // the same path here. (No early `continue`: after the catch-up request every lane is still
                // parked, so the rest of this iteration does nothing; after a new slice opens, this
                // iteration's actions are those the next one would take.)
                if (!synced) {
                    synced = true;
                    want = ppu_calls < slice ? slice : -1;
                } else {
                    if (__all(slice >= last_call)) break;
                    if (slice < last_call) { slice = next_slice(last_call); parked = false; }
                    synced = false;
                }
            }
            // One action per lane and iteration, chosen through `act` rather than early exits from the
            // loop body (each exit is a path whose state the next iteration must merge): park at the
            // slice end, ask for a catch-up, fast-forward, or run one instruction.
            const int32_t j = exec_at;
            const int32_t tgt = 3 * (j + 1);
            bool act = !parked;
            if (act && (j >= end || tgt > slice)) { parked = true; act = false; }
            if (act && tgt >= nmi_thresh && ppu_calls < tgt) { want = tgt; act = false; }
            {   // at most LONE_MAX_ENVS consoles left to run instructions and no catch-up asked for: each one's
                // run of lone instructions, one console after the other (its own lanes only)
                const uint64_t go = __ballot(act);
                // (a run of at least one instruction is this iteration's action: no early `continue`, whose
                // extra path into the loop top would make the compiler merge the console state there)
                if (go && __popcll(go) <= LONE_MAX_ENVS * LANES_PER_ENV && !__any(want >= 0)) {
                    uint64_t rest = go;
                    do {   // wave-uniform: rest is a ballot
                        const uint64_t env = PART_LANES << (__builtin_ctzll(rest) & (ENVS_PER_WAVE - 1));
                        if ((env >> __lane_id()) & 1u)
                            if (act && lone_run(end, slice) != 0) act = false;
                        rest &= ~env;
                    } while (rest);
                }
            }
            // PRG bytes pc .. pc + 6 for the fast paths, from three aligned LDS words and two byte-aligns (the
            // words past the last PRG word are the staged CHR bank's first ones: in bounds, and the bytes taken
            // from them are not used); the idle check reads 0xff past 0xffff
            const bool in_prg = pc >= 0x8000;
            const uint32_t pa = pc & 0x7fffu;
            const uint32_t* pw = (const uint32_t*)cart.prg + (pa >> 2);
            const uint32_t w0 = pw[0], w1 = pw[1], w2 = pw[2];
            const uint32_t b0 = __builtin_amdgcn_alignbyte(w1, w0, pa & 3u);   // bytes pc .. pc + 3
            const uint32_t b4 = __builtin_amdgcn_alignbyte(w2, w1, pa & 3u);   // bytes pc + 4 .. pc + 7
            const uint8_t op0 = in_prg ? (uint8_t)b0 : (uint8_t)0;
            const uint8_t q1 = in_prg && pc != 0xffff ? (uint8_t)(b0 >> 8) : (uint8_t)0xff;
            const uint8_t q2 = in_prg && pc < 0xfffe ? (uint8_t)(b0 >> 16) : (uint8_t)0xff;
            if (act && in_prg && op0 == 0x4c && (uint16_t)(q1 | q2 << 8) == pc) {
                const int32_t lim_end = end - j, lim_nmi = nmi_thresh - tgt;
                const int32_t k1 = lim_end > 0 ? (lim_end + 2) / 3 : 0;
                const int32_t k2 = lim_nmi > 0 ? (lim_nmi + 8) / 9 : 0;
                const int32_t k = k1 < k2 ? k1 : k2;
                if (k > 1) { exec_at = j + 3 * (k - 1); zero_skip = 0; act = false; }
            }
            // LDA $2002 / AND #$40 / BEQ|BNE back to the LDA: bytes AD 02 20 29 40 (F0|D0) F9
            if (act && in_prg && pc <= 0xfff8 && b0 == 0x292002adu && (b4 & 0x00ff00ffu) == 0x00f90040u) {
                const uint8_t br = (uint8_t)(b4 >> 8);
                if (br == 0xf0 || br == 0xd0) {
                    if (ppu_calls < tgt) { want = tgt; act = false; }   // the sync of the LDA $2002 at j
                    else if (poll_skip(j, end, br == 0xf0)) act = false;
                }
            }
            if (act && !instruction(j, tgt, in_prg && pc <= 0xfffd, op0, q1, q2)) want = tgt;
        }
        // rebase the frame-relative counters on the new frame start
        exec_at -= FRAME_ITERS;
        ppu_calls -= 3 * FRAME_ITERS;
        nmi_thresh -= 3 * FRAME_ITERS;
        const uint32_t lo = iter_lo + FRAME_ITERS;
        iter_hi += lo < iter_lo;
        iter_lo = lo;
    }
};

}  // namespace mh
