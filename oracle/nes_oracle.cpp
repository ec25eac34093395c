// CPU oracle for the batched SMB env step — TEST INFRASTRUCTURE ONLY (see nes_oracle.h).
//
// A plain, single-threaded restatement of the reference algorithm. It is written for readability,
// not speed: the PPU renders dot by dot, sprite lines are recomputed per dot, state snapshots are
// struct copies. Every quirk of the reference (which reproduces nes-py 8.2.1) is kept on purpose;
// the comment on each function names the reference lines it follows.
#include "nes_oracle.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace orc {

// ------------------------------------------------------------------ constants
// Status-flag bits in nes-py's bitfield byte layout (N is the least significant bit). nes_core.hpp:36-38
enum : uint8_t { FN = 0x01, FV = 0x02, FONE = 0x04, FB = 0x08, FD = 0x10, FI = 0x20, FZ = 0x40, FC = 0x80 };
enum : uint8_t { ST_PRE = 0, ST_RENDER = 1, ST_POST = 2, ST_VBLANK = 3 };

// Base cycles per opcode (0 = not an official opcode). Data table of nes_core.hpp:42-51.
static const uint8_t kCycles[256] = {
    7, 6, 0, 0, 0, 3, 5, 0, 3, 2, 2, 0, 0, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    6, 6, 0, 0, 3, 3, 5, 0, 4, 2, 2, 0, 4, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    6, 6, 0, 0, 0, 3, 5, 0, 3, 2, 2, 0, 3, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    6, 6, 0, 0, 0, 3, 5, 0, 4, 2, 2, 0, 5, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    0, 6, 0, 0, 3, 3, 3, 0, 2, 0, 2, 0, 4, 4, 4, 0, 2, 6, 0, 0, 4, 4, 4, 0, 2, 5, 2, 0, 0, 5, 0, 0,
    2, 6, 2, 0, 3, 3, 3, 0, 2, 2, 2, 0, 4, 4, 4, 0, 2, 5, 0, 0, 4, 4, 4, 0, 2, 4, 2, 0, 4, 4, 4, 0,
    2, 6, 0, 0, 3, 3, 5, 0, 2, 2, 2, 0, 4, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
    2, 6, 0, 0, 3, 3, 5, 0, 2, 2, 2, 2, 4, 4, 6, 0, 2, 5, 0, 0, 0, 4, 6, 0, 2, 4, 0, 0, 0, 4, 7, 0,
};
static const int kFrameIters = 29781;     // CPU iterations per nes-py Emulator::step
static const int kLineEnd = 341;

// nes-py master palette, 0xRRGGBB (fastmario.cpp:26-34).
static const uint32_t kPalette[64] = {
    0x7C7C7C, 0x0000FC, 0x0000BC, 0x4428BC, 0x940084, 0xA80020, 0xA81000, 0x881400,
    0x503000, 0x007800, 0x006800, 0x005800, 0x004058, 0x000000, 0x000000, 0x000000,
    0xBCBCBC, 0x0078F8, 0x0058F8, 0x6844FC, 0xD800CC, 0xE40058, 0xF83800, 0xE45C10,
    0xAC7C00, 0x00B800, 0x00A800, 0x00A844, 0x008888, 0x000000, 0x000000, 0x000000,
    0xF8F8F8, 0x3CBCFC, 0x6888FC, 0x9878F8, 0xF878F8, 0xF85898, 0xF87858, 0xFCA044,
    0xF8B800, 0xB8F818, 0x58D854, 0x58F898, 0x00E8D8, 0x787878, 0x000000, 0x000000,
    0xFCFCFC, 0xA4E4FC, 0xB8B8F8, 0xD8B8F8, 0xF8B8F8, 0xF8A4C0, 0xF0D0B0, 0xFCE0A8,
    0xF8D878, 0xD8F878, 0xB8F8B8, 0xB8F8D8, 0x00FCFC, 0xF8D8F8, 0x000000, 0x000000};

// JoypadSpace(SIMPLE_MOVEMENT) action -> button byte (fastmario.cpp:36).
static const uint8_t kButtons[7] = {0x00, 0x80, 0x81, 0x82, 0x83, 0x01, 0x40};

// ------------------------------------------------------------------ cartridge (nes_core.hpp:59-87)
struct Rom {
    uint8_t prg[0x8000];
    uint8_t chr[0x2000];
    uint16_t nt[4];
};

static int rom_load(Rom* r, const uint8_t* d, size_t n) {
    if (n < 16 || d[0] != 'N' || d[1] != 'E' || d[2] != 'S' || d[3] != 0x1a) return -1;
    int mapper = ((d[6] >> 4) & 0xf) | (d[7] & 0xf0);
    if (mapper != 0 || (d[6] & 0x2) || (d[6] & 0x4)) return -2;
    int banks = d[4];
    if (banks < 1 || banks > 2 || d[5] != 1) return -3;
    if (n < 16 + 0x4000u * banks + 0x2000u) return -4;
    memset(r, 0, sizeof(*r));
    for (int i = 0; i < 0x8000; i++) r->prg[i] = d[16 + (i % (0x4000 * banks))];
    memcpy(r->chr, d + 16 + 0x4000 * banks, 0x2000);
    switch (d[6] & 0xB) {
        case 0: r->nt[0] = 0; r->nt[1] = 0; r->nt[2] = 0x400; r->nt[3] = 0x400; break;
        case 1: r->nt[0] = 0; r->nt[1] = 0x400; r->nt[2] = 0; r->nt[3] = 0x400; break;
        default: r->nt[0] = r->nt[1] = r->nt[2] = r->nt[3] = 0; break;
    }
    return 0;
}

// ------------------------------------------------------------------ machine state (nes_core.hpp:90-114)
struct Machine {
    int64_t iter, exec_at, ppu_calls, nmi_thresh;
    uint8_t zero_skip;
    uint16_t pc;
    uint8_t sp, a, x, y, p;
    uint8_t joy_strobe[2], joy_buttons[2], joy_bits[2];
    uint8_t pstate, even, vblank, s0hit, first_write, data_buffer, oam_addr, fine_x;
    uint8_t show_bg, show_spr, hide_edge_bg, hide_edge_spr, long_spr, nmi_en, bg_page, spr_page;
    uint8_t nsl, sl[8];
    int32_t pcyc, scanline;
    uint16_t v, t, inc;
    uint8_t oam[256], pal[32], vram[0x800], ram[0x800];
};

static void canon(const Machine& m, uint8_t* o) {
    memset(o, 0, OR_CANON_BYTES);
    memcpy(o + 0, &m.iter, 8); memcpy(o + 8, &m.exec_at, 8); memcpy(o + 16, &m.ppu_calls, 8);
    memcpy(o + 24, &m.pcyc, 4); memcpy(o + 28, &m.scanline, 4);
    memcpy(o + 32, &m.pc, 2); memcpy(o + 34, &m.v, 2); memcpy(o + 36, &m.t, 2); memcpy(o + 38, &m.inc, 2);
    const uint8_t b1[] = {m.sp, m.a, m.x, m.y, m.p, m.zero_skip, m.joy_strobe[0], m.joy_strobe[1],
                          m.joy_buttons[0], m.joy_buttons[1], m.joy_bits[0], m.joy_bits[1],
                          m.pstate, m.even, m.vblank, m.s0hit, m.first_write, m.data_buffer, m.oam_addr, m.fine_x,
                          m.show_bg, m.show_spr, m.hide_edge_bg, m.hide_edge_spr, m.long_spr, m.nmi_en,
                          m.bg_page, m.spr_page, m.nsl};
    memcpy(o + 40, b1, sizeof(b1));
    for (int i = 0; i < m.nsl && i < 8; i++) o[69 + i] = m.sl[i];
    memcpy(o + 80, m.oam, 256); memcpy(o + 336, m.pal, 32);
    memcpy(o + 368, m.vram, 0x800); memcpy(o + 2416, m.ram, 0x800);
}

// ------------------------------------------------------------------ console
struct Console {
    Machine m;
    const Rom* rom = nullptr;
    bool render = false;
    uint8_t* screen = nullptr;          // optional 240*256 palette values
    uint8_t* gray = nullptr;            // optional 240*256 gray values
    const uint8_t* lut = nullptr;       // palette value -> gray
    int64_t cur = 0;                    // iteration of the executing instruction
    int skip = 0;                       // cycles added by the executing instruction
    int64_t bad_ops = 0, instructions = 0;

    // nes_core.hpp:123-147 (Emulator construction with zeroed memory, then CPU/PPU reset)
    void power_on(const Rom* r) {
        rom = r;
        memset(&m, 0, sizeof(m));
        m.joy_strobe[0] = m.joy_strobe[1] = 1;
        m.zero_skip = 0;
        m.a = m.x = m.y = 0;
        m.p = 0x34;
        m.pc = (uint16_t)(prg(0xfffc) | prg(0xfffd) << 8);
        m.sp = 0xfd;
        m.iter = m.exec_at = m.ppu_calls = 0;
        m.long_spr = 0; m.nmi_en = 0; m.vblank = 0; m.show_bg = 1; m.show_spr = 1; m.even = 1;
        m.first_write = 1; m.bg_page = 0; m.spr_page = 0; m.v = 0; m.pcyc = 0; m.scanline = 0;
        m.oam_addr = 0; m.fine_x = 0; m.t = 0; m.inc = 1; m.pstate = ST_PRE; m.nsl = 0;
        nmi_threshold();
    }

    uint8_t prg(uint16_t a) const { return rom->prg[a & 0x7fff]; }

    // ---- CPU bus, nes_core.hpp:150-208
    uint8_t read(uint16_t a) {
        if (a >= 0x8000) return prg(a);
        if (a < 0x2000) return m.ram[a & 0x7ff];
        if (a < 0x4000) {
            uint16_t r = a & 0x2007;
            if (r == 0x2002) { catch_up(); return status_read(); }
            if (r == 0x2007) { catch_up(); return data_read(); }
            if (r == 0x2004) return m.oam[m.oam_addr];
            return 0;
        }
        if (a == 0x4016) return pad_read(0);
        if (a == 0x4017) return pad_read(1);
        return 0;
    }
    void write(uint16_t a, uint8_t val) {
        if (a < 0x2000) { m.ram[a & 0x7ff] = val; return; }
        if (a < 0x4000) {
            switch (a & 0x2007) {
                case 0x2000: catch_up(); ctrl_write(val); break;
                case 0x2001: catch_up(); mask_write(val); break;
                case 0x2003: catch_up(); m.oam_addr = val; break;
                case 0x2004: catch_up(); m.oam[m.oam_addr] = val; m.oam_addr++; break;
                case 0x2005: catch_up(); scroll_write(val); break;
                case 0x2006: catch_up(); addr_write(val); break;
                case 0x2007: catch_up(); data_write(val); break;
                default: break;
            }
            return;
        }
        if (a == 0x4014) {  // OAM DMA: 513 or 514 cycles, copies only from RAM pages
            catch_up();
            skip += 513 + (int)((cur + 1) & 1);
            uint16_t src = (uint16_t)(val << 8);
            if (src < 0x2000)
                for (int i = 0; i < 256; i++) m.oam[(m.oam_addr + i) & 0xff] = m.ram[(src + i) & 0x7ff];
            return;
        }
        if (a == 0x4016) {
            for (int i = 0; i < 2; i++) {
                m.joy_strobe[i] = val & 1;
                if (!m.joy_strobe[i]) m.joy_bits[i] = m.joy_buttons[i];
            }
        }
    }
    uint8_t pad_read(int i) {
        uint8_t bit;
        if (m.joy_strobe[i]) bit = m.joy_buttons[i] & 1;
        else { bit = m.joy_bits[i] & 1; m.joy_bits[i] >>= 1; }
        return bit | 0x40;
    }

    // ---- PPU registers, nes_core.hpp:211-260
    void ctrl_write(uint8_t c) {
        m.nmi_en = (c >> 7) & 1;
        m.long_spr = (c >> 5) & 1;
        m.bg_page = (c >> 4) & 1;
        m.spr_page = (c >> 3) & 1;
        m.inc = (c & 4) ? 32 : 1;
        m.t = (uint16_t)((m.t & 0xf3ff) | ((c & 3) << 10));
    }
    void mask_write(uint8_t k) {
        m.hide_edge_bg = !(k & 2);
        m.hide_edge_spr = !(k & 4);
        m.show_bg = (k >> 3) & 1;
        m.show_spr = (k >> 4) & 1;
    }
    uint8_t status_read() {
        uint8_t r = (uint8_t)((m.s0hit << 6) | (m.vblank << 7));
        m.vblank = 0;
        m.first_write = 1;
        return r;
    }
    void addr_write(uint8_t d) {
        if (m.first_write) { m.t = (uint16_t)((m.t & 0x00ff) | ((d & 0x3f) << 8)); m.first_write = 0; }
        else { m.t = (uint16_t)((m.t & 0xff00) | d); m.v = m.t; m.first_write = 1; }
    }
    uint8_t data_read() {
        uint8_t d = vbus_read(m.v);
        m.v = (uint16_t)(m.v + m.inc);
        if (m.v < 0x3f00) { uint8_t buffered = m.data_buffer; m.data_buffer = d; d = buffered; }
        return d;
    }
    void data_write(uint8_t d) {
        vbus_write(m.v, d);
        m.v = (uint16_t)(m.v + m.inc);
    }
    void scroll_write(uint8_t d) {
        if (m.first_write) { m.t = (uint16_t)((m.t & ~0x1f) | (d >> 3)); m.fine_x = d & 7; m.first_write = 0; }
        else { m.t = (uint16_t)((m.t & ~0x73e0) | ((d & 7) << 12) | ((d & 0xf8) << 2)); m.first_write = 1; }
    }

    // ---- picture bus, nes_core.hpp:263-285
    int nt_index(uint16_t a) const { return a < 0x2400 ? 0 : a < 0x2800 ? 1 : a < 0x2c00 ? 2 : 3; }
    uint8_t vbus_read(uint16_t a) const {
        if (a < 0x2000) return rom->chr[a];
        if (a < 0x3eff) return m.vram[rom->nt[nt_index(a)] + (a & 0x3ff)];
        if (a < 0x3fff) return m.pal[a & 0x1f];
        return 0;
    }
    void vbus_write(uint16_t a, uint8_t d) {
        if (a < 0x2000) return;
        if (a < 0x3eff) m.vram[rom->nt[nt_index(a)] + (a & 0x3ff)] = d;
        else if (a < 0x3fff) m.pal[a == 0x3f10 ? 0 : (a & 0x1f)] = d;
    }
    uint8_t nametable(uint16_t a) const { return m.vram[rom->nt[(a >> 10) & 3] + (a & 0x3ff)]; }

    // ---- PPU timing, nes_core.hpp:289-308
    void nmi_threshold() {
        int line = m.pstate == ST_PRE ? -1 : m.pstate == ST_POST ? 240 : m.scanline;
        int64_t pos = (int64_t)(line + 1) * 341 + (m.pcyc - 1);
        const int64_t vbl = 242LL * 341;
        int64_t d = pos <= vbl ? vbl - pos + 1 : (262LL * 341 - pos) + vbl + 1;
        m.nmi_thresh = m.ppu_calls + d - 8;
    }
    void advance_to(int64_t target) {
        if (target > m.ppu_calls) { ppu_run(target - m.ppu_calls); nmi_threshold(); }
    }
    void catch_up() { advance_to(3 * (cur + 1)); }

    // ---- scroll helpers, nes_core.hpp:310-334
    void coarse_x_add(int n) {
        if (n <= 0) return;
        int tot = (m.v & 0x1f) + n;
        m.v = (uint16_t)((m.v & ~0x1f) | (tot & 31));
        if ((tot >> 5) & 1) m.v ^= 0x400;
    }
    void fine_y_step() {
        if ((m.v & 0x7000) != 0x7000) { m.v += 0x1000; return; }
        m.v &= ~0x7000;
        int y = (m.v >> 5) & 31;
        if (y == 29) { y = 0; m.v ^= 0x800; }
        else if (y == 31) y = 0;
        else y++;
        m.v = (uint16_t)((m.v & ~0x3e0) | (y << 5));
    }
    void copy_h() { m.v = (uint16_t)((m.v & ~0x41f) | (m.t & 0x41f)); }
    void copy_v() { m.v = (uint16_t)((m.v & ~0x7be0) | (m.t & 0x7be0)); }

    // per-line sprite list, scanning from oam_addr/4 (nes_core.hpp:336-349)
    void eval_sprites() {
        m.nsl = 0;
        int h = m.long_spr ? 16 : 8;
        for (int i = m.oam_addr / 4; i < 64 && m.nsl < 8; i++) {
            int d = m.scanline - m.oam[i * 4];
            if (d >= 0 && d < h) m.sl[m.nsl++] = (uint8_t)i;
        }
    }

    // background: 2-bit pattern value plus attribute bits at dot x for the current v (nes_core.hpp:352-367)
    uint8_t bg_colour(int x, uint8_t* pattern) const {
        int xf = (m.fine_x + x) % 8;
        uint8_t tile = nametable((uint16_t)(0x2000 | (m.v & 0x0fff)));
        uint16_t pa = (uint16_t)(((tile * 16) + ((m.v >> 12) & 7)) | (m.bg_page << 12));
        uint8_t c = (uint8_t)(((rom->chr[pa] >> (7 ^ xf)) & 1) | (((rom->chr[pa + 8] >> (7 ^ xf)) & 1) << 1));
        *pattern = c;
        uint16_t aa = (uint16_t)(0x23c0 | (m.v & 0x0c00) | ((m.v >> 4) & 0x38) | ((m.v >> 2) & 7));
        int sh = ((m.v >> 4) & 4) | (m.v & 2);
        return (uint8_t)(c | (((nametable(aa) >> sh) & 3) << 2));
    }
    // sprite i's 2-bit pattern value at (x, y), with C++ int semantics for stale lists (nes_core.hpp:369-391)
    uint8_t sprite_pattern(int i, int x, int y) const {
        uint8_t sx = m.oam[i * 4 + 3];
        uint8_t sy = (uint8_t)(m.oam[i * 4] + 1), tile = m.oam[i * 4 + 1], attr = m.oam[i * 4 + 2];
        int h = m.long_spr ? 16 : 8;
        int xs = (x - sx) % 8, yo = (y - sy) % h;
        if (!(attr & 0x40)) xs ^= 7;
        if (attr & 0x80) yo ^= (h - 1);
        uint16_t a;
        if (!m.long_spr) {
            a = (uint16_t)(tile * 16 + yo);
            if (m.spr_page) a += 0x1000;
        } else {
            yo = (yo & 7) | ((yo & 8) << 1);
            a = (uint16_t)((tile >> 1) * 32 + yo);
            a |= (tile & 1) << 12;
        }
        return (uint8_t)(((vbus_read(a) >> xs) & 1) | (((vbus_read((uint16_t)(a + 8)) >> xs) & 1) << 1));
    }

    // visible dots [x0, x1) without pixel output: only CPU-visible effects (nes_core.hpp:394-413)
    void dots_quiet(int x0, int x1) {
        if (!m.show_bg) return;
        bool s0_window = !m.s0hit && m.show_spr && m.nsl > 0 && m.sl[0] == 0;
        for (int x = x0; x < x1; x++) {
            if (s0_window && !m.s0hit && x >= m.oam[3] && x < m.oam[3] + 8 && (!m.hide_edge_spr || x >= 8) &&
                (!m.hide_edge_bg || x >= 8)) {
                uint8_t pat;
                bg_colour(x, &pat);
                if (pat && sprite_pattern(0, x, m.scanline)) m.s0hit = 1;
            }
            if ((m.fine_x + x) % 8 == 7) coarse_x_add(1);
        }
    }

    // visible dots [x0, x1) with pixel output (nes_core.hpp:467-513; per-dot form of the span renderer)
    void dots_drawn(int x0, int x1) {
        const int y = m.scanline;
        for (int x = x0; x < x1; x++) {
            uint8_t pa = 0, bg_op = 0;
            if (m.show_bg) {
                uint8_t pat;
                uint8_t c = bg_colour(x, &pat);
                if (!(m.hide_edge_bg && x < 8) && pat) { pa = c; bg_op = pat; }
                if ((m.fine_x + x) % 8 == 7) coarse_x_add(1);
            }
            if (m.show_spr && m.nsl && !(m.hide_edge_spr && x < 8)) {
                for (int k = 0; k < m.nsl; k++) {   // first opaque sprite of the list wins
                    int i = m.sl[k];
                    int sx = m.oam[i * 4 + 3];
                    if (x < sx || x >= sx + 8) continue;
                    uint8_t c = sprite_pattern(i, x, y);
                    if (!c) continue;
                    uint8_t attr = m.oam[i * 4 + 2];
                    if (i == 0 && bg_op && !m.s0hit && m.show_bg) m.s0hit = 1;
                    if (!bg_op || !(attr & 0x20)) pa = (uint8_t)(c | 0x10 | ((attr & 3) << 2));
                    break;
                }
            }
            if (screen) screen[y * 256 + x] = m.pal[pa];
            if (gray) gray[y * 256 + x] = lut[m.pal[pa]];
        }
    }

    // NMI raised by PPU call `call` (1-based); nes_core.hpp:520-531
    void nmi(int64_t call) {
        int64_t it = (call - 1) / 3;
        push((uint8_t)(m.pc >> 8));
        push((uint8_t)m.pc);
        push((uint8_t)(m.p | 0x20));
        m.p |= FI;
        m.pc = (uint16_t)(prg(0xfffa) | prg(0xfffb) << 8);
        int64_t d = (m.zero_skip && it == m.exec_at) ? 0 : (m.exec_at - it + 1);
        m.exec_at = it + d + 6;
        m.zero_skip = 0;
    }

    // advance the PPU by n calls (nes_core.hpp:539-616)
    void ppu_run(int64_t n) {
        while (n > 0) {
            int c = m.pcyc;
            if (m.pstate == ST_PRE) {
                bool on = m.show_bg && m.show_spr;
                int end = kLineEnd - (!m.even && on);
                int64_t k = c >= end ? 1 : (n < end - c ? n : end - c);
                int a = c, b = (int)(c + k);
                if (a <= 1 && 1 < b) m.vblank = m.s0hit = 0;
                if (on) {
                    if (a <= 258 && 258 < b) copy_h();
                    if (a <= 304 && 281 < b) copy_v();
                }
                m.ppu_calls += k; n -= k;
                if (b - 1 >= end) { m.pstate = ST_RENDER; m.scanline = 0; m.pcyc = 1; }
                else m.pcyc = b;
            } else if (m.pstate == ST_RENDER) {
                if (c >= 1 && c <= 256) {
                    int64_t k = n < 257 - c ? n : 257 - c;
                    if (render) dots_drawn(c - 1, (int)(c - 1 + k));
                    else dots_quiet(c - 1, (int)(c - 1 + k));
                    m.pcyc += (int)k; m.ppu_calls += k; n -= k;
                } else if (c == 257) {
                    if (m.show_bg) fine_y_step();
                    m.pcyc++; m.ppu_calls++; n--;
                } else if (c == 258) {
                    if (m.show_bg && m.show_spr) copy_h();
                    m.pcyc++; m.ppu_calls++; n--;
                } else if (c > 258 && c < kLineEnd) {
                    int64_t k = n < kLineEnd - c ? n : kLineEnd - c;
                    m.pcyc += (int)k; m.ppu_calls += k; n -= k;
                } else if (c >= kLineEnd) {
                    eval_sprites();
                    m.scanline++;
                    m.pcyc = 1; m.ppu_calls++; n--;
                    if (m.scanline >= 240) m.pstate = ST_POST;
                } else {
                    m.pcyc++; m.ppu_calls++; n--;
                }
            } else if (m.pstate == ST_POST) {
                if (c >= kLineEnd) {
                    m.scanline++; m.pcyc = 1; m.pstate = ST_VBLANK;
                    m.ppu_calls++; n--;
                } else {
                    int64_t k = n < kLineEnd - c ? n : kLineEnd - c;
                    m.pcyc += (int)k; m.ppu_calls += k; n -= k;
                }
            } else {
                if (c >= kLineEnd) {
                    m.scanline++;
                    m.pcyc = 1;
                    if (m.scanline >= 261) { m.pstate = ST_PRE; m.scanline = 0; m.even = !m.even; }
                    m.ppu_calls++; n--;
                } else if (c == 1 && m.scanline == 241) {
                    m.vblank = 1;
                    m.ppu_calls++; n--;
                    m.pcyc = 2;
                    if (m.nmi_en) nmi(m.ppu_calls);
                } else {
                    int lim = kLineEnd - c;
                    if (m.scanline == 241 && c < 1) lim = 1 - c;
                    int64_t k = n < lim ? n : lim;
                    m.pcyc += (int)k; m.ppu_calls += k; n -= k;
                }
            }
        }
    }

    // ---- CPU helpers, nes_core.hpp:619-642
    void set_nz(uint8_t r) { m.p = (uint8_t)((m.p & ~(FZ | FN)) | (r ? 0 : FZ) | ((r & 0x80) ? FN : 0)); }
    void flag(uint8_t f, bool on) { m.p = on ? (uint8_t)(m.p | f) : (uint8_t)(m.p & ~f); }
    bool has(uint8_t f) const { return (m.p & f) != 0; }
    uint16_t read16(uint16_t a) { uint8_t lo = read(a); uint8_t hi = read((uint16_t)(a + 1)); return (uint16_t)(lo | hi << 8); }
    void push(uint8_t d) { m.ram[(0x100 | m.sp) & 0x7ff] = d; m.sp--; }
    uint8_t pull() { m.sp++; return m.ram[(0x100 | m.sp) & 0x7ff]; }
    void cross_penalty(uint16_t a, uint16_t b, int k) { if ((a & 0xff00) != (b & 0xff00)) skip += k; }

    // implied-class opcodes (nes_core.hpp:644-690)
    bool op_implied(uint8_t op) {
        switch (op) {
            case 0x00:  // BRK: pushes p | 0x30 in this layout (I and D), vector $FFFE
                m.pc++;
                push((uint8_t)(m.pc >> 8)); push((uint8_t)m.pc);
                push((uint8_t)(m.p | 0x30));
                m.p |= FI;
                m.pc = read16(0xfffe);
                skip += 7;
                return true;
            case 0x08: push(m.p); return true;
            case 0x18: flag(FC, false); return true;
            case 0x20: {
                uint16_t ret = (uint16_t)(m.pc + 1);
                push((uint8_t)(ret >> 8)); push((uint8_t)ret);
                m.pc = read16(m.pc);
                return true;
            }
            case 0x28: m.p = pull(); return true;
            case 0x38: flag(FC, true); return true;
            case 0x40: { m.p = pull(); uint8_t lo = pull(); uint8_t hi = pull(); m.pc = (uint16_t)(lo | hi << 8); return true; }
            case 0x48: push(m.a); return true;
            case 0x4c: m.pc = read16(m.pc); return true;
            case 0x58: flag(FI, false); return true;
            case 0x60: { uint8_t lo = pull(); uint8_t hi = pull(); m.pc = (uint16_t)((lo | hi << 8) + 1); return true; }
            case 0x68: m.a = pull(); set_nz(m.a); return true;
            case 0x6c: {  // JMP (ind) with the page-wrap of the pointer's high byte
                uint16_t ptr = read16(m.pc);
                uint8_t lo = read(ptr);
                uint8_t hi = read((uint16_t)((ptr & 0xff00) | ((ptr + 1) & 0xff)));
                m.pc = (uint16_t)(lo | hi << 8);
                return true;
            }
            case 0x78: flag(FI, true); return true;
            case 0x88: m.y--; set_nz(m.y); return true;
            case 0x8a: m.a = m.x; set_nz(m.a); return true;
            case 0x98: m.a = m.y; set_nz(m.a); return true;
            case 0x9a: m.sp = m.x; return true;
            case 0xa8: m.y = m.a; set_nz(m.y); return true;
            case 0xaa: m.x = m.a; set_nz(m.x); return true;
            case 0xb8: flag(FV, false); return true;
            case 0xba: m.x = m.sp; set_nz(m.x); return true;
            case 0xc8: m.y++; set_nz(m.y); return true;
            case 0xca: m.x--; set_nz(m.x); return true;
            case 0xd8: flag(FD, false); return true;
            case 0xe8: m.x++; set_nz(m.x); return true;
            case 0xea: return true;
            case 0xf8: flag(FD, true); return true;
            default: return false;
        }
    }

    // branches: one extra cycle when taken, two more on a page cross (nes_core.hpp:692-710)
    bool op_branch(uint8_t op) {
        if ((op & 0x1f) != 0x10) return false;
        static const uint8_t which[4] = {FN, FV, FC, FZ};
        bool want = (op & 0x20) != 0;
        bool take = has(which[op >> 6]) == want;
        if (take) {
            int8_t off = (int8_t)read(m.pc++);
            skip += 1;
            uint16_t to = (uint16_t)(m.pc + off);
            cross_penalty(m.pc, to, 2);
            m.pc = to;
        } else {
            m.pc++;
        }
        return true;
    }

    // group 0 (op & 3 == 0): BIT/STY/LDY/CPY/CPX (nes_core.hpp:712-752)
    bool op_group0(uint8_t op) {
        if ((op & 3) != 0) return false;
        uint16_t ea;
        switch ((op >> 2) & 7) {
            case 0: ea = m.pc++; break;
            case 1: ea = read(m.pc++); break;
            case 3: ea = read16(m.pc); m.pc += 2; break;
            case 5: ea = (uint8_t)(read(m.pc++) + m.x); break;
            case 7: ea = read16(m.pc); m.pc += 2; cross_penalty(ea, (uint16_t)(ea + m.x), 1); ea = (uint16_t)(ea + m.x); break;
            default: return false;
        }
        switch (op >> 5) {
            case 1: { uint8_t d = read(ea); flag(FZ, !(m.a & d)); flag(FV, d & 0x40); flag(FN, d & 0x80); return true; }
            case 4: write(ea, m.y); return true;
            case 5: m.y = read(ea); set_nz(m.y); return true;
            case 6: { uint16_t r = (uint16_t)(m.y - read(ea)); flag(FC, !(r & 0x100)); set_nz((uint8_t)r); return true; }
            case 7: { uint16_t r = (uint16_t)(m.x - read(ea)); flag(FC, !(r & 0x100)); set_nz((uint8_t)r); return true; }
            default: return false;
        }
    }

    // group 1 (op & 3 == 1): ORA AND EOR ADC STA LDA CMP SBC, every mode (nes_core.hpp:754-823)
    bool op_group1(uint8_t op) {
        if ((op & 3) != 1) return false;
        int fn = op >> 5;
        bool store = fn == 4;
        uint16_t ea;
        switch ((op >> 2) & 7) {
            case 0: { uint8_t z = (uint8_t)(m.x + read(m.pc++)); uint8_t lo = read(z); uint8_t hi = read((uint8_t)(z + 1)); ea = (uint16_t)(lo | hi << 8); break; }
            case 1: ea = read(m.pc++); break;
            case 2: ea = m.pc++; break;
            case 3: ea = read16(m.pc); m.pc += 2; break;
            case 4: {
                uint8_t z = read(m.pc++); uint8_t lo = read(z); uint8_t hi = read((uint8_t)(z + 1));
                ea = (uint16_t)(lo | hi << 8);
                if (!store) cross_penalty(ea, (uint16_t)(ea + m.y), 1);
                ea = (uint16_t)(ea + m.y);
                break;
            }
            case 5: ea = (uint8_t)(read(m.pc++) + m.x); break;
            case 6: ea = read16(m.pc); m.pc += 2; if (!store) cross_penalty(ea, (uint16_t)(ea + m.y), 1); ea = (uint16_t)(ea + m.y); break;
            default: ea = read16(m.pc); m.pc += 2; if (!store) cross_penalty(ea, (uint16_t)(ea + m.x), 1); ea = (uint16_t)(ea + m.x); break;
        }
        switch (fn) {
            case 0: m.a |= read(ea); set_nz(m.a); break;
            case 1: m.a &= read(ea); set_nz(m.a); break;
            case 2: m.a ^= read(ea); set_nz(m.a); break;
            case 3: {
                uint8_t d = read(ea);
                uint16_t s = (uint16_t)(m.a + d + (has(FC) ? 1 : 0));
                flag(FC, s & 0x100);
                flag(FV, (m.a ^ s) & (d ^ s) & 0x80);
                m.a = (uint8_t)s; set_nz(m.a);
                break;
            }
            case 4: write(ea, m.a); break;
            case 5: m.a = read(ea); set_nz(m.a); break;
            case 6: { uint16_t r = (uint16_t)(m.a - read(ea)); flag(FC, !(r & 0x100)); set_nz((uint8_t)r); break; }
            default: {
                uint16_t d = read(ea);
                uint16_t r = (uint16_t)(m.a - d - (has(FC) ? 0 : 1));
                flag(FC, !(r & 0x100));
                flag(FV, (m.a ^ r) & (~d ^ r) & 0x80);
                m.a = (uint8_t)r; set_nz((uint8_t)r);
                break;
            }
        }
        return true;
    }

    // group 2 (op & 3 == 2): ASL ROL LSR ROR STX LDX DEC INC (nes_core.hpp:825-889); every abs,X/abs,Y
    // form pays the page-cross cycle, including the read-modify-write ones.
    bool op_group2(uint8_t op) {
        if ((op & 3) != 2) return false;
        int fn = op >> 5, mode = (op >> 2) & 7;
        bool xy = fn == 4 || fn == 5;          // STX/LDX index with Y
        uint16_t ea = 0;
        switch (mode) {
            case 0: ea = m.pc++; break;
            case 1: ea = read(m.pc++); break;
            case 2: break;
            case 3: ea = read16(m.pc); m.pc += 2; break;
            case 5: ea = (uint8_t)(read(m.pc++) + (xy ? m.y : m.x)); break;
            case 7: { ea = read16(m.pc); m.pc += 2; uint8_t ix = xy ? m.y : m.x; cross_penalty(ea, (uint16_t)(ea + ix), 1); ea = (uint16_t)(ea + ix); break; }
            default: return false;
        }
        switch (fn) {
            case 0: case 1: {
                bool cin = has(FC) && fn == 1;
                if (mode == 2) { flag(FC, m.a & 0x80); m.a = (uint8_t)((m.a << 1) | cin); set_nz(m.a); }
                else { uint8_t d = read(ea); flag(FC, d & 0x80); d = (uint8_t)((d << 1) | cin); set_nz(d); write(ea, d); }
                break;
            }
            case 2: case 3: {
                bool cin = has(FC) && fn == 3;
                if (mode == 2) { flag(FC, m.a & 1); m.a = (uint8_t)((m.a >> 1) | (cin << 7)); set_nz(m.a); }
                else { uint8_t d = read(ea); flag(FC, d & 1); d = (uint8_t)((d >> 1) | (cin << 7)); set_nz(d); write(ea, d); }
                break;
            }
            case 4: write(ea, m.x); break;
            case 5: m.x = read(ea); set_nz(m.x); break;
            case 6: { uint8_t d = (uint8_t)(read(ea) - 1); set_nz(d); write(ea, d); break; }
            default: { uint8_t d = (uint8_t)(read(ea) + 1); set_nz(d); write(ea, d); break; }
        }
        return true;
    }

    // one instruction; returns the cycles it takes (nes_core.hpp:892-899, 901-1163)
    int step_instruction() {
        skip = 0;
        uint8_t op = read(m.pc++);
        instructions++;
        if (op_implied(op) || op_branch(op) || op_group1(op) || op_group2(op) || op_group0(op)) skip += kCycles[op];
        else bad_ops++;
        return skip;
    }

    // one nes-py Emulator::step (nes_core.hpp:1166-1204), with the exact `JMP *` idle fast-forward
    void frame() {
        const int64_t end = m.iter + kFrameIters;
        while (m.exec_at < end) {
            const int64_t j = m.exec_at;
            if (3 * (j + 1) >= m.nmi_thresh) {
                cur = j;
                advance_to(3 * (j + 1));
                if (m.exec_at != j) continue;
            }
            uint16_t pc = m.pc;
            auto fetch = [&](uint16_t a) -> uint8_t { return a >= 0x8000 ? prg(a) : 0xff; };
            if (fetch(pc) == 0x4c && (uint16_t)(fetch((uint16_t)(pc + 1)) | fetch((uint16_t)(pc + 2)) << 8) == pc) {
                int64_t lim_end = end - j, lim_nmi = m.nmi_thresh - 3 * (j + 1);
                int64_t k1 = lim_end > 0 ? (lim_end + 2) / 3 : 0;
                int64_t k2 = lim_nmi > 0 ? (lim_nmi + 8) / 9 : 0;
                int64_t k = k1 < k2 ? k1 : k2;
                if (k > 1) { m.exec_at = j + 3 * (k - 1); m.zero_skip = 0; continue; }
            }
            cur = j;
            int s = step_instruction();
            m.exec_at = j + (s >= 1 ? s : 1);
            m.zero_skip = s <= 0;
        }
        advance_to(3 * end);
        m.iter = end;
    }
};

// ------------------------------------------------------------------ numpy PCG64 (fastmario.cpp:39-78)
struct Pcg {
    unsigned __int128 state = 0, inc = 0;
    int has32 = 0;
    uint32_t half = 0;
    uint64_t next64() {
        const unsigned __int128 mul = ((unsigned __int128)0x2360ED051FC65DA4ULL << 64) | 0x4385DF649FCCF645ULL;
        state = state * mul + inc;
        uint64_t x = (uint64_t)(state >> 64) ^ (uint64_t)state;
        unsigned r = (unsigned)(state >> 122);
        return (x >> r) | (x << ((64 - r) & 63));
    }
    uint32_t next32() {
        if (has32) { has32 = 0; return half; }
        uint64_t v = next64();
        has32 = 1; half = (uint32_t)(v >> 32);
        return (uint32_t)v;
    }
    double random() { return (double)(next64() >> 11) * (1.0 / 9007199254740992.0); }
    int64_t integers(int64_t high) {   // Generator.integers(0, high), 32-bit Lemire with rejection
        uint64_t rng = (uint64_t)(high - 1);
        if (rng == 0) return 0;
        if (rng == 0xffffffffULL) return next32();
        uint32_t excl = (uint32_t)rng + 1;
        uint64_t prod = (uint64_t)next32() * excl;
        uint32_t left = (uint32_t)prod;
        if (left < excl) {
            uint32_t thr = (uint32_t)((0xffffffffu - (uint32_t)rng) % excl);
            while (left < thr) { prod = (uint64_t)next32() * excl; left = (uint32_t)prod; }
        }
        return (int64_t)(prod >> 32);
    }
};

// ------------------------------------------------------------------ INTER_AREA (fastmario.cpp:80-130)
struct Tap { int di, si; float w; };
static int area_tab(int ssize, int dsize, Tap* t) {
    double scale = 1.0 / ((double)dsize / ssize);
    int k = 0;
    for (int dx = 0; dx < dsize; dx++) {
        double f1 = dx * scale, f2 = f1 + scale;
        double cell = scale < ssize - f1 ? scale : ssize - f1;
        int s1 = (int)std::ceil(f1), s2 = (int)std::floor(f2);
        if (s2 > ssize - 1) s2 = ssize - 1;
        if (s1 > s2) s1 = s2;
        if (s1 - f1 > 1e-3) t[k++] = {dx, s1 - 1, (float)((s1 - f1) / cell)};
        for (int s = s1; s < s2; s++) t[k++] = {dx, s, (float)(1.0 / cell)};
        if (f2 - s2 > 1e-3) {
            double w = f2 - s2 < 1.0 ? f2 - s2 : 1.0;
            if (cell < w) w = cell;
            t[k++] = {dx, s2, (float)(w / cell)};
        }
    }
    return k;
}
static uint8_t round_sat(float v) {
    long r = lrintf(v);
    return (uint8_t)(r < 0 ? 0 : r > 255 ? 255 : r);
}
// 240x256 -> 84x84 in OpenCV's float order: per source row a horizontal tap sum, then the vertical
// sum of weighted rows, flushed when the output row changes.
static void area_resize(const uint8_t* src, uint8_t* dst) {
    static Tap xt[512], yt[512];
    static int xn = 0, yn = 0;
    if (!xn) { xn = area_tab(256, 84, xt); yn = area_tab(240, 84, yt); }
    float row[84], acc[84];
    int cur = yt[0].di;
    for (int d = 0; d < 84; d++) acc[d] = 0.f;
    for (int j = 0; j < yn; j++) {
        const uint8_t* s = src + yt[j].si * 256;
        for (int d = 0; d < 84; d++) row[d] = 0.f;
        for (int k = 0; k < xn; k++) row[xt[k].di] += s[xt[k].si] * xt[k].w;
        float beta = yt[j].w;
        if (yt[j].di != cur) {
            for (int d = 0; d < 84; d++) { dst[cur * 84 + d] = round_sat(acc[d]); acc[d] = beta * row[d]; }
            cur = yt[j].di;
        } else {
            for (int d = 0; d < 84; d++) acc[d] += beta * row[d];
        }
    }
    for (int d = 0; d < 84; d++) dst[cur * 84 + d] = round_sat(acc[d]);
}

// ------------------------------------------------------------------ SMB RAM protocol (fastmario.cpp:204-250)
static int64_t dec_digits(const uint8_t* r, int n) {   // int(''.join(map(str, ram[a:a+n])))
    int64_t v = 0;
    for (int i = 0; i < n; i++) v = v * (r[i] >= 100 ? 1000 : r[i] >= 10 ? 100 : 10) + r[i];
    return v;
}
struct Info { int64_t v[10]; };   // x_pos flag_get life score time world stage coins y_pos status
static int64_t smb_x(const uint8_t* r) { return (int64_t)r[0x6d] * 256 + r[0x86]; }
static int64_t smb_time(const uint8_t* r) { return dec_digits(r + 0x7f8, 3); }
static bool smb_dying(const uint8_t* r) { return r[0x0e] == 0x0b || r[0xb5] > 1; }
static bool smb_dead(const uint8_t* r) { return r[0x0e] == 0x06; }
static bool smb_busy(const uint8_t* r) { return r[0x0e] <= 5 || r[0x0e] == 7; }
static bool smb_world_over(const uint8_t* r) { return r[0x770] == 2; }
static bool smb_stage_over(const uint8_t* r) {
    for (int a = 0x16; a <= 0x1a; a++)
        if (r[a] == 0x2d || r[a] == 0x31) return r[0x1d] == 3;
    return false;
}
static Info smb_info(const uint8_t* r) {
    Info i;
    i.v[0] = smb_x(r);
    i.v[1] = smb_world_over(r) || smb_stage_over(r);
    i.v[2] = r[0x75a];
    i.v[3] = dec_digits(r + 0x7de, 6);
    i.v[4] = smb_time(r);
    i.v[5] = r[0x75f] + 1;
    i.v[6] = r[0x75c] + 1;
    i.v[7] = dec_digits(r + 0x7ed, 2);
    i.v[8] = r[0xb5] < 1 ? 255 + (255 - r[0x3b8]) : 255 - r[0x3b8];
    i.v[9] = r[0x756] == 0 ? 0 : r[0x756] == 1 ? 1 : 2;
    return i;
}

// ------------------------------------------------------------------ env (fastmario.cpp:260-411)
static const int kGray = 256 * 240, kObs = 84 * 84;

struct Level {
    int world, stage, area;
    Machine boot;
    int64_t x0, time0;
    uint8_t obs0[kObs];
};

struct Cfg { int skip, max_steps, noop_max, maxpool, stack; double sticky; };

struct Env {
    Console con;
    const Level* lvl = nullptr;
    const Cfg* cfg = nullptr;
    Pcg rng;
    int64_t x_last = 0, time_last = 0;
    int prev = 0, lives = -1, t = 0, ep_len = 0;
    double ep_ret = 0.0;
    bool shows_boot = false, pooled = false;
    std::vector<uint8_t> g, g_prev;
    Info info{};
    int64_t frames = 0;
    int reemu_kind = -1;             // branch of the last agent step's early termination (-1: none)
    bool reemu_k2 = false;           // ... and it ended at frame K-2 under max-pool
    int64_t reemu[3] = {0, 0, 0};    // env steps (not reset no-ops) by kind: re-ran last alone, with last-1, K-2 ends

    void restore() { con.m = lvl->boot; x_last = lvl->x0; time_last = lvl->time0; shows_boot = true; }
    void nes_frame(uint8_t buttons, bool render) {
        con.m.joy_buttons[0] = buttons;
        con.render = render;
        con.frame();
        frames++;
        if (render) shows_boot = false;
    }
    // _skip_change_area / _skip_occupied_states of a not-done env (fastmario.cpp:297-308)
    void skip_busy(bool render) {
        uint8_t* r = con.m.ram;
        if (r[0x6de] > 1 && r[0x6de] < 255) r[0x6de] = 1;
        while (smb_busy(r) || smb_world_over(r)) { r[0x7a0] = 0; nes_frame(0, render); }
    }
    // nes-py step: reward, done, info, then the hacks (fastmario.cpp:310-334)
    double frame_step(uint8_t buttons, bool render, bool* done) {
        nes_frame(buttons, render);
        const uint8_t* r = con.m.ram;
        int64_t x = smb_x(r), dx = x - x_last;
        x_last = x;
        if (dx < -5 || dx > 5) dx = 0;
        int64_t tm = smb_time(r), dt = tm - time_last;
        time_last = tm;
        if (dt > 0) dt = 0;
        bool die = smb_dying(r) || smb_dead(r);
        int64_t rew = dx + dt + (die ? -25 : 0);
        if (rew < -15) rew = -15;
        if (rew > 15) rew = 15;
        info = smb_info(r);
        *done = die || info.v[1];
        if (!*done) skip_busy(render);
        return (double)rew;
    }
    // sticky + frame skip + max-pool + early termination + life loss (fastmario.cpp:336-374)
    double agent_step(int a, bool want_obs, bool* term) {
        const int K = cfg->skip;
        const bool mp = cfg->maxpool != 0;
        Machine snaps[16];
        uint8_t acts[16];
        double total = 0.0;
        bool done = false;
        int i;
        for (i = 0; i < K; i++) {
            int act = a;
            if (cfg->sticky != 0.0 && rng.random() < cfg->sticky) act = prev;
            prev = act;
            bool render = want_obs && (i == K - 1 || (mp && i == K - 2));
            if (want_obs) snaps[i] = con.m;
            acts[i] = (uint8_t)act;
            total += frame_step(kButtons[act], render, &done);
            if (want_obs && mp && i == K - 2) g_prev = g;
            if (done) break;
        }
        int last = done ? i : K - 1;
        reemu_kind = -1;
        if (want_obs && done && last < K - 1) {
            reemu_kind = (mp && last >= 1) ? 1 : 0;
            reemu_k2 = mp && last == K - 2;
            if (mp && last >= 1) {
                con.m = snaps[last - 1];
                nes_frame(kButtons[acts[last - 1]], true);
                skip_busy(true);
                g_prev = g;
            } else {
                con.m = snaps[last];
            }
            nes_frame(kButtons[acts[last]], true);
        }
        if (want_obs) pooled = mp && last >= 1;
        bool tm = done;
        int life = (int)info.v[2];
        if (lives >= 0 && life < lives) tm = true;
        lives = life;
        if (info.v[1]) tm = true;
        *term = tm;
        return total;
    }
    void observe(uint8_t* out, bool allow_pool) {   // fastmario.cpp:377-386
        if (shows_boot) { memcpy(out, lvl->obs0, kObs); return; }
        if (allow_pool && pooled) {
            std::vector<uint8_t> mx(kGray);
            for (int k = 0; k < kGray; k++) mx[k] = g_prev[k] > g[k] ? g_prev[k] : g[k];
            area_resize(mx.data(), out);
        } else {
            area_resize(g.data(), out);
        }
    }
    void reset(uint8_t* out) {   // fastmario.cpp:389-401
        restore(); prev = 0; lives = -1;
        if (cfg->noop_max) {
            int64_t k = rng.integers(cfg->noop_max + 1);
            for (int64_t j = 0; j < k; j++) {
                bool tm;
                agent_step(0, j == k - 1, &tm);
                if (tm) { restore(); prev = 0; lives = -1; }
            }
        }
        t = 0; ep_ret = 0.0; ep_len = 0;
        observe(out, false);
    }
    void step(int a, uint8_t* out, float* rew, bool* term, bool* trunc) {   // fastmario.cpp:403-411
        bool tm;
        double r = agent_step(a, true, &tm);
        if (reemu_kind >= 0) { reemu[reemu_kind]++; reemu[2] += reemu_k2; }
        t++;
        *trunc = t >= cfg->max_steps;
        ep_ret += r; ep_len++;
        *rew = (float)r; *term = tm;
        observe(out, true);
    }
};

// power-on + title sequence with the target level written into RAM (fastmario.cpp:414-445)
static void boot_level(const Rom* rom, const uint8_t* lut, Level* L) {
    Console c;
    std::vector<uint8_t> g(kGray, 0);
    c.gray = g.data(); c.lut = lut;
    c.power_on(rom);
    auto fr = [&](uint8_t b) { c.m.joy_buttons[0] = b; c.render = true; c.frame(); };
    uint8_t* r = c.m.ram;
    fr(8); fr(0);
    while (smb_time(r) == 0) {
        fr(8);
        r[0x75f] = (uint8_t)(L->world - 1); r[0x75c] = (uint8_t)(L->stage - 1); r[0x760] = (uint8_t)(L->area - 1);
        fr(0);
        r[0x7a0] = 0;
    }
    int64_t tl = smb_time(r);
    while (smb_time(r) >= tl) { tl = smb_time(r); fr(8); fr(0); }
    L->boot = c.m;
    L->x0 = smb_x(r);
    L->time0 = smb_time(r);
    area_resize(g.data(), L->obs0);
}

struct Vec {
    int n = 0, K = 4;
    Cfg cfg{};
    Rom rom;
    uint8_t lut[256];
    std::vector<Level*> levels;
    std::vector<int> env_level;
    std::vector<Env> envs;
    uint8_t *obs = nullptr, *fin = nullptr, *term = nullptr, *trunc = nullptr;
    float* rew = nullptr;
    int64_t *info = nullptr, *ep_len = nullptr;
    double* ep_ret = nullptr;
    ~Vec() { for (auto* l : levels) delete l; }

    // frame stack shift, final_obs and auto-reset (fastmario.cpp:477-504)
    void step_env(int i, int act) {
        Env& e = envs[i];
        uint8_t* st = obs + (size_t)i * K * kObs;
        uint8_t o[kObs];
        float r; bool te, tr;
        e.step(act, o, &r, &te, &tr);
        rew[i] = r; term[i] = te; trunc[i] = tr;
        for (int k = 0; k < 10; k++) info[(size_t)i * 10 + k] = e.info.v[k];
        memmove(st, st + kObs, (size_t)(K - 1) * kObs);
        if (te || tr) {
            uint8_t* fo = fin + (size_t)i * K * kObs;
            memcpy(fo, st, (size_t)(K - 1) * kObs);
            memcpy(fo + (size_t)(K - 1) * kObs, o, kObs);
            ep_ret[i] = e.ep_ret; ep_len[i] = e.ep_len;
            e.reset(o);
            memset(st, 0, (size_t)(K - 1) * kObs);
        }
        memcpy(st + (size_t)(K - 1) * kObs, o, kObs);
    }
    void reset_env(int i) {
        uint8_t* st = obs + (size_t)i * K * kObs;
        uint8_t o[kObs];
        envs[i].reset(o);
        memset(st, 0, (size_t)K * kObs);
        memcpy(st + (size_t)(K - 1) * kObs, o, kObs);
    }
};

struct Raw {
    Rom rom;
    Console c;
    Machine saved;
    std::vector<uint8_t> screen, g;
    uint8_t lut[256];
};

}  // namespace orc

using namespace orc;

extern "C" {

void* or_raw_create(const uint8_t* rom, int64_t len) {
    Raw* r = new Raw();
    if (rom_load(&r->rom, rom, (size_t)len) != 0) { delete r; return nullptr; }
    r->screen.assign(kGray, 0); r->g.assign(kGray, 0);
    for (int i = 0; i < 256; i++) r->lut[i] = (uint8_t)i;
    r->c.screen = r->screen.data(); r->c.gray = r->g.data(); r->c.lut = r->lut;
    r->c.power_on(&r->rom);
    return r;
}
void or_raw_frame(void* h, int buttons, int render) {
    Raw* r = (Raw*)h;
    r->c.m.joy_buttons[0] = (uint8_t)buttons;
    r->c.render = render != 0;
    r->c.frame();
}
const uint8_t* or_raw_ram(void* h) { return ((Raw*)h)->c.m.ram; }
const uint8_t* or_raw_screen(void* h) { return ((Raw*)h)->screen.data(); }
void or_raw_backup(void* h) { Raw* r = (Raw*)h; r->saved = r->c.m; }
void or_raw_restore(void* h) { Raw* r = (Raw*)h; r->c.m = r->saved; }
int64_t or_raw_bad_ops(void* h) { return ((Raw*)h)->c.bad_ops; }
int64_t or_raw_instructions(void* h) { return ((Raw*)h)->c.instructions; }
void or_raw_canon(void* h, uint8_t* out) { canon(((Raw*)h)->c.m, out); }
void or_raw_destroy(void* h) { delete (Raw*)h; }

void* or_create(const uint8_t* rom, int64_t rom_len, int n, const int* levels, const uint8_t* lut,
                int skip, int max_steps, double sticky, int noop_max, int maxpool, int frame_stack,
                const uint64_t* rng) {
    if (skip < 1 || skip > 16 || n < 1 || frame_stack < 1) return nullptr;
    Vec* v = new Vec();
    if (rom_load(&v->rom, rom, (size_t)rom_len) != 0) { delete v; return nullptr; }
    v->n = n; v->K = frame_stack;
    v->cfg = Cfg{skip, max_steps, noop_max, maxpool, frame_stack, sticky};
    memcpy(v->lut, lut, 256);
    v->envs.resize(n);
    v->env_level.resize(n);
    for (int i = 0; i < n; i++) {
        int w = levels[3 * i], s = levels[3 * i + 1], a = levels[3 * i + 2];
        int li = -1;
        for (size_t k = 0; k < v->levels.size(); k++)
            if (v->levels[k]->world == w && v->levels[k]->stage == s && v->levels[k]->area == a) li = (int)k;
        if (li < 0) {
            Level* L = new Level();
            L->world = w; L->stage = s; L->area = a;
            boot_level(&v->rom, v->lut, L);
            v->levels.push_back(L);
            li = (int)v->levels.size() - 1;
        }
        v->env_level[i] = li;
        Env& e = v->envs[i];
        e.lvl = v->levels[li];
        e.cfg = &v->cfg;
        e.g.assign(kGray, 0); e.g_prev.assign(kGray, 0);
        e.con.rom = &v->rom; e.con.lut = v->lut; e.con.gray = e.g.data();
        e.restore();
        const uint64_t* r = rng + 6 * i;
        e.rng.state = ((unsigned __int128)r[0] << 64) | r[1];
        e.rng.inc = ((unsigned __int128)r[2] << 64) | r[3];
        e.rng.has32 = (int)r[4];
        e.rng.half = (uint32_t)r[5];
    }
    return v;
}
void or_set_buffers(void* h, uint8_t* obs, uint8_t* fin, float* rew, uint8_t* term, uint8_t* trunc,
                    int64_t* info, double* ep_ret, int64_t* ep_len) {
    Vec* v = (Vec*)h;
    v->obs = obs; v->fin = fin; v->rew = rew; v->term = term; v->trunc = trunc;
    v->info = info; v->ep_ret = ep_ret; v->ep_len = ep_len;
}
void or_reset(void* h) { Vec* v = (Vec*)h; for (int i = 0; i < v->n; i++) v->reset_env(i); }
void or_step(void* h, const int64_t* actions) {
    Vec* v = (Vec*)h;
    for (int i = 0; i < v->n; i++) v->step_env(i, (int)actions[i]);
}
int64_t or_frames(void* h) { int64_t f = 0; for (auto& e : ((Vec*)h)->envs) f += e.frames; return f; }
int64_t or_bad_ops(void* h) { int64_t f = 0; for (auto& e : ((Vec*)h)->envs) f += e.con.bad_ops; return f; }
int64_t or_instructions(void* h) { int64_t f = 0; for (auto& e : ((Vec*)h)->envs) f += e.con.instructions; return f; }
void or_reemulations(void* h, int64_t* out) {
    out[0] = out[1] = out[2] = 0;
    for (auto& e : ((Vec*)h)->envs) for (int k = 0; k < 3; k++) out[k] += e.reemu[k];
}
void or_env_ram(void* h, int i, uint8_t* out) { memcpy(out, ((Vec*)h)->envs[i].con.m.ram, 0x800); }
void or_env_canon(void* h, int i, uint8_t* out) { canon(((Vec*)h)->envs[i].con.m, out); }
void or_env_gray(void* h, int i, uint8_t* out) { memcpy(out, ((Vec*)h)->envs[i].g.data(), kGray); }
void or_level_canon(void* h, int level, uint8_t* out) { canon(((Vec*)h)->levels[level]->boot, out); }
void or_level_obs(void* h, int level, uint8_t* out) { memcpy(out, ((Vec*)h)->levels[level]->obs0, kObs); }
void or_destroy(void* h) { delete (Vec*)h; }

void or_pcg_run(const uint64_t* st, const int64_t* ops, int n, uint64_t* out, uint64_t* state_out) {
    Pcg g;
    g.state = ((unsigned __int128)st[0] << 64) | st[1];
    g.inc = ((unsigned __int128)st[2] << 64) | st[3];
    g.has32 = (int)st[4];
    g.half = (uint32_t)st[5];
    for (int i = 0; i < n; i++) {
        if (ops[i] == 0) { double d = g.random(); memcpy(&out[i], &d, 8); }
        else out[i] = (uint64_t)g.integers(ops[i]);
    }
    state_out[0] = (uint64_t)(g.state >> 64); state_out[1] = (uint64_t)g.state;
    state_out[2] = (uint64_t)(g.inc >> 64); state_out[3] = (uint64_t)g.inc;
    state_out[4] = (uint64_t)g.has32; state_out[5] = g.half;
}
void or_palette(uint32_t* out) { memcpy(out, kPalette, sizeof(kPalette)); }
void or_resize(const uint8_t* src, uint8_t* dst) { area_resize(src, dst); }
int or_area_tab(int ssize, int dsize, int* di, int* si, float* alpha) {
    std::vector<Tap> t((size_t)ssize * 2 + 8);
    int k = area_tab(ssize, dsize, t.data());
    for (int i = 0; i < k; i++) { di[i] = t[i].di; si[i] = t[i].si; alpha[i] = t[i].w; }
    return k;
}

}  // extern "C"
