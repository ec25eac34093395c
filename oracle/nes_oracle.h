/* CPU oracle for the batched Super Mario Bros env step — TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker the GPU path is compared against. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it; the product (fast-mario-env_amd/) never does.
 *
 * It restates, in plain single-threaded C++, the algorithm of the reference's C++ FastVecEnv:
 *   csrc/nes_core.hpp   (NROM cart, nes-py-exact 6502, catch-up PPU, renderer, frame loop)
 *   csrc/fastmario.cpp  (PCG64, INTER_AREA, SMB reward/done/info, frame skip, sticky, max-pool,
 *                        early termination, no-op reset, boot, frame stack / auto-reset)
 * Each function cites the reference file:line it follows.
 *
 * Pinning (tests/test_oracle.py): frame-by-frame RAM + rendered screen and env-level obs / reward /
 * done / info / RAM against oracle/_ref (the reference C++ compiled from its own sources) on the
 * synthetic NROM images under tests/golden/roms, committed golden traces for boxes without the
 * reference tree, numpy for PCG64, closed forms for the gray LUT and area tables, and textbook
 * 8-bit arithmetic for the ALU.
 */
#ifndef NES_ORACLE_H
#define NES_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Canonical console-state dump shared with the GPU library: a fixed little-endian byte layout, so a
 * test can compare whole machine states byte for byte.
 *   0 iter i64 | 8 exec_at i64 | 16 ppu_calls i64 | 24 pcyc i32 | 28 scanline i32
 *  32 pc u16 | 34 v u16 | 36 t u16 | 38 inc u16 | 40 sp a x y p zero_skip
 *  46 joy_strobe[2] joy_buttons[2] joy_bits[2]
 *  52 pstate even vblank s0hit first_write data_buffer oam_addr fine_x
 *  60 show_bg show_spr hide_edge_bg hide_edge_spr long_spr nmi_en bg_page spr_page
 *  68 nsl | 69 sl[8] (entries >= nsl are zero: never observable) | 77..79 zero
 *  80 oam[256] | 336 pal[32] | 368 vram[2048] | 2416 ram[2048] | 4464 end */
#define OR_CANON_BYTES 4464

/* ---- raw console (one emulator, frame stepping, like the reference's fm_raw_*) ---- */
void*   or_raw_create(const uint8_t* rom, int64_t len);
void    or_raw_frame(void* h, int buttons, int render);
const uint8_t* or_raw_ram(void* h);
const uint8_t* or_raw_screen(void* h);       /* 240*256 palette values of the last rendered dots */
void    or_raw_backup(void* h);
void    or_raw_restore(void* h);
int64_t or_raw_bad_ops(void* h);
int64_t or_raw_instructions(void* h);        /* 6502 instructions retired (idle-skip iterations excluded) */
void    or_raw_canon(void* h, uint8_t* out); /* OR_CANON_BYTES */
void    or_raw_destroy(void* h);

/* ---- vector env (FastVecEnv semantics, single thread) ---- */
void* or_create(const uint8_t* rom, int64_t rom_len, int n, const int* levels, const uint8_t* lut,
                int skip, int max_steps, double sticky, int noop_max, int maxpool, int frame_stack,
                const uint64_t* rng);
void    or_set_buffers(void* h, uint8_t* obs, uint8_t* fin, float* rew, uint8_t* term, uint8_t* trunc,
                       int64_t* info, double* ep_ret, int64_t* ep_len);
void    or_reset(void* h);
void    or_step(void* h, const int64_t* actions);
int64_t or_frames(void* h);
int64_t or_bad_ops(void* h);
int64_t or_instructions(void* h);
/* Early-termination re-emulations of env steps (reset no-op steps excluded), by the branch of
 * fastmario.cpp:351-362: out[0] frame last re-run alone, out[1] with its max-pool partner last-1,
 * out[2] of both, the episode ends at frame K-2 under max-pool. */
void    or_reemulations(void* h, int64_t* out);
void    or_env_ram(void* h, int i, uint8_t* out);
void    or_env_canon(void* h, int i, uint8_t* out);
void    or_env_gray(void* h, int i, uint8_t* out);      /* 240*256 gray buffer of env i */
void    or_level_canon(void* h, int level, uint8_t* out); /* boot state of a level */
void    or_level_obs(void* h, int level, uint8_t* out);   /* 84*84 boot observation */
void    or_destroy(void* h);

/* ---- helpers ---- */
/* PCG64 stream from the 6 state words; ops[i] = 0 -> out[i] = random() as double bits,
 * ops[i] = h > 0 -> out[i] = integers(0, h). Lets tests compare the interleaved sequence with numpy. */
void    or_pcg_run(const uint64_t* state6, const int64_t* ops, int n, uint64_t* out, uint64_t* state_out);
void    or_palette(uint32_t* out);                       /* 64 x 0xRRGGBB */
void    or_resize(const uint8_t* src, uint8_t* dst);     /* 240x256 -> 84x84 INTER_AREA */
int     or_area_tab(int ssize, int dsize, int* di, int* si, float* alpha); /* returns entry count */

#ifdef __cplusplus
}
#endif
#endif
