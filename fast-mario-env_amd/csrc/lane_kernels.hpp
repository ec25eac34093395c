// Per-lane bodies of the env kernels (one env / level / cache entry per lane). The __global__ wrappers
// in mario_hip.hip stage the cartridge in LDS and call these.
#pragma once
#include <cmath>

#include "env_device.hpp"

namespace mh {

constexpr int OBS_PIX = 84 * 84;
constexpr int TAPS = 6;   // max area-filter taps per output row / column

// ------------------------------------------------------------------ INTER_AREA tables
// OpenCV computeResizeAreaTab in double precision (fastmario.cpp:83-100): per output index the source
// indices and float weights, in the order the float sums are taken.
struct AreaTables {
    int32_t xs[84 * TAPS], ys[84 * TAPS];
    float xw[84 * TAPS], yw[84 * TAPS];
    int32_t xn[84], yn[84];
};

// Host and device: the device computes the same IEEE double arithmetic (division, ceil, floor and the
// double -> float conversion are correctly rounded on both).
__host__ __device__ inline void area_taps(int ssize, int dsize, int32_t* idx, float* w, int32_t* cnt) {
    double scale = 1.0 / ((double)dsize / ssize);
    for (int d = 0; d < dsize; d++) cnt[d] = 0;
    auto add = [&](int d, int s, float a) { idx[d * TAPS + cnt[d]] = s; w[d * TAPS + cnt[d]] = a; cnt[d]++; };
    for (int d = 0; d < dsize; d++) {
        double f1 = d * scale, f2 = f1 + scale;
        double cell = scale < ssize - f1 ? scale : ssize - f1;
        int s1 = (int)__builtin_ceil(f1), s2 = (int)__builtin_floor(f2);
        if (s2 > ssize - 1) s2 = ssize - 1;
        if (s1 > s2) s1 = s2;
        if (s1 - f1 > 1e-3) add(d, s1 - 1, (float)((s1 - f1) / cell));
        for (int s = s1; s < s2; s++) add(d, s, (float)(1.0 / cell));
        if (f2 - s2 > 1e-3) {
            double ww = f2 - s2 < 1.0 ? f2 - s2 : 1.0;
            if (cell < ww) ww = cell;
            add(d, s2, (float)(ww / cell));
        }
    }
}

__host__ __device__ inline void area_tables(AreaTables* T) {
    for (int i = 0; i < 84 * TAPS; i++) { T->xs[i] = T->ys[i] = 0; T->xw[i] = T->yw[i] = 0.f; }
    area_taps(256, 84, T->xs, T->xw, T->xn);
    area_taps(240, 84, T->ys, T->yw, T->yn);
}

// The first source column of each output column's taps, at compile time: area_taps(256, 84)'s steps for the
// start index (the same double operations; ceil and floor of non-negative values by truncation), so that a
// kernel can address a column's pixels with constant word and byte indices. The library checks at start-up that
// they equal the run-time tables' (x_cols_match()); the taps of a column are at most 4 consecutive pixels.
struct XCols { int x0[84]; };
constexpr XCols x_cols() {
    XCols r{};
    const double scale = 1.0 / ((double)84 / 256);
    for (int d = 0; d < 84; d++) {
        const double f1 = d * scale, f2 = f1 + scale;
        int s1 = (int)f1;
        if ((double)s1 < f1) s1++;
        int s2 = (int)f2;
        if (s2 > 255) s2 = 255;
        if (s1 > s2) s1 = s2;
        r.x0[d] = s1 - f1 > 1e-3 ? s1 - 1 : s1;
    }
    return r;
}
constexpr XCols kXCols = x_cols();
inline bool x_cols_match(const AreaTables& T) {
    for (int d = 0; d < 84; d++) {
        if (T.xs[d * TAPS] != kXCols.x0[d] || T.xn[d] < 1 || T.xn[d] > 4) return false;
        for (int k = 1; k < T.xn[d]; k++)
            if (T.xs[d * TAPS + k] != kXCols.x0[d] + k) return false;
        for (int k = T.xn[d]; k < 4; k++)
            if (T.xw[d * TAPS + k] != 0.f) return false;
    }
    return true;
}

__device__ __forceinline__ uint8_t round_sat(float v) {
    float r = __builtin_rintf(v);           // round half to even, like lrintf
    int iv = (int)r;
    return (uint8_t)(iv < 0 ? 0 : iv > 255 ? 255 : iv);
}

// Frame buffers (GRAY) hold 4 pixels per 32-bit word, lane-interleaved: pixel p of lane e of a
// buffer with np lanes is byte ((p / 4) * np + e) * 4 + p % 4. An Image addresses one lane's frame
// in such a buffer, or a plain row-major 256x240 frame when np == 0.
struct Image {
    const uint8_t* base;
    uint32_t np, e;
    __device__ __forceinline__ uint8_t operator()(uint32_t p) const {
        return np ? base[((size_t)(p >> 2) * np + e) * 4 + (p & 3)] : base[p];
    }
};
__host__ __device__ __forceinline__ size_t gray_lane_offset(uint32_t e) { return (size_t)e * 4; }

// INTER_AREA output pixel o of one image, max-pooled with a second one if `pool`.
__device__ __forceinline__ uint8_t area_pixel(const Image& g0, const Image& g1, bool pool, int o, const AreaTables* T) {
    const int dy = o / 84, dx = o - dy * 84;
    const int ny = T->yn[dy], nx = T->xn[dx];
    float acc = 0.f;
    for (int j = 0; j < ny; j++) {
        const int sy = T->ys[dy * TAPS + j];
        float row = 0.f;
        for (int k = 0; k < nx; k++) {
            const uint32_t p = (uint32_t)(sy * 256 + T->xs[dx * TAPS + k]);
            uint8_t s = g0(p);
            if (pool) { uint8_t s1 = g1(p); s = s1 > s ? s1 : s; }
            row += (float)s * T->xw[dx * TAPS + k];
        }
        const float term = T->yw[dy * TAPS + j] * row;
        acc = j == 0 ? term : acc + term;
    }
    return round_sat(acc);
}

// bytewise max of two words (in 16-bit lanes: 256 + a - b has bit 8 set exactly when a >= b)
__device__ __forceinline__ uint32_t max_u8x4(uint32_t a, uint32_t b) {
    const uint32_t a0 = a & 0x00ff00ffu, b0 = b & 0x00ff00ffu, a1 = (a >> 8) & 0x00ff00ffu, b1 = (b >> 8) & 0x00ff00ffu;
    const uint32_t t0 = ((a0 | 0x01000100u) - b0) & 0x01000100u, t1 = ((a1 | 0x01000100u) - b1) & 0x01000100u;
    const uint32_t k0 = t0 - (t0 >> 8), k1 = t1 - (t1 >> 8);
    return ((a0 & k0) | (b0 & ~k0)) | (((a1 & k1) | (b1 & ~k1)) << 8);
}
// ---- INTER_AREA of a staged source row, by column groups (k_obs)
constexpr int OBS_COLS = 24;   // output columns one row-sum call covers: 20 G .. 20 G + 23

// The horizontal sums of one source row for output columns 20 G .. 20 G + 23 of one env: word i of the row
// (pixels 4 i .. 4 i + 3, max-pooled if the env pools) at rw[i * stride + lane]; xw[c]: column c's 4 tap
// weights (+0 past its tap count). The words these columns' taps cover are read once, and every tap is a
// constant byte of one of them (kXCols). Always 4 taps: adding +0 * pixel leaves the non-negative sum
// unchanged, bit for bit, and the pixel is still inside the row.
template <int G>
__device__ __forceinline__ void obs_row_sums(const uint32_t* rw, uint32_t stride, uint32_t lane, const float (*xw)[4],
                                             float (&rs)[OBS_COLS]) {
    constexpr int c0 = 20 * G, wlo = kXCols.x0[c0] >> 2, whi = (kXCols.x0[c0 + OBS_COLS - 1] + 3) >> 2;
    constexpr int NW = whi - wlo + 1;
    static_assert(G >= 0 && G <= 3 && c0 + OBS_COLS <= 84 && whi < 64, "columns and taps inside the row");
    uint32_t wv[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) wv[i] = rw[(uint32_t)(wlo + i) * stride + lane];
#pragma unroll
    for (int q = 0; q < OBS_COLS; q++) {
        const int c = c0 + q;
        float row = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int px = kXCols.x0[c] + k;
            row += (float)((wv[(px >> 2) - wlo] >> (8 * (px & 3))) & 0xffu) * xw[c][k];
        }
        rs[q] = row;
    }
}
__device__ __forceinline__ void obs_row_sums(int g, const uint32_t* rw, uint32_t stride, uint32_t lane,
                                             const float (*xw)[4], float (&rs)[OBS_COLS]) {
    switch (g) {
        case 0: obs_row_sums<0>(rw, stride, lane, xw, rs); break;
        case 1: obs_row_sums<1>(rw, stride, lane, xw, rs); break;
        case 2: obs_row_sums<2>(rw, stride, lane, xw, rs); break;
        default: obs_row_sums<3>(rw, stride, lane, xw, rs); break;
    }
}

// The vertical step for source row sy: every (output row dy, tap j) from the current (dy, j) on, up to output
// row dy_end, that takes row sy, in order (consecutive output rows take consecutive source rows, the one they
// share summed once); emit(dy, acc) when output row dy is complete.
template <class Emit>
__device__ __forceinline__ void obs_rows_take(int sy, int& dy, int& j, int dy_end, const int32_t* ys, const float* yw,
                                              const int32_t* yn, const float (&rs)[OBS_COLS], float (&acc)[OBS_COLS],
                                              Emit&& emit) {
    while (dy < dy_end && ys[dy * TAPS + j] == sy) {
        const float w = yw[dy * TAPS + j];
#pragma unroll
        for (int q = 0; q < OBS_COLS; q++) {
            const float term = w * rs[q];
            acc[q] = j == 0 ? term : acc[q] + term;
        }
        if (++j == yn[dy]) { emit(dy); dy++; j = 0; }
    }
}

// output pixels 4 wq .. 4 wq + 3 of a column group as one word (pixel 4 wq + i in byte i)
__device__ __forceinline__ uint32_t obs_word(const float (&acc)[OBS_COLS], int wq) {
    return (uint32_t)round_sat(acc[4 * wq]) | (uint32_t)round_sat(acc[4 * wq + 1]) << 8 |
           (uint32_t)round_sat(acc[4 * wq + 2]) << 16 | (uint32_t)round_sat(acc[4 * wq + 3]) << 24;
}

// ------------------------------------------------------------------ arguments
constexpr int MAX_CHR_BANKS = 4;   // ROMs per env instance: one PRG, a CHR bank each (the rom_mode variants)

struct RomArgs {
    const uint8_t* rom;      // 0x8000 PRG (mirrored) + n_chr x 0x2000 CHR
    const uint8_t* lut;      // 256
    uint32_t nt_bits;        // bit k: name table k maps to VRAM $400
    int n_chr;               // CHR banks, 1 .. MAX_CHR_BANKS
};

__device__ __forceinline__ Cart make_cart(const RomArgs& R, const uint8_t* s_rom, const uint32_t* s_dec) {
    Cart c;
    c.prg = s_rom;
    c.gprg = R.rom;
    c.chr = s_rom + 0x8000;
    c.dec = s_dec;
    c.nt_bits = R.nt_bits;
    return c;
}

// What a lane needs from its block: the staged cartridge, the gray LUT and its LDS render buffers.
struct LaneCtx {
    Cart cart;
    const uint8_t* lut;
    uint32_t* sp;     // this lane's sprite line buffer (stride LDS_LANES words)
    uint32_t* gp;     // this lane's gray palette, tile row and OAM (stride LDS_LANES words)
    uint8_t part;     // which of the env's LANES_PER_ENV lanes this is
};

// console e of the memory block `mem` (np consoles), on CHR bank `bank` of the staged cartridge
__device__ __forceinline__ void attach(Console& c, const LaneCtx& x, uint8_t* mem, uint32_t np, uint32_t e,
                                       uint32_t bank = 0) {
    c.mem = mem + e; c.vmem = mem + vram_word_offset(np, e, 0); c.np = np;
    c.cart = x.cart; c.cart.chr += bank * 0x2000u; c.lut = x.lut; c.lds_sp = x.sp; c.lds_gp = x.gp;
    c.lds_bg = x.gp + LDS_GP_WORDS * LDS_LANES; c.bg_key = -1;
    c.lds_oam = x.gp + (LDS_GP_WORDS + LDS_BG_WORDS) * LDS_LANES;
    c.part = x.part;
    c.bad_ops = 0; c.instructions = 0; c.ff_instructions = 0;
    c.pend_line = -1; c.sp_line = -1; c.pal_dirty = true;
}

struct BootArgs {
    RomArgs R;
    int nl;
    uint32_t nlp;
    const int* levels;           // 3 * nl
    const uint8_t* key_bank;     // nl: CHR bank of each (level, ROM) key
    uint8_t* mem; uint32_t* sc;  // boot consoles [row * nlp + l]
    uint8_t* gray;               // frame buffer of nlp lanes (4-pixel words)
    int64_t* x0; int64_t* t0;
    uint32_t* err;
};

struct CacheArgs {
    RomArgs R;
    Cfg cfg;
    const uint8_t* key_bank;     // CHR bank of each (level, ROM) key
    int nl, nk, nc;
    uint32_t nlp, ncp;
    const uint8_t* boot_mem; const uint32_t* boot_sc; const int64_t* x0; const int64_t* t0;
    uint8_t* mem; uint32_t* sc;          // cache consoles [row * ncp + c]
    uint8_t* gray;                       // 2 frame buffers of ncp lanes (4-pixel words)
    uint8_t* snap_mem; uint32_t* snap_sc;  // 2 snapshot slots of the cache consoles' layout
    int64_t* cx; int64_t* ct; int32_t* clives; int32_t* cdraws; uint8_t* cboot;
    uint64_t* cframes; uint64_t* cinstr; uint64_t* cff; uint32_t* cbad;
};

struct StepArgs {
    RomArgs R;
    Cfg cfg;
    int n;
    uint32_t np;
    uint8_t* mem; uint32_t* sc;
    uint32_t* ev;                 // env words [w * np + e]
    uint8_t* gray;                // 2 frame buffers of np lanes (4-pixel words)
    uint8_t* snap_mem; uint32_t* snap_sc;   // 2 snapshot slots of the live layout (re-emulation)
    const int64_t* actions;
    float* rew; uint8_t* term; uint8_t* trunc; int32_t* info; double* ep_ret_out; int32_t* ep_len_out;
    const uint8_t* key_bank;      // CHR bank of each (level, ROM) key (E_LEVEL)
    const int32_t* slot_env;      // env of each console slot (actions in and outputs out are in env order)
};

struct ResetArgs {
    int n; uint32_t np;
    Cfg cfg;
    int nk; uint32_t ncp;
    uint8_t* mem; uint32_t* sc; uint32_t* ev;
    const uint8_t* cmem; const uint32_t* csc;
    const int64_t* cx; const int64_t* ct; const int32_t* clives; const int32_t* cdraws; const uint8_t* cboot;
    const uint64_t* cframes; const uint64_t* cinstr; const uint64_t* cff; const uint32_t* cbad;
    int all;
};

struct RawArgs {
    RomArgs R;
    int n; uint32_t np;
    uint8_t* mem; uint32_t* sc;
    uint8_t* screen;             // [pix * np + e], palette values
    const uint8_t* buttons;      // n
    int render;
    uint32_t* bad; uint32_t* instr; uint32_t* ff;
    int power_on;
};

// ------------------------------------------------------------------ env words
__device__ __forceinline__ void load_env(EnvRegs& ev, const uint32_t* E, uint32_t np, uint32_t e) {
    auto w = [&](int k) { return E[(size_t)k * np + e]; };
    ev.x_last = (int64_t)((uint64_t)w(E_XLAST_LO) | ((uint64_t)w(E_XLAST_HI) << 32));
    ev.time_last = (int64_t)((uint64_t)w(E_TLAST_LO) | ((uint64_t)w(E_TLAST_HI) << 32));
    ev.prev = (int)w(E_PREV); ev.lives = (int)w(E_LIVES); ev.t = (int)w(E_T); ev.ep_len = (int)w(E_EP_LEN);
    uint64_t r = (uint64_t)w(E_EPRET_LO) | ((uint64_t)w(E_EPRET_HI) << 32);
    ev.ep_ret = __longlong_as_double((long long)r);
    ev.shows_boot = w(E_SHOWS_BOOT) != 0; ev.pooled = (w(E_POOLED) & 1) != 0; ev.slot_swap = (w(E_POOLED) & 2) != 0;
    ev.frames = 0; ev.draws = 0;
}
__device__ __forceinline__ void store_env(const EnvRegs& ev, uint32_t* E, uint32_t np, uint32_t e) {
    auto w = [&](int k, uint32_t v) { E[(size_t)k * np + e] = v; };
    w(E_XLAST_LO, (uint32_t)ev.x_last); w(E_XLAST_HI, (uint32_t)((uint64_t)ev.x_last >> 32));
    w(E_TLAST_LO, (uint32_t)ev.time_last); w(E_TLAST_HI, (uint32_t)((uint64_t)ev.time_last >> 32));
    w(E_PREV, (uint32_t)ev.prev); w(E_LIVES, (uint32_t)ev.lives); w(E_T, (uint32_t)ev.t);
    w(E_EP_LEN, (uint32_t)ev.ep_len);
    uint64_t r = (uint64_t)__double_as_longlong(ev.ep_ret);
    w(E_EPRET_LO, (uint32_t)r); w(E_EPRET_HI, (uint32_t)(r >> 32));
    w(E_SHOWS_BOOT, ev.shows_boot); w(E_POOLED, (ev.pooled ? 1u : 0u) | (ev.slot_swap ? 2u : 0u));
}
__device__ __forceinline__ void add_counter(uint32_t* E, uint32_t np, uint32_t e, int lo_word, uint64_t add) {
    uint64_t v = (uint64_t)E[(size_t)lo_word * np + e] | ((uint64_t)E[(size_t)(lo_word + 1) * np + e] << 32);
    v += add;
    E[(size_t)lo_word * np + e] = (uint32_t)v;
    E[(size_t)(lo_word + 1) * np + e] = (uint32_t)(v >> 32);
}

// ------------------------------------------------------------------ lane bodies
// Power-on and title sequence with the target level written into RAM (fastmario.cpp:414-445).
__device__ inline void boot_lane(const BootArgs& A, const LaneCtx& x, int l) {
    Console c;
    attach(c, x, A.mem, A.nlp, (uint32_t)l, A.key_bank[l]);
    c.gray = A.gray + gray_lane_offset(l); c.render = true;
    c.power_on();
    auto fr = [&](uint8_t b) { c.set_buttons0(b); c.frame(); };
    const int w = A.levels[3 * l], s = A.levels[3 * l + 1], ar = A.levels[3 * l + 2];
    fr(8); fr(0);
    int guard = 0;
    while (smb_time(c) == 0) {
        if (++guard > HACK_FRAME_LIMIT) { atomicOr(A.err, 1u); break; }
        fr(8);
        c.st(ROW_RAM + 0x75f, (uint8_t)(w - 1)); c.st(ROW_RAM + 0x75c, (uint8_t)(s - 1));
        c.st(ROW_RAM + 0x760, (uint8_t)(ar - 1));
        fr(0);
        c.st(ROW_RAM + 0x7a0, 0);
    }
    int64_t tl = smb_time(c);
    guard = 0;
    while (smb_time(c) >= tl) {
        if (++guard > HACK_FRAME_LIMIT) { atomicOr(A.err, 2u); break; }
        tl = smb_time(c); fr(8); fr(0);
    }
    c.store(A.sc, l);
    A.x0[l] = smb_x(c);
    A.t0[l] = smb_time(c);
}

// Reset cache: the state after k no-op agent steps from the boot state of a level, k in 0..noop_max
// (fastmario.cpp:389-401), restarting on termination like the reference. The sticky draws only choose
// between action 0 and prev == 0, so their count is recorded, not their values.
__device__ inline void cache_lane(const CacheArgs& A, const LaneCtx& x, int ci) {
    const int lvl = ci / A.nk, k = ci - lvl * A.nk;
    Region boot{(uint8_t*)A.boot_mem, (uint32_t*)A.boot_sc, A.nlp, (uint32_t)lvl};
    Region live{A.mem, A.sc, A.ncp, (uint32_t)ci};
    copy_console(live, boot);
    Console c;
    attach(c, x, A.mem, A.ncp, (uint32_t)ci, A.key_bank[lvl]);
    c.load(A.sc, ci);
    EnvRegs ev{};
    ev.x_last = A.x0[lvl]; ev.time_last = A.t0[lvl];
    ev.prev = 0; ev.lives = -1; ev.shows_boot = true; ev.frames = 0; ev.draws = 0;
    Stepper stp{c, ev, A.cfg, nullptr, A.gray + gray_lane_offset(ci), A.gray + (size_t)GRAY_PIX * A.ncp + gray_lane_offset(ci),
                live, A.snap_mem, A.snap_sc};
    for (int j = 0; j < k; j++) {
        bool term;
        stp.agent_step(0, j == k - 1, &term);
        if (term) {
            copy_console(live, boot);
            c.load(A.sc, ci);
            ev.x_last = A.x0[lvl]; ev.time_last = A.t0[lvl];
            ev.prev = 0; ev.lives = -1; ev.shows_boot = true;
        }
    }
    c.store(A.sc, ci);
    A.cx[ci] = ev.x_last; A.ct[ci] = ev.time_last; A.clives[ci] = ev.lives;
    A.cdraws[ci] = (int32_t)ev.draws; A.cboot[ci] = ev.shows_boot;
    A.cframes[ci] = ev.frames; A.cinstr[ci] = c.instructions; A.cff[ci] = c.ff_instructions; A.cbad[ci] = c.bad_ops;
}

// One agent step of the env in console slot e (fastmario.cpp:403-411 + 336-374).
__device__ inline void step_lane(const StepArgs& A, const LaneCtx& x, uint32_t e) {
    const uint32_t o = (uint32_t)A.slot_env[e];   // the env's index in the action and output arrays
    Console c;
    attach(c, x, A.mem, A.np, e, A.key_bank[A.ev[(size_t)E_LEVEL * A.np + e]]);
    c.load(A.sc, e);
    EnvRegs ev;
    load_env(ev, A.ev, A.np, e);
    Pcg rng;
    rng.load(A.ev, A.np, e);
    int64_t a64 = A.actions[o];
    const int act = (a64 >= 0 && a64 < 7) ? (int)a64 : 0;
    Stepper stp{c, ev, A.cfg, &rng, A.gray + gray_lane_offset(e), A.gray + (size_t)GRAY_PIX * A.np + gray_lane_offset(e),
                Region{A.mem, A.sc, A.np, e}, A.snap_mem, A.snap_sc};
    bool tm;
    double r = stp.agent_step(act, true, &tm);
    ev.t++;
    const bool tr = ev.t >= A.cfg.max_steps;
    ev.ep_ret += r; ev.ep_len++;
    A.rew[o] = (float)r;
    A.term[o] = tm;
    A.trunc[o] = tr;
    for (int k = 0; k < 10; k++) A.info[(size_t)o * 10 + k] = (int32_t)ev.info.v[k];
    const bool done = tm || tr;
    if (done) { A.ep_ret_out[o] = ev.ep_ret; A.ep_len_out[o] = ev.ep_len; }
    c.store(A.sc, e);
    store_env(ev, A.ev, A.np, e);
    rng.store(A.ev, A.np, e);
    A.ev[(size_t)E_DONE * A.np + e] = done;
    add_counter(A.ev, A.np, e, E_FRAMES_LO, ev.frames);
    add_counter(A.ev, A.np, e, E_INSTR_LO, c.instructions);
    add_counter(A.ev, A.np, e, E_FF_LO, c.ff_instructions);
    A.ev[(size_t)E_BAD * A.np + e] += c.bad_ops;
    for (int k = 0; k < 3; k++)
        if ((ev.reemu >> k) & 1u) A.ev[(size_t)(E_REEMU_ONE + k) * A.np + e] += 1;
    A.ev[(size_t)E_HACK_REDRAWS * A.np + e] += ev.hack_redraws;
}

// Auto-reset (fastmario.cpp:389-401): k = integers(noop_max + 1) from the env's stream, the draws of
// the k no-op steps are skipped, and the cached state of (level, k) is installed. Returns the cache
// entry whose console the env takes (the caller copies it, see copy_console_wave), or -1.
__device__ inline int reset_lane(const ResetArgs& A, uint32_t e) {
    uint32_t* E = A.ev;
    const size_t np = A.np;
    if (!A.all && !E[E_DONE * np + e]) { E[E_RESET_IDX * np + e] = 0xffffffffu; return -1; }
    Pcg rng;
    rng.load(E, A.np, e);
    int k = 0;
    if (A.cfg.noop_max) k = (int)rng.integers(A.cfg.noop_max + 1);
    const int lvl = (int)E[E_LEVEL * np + e];
    const int ci = lvl * A.nk + k;
    if (A.cfg.sticky != 0.0)
        for (int d = 0; d < A.cdraws[ci]; d++) rng.next64();
    rng.store(E, A.np, e);
    EnvRegs ev{};
    ev.x_last = A.cx[ci]; ev.time_last = A.ct[ci]; ev.lives = A.clives[ci]; ev.prev = 0;
    ev.t = 0; ev.ep_len = 0; ev.ep_ret = 0.0; ev.shows_boot = A.cboot[ci] != 0; ev.pooled = false; ev.slot_swap = false;
    store_env(ev, E, A.np, e);
    E[E_RESET_IDX * np + e] = (uint32_t)ci;
    // the no-op steps count as emulated work, as on the reference CPU path
    add_counter(E, A.np, e, E_FRAMES_LO, A.cframes[ci]);
    add_counter(E, A.np, e, E_INSTR_LO, A.cinstr[ci]);
    add_counter(E, A.np, e, E_FF_LO, A.cff[ci]);
    E[E_BAD * np + e] += A.cbad[ci];
    return ci;
}

// One nes-py frame of raw console e (fastmario.cpp:656-661); power_on != 0 boots it instead.
__device__ inline void raw_lane(const RawArgs& A, const LaneCtx& x, uint32_t e) {
    Console c;
    attach(c, x, A.mem, A.np, e);
    c.gray = A.screen + gray_lane_offset(e);
    if (A.power_on) {
        c.power_on();
    } else {
        c.load(A.sc, e);
        c.set_buttons0(A.buttons[e]);
        c.render = A.render != 0;
        c.frame();
    }
    c.store(A.sc, e);
    A.bad[e] += c.bad_ops;
    A.instr[e] += c.instructions;
    A.ff[e] += c.ff_instructions;
}

// Canonical state dump of console e (layout in include/mario_hip.h).
__device__ inline void canon_lane(const uint8_t* mem, const uint32_t* sc, uint32_t np, uint32_t e, uint8_t* o) {
    auto w = [&](int k) { return sc[(size_t)k * np + e]; };
    auto put = [&](int off, uint64_t v, int bytes) { for (int b = 0; b < bytes; b++) o[off + b] = (uint8_t)(v >> (8 * b)); };
    for (int i = 0; i < 80; i++) o[i] = 0;
    const uint64_t iter = (uint64_t)w(S_ITER_LO) | ((uint64_t)w(S_ITER_HI) << 32);
    put(0, iter, 8);
    put(8, iter + (int64_t)(int32_t)w(S_EXEC_REL), 8);
    put(16, 3 * iter, 8);
    put(24, w(S_PCYC), 4); put(28, w(S_SCANLINE), 4);
    put(32, w(S_PC), 2); put(34, w(S_V), 2); put(36, w(S_T), 2); put(38, w(S_INC), 2);
    const int order[] = {S_SP, S_A, S_X, S_Y, S_P, S_ZERO_SKIP, S_JOY_STROBE0, S_JOY_STROBE1, S_JOY_BUTTONS0,
                         S_JOY_BUTTONS1, S_JOY_BITS0, S_JOY_BITS1, S_PSTATE, S_EVEN, S_VBLANK, S_S0HIT,
                         S_FIRST_WRITE, S_DATA_BUFFER, S_OAM_ADDR, S_FINE_X, S_SHOW_BG, S_SHOW_SPR,
                         S_HIDE_EDGE_BG, S_HIDE_EDGE_SPR, S_LONG_SPR, S_NMI_EN, S_BG_PAGE, S_SPR_PAGE, S_NSL};
    for (int i = 0; i < 29; i++) o[40 + i] = (uint8_t)w(order[i]);
    const uint32_t nsl = w(S_NSL);
    const uint64_t sl = (uint64_t)w(S_SL_LO) | ((uint64_t)w(S_SL_HI) << 32);
    for (uint32_t i = 0; i < 8; i++) o[69 + i] = i < nsl ? (uint8_t)(sl >> (8 * i)) : 0;
    const uint32_t rows[3][3] = {{80, ROW_OAM, 256}, {336, ROW_PAL, 32}, {2416, ROW_RAM, 2048}};
    for (int k = 0; k < 3; k++)
        for (uint32_t i = 0; i < rows[k][2]; i++) o[rows[k][0] + i] = mem[(size_t)(rows[k][1] + i) * np + e];
    for (uint32_t i = 0; i < 2048; i++) o[368 + i] = mem[vram_word_offset(np, e, i >> 2) + (i & 3)];
}

}  // namespace mh
