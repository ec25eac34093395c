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

// ---- The INTER_AREA tables by periods
// 256 -> 84 columns and 240 -> 84 rows are ratios 64 : 21 and 20 : 7, and the tables repeat with them: output
// column 21 g + q takes source pixels 64 g + (those of column q) with column q's weights, output row 7 p + q
// source rows 20 p + (those of row q) with row q's weights, and no source pixel or row is shared across a
// period boundary. AreaPeriod holds one period of each, computed at compile time by area_taps's steps (the same
// double operations; ceil and floor of non-negative values by truncation), so that a kernel can take every
// tap's position and weight as a constant. The library checks at start-up that the run-time tables are these
// periods repeated (area_period_match()).
struct AreaPeriod {
    int x0[21], xn[21];    // output column q: source pixels x0 .. x0 + xn - 1 of its 64-pixel period
    float xw[21][4];
    int y0[7], yn[7];      // output row q: source rows y0 .. y0 + yn - 1 of its 20-row period
    float yw[7][4];
};
constexpr void area_taps_cx(int ssize, int dsize, int d, int* idx, float* w, int& cnt) {
    const double scale = 1.0 / ((double)dsize / ssize);
    const double f1 = d * scale, f2 = f1 + scale;
    const double cell = scale < ssize - f1 ? scale : ssize - f1;
    int s1 = (int)f1;
    if ((double)s1 < f1) s1++;
    int s2 = (int)f2;
    if (s2 > ssize - 1) s2 = ssize - 1;
    if (s1 > s2) s1 = s2;
    cnt = 0;
    if (s1 - f1 > 1e-3) { idx[cnt] = s1 - 1; w[cnt] = (float)((s1 - f1) / cell); cnt++; }
    for (int s = s1; s < s2; s++) { idx[cnt] = s; w[cnt] = (float)(1.0 / cell); cnt++; }
    if (f2 - s2 > 1e-3) {
        double ww = f2 - s2 < 1.0 ? f2 - s2 : 1.0;
        if (cell < ww) ww = cell;
        idx[cnt] = s2; w[cnt] = (float)(ww / cell); cnt++;
    }
}
constexpr AreaPeriod area_period() {
    AreaPeriod r{};
    for (int q = 0; q < 21; q++) {
        int idx[TAPS] = {}, n = 0;
        float w[TAPS] = {};
        area_taps_cx(256, 84, q, idx, w, n);
        r.x0[q] = idx[0]; r.xn[q] = n;
        for (int k = 0; k < n && k < 4; k++) r.xw[q][k] = w[k];
    }
    for (int q = 0; q < 7; q++) {
        int idx[TAPS] = {}, n = 0;
        float w[TAPS] = {};
        area_taps_cx(240, 84, q, idx, w, n);
        r.y0[q] = idx[0]; r.yn[q] = n;
        for (int k = 0; k < n && k < 4; k++) r.yw[q][k] = w[k];
    }
    return r;
}
constexpr AreaPeriod kArea = area_period();
constexpr bool area_period_shape() {
    for (int q = 0; q < 21; q++)
        if (kArea.xn[q] != 4 || kArea.x0[q] < 0 || kArea.x0[q] + 4 > 64) return false;
    for (int q = 0; q < 7; q++) {
        if (kArea.yn[q] < 1 || kArea.yn[q] > 4 || kArea.y0[q] < 0 || kArea.y0[q] + kArea.yn[q] > 20) return false;
        // consecutive rows share at most their boundary row
        if (q > 0 && kArea.y0[q] < kArea.y0[q - 1] + kArea.yn[q - 1] - 1) return false;
    }
    return kArea.y0[0] == 0 && kArea.y0[6] + kArea.yn[6] == 20;
}
static_assert(area_period_shape(), "every column takes 4 pixels of its period, every row 1-4 rows of its period");

// The whole tables at compile time: area_taps_cx for every output index (the same double operations as
// area_taps), for kernels that take the tables from a statically initialised device array.
constexpr AreaTables area_tables_cx() {
    AreaTables T{};
    for (int d = 0; d < 84; d++) {
        int idx[TAPS] = {}, n = 0;
        float w[TAPS] = {};
        area_taps_cx(256, 84, d, idx, w, n);
        T.xn[d] = n;
        for (int k = 0; k < n; k++) { T.xs[d * TAPS + k] = idx[k]; T.xw[d * TAPS + k] = w[k]; }
        int jdx[TAPS] = {}, m = 0;
        float v[TAPS] = {};
        area_taps_cx(240, 84, d, jdx, v, m);
        T.yn[d] = m;
        for (int k = 0; k < m; k++) { T.ys[d * TAPS + k] = jdx[k]; T.yw[d * TAPS + k] = v[k]; }
    }
    return T;
}
constexpr AreaTables kAreaTables = area_tables_cx();

// Two tables equal entry for entry (weights compared as bit patterns).
inline bool area_tables_equal(const AreaTables& a, const AreaTables& b) {
    for (int i = 0; i < 84 * TAPS; i++)
        if (a.xs[i] != b.xs[i] || a.ys[i] != b.ys[i] || __builtin_bit_cast(uint32_t, a.xw[i]) != __builtin_bit_cast(uint32_t, b.xw[i]) ||
            __builtin_bit_cast(uint32_t, a.yw[i]) != __builtin_bit_cast(uint32_t, b.yw[i]))
            return false;
    for (int d = 0; d < 84; d++)
        if (a.xn[d] != b.xn[d] || a.yn[d] != b.yn[d]) return false;
    return true;
}

inline bool area_period_match(const AreaTables& T) {
    for (int d = 0; d < 84; d++) {
        const int q = d % 21, g = d / 21;
        if (T.xn[d] != kArea.xn[q]) return false;
        for (int k = 0; k < T.xn[d]; k++)
            if (T.xs[d * TAPS + k] != 64 * g + kArea.x0[q] + k || T.xw[d * TAPS + k] != kArea.xw[q][k]) return false;
        const int r = d % 7, p = d / 7;
        if (T.yn[d] != kArea.yn[r]) return false;
        for (int j = 0; j < T.yn[d]; j++)
            if (T.ys[d * TAPS + j] != 20 * p + kArea.y0[r] + j || T.yw[d * TAPS + j] != kArea.yw[r][j]) return false;
    }
    return true;
}

// What source row r of a 20-row period does: its sums, times `wa`, are added to the open output row (row q of
// the period); if `last`, that row is then complete, and the next one opens with the row's sums times `wb`
// (+0 when the next row starts at the following source row).
struct RowStep { float wa, wb; int q; int last; };
struct RowSteps { RowStep s[20]; };
constexpr RowSteps row_steps() {
    RowSteps t{};
    for (int r = 0; r < 20; r++) {
        int q = 0;
        while (!(kArea.y0[q] <= r && r < kArea.y0[q] + kArea.yn[q])) q++;
        const int j = r - kArea.y0[q];
        t.s[r].wa = kArea.yw[q][j];
        t.s[r].q = q;
        t.s[r].last = j == kArea.yn[q] - 1;
        t.s[r].wb = (t.s[r].last && q + 1 < 7 && kArea.y0[q + 1] == r) ? kArea.yw[q + 1][0] : 0.f;
    }
    return t;
}
constexpr RowSteps kRows = row_steps();

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

// Bytewise max of two words by packed 16-bit maxima: max_even_bytes holds the maxima of bytes 0 and 2 in bytes
// 0 and 2 (the other bytes masked to 0 first); max_odd_bytes those of bytes 1 and 3 in bytes 1 and 3 (the high
// byte of a 16-bit maximum is the maximum of the high bytes, whatever the low bytes are).
typedef unsigned short mh_u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t max_even_bytes(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(mh_u16x2, a & 0x00ff00ffu),
                                                                  __builtin_bit_cast(mh_u16x2, b & 0x00ff00ffu)));
}
__device__ __forceinline__ uint32_t max_odd_bytes(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(mh_u16x2, a),
                                                                  __builtin_bit_cast(mh_u16x2, b)));
}
// ---- INTER_AREA by periods (the step kernel's observation)
// The horizontal sums of source row pixels 64 g .. 64 g + 63 for output columns 21 g .. 21 g + 20: per column
// its 4 taps in order, as area_pixel's row sum (whose first step, +0 + a non-negative product, is the product
// itself). Pixel 4 i + j (max-pooled if the env pools) is byte j of ev[i] for even j and of od[i] for odd j, so
// that a max-pooled row needs no merge of the two packed maxima (both arrays are the row's words otherwise).
__device__ __forceinline__ void obs_period_sums(const uint32_t (&ev)[16], const uint32_t (&od)[16], float (&rs)[21]) {
#pragma unroll
    for (int q = 0; q < 21; q++) {
        float row = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int px = kArea.x0[q] + k;
            const uint32_t w = (px & 1) ? od[px >> 2] : ev[px >> 2];
            const float t = (float)((w >> (8 * (px & 3))) & 0xffu) * kArea.xw[q][k];
            row = k == 0 ? t : row + t;
        }
        rs[q] = row;
    }
}

// The vertical step for source row sy (0 .. 239) with its sums rs: adds them to the open output row `acc`
// (which starts at +0: +0 + the first non-negative term is that term, as area_pixel's first step), and when the
// row is complete calls emit(output row, acc) and opens the next one. The step is the same for every lane
// (sy is uniform in the kernel), so its weights come from one table entry.
template <class Emit>
__device__ __forceinline__ void obs_period_take(int sy, const float (&rs)[21], float (&acc)[21], Emit&& emit) {
    const int p = sy / 20;
    const RowStep st = kRows.s[sy - 20 * p];
#pragma unroll
    for (int q = 0; q < 21; q++) acc[q] = acc[q] + st.wa * rs[q];
    if (st.last) {
        emit(7 * p + st.q, acc);
#pragma unroll
        for (int q = 0; q < 21; q++) acc[q] = st.wb * rs[q];
    }
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
    c.mbase = mem; c.eo = e; c.vo = (uint32_t)vram_word_offset(np, e, 0); c.np = np;
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
    uint8_t* fresh;               // new observation of each slot: [e * OBS_PIX + o]
    const uint8_t* boot_obs;      // boot observation of each level: [level * OBS_PIX + o]
    uint32_t* obs_order;          // [0]: waves that finished their frame loop (0 at launch); [1 + k]: the first
                                  // slot of the wave whose ticket is obs_late_from + k
    uint32_t obs_late_from;       // waves with a ticket in [obs_late_from, obs_late_to) leave their
    uint32_t obs_late_to;         // observations to k_obs_late (obs_late_to: the waves with live envs)
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
    int cpw;                     // consoles per wave (k_raw): 1, 2, 4, 8 or ENVS_PER_WAVE
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
// Returns what the env's new observation needs: bit 0 pool, bit 1 the last frame is in frame buffer 1, bit 2
// the boot observation, bits 8.. the level.
__device__ inline uint32_t step_lane(const StepArgs& A, const LaneCtx& x, uint32_t e) {
    const uint32_t o = (uint32_t)A.slot_env[e];   // the env's index in the action and output arrays
    Console c;
    const uint32_t level = A.ev[(size_t)E_LEVEL * A.np + e];
    attach(c, x, A.mem, A.np, e, A.key_bank[level]);
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
    return (ev.pooled ? 1u : 0u) | (ev.slot_swap ? 2u : 0u) | (ev.shows_boot ? 4u : 0u) | level << 8;
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
