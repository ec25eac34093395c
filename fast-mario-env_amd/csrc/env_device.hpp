// Device-side env layer: gym-super-mario-bros reward / done / info, the wrapper stack (sticky actions,
// frame skip, 2-frame max-pool, early termination, life loss, no-op starts, time limit) and the level
// boot, as in the reference's csrc/fastmario.cpp:204-445.
#pragma once
#include "nes_device.hpp"

namespace mh {

// Per-env words beside the console state, interleaved as EV[w * NP + e].
enum EnvWord : int {
    E_XLAST_LO = 0, E_XLAST_HI, E_TLAST_LO, E_TLAST_HI, E_PREV, E_LIVES, E_T, E_EP_LEN,
    E_EPRET_LO, E_EPRET_HI, E_SHOWS_BOOT, E_POOLED, E_LEVEL, E_FRAMES_LO, E_FRAMES_HI,
    E_BAD, E_INSTR_LO, E_INSTR_HI,
    E_RNG_S0, E_RNG_S1, E_RNG_S2, E_RNG_S3, E_RNG_I0, E_RNG_I1, E_RNG_I2, E_RNG_I3,   // little-endian u32 limbs
    E_RNG_HAS32, E_RNG_HALF, E_DONE, E_RESET_IDX,
    E_FF_LO, E_FF_HI,                                  // poll-loop instructions fast-forwarded (in E_INSTR too)
    E_REEMU_ONE, E_REEMU_PAIR, E_REEMU_K2,             // early-termination re-emulations by kind (REEMU_*)
    E_HACK_REDRAWS,                                     // hack frames run a second time to be drawn
    E_COUNT
};

constexpr int MAX_SKIP = 16;
// Kinds of early-termination re-emulation (an agent step whose episode ended at frame last < K-1), by the
// reference's branches (fastmario.cpp:351-362): ONE re-runs frame last alone, PAIR re-runs its max-pool
// partner last-1 too; K2 marks an end at frame K-2 under max-pool, where frame last was rendered in the
// first pass and only the partner runs again.
enum : uint32_t { REEMU_ONE = 1u, REEMU_PAIR = 2u, REEMU_K2 = 4u };
constexpr int HACK_FRAME_LIMIT = 20000;   // guard against a game stuck in a busy state (the reference loops forever)

__device__ __constant__ static const uint8_t kButtons[8] = {0x00, 0x80, 0x81, 0x82, 0x83, 0x01, 0x40, 0x00};

// numpy PCG64 (XSL-RR 128/64) with Generator.random() and the 32-bit Lemire integers() path
// (fastmario.cpp:39-78; numpy's bit generator and `random_bounded_uint64` for ranges < 2^32).
struct Pcg {
    unsigned __int128 state, inc;
    uint32_t has32, half;
    __device__ uint64_t next64() {
        const unsigned __int128 mul = ((unsigned __int128)0x2360ED051FC65DA4ULL << 64) | 0x4385DF649FCCF645ULL;
        state = state * mul + inc;
        uint64_t xs = (uint64_t)(state >> 64) ^ (uint64_t)state;
        unsigned r = (unsigned)(state >> 122);
        return (xs >> r) | (xs << ((64 - r) & 63));
    }
    __device__ uint32_t next32() {
        if (has32) { has32 = 0; return half; }
        uint64_t w = next64();
        has32 = 1; half = (uint32_t)(w >> 32);
        return (uint32_t)w;
    }
    __device__ double random() { return (double)(next64() >> 11) * (1.0 / 9007199254740992.0); }
    __device__ int64_t integers(int64_t high) {
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
    __device__ void load(const uint32_t* ev, uint32_t np, uint32_t e) {
        auto w = [&](int k) { return (unsigned __int128)ev[(size_t)k * np + e]; };
        state = w(E_RNG_S0) | (w(E_RNG_S1) << 32) | (w(E_RNG_S2) << 64) | (w(E_RNG_S3) << 96);
        inc = w(E_RNG_I0) | (w(E_RNG_I1) << 32) | (w(E_RNG_I2) << 64) | (w(E_RNG_I3) << 96);
        has32 = ev[(size_t)E_RNG_HAS32 * np + e];
        half = ev[(size_t)E_RNG_HALF * np + e];
    }
    __device__ void store(uint32_t* ev, uint32_t np, uint32_t e) const {
        for (int k = 0; k < 4; k++) {
            ev[(size_t)(E_RNG_S0 + k) * np + e] = (uint32_t)(state >> (32 * k));
            ev[(size_t)(E_RNG_I0 + k) * np + e] = (uint32_t)(inc >> (32 * k));
        }
        ev[(size_t)E_RNG_HAS32 * np + e] = has32;
        ev[(size_t)E_RNG_HALF * np + e] = half;
    }
};

// ------------------------------------------------------------------ SMB RAM protocol (fastmario.cpp:204-250)
// x_pos flag_get life score time world stage coins y_pos status, as the int32 values of the C ABI
struct Info { int32_t v[10]; };

__device__ __forceinline__ int64_t dec_digits(const Console& c, uint32_t ad, int n) {
    int64_t val = 0;
    for (int i = 0; i < n; i++) {
        int b = c.ram(ad + i);
        val = val * (b >= 100 ? 1000 : b >= 10 ? 100 : 10) + b;
    }
    return val;
}
__device__ __forceinline__ int64_t smb_x(const Console& c) { return (int64_t)c.ram(0x6d) * 256 + c.ram(0x86); }
__device__ __forceinline__ int64_t smb_time(const Console& c) { return dec_digits(c, 0x7f8, 3); }
__device__ __forceinline__ bool smb_busy(const Console& c) { uint8_t s = c.ram(0x0e); return s <= 5 || s == 7; }
__device__ __forceinline__ bool smb_world_over(const Console& c) { return c.ram(0x770) == 2; }
__device__ __forceinline__ bool smb_stage_over(const Console& c) {
    for (uint32_t ad = 0x16; ad <= 0x1a; ad++) {
        uint8_t id = c.ram(ad);
        if (id == 0x2d || id == 0x31) return c.ram(0x1d) == 3;
    }
    return false;
}
__device__ __forceinline__ Info smb_info(const Console& c) {
    Info i;
    i.v[0] = (int32_t)smb_x(c);
    i.v[1] = smb_world_over(c) || smb_stage_over(c);
    i.v[2] = c.ram(0x75a);
    i.v[3] = (int32_t)dec_digits(c, 0x7de, 6);
    i.v[4] = (int32_t)smb_time(c);
    i.v[5] = c.ram(0x75f) + 1;
    i.v[6] = c.ram(0x75c) + 1;
    i.v[7] = (int32_t)dec_digits(c, 0x7ed, 2);
    uint8_t yp = c.ram(0x3b8);
    i.v[8] = c.ram(0xb5) < 1 ? 255 + (255 - yp) : 255 - yp;
    uint8_t st = c.ram(0x756);
    i.v[9] = st == 0 ? 0 : st == 1 ? 1 : 2;
    return i;
}

struct Cfg {
    int skip, max_steps, noop_max, maxpool;
    double sticky;
};

// Memory region of consoles with the same layout as the live state (reset cache, boot states).
struct Region {
    uint8_t* mem;       // row-major [row * np + idx], VRAM word-interleaved (vram_word_offset)
    uint32_t* sc;       // [word * np + idx]
    uint32_t np;
    uint32_t idx;
};

__device__ inline void copy_console(const Region& dst, const Region& src) {
    for (uint32_t r = 0; r < MEM_ROWS; r++)
        if (r < ROW_VRAM || r >= ROW_VRAM + 2048) dst.mem[(size_t)r * dst.np + dst.idx] = src.mem[(size_t)r * src.np + src.idx];
    for (uint32_t w = 0; w < 512; w++)
        *(uint32_t*)(dst.mem + vram_word_offset(dst.np, dst.idx, w)) =
            *(const uint32_t*)(src.mem + vram_word_offset(src.np, src.idx, w));
    for (int w = 0; w < S_COUNT; w++) dst.sc[(size_t)w * dst.np + dst.idx] = src.sc[(size_t)w * src.np + src.idx];
}

// copy_console by the `lanes` lanes of a wave together, lane `lane` taking every lanes-th byte row, VRAM
// word and register word: one console is a few thousand independent accesses, too many for one lane.
__device__ inline void copy_console_wave(const Region& dst, const Region& src, uint32_t lane, uint32_t lanes) {
    constexpr uint32_t BYTE_ROWS = MEM_ROWS - 2048;   // every row but the VRAM span
    for (uint32_t i = lane; i < BYTE_ROWS; i += lanes) {
        const uint32_t r = i < (uint32_t)ROW_VRAM ? i : i + 2048;
        dst.mem[(size_t)r * dst.np + dst.idx] = src.mem[(size_t)r * src.np + src.idx];
    }
    for (uint32_t w = lane; w < 512; w += lanes)
        *(uint32_t*)(dst.mem + vram_word_offset(dst.np, dst.idx, w)) =
            *(const uint32_t*)(src.mem + vram_word_offset(src.np, src.idx, w));
    for (uint32_t w = lane; w < (uint32_t)S_COUNT; w += lanes)
        dst.sc[(size_t)w * dst.np + dst.idx] = src.sc[(size_t)w * src.np + src.idx];
}

// The memory rows of copy_console (not the register words), by one lane: the loads of a batch of 32 are
// issued before its stores, so the lane keeps 32 accesses in flight instead of waiting for each one.
__device__ inline void copy_rows_lane(const Region& dst, const Region& src) {
    constexpr uint32_t B = 32, BYTE_ROWS = MEM_ROWS - 2048;   // the VRAM span aside
    static_assert(BYTE_ROWS % B == 0 && ROW_VRAM % B == 0 && 512 % B == 0, "batches must not straddle the VRAM span");
    for (uint32_t i0 = 0; i0 < BYTE_ROWS; i0 += B) {
        const uint32_t r0 = i0 < (uint32_t)ROW_VRAM ? i0 : i0 + 2048;
        uint8_t t[B];
#pragma unroll
        for (uint32_t b = 0; b < B; b++) t[b] = src.mem[(size_t)(r0 + b) * src.np + src.idx];
#pragma unroll
        for (uint32_t b = 0; b < B; b++) dst.mem[(size_t)(r0 + b) * dst.np + dst.idx] = t[b];
    }
    for (uint32_t w0 = 0; w0 < 512; w0 += B) {
        uint32_t t[B];
#pragma unroll
        for (uint32_t b = 0; b < B; b++) t[b] = *(const uint32_t*)(src.mem + vram_word_offset(src.np, src.idx, w0 + b));
#pragma unroll
        for (uint32_t b = 0; b < B; b++) *(uint32_t*)(dst.mem + vram_word_offset(dst.np, dst.idx, w0 + b)) = t[b];
    }
}

// Snapshot of a console between two frames into `dst` (a region of the same np, at the console's own
// index): store() of the registers (and of the LDS copy of OAM into the console's rows), then its rows.
__device__ inline void save_console(Console& c, const Region& live, const Region& dst) {
    c.store(dst.sc, dst.idx);
    copy_rows_lane(dst, live);
}
// The console as snapshotted: rows back, then load() of the registers (OAM to LDS, derived caches reset).
// The instruction and bad-op counters are not part of the snapshot and keep counting.
__device__ inline void restore_console(Console& c, const Region& live, const Region& src) {
    copy_rows_lane(live, src);
    c.load(src.sc, src.idx);
}

// One env's layer state in registers.
struct EnvRegs {
    int64_t x_last, time_last;
    int prev, lives, t, ep_len;
    double ep_ret;
    bool shows_boot, pooled, slot_swap;   // slot_swap: the last frame is in frame buffer 1
    uint64_t frames;
    uint32_t draws;     // sticky draws taken (counted by the reset-cache builder)
    uint32_t reemu;     // REEMU_* bits of the last agent step
    uint32_t hack_redraws;   // hack frames run again to be drawn in the last agent step
    Info info;
};

struct Stepper {
    Console& c;
    EnvRegs& ev;
    const Cfg& cfg;
    Pcg* rng;             // null: draws are counted, not taken (reset cache: action 0 == prev 0)
    uint8_t* gray0;       // frame buffer of frames K-1, K-3, ... of the agent step
    uint8_t* gray1;       // frame buffer of frames K-2, K-4, ...
    Region live;          // the console's own rows and register words
    uint8_t* snap_mem;    // two snapshot slots of live's layout: rows of slot s at snap_mem + s MEM_ROWS np,
    uint32_t* snap_sc;    // register words at snap_sc + s S_COUNT np

    __device__ __forceinline__ Region snap(int s) const {
        return Region{snap_mem + (size_t)s * MEM_ROWS * live.np, snap_sc + (size_t)s * S_COUNT * live.np, live.np, live.idx};
    }
    __device__ __forceinline__ bool busy() { return smb_busy(c) || smb_world_over(c); }
    // _skip_change_area before the _skip_occupied_states loop (fastmario.cpp:297-300)
    __device__ __forceinline__ void fix_change_area() {
        const uint8_t cat = c.ram(0x6de);
        if (cat > 1 && cat < 255) c.st(ROW_RAM + 0x6de, 1);
    }
    // reward, done and info after an agent frame (fastmario.cpp:310-334)
    __device__ __forceinline__ double frame_reward(bool* done) {
        int64_t xx = smb_x(c), dx = xx - ev.x_last;
        ev.x_last = xx;
        if (dx < -5 || dx > 5) dx = 0;
        int64_t tm = smb_time(c), dt = tm - ev.time_last;
        ev.time_last = tm;
        if (dt > 0) dt = 0;
        uint8_t ps = c.ram(0x0e);
        bool die = ps == 0x0b || c.ram(0xb5) > 1 || ps == 0x06;
        int64_t r = dx + dt + (die ? -25 : 0);
        if (r < -15) r = -15;
        if (r > 15) r = 15;
        ev.info = smb_info(c);
        *done = die || ev.info.v[1];
        return (double)r;
    }

    // Sticky actions + frame skip + max-pool + early termination + life loss (fastmario.cpp:336-374),
    // with the hack frames of _skip_change_area / _skip_occupied_states (fastmario.cpp:297-308) after
    // every agent frame that did not end the episode.
    //
    // When an observation is wanted, frames K-1 and (max-pool) K-2 are rendered with their hack frames,
    // K-1 into gray0 and K-2 into gray1. Before every frame that a re-emulation could start from, the
    // console is snapshotted into slot (frame & 1). When the episode ends at a frame last < K-1, the
    // reference restores the snapshot of frame last-1 (max-pool, last >= 1) or of frame last and runs those
    // frames again with pixels on, last-1 with its hack frames (fastmario.cpp:351-362); the re-emulated
    // frames count like any other. Frames that were not rendered are re-emulated here the same way. Frame
    // K-2 (max-pool) was rendered in the first pass, and running it again from the same state with the same
    // buttons repeats it exactly: its state after the first pass is saved instead, only its partner K-3 runs
    // again, the saved state is restored, and frame K-2 is counted a second time. No lane then runs more
    // than K frames (plus hack frames) in a step, which would hold up its whole wave.
    // Written as a state machine around ONE console frame so that the emulator is inlined once: a lane that
    // re-emulates does so while the other lanes of its wave still run their remaining agent frames, and it
    // waits (skipping the frame call) until the iterations of the wave's own rendered frames, K-2 and K-1,
    // so that its rendered re-emulation does not turn an unrendered iteration of the wave into a rendered one.
    __device__ __forceinline__ double agent_step(int act0, bool want_obs, bool* term) {
        const int K = cfg.skip;
        const bool mp = cfg.maxpool != 0;
        double total = 0.0;
        bool done = false, hack = false, render = false;
        bool keep_last = false;            // the state after frame last is in slot last & 1
        int i = 0, guard = 0;
        int rf = -1;                       // agent frame being re-emulated (-1: the first pass)
        uint8_t b_prev = 0, b_cur = 0;     // buttons of agent frames i-1 and i
        uint32_t n0 = 0, b0 = 0, f0 = 0;   // instruction, bad-op and fast-forward counters at the start of agent frame i
        int it = 0, resume_at = 0;         // loop iterations so far; the iteration a re-emulation starts at
        uint8_t* slot = gray0;
        bool undrawn = false;              // the hack frame just run was not drawn; its start state is in slot 0
        bool redraw = false;               // this iteration runs that hack frame again, drawn
        uint32_t hn = 0, hb = 0, hf = 0;   // instruction, bad-op and fast-forward counters at that start state
        ev.hack_redraws = 0;
        for (;;) {
            if (rf >= 0 && it < resume_at) { it++; continue; }   // waiting for the wave's rendered frames
            it++;
            uint8_t buttons = 0;
            if (hack) {
                c.st(ROW_RAM + 0x7a0, 0);
                // A hack frame of a drawn agent frame is drawn only if it ends the busy run: it runs undrawn
                // from a snapshot and, when busy() clears after it, runs again drawn (below). A CPU frame
                // covers a whole PPU frame, so the last frame's pixels are the whole picture, as in the
                // reference, which draws every one. Slot 0 is free: a drawn agent frame followed by hack
                // frames did not end the episode, so no re-emulation can follow in this step.
                undrawn = rf < 0 && render && !redraw;
                if (undrawn) {
                    save_console(c, live, snap(0));
                    hn = c.instructions; hb = c.bad_ops; hf = c.ff_instructions;
                }
            } else if (rf < 0) {
                int act = act0;
                if (cfg.sticky != 0.0) {
                    if (rng) { if (rng->random() < cfg.sticky) act = ev.prev; }
                    else ev.draws++;
                }
                ev.prev = act;
                b_prev = b_cur; b_cur = kButtons[act];
                buttons = b_cur;
                render = want_obs && (i == K - 1 || (mp && i == K - 2));
                slot = ((K - 1 - i) & 1) ? gray1 : gray0;
                n0 = c.instructions; b0 = c.bad_ops; f0 = c.ff_instructions;
                // re-emulations start at frame last-1 (max-pool, last >= 1) or last, for last < K-1, and
                // never at K-2 (max-pool)
                if (want_obs && i < K - 1 && (!mp || i <= K - 3)) save_console(c, live, snap(i & 1));
            } else {
                buttons = rf == i ? b_cur : b_prev;
                render = true;
                slot = ((K - 1 - rf) & 1) ? gray1 : gray0;
            }
            c.set_buttons0(buttons);
            c.render = render && !undrawn;
            c.gray = slot;
            c.frame();
            ev.frames++;
            if (render) ev.shows_boot = false;
            if (rf < 0) {
                if (!hack) {
                    total += frame_reward(&done);
                    if (!done) { fix_change_area(); guard = 0; }
                }
                if (!done && busy()) {
                    if (++guard <= HACK_FRAME_LIMIT) { hack = true; continue; }
                    c.bad_ops |= ERR_HACK_LIMIT;
                }
                if (undrawn && !(c.bad_ops & ERR_HACK_LIMIT)) {
                    // the busy run ended with an undrawn hack frame: back to its start, counted once
                    restore_console(c, live, snap(0));
                    c.instructions = hn; c.bad_ops = hb; c.ff_instructions = hf;
                    ev.frames--;
                    ev.hack_redraws++;
                    undrawn = false;
                    redraw = true;
                    continue;
                }
                undrawn = redraw = false;
                hack = false;
                if (!done && i < K - 1) { i++; continue; }
                // the first pass ended at agent frame i
                if (!(want_obs && done && i < K - 1)) break;
                if (mp && i == K - 2) {
                    // frame i was rendered: count its re-emulation (it ended the episode, so it had no hack
                    // frames), and re-emulate its max-pool partner i-1 if there is one
                    ev.frames++;
                    const uint32_t dn = c.instructions - n0, db = (c.bad_ops - b0) & ~ERR_FLAGS;
                    c.instructions += dn;
                    c.bad_ops += db;
                    c.ff_instructions += c.ff_instructions - f0;
                    if (i == 0) break;
                    save_console(c, live, snap(i & 1));
                    keep_last = true;
                    rf = i - 1;
                } else {
                    rf = (mp && i >= 1) ? i - 1 : i;
                }
                resume_at = K - (keep_last ? 1 : i - rf + 1);   // K minus the frames to run again
                restore_console(c, live, snap(rf & 1));
            } else if (rf < i) {
                // frame last-1 again, then its hack frames (it did not end the episode)
                if (!hack) { fix_change_area(); guard = 0; }
                if (busy()) {
                    if (++guard <= HACK_FRAME_LIMIT) { hack = true; continue; }
                    c.bad_ops |= ERR_HACK_LIMIT;
                }
                hack = false;
                if (keep_last) { restore_console(c, live, snap(i & 1)); break; }
                rf++;
            } else {
                break;
            }
        }
        const int last = i;
        ev.reemu = (want_obs && done && last < K - 1)
                       ? ((mp && last >= 1) ? REEMU_PAIR : REEMU_ONE) | ((mp && last == K - 2) ? REEMU_K2 : 0u)
                       : 0u;
        if (want_obs) {
            ev.pooled = mp && last >= 1;
            ev.slot_swap = ((K - 1 - last) & 1) != 0;
        }
        bool tm = done;
        int life = (int)ev.info.v[2];
        if (ev.lives >= 0 && life < ev.lives) tm = true;
        ev.lives = life;
        if (ev.info.v[1]) tm = true;
        *term = tm;
        return total;
    }
};

}  // namespace mh
