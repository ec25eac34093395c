// Host build of the device code (test infrastructure only).
//
// Compiles fast-mario-env_amd/csrc/lane_kernels.hpp (with env_device.hpp and nes_device.hpp) as x86 C++ for
// one lane per env (the include path puts tests/hostbuild/hip/hip_runtime.h in front of HIP's) and drives
// the same lane bodies the GPU kernels call, one console after another, so that the device code itself runs
// under AddressSanitizer and UndefinedBehaviorSanitizer. The orchestration around the lane bodies (boot,
// reset cache, reset, step, observation, frame stack) follows libmario_hip.so's host side and kernels
// (mario_hip.hip); the arrays have the GPU's lane-interleaved layouts, sized exactly, so an access outside a
// console's rows is an access outside its buffer.
//
// Protocol on stdin / stdout (little-endian binary), one session per process:
//   raw <rom file>:  'F' buttons:u8 render:u8 -> ram[2048] screen[61440]; 'B' backup; 'S' restore;
//                    'Q' -> bad_ops:i64 instructions:i64 ff_instructions:i64, exit
//   env <config file> (rom_len:i64 rom n:i32 levels:i32[3n] lut:u8[256] skip max_steps:i32 sticky:f64
//                    noop_max maxpool frame_stack:i32 rng:u64[6n]):
//                    'R' -> obs;  'T' actions:i64[n] -> obs rew:f32[n] term:u8[n] trunc:u8[n] info:i64[10n]
//                    ram[2048 n] fin ep_ret:f64[n] ep_len:i64[n];  'Q' -> frames bad_ops instructions ff
//                    hack_redraws:i64, exit
//   plant <bytes>:   reads one byte past a buffer of that size (the tests check that the sanitizers catch it)
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "lane_kernels.hpp"

using namespace mh;

namespace {

[[noreturn]] void die(const char* m) { std::fprintf(stderr, "host_driver: %s\n", m); std::exit(2); }

void get(void* p, size_t n) { if (std::fread(p, 1, n, stdin) != n) die("short read on stdin"); }
template <class T> T get1() { T v; get(&v, sizeof v); return v; }
void put(const void* p, size_t n) { if (std::fwrite(p, 1, n, stdout) != n) die("short write"); }

uint32_t pad64(int n) { return (uint32_t)((n + 63) / 64 * 64); }

// iNES NROM -> PRG (16 KB mirrored to 32 KB) + CHR, name-table bits (the steps of mario_hip.hip's load_cart)
void load_cart(const std::vector<uint8_t>& d, std::vector<uint8_t>& img, uint32_t& nt_bits) {
    if (d.size() < 16 || d[0] != 'N' || d[1] != 'E' || d[2] != 'S' || d[3] != 0x1a) die("not an iNES image");
    const int banks = d[4];
    if (banks < 1 || banks > 2 || d[5] != 1 || (d[6] >> 4) || (d[7] & 0xf0) || (d[6] & 6)) die("not an NROM image");
    if (d.size() < 16 + 0x4000u * banks + 0x2000u) die("truncated ROM");
    img.assign(0xa000, 0);
    for (int i = 0; i < 0x8000; i++) img[i] = d[16 + (i % (0x4000 * banks))];
    for (int i = 0; i < 0x2000; i++) img[0x8000 + i] = d[16 + 0x4000 * banks + i];
    const int m = d[6] & 0xB;
    const uint16_t nt[4] = {0, (uint16_t)(m == 1 ? 0x400 : 0), (uint16_t)(m == 0 ? 0x400 : 0), (uint16_t)(m <= 1 ? 0x400 : 0)};
    nt_bits = 0;
    for (int i = 0; i < 4; i++) nt_bits |= (nt[i] ? 1u : 0u) << i;
}

// The block-shared LDS of the emulator kernels for one block of LDS_LANES env slots. Consoles run one after
// another here, so consoles of different blocks reuse one block's per-slot buffers.
struct Lds {
    std::vector<uint8_t> rom, lut;
    std::vector<uint32_t> dec, sp, gp;
    RomArgs R{};
    Lds(const std::vector<uint8_t>& img, const uint8_t* lut256, uint32_t nt_bits)
        : rom(img), lut(lut256, lut256 + 256), dec(256), sp((size_t)LDS_SP_WORDS * LDS_LANES),
          gp((size_t)LDS_GP_REGION * LDS_LANES) {
        for (int i = 0; i < 256; i++) dec[i] = kDecode.w[i];
        R.rom = rom.data(); R.lut = lut.data(); R.nt_bits = nt_bits; R.n_chr = 1;
    }
    LaneCtx ctx(uint32_t index) {
        const uint32_t slot = index % LDS_LANES;
        return LaneCtx{make_cart(R, rom.data(), dec.data()), lut.data(), sp.data() + slot, gp.data() + slot, 0};
    }
};

// ------------------------------------------------------------------ raw consoles
int run_raw(const char* rom_file) {
    FILE* f = std::fopen(rom_file, "rb");
    if (!f) die("cannot open the ROM");
    std::vector<uint8_t> d;
    for (int c; (c = std::fgetc(f)) != EOF;) d.push_back((uint8_t)c);
    std::fclose(f);
    std::vector<uint8_t> img;
    uint32_t nt_bits;
    load_cart(d, img, nt_bits);
    std::vector<uint8_t> ident(256);
    for (int i = 0; i < 256; i++) ident[i] = (uint8_t)i;
    Lds L(img, ident.data(), nt_bits);
    const int n = 1;
    const uint32_t np = pad64(n);
    std::vector<uint8_t> mem((size_t)MEM_ROWS * np), bk_mem(mem.size()), screen((size_t)GRAY_PIX * np);
    std::vector<uint32_t> sc((size_t)S_COUNT * np), bk_sc(sc.size()), bad(np), instr(np), ff(np);
    std::vector<uint8_t> buttons(np);
    RawArgs A{L.R, n, np, mem.data(), sc.data(), screen.data(), buttons.data(), 0, bad.data(), instr.data(), ff.data(), 1, 1};
    raw_lane(A, L.ctx(0), 0);
    A.power_on = 0;
    for (;;) {
        const char c = get1<char>();
        if (c == 'F') {
            buttons[0] = get1<uint8_t>();
            A.render = get1<uint8_t>();
            raw_lane(A, L.ctx(0), 0);
            uint8_t ram[2048];
            for (int i = 0; i < 2048; i++) ram[i] = mem[(size_t)(ROW_RAM + i) * np];
            std::vector<uint8_t> scr(GRAY_PIX);
            for (int p = 0; p < GRAY_PIX; p++) scr[p] = screen[((size_t)(p >> 2) * np) * 4 + (p & 3)];
            put(ram, sizeof ram);
            put(scr.data(), scr.size());
            std::fflush(stdout);
        } else if (c == 'B') {
            bk_mem = mem; bk_sc = sc;
        } else if (c == 'S') {
            mem = bk_mem; sc = bk_sc;
        } else if (c == 'Q') {
            const int64_t out[3] = {bad[0], instr[0], ff[0]};
            put(out, sizeof out);
            std::fflush(stdout);
            return 0;
        } else {
            die("unknown raw command");
        }
    }
}

// ------------------------------------------------------------------ vector env
struct Vec {
    int n, K, nl, nk, nc;
    uint32_t np, nlp, ncp;
    Cfg cfg;
    std::vector<uint8_t> img;
    uint32_t nt_bits;
    std::vector<int> lv;
    std::vector<uint8_t> key_bank;
    std::vector<uint8_t> mem, gray, snap_mem, fresh, boot_mem, boot_gray, boot_obs, cmem, cgray, csnap_mem, cobs, cboot;
    std::vector<uint32_t> sc, ev, snap_sc, boot_sc, csc, csnap_sc, cbad;
    std::vector<int64_t> x0, t0, cx, ct;
    std::vector<int32_t> clives, cdraws, slot_env;
    std::vector<uint64_t> cframes, cinstr, cff;
    std::vector<uint8_t> obs, fin, term, trunc;
    std::vector<float> rew;
    std::vector<int32_t> info, ep_len;
    std::vector<double> ep_ret;
    AreaTables T;
};

// INTER_AREA of one frame-buffer lane, or a boot observation (k_small_obs)
void small_obs(const Vec& v, const std::vector<uint8_t>& gray, uint32_t stride, const uint8_t* use_boot, int count,
               std::vector<uint8_t>& out) {
    for (int i = 0; i < count; i++)
        for (int o = 0; o < OBS_PIX; o++)
            out[(size_t)i * OBS_PIX + o] = (use_boot && use_boot[i])
                ? v.boot_obs[(size_t)(i / v.nk) * OBS_PIX + o]
                : area_pixel(Image{gray.data(), stride, (uint32_t)i}, Image{}, false, o, &v.T);
}

int run_env(const char* cfg_file) {
    FILE* f = std::fopen(cfg_file, "rb");
    if (!f) die("cannot open the config");
    auto rd = [&](void* p, size_t k) { if (std::fread(p, 1, k, f) != k) die("short config"); };
    Vec v;
    int64_t rom_len;
    rd(&rom_len, 8);
    std::vector<uint8_t> rom((size_t)rom_len);
    rd(rom.data(), rom.size());
    int32_t n;
    rd(&n, 4);
    std::vector<int32_t> levels(3 * (size_t)n);
    rd(levels.data(), levels.size() * 4);
    uint8_t lut[256];
    rd(lut, 256);
    int32_t skip, max_steps, noop_max, maxpool, stack;
    double sticky;
    rd(&skip, 4); rd(&max_steps, 4); rd(&sticky, 8); rd(&noop_max, 4); rd(&maxpool, 4); rd(&stack, 4);
    std::vector<uint64_t> rng(6 * (size_t)n);
    rd(rng.data(), rng.size() * 8);
    std::fclose(f);
    load_cart(rom, v.img, v.nt_bits);
    Lds L(v.img, lut, v.nt_bits);
    v.n = n; v.K = stack; v.np = pad64(n);
    v.cfg = Cfg{skip, max_steps, noop_max, maxpool ? 1 : 0, sticky};
    // distinct levels in order of first appearance (one ROM here)
    std::vector<int> env_level(n);
    for (int i = 0; i < n; i++) {
        int li = -1;
        for (size_t k = 0; k < v.lv.size() / 3; k++)
            if (v.lv[3 * k] == levels[3 * i] && v.lv[3 * k + 1] == levels[3 * i + 1] && v.lv[3 * k + 2] == levels[3 * i + 2]) li = (int)k;
        if (li < 0) { li = (int)v.lv.size() / 3; v.lv.insert(v.lv.end(), &levels[3 * i], &levels[3 * i] + 3); }
        env_level[i] = li;
    }
    v.nl = (int)v.lv.size() / 3; v.nlp = pad64(v.nl);
    v.nk = noop_max + 1; v.nc = v.nl * v.nk; v.ncp = pad64(v.nc);
    v.key_bank.assign(v.nl, 0);
    v.slot_env.resize(v.np);
    for (uint32_t s = 0; s < v.np; s++) v.slot_env[s] = (int32_t)s;
    const uint32_t np = v.np, nlp = v.nlp, ncp = v.ncp;
    v.mem.assign((size_t)MEM_ROWS * np, 0); v.sc.assign((size_t)S_COUNT * np, 0); v.ev.assign((size_t)E_COUNT * np, 0);
    v.gray.assign((size_t)2 * GRAY_PIX * np, 0);
    v.snap_mem.assign((size_t)2 * MEM_ROWS * np, 0); v.snap_sc.assign((size_t)2 * S_COUNT * np, 0);
    v.fresh.assign((size_t)OBS_PIX * np, 0);
    v.boot_mem.assign((size_t)MEM_ROWS * nlp, 0); v.boot_sc.assign((size_t)S_COUNT * nlp, 0);
    v.boot_gray.assign((size_t)GRAY_PIX * nlp, 0); v.boot_obs.assign((size_t)OBS_PIX * v.nl, 0);
    v.x0.assign(v.nl, 0); v.t0.assign(v.nl, 0);
    v.cmem.assign((size_t)MEM_ROWS * ncp, 0); v.csc.assign((size_t)S_COUNT * ncp, 0);
    v.cgray.assign((size_t)2 * GRAY_PIX * ncp, 0);
    v.csnap_mem.assign((size_t)2 * MEM_ROWS * ncp, 0); v.csnap_sc.assign((size_t)2 * S_COUNT * ncp, 0);
    v.cobs.assign((size_t)OBS_PIX * v.nc, 0); v.cboot.assign(v.nc, 0);
    v.cx.assign(v.nc, 0); v.ct.assign(v.nc, 0); v.clives.assign(v.nc, 0); v.cdraws.assign(v.nc, 0);
    v.cframes.assign(v.nc, 0); v.cinstr.assign(v.nc, 0); v.cff.assign(v.nc, 0); v.cbad.assign(v.nc, 0);
    const size_t stack_bytes = (size_t)n * stack * OBS_PIX;
    v.obs.assign(stack_bytes, 0); v.fin.assign(stack_bytes, 0); v.term.assign(n, 0); v.trunc.assign(n, 0);
    v.rew.assign(n, 0.f); v.info.assign((size_t)10 * n, 0); v.ep_ret.assign(n, 0.0); v.ep_len.assign(n, 0);
    area_tables(&v.T);
    // the library creates an env only if the run-time tables are the compiled-in periods that obs_tail uses
    if (!area_period_match(v.T)) die("INTER_AREA tables differ from the compiled-in periods");
    // and the allocation-free resize takes the whole tables from a device array initialised at compile time
    if (!area_tables_equal(v.T, kAreaTables)) die("INTER_AREA tables differ from the compile-time tables");
    for (int i = 0; i < n; i++) {
        auto w = [&](int k) -> uint32_t& { return v.ev[(size_t)k * np + i]; };
        w(E_LEVEL) = (uint32_t)env_level[i];
        const uint64_t* r = &rng[6 * (size_t)i];
        w(E_RNG_S3) = (uint32_t)(r[0] >> 32); w(E_RNG_S2) = (uint32_t)r[0];
        w(E_RNG_S1) = (uint32_t)(r[1] >> 32); w(E_RNG_S0) = (uint32_t)r[1];
        w(E_RNG_I3) = (uint32_t)(r[2] >> 32); w(E_RNG_I2) = (uint32_t)r[2];
        w(E_RNG_I1) = (uint32_t)(r[3] >> 32); w(E_RNG_I0) = (uint32_t)r[3];
        w(E_RNG_HAS32) = (uint32_t)r[4]; w(E_RNG_HALF) = (uint32_t)r[5];
        w(E_LIVES) = 0xffffffffu; w(E_SHOWS_BOOT) = 1; w(E_RESET_IDX) = 0xffffffffu;
    }
    // level boots and the reset cache (k_boot, k_small_obs, k_cache, k_small_obs)
    uint32_t err = 0;
    BootArgs ba{L.R, v.nl, nlp, v.lv.data(), v.key_bank.data(), v.boot_mem.data(), v.boot_sc.data(), v.boot_gray.data(),
                v.x0.data(), v.t0.data(), &err};
    for (int l = 0; l < v.nl; l++) boot_lane(ba, L.ctx(l), l);
    if (err) die("level boot did not finish");
    small_obs(v, v.boot_gray, nlp, nullptr, v.nl, v.boot_obs);
    CacheArgs ca{L.R, v.cfg, v.key_bank.data(), v.nl, v.nk, v.nc, nlp, ncp, v.boot_mem.data(), v.boot_sc.data(),
                 v.x0.data(), v.t0.data(), v.cmem.data(), v.csc.data(), v.cgray.data(), v.csnap_mem.data(),
                 v.csnap_sc.data(), v.cx.data(), v.ct.data(), v.clives.data(), v.cdraws.data(), v.cboot.data(),
                 v.cframes.data(), v.cinstr.data(), v.cff.data(), v.cbad.data()};
    for (int c = 0; c < v.nc; c++) cache_lane(ca, L.ctx(c), c);
    small_obs(v, v.cgray, ncp, v.cboot.data(), v.nc, v.cobs);

    auto reset_args = [&](int all) {
        return ResetArgs{n, np, v.cfg, v.nk, ncp, v.mem.data(), v.sc.data(), v.ev.data(), v.cmem.data(), v.csc.data(),
                         v.cx.data(), v.ct.data(), v.clives.data(), v.cdraws.data(), v.cboot.data(), v.cframes.data(),
                         v.cinstr.data(), v.cff.data(), v.cbad.data(), all};
    };
    // k_reset: draw each env's reset, install the chosen cache console
    auto do_reset = [&](int all) {
        const ResetArgs ra = reset_args(all);
        for (int e = 0; e < n; e++) {
            const int ci = reset_lane(ra, (uint32_t)e);
            if (ci >= 0)
                copy_console_wave(Region{v.mem.data(), v.sc.data(), np, (uint32_t)e},
                                  Region{v.cmem.data(), v.csc.data(), ncp, (uint32_t)ci}, 0, 1);
        }
    };
    const size_t nw = OBS_PIX / 4, fw = nw * stack;
    auto word = [](std::vector<uint8_t>& b, size_t i) -> uint8_t* { return b.data() + 4 * i; };
    // k_stack (mode 1: reset stacks; mode 0: shift, final_obs, reset observation)
    auto do_stack = [&](int mode) {
        for (int e = 0; e < n; e++) {
            const uint32_t ri = v.ev[(size_t)E_RESET_IDX * np + e];
            for (size_t w = 0; w < nw; w++) {
                uint8_t* st0 = word(v.obs, e * fw);
                auto st = [&](size_t s) { return st0 + 4 * (s * nw + w); };
                uint8_t fresh[4];
                for (int b = 0; b < 4; b++) fresh[b] = v.fresh[(size_t)e * OBS_PIX + 4 * w + b];
                const uint8_t* cw = v.cobs.data() + 4 * ((size_t)ri * nw + w);
                if (mode == 1) {
                    for (int s = 0; s < stack - 1; s++) memset(st(s), 0, 4);
                    memcpy(st(stack - 1), cw, 4);
                } else if (ri != 0xffffffffu) {
                    uint8_t* fo0 = word(v.fin, e * fw);
                    for (int s = 0; s < stack - 1; s++) { memcpy(fo0 + 4 * (s * nw + w), st(s + 1), 4); memset(st(s), 0, 4); }
                    memcpy(fo0 + 4 * ((stack - 1) * nw + w), fresh, 4);
                    memcpy(st(stack - 1), cw, 4);
                } else {
                    for (int s = 0; s < stack - 1; s++) memcpy(st(s), st(s + 1), 4);
                    memcpy(st(stack - 1), fresh, 4);
                }
            }
        }
    };
    // k_step's obs_tail: the boot observation right after a reset, else INTER_AREA of the last frame,
    // max-pooled; per env its 4 column periods one after another, with the kernel's row sums and vertical steps
    // (bits: what step_lane returned for the env)
    auto do_obs = [&](const std::vector<uint32_t>& bits) {
        for (int e = 0; e < n; e++) {
            uint8_t* out = v.fresh.data() + (size_t)e * OBS_PIX;
            const uint32_t b = bits[e];
            if (b & 4) {
                memcpy(out, v.boot_obs.data() + (size_t)(b >> 8) * OBS_PIX, OBS_PIX);
                continue;
            }
            const uint32_t* g0 = (const uint32_t*)v.gray.data();
            const uint32_t* g1 = (const uint32_t*)(v.gray.data() + (size_t)GRAY_PIX * np);
            for (int g = 0; g < 4; g++) {
                float acc[21] = {}, rs[21];
                for (int sy = 0; sy < 240; sy++) {
                    uint32_t ev[16], od[16];
                    for (int i = 0; i < 16; i++) {
                        const size_t wi = (size_t)(sy * 64 + 16 * g + i) * np + e;
                        const uint32_t w = (b & 2) ? g1[wi] : g0[wi];
                        ev[i] = (b & 1) ? max_even_bytes(g0[wi], g1[wi]) : w;
                        od[i] = (b & 1) ? max_odd_bytes(g0[wi], g1[wi]) : w;
                    }
                    obs_period_sums(ev, od, rs);
                    obs_period_take(sy, rs, acc, [&](int dy, const float (&a)[21]) {
                        for (int q = 0; q < 21; q++) out[dy * 84 + 21 * g + q] = round_sat(a[q]);
                    });
                }
            }
        }
    };
    std::vector<int64_t> actions(n);
    for (;;) {
        const char c = get1<char>();
        if (c == 'R') {
            do_reset(1);
            do_stack(1);
            put(v.obs.data(), v.obs.size());
            std::fflush(stdout);
        } else if (c == 'T') {
            get(actions.data(), actions.size() * 8);
            StepArgs sa{L.R, v.cfg, n, np, v.mem.data(), v.sc.data(), v.ev.data(), v.gray.data(), v.snap_mem.data(),
                        v.snap_sc.data(), actions.data(), v.rew.data(), v.term.data(), v.trunc.data(), v.info.data(),
                        v.ep_ret.data(), v.ep_len.data(), v.key_bank.data(), v.slot_env.data(), v.fresh.data(),
                        v.boot_obs.data()};
            std::vector<uint32_t> bits(n);
            for (int e = 0; e < n; e++) bits[e] = step_lane(sa, L.ctx(e), (uint32_t)e);
            do_obs(bits);
            do_reset(0);
            do_stack(0);
            std::vector<int64_t> info64(v.info.begin(), v.info.end()), epl64(v.ep_len.begin(), v.ep_len.end());
            std::vector<uint8_t> ram((size_t)2048 * n);
            for (int e = 0; e < n; e++)
                for (int i = 0; i < 2048; i++) ram[(size_t)e * 2048 + i] = v.mem[(size_t)(ROW_RAM + i) * np + e];
            put(v.obs.data(), v.obs.size());
            put(v.rew.data(), 4 * (size_t)n);
            put(v.term.data(), n);
            put(v.trunc.data(), n);
            put(info64.data(), 8 * info64.size());
            put(ram.data(), ram.size());
            put(v.fin.data(), v.fin.size());
            put(v.ep_ret.data(), 8 * (size_t)n);
            put(epl64.data(), 8 * (size_t)n);
            std::fflush(stdout);
        } else if (c == 'Q') {
            int64_t out[5] = {0, 0, 0, 0, 0};
            for (int e = 0; e < n; e++) {
                auto w = [&](int k) { return (uint64_t)v.ev[(size_t)k * np + e]; };
                out[0] += (int64_t)(w(E_FRAMES_LO) | w(E_FRAMES_HI) << 32);
                out[1] += (int64_t)w(E_BAD);
                out[2] += (int64_t)(w(E_INSTR_LO) | w(E_INSTR_HI) << 32);
                out[3] += (int64_t)(w(E_FF_LO) | w(E_FF_HI) << 32);
                out[4] += (int64_t)w(E_HACK_REDRAWS);
            }
            put(out, sizeof out);
            std::fflush(stdout);
            return 0;
        } else {
            die("unknown env command");
        }
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) die("usage: host_driver raw <rom> | env <config>");
    const std::string mode = argv[1];
    if (mode == "raw") return run_raw(argv[2]);
    if (mode == "env") return run_env(argv[2]);
    if (mode == "plant") {   // a deliberate out-of-bounds read: the sanitizer build must abort on it
        std::vector<uint8_t> row(std::atoi(argv[2]));
        volatile uint8_t v = row.data()[row.size()];
        return v;
    }
    die("unknown mode");
}
