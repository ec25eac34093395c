// mario_hip: batched Super Mario Bros env stepping on gfx950 — kernels and the C-ABI (include/mario_hip.h).
//
// One agent step of N envs is three kernels on the caller's stream:
//   k_step          4 lanes per env: sticky draw, K frames of 6502 + catch-up PPU, reward/done/info,
//                   hack frames, gray rendering of every frame into two alternating frame buffers; then, per
//                   wave, the 2-frame max + INTER_AREA of its envs' last frames (obs_tail)
//   k_reset         one lane per env: finished envs take a cached (level, no-op count) start state
//   k_stack         frame-stack shift, final_obs, reset observation
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <tuple>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/mario_hip.h"
#include "lane_kernels.hpp"
#include "replay.hpp"

using namespace mh;

namespace {

// Stage PRG and the CHR banks (32 KB + 8 KB each), the gray LUT and the decode table in LDS; every thread of
// the block must call this.
__device__ __forceinline__ void stage_rom(const RomArgs& R, uint8_t* s_rom, uint8_t* s_lut, uint32_t* s_dec) {
    const uint4* src = (const uint4*)R.rom;
    uint4* dst = (uint4*)s_rom;
    const int words = (0x8000 + R.n_chr * 0x2000) / 16;
    for (int i = threadIdx.x; i < words; i += blockDim.x) dst[i] = src[i];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) { s_lut[i] = R.lut[i]; s_dec[i] = kDecode.w[i]; }
    __syncthreads();
}

// Block-shared LDS of the emulator kernels: the cartridge, the gray LUT and per-lane render buffers.
#define ROM_LDS                                                     \
    __shared__ __attribute__((aligned(16))) uint8_t s_rom[0x8000 + MAX_CHR_BANKS * 0x2000]; \
    __shared__ uint8_t s_lut[256];                                  \
    __shared__ uint32_t s_dec[256];                                 \
    __shared__ uint32_t s_sp[LDS_SP_WORDS * LDS_LANES];              \
    __shared__ uint32_t s_gp[LDS_GP_REGION * LDS_LANES];

// Env slot of this thread within its block (0 .. LDS_LANES-1). Lanes l, l + ENVS_PER_WAVE, ... of a wave are
// the parts of one env: they run its console in lockstep (identical state, identical loads and stores of
// identical values) and share its LDS buffers; only the renderer and the sprite evaluation give them
// different work.
__device__ __forceinline__ int lane_slot() {
    return (int)(threadIdx.x >> 6) * ENVS_PER_WAVE + (int)(threadIdx.x & (ENVS_PER_WAVE - 1));
}
__device__ __forceinline__ uint8_t lane_part() {
    return (uint8_t)(((threadIdx.x & 63u) / ENVS_PER_WAVE) & (LANES_PER_ENV - 1));
}

__device__ __forceinline__ LaneCtx lane_ctx(const RomArgs& R, const uint8_t* s_rom, const uint8_t* s_lut,
                                            const uint32_t* s_dec, uint32_t* s_sp, uint32_t* s_gp, int slot) {
    return LaneCtx{make_cart(R, s_rom, s_dec), s_lut, s_sp + slot, s_gp + slot, lane_part()};
}

constexpr int EMU_THREADS = 64 * WAVES_PER_BLOCK;
#define EMU_BOUNDS __launch_bounds__(EMU_THREADS, EMU_WAVES_PER_SIMD)
// blocks of an emulator kernel over `count` envs
// Launch shape of an emulator kernel over `count` consoles on a GPU with `cus` compute units: blocks of up to
// WAVES_PER_BLOCK waves (one block per CU: its LDS). When count is too small to give every CU a full block, the
// blocks shrink (down to one wave) so that the waves spread over all CUs instead of sharing a few CUs' SIMDs.
struct EmuLaunch { dim3 grid, block; };
static inline EmuLaunch emu_launch(int count, int cus) {
    const int per_full_wave = ENVS_PER_WAVE * (cus > 0 ? cus : 1);
    int waves = (count + per_full_wave - 1) / per_full_wave;
    waves = waves < 1 ? 1 : waves > WAVES_PER_BLOCK ? WAVES_PER_BLOCK : waves;
    const int slots = waves * ENVS_PER_WAVE;
    return EmuLaunch{dim3((unsigned)((count + slots - 1) / slots)), dim3((unsigned)(64 * waves))};
}
// Launch shape of k_raw over `count` consoles: fewer consoles per wave (a power of two, cpw) where the count is too
// small to give every SIMD two waves of 16. A raw batch of 4,096 consoles is then 2,048 waves of 2 instead of 256
// waves of 16 (one per CU, three of its four SIMDs idle): a wave's iterations follow the union of its consoles'
// instruction streams and slice waits, so fewer consoles per wave also means fewer iterations per console, and
// the lanes a wave leaves idle would have had no SIMD to run on anyway. force > 0 sets cpw instead (one of 1, 2, 4,
// 8, 16: the MH_RAW_CONSOLES_PER_WAVE environment variable at mh_raw_create).
static inline EmuLaunch raw_launch(int count, int cus, int force, int& cpw) {
    const int target = 4 * EMU_WAVES_PER_SIMD * (cus > 0 ? cus : 1);   // waves that fill every SIMD
    cpw = ENVS_PER_WAVE;
    while (force <= 0 && cpw > 1 && (count + cpw / 2 - 1) / (cpw / 2) <= target) cpw /= 2;
    if (force > 0) cpw = force;
    const int waves = (count + cpw - 1) / cpw;
    int wpb = (waves + (cus > 0 ? cus : 1) - 1) / (cus > 0 ? cus : 1);   // waves per block: spread over the CUs
    wpb = wpb < 1 ? 1 : wpb > WAVES_PER_BLOCK ? WAVES_PER_BLOCK : wpb;
    return EmuLaunch{dim3((unsigned)((waves + wpb - 1) / wpb)), dim3((unsigned)(64 * wpb))};
}
// first console slot of this block (blocks of blockDim.x / 64 waves)
__device__ __forceinline__ uint32_t block_base() { return blockIdx.x * ((blockDim.x >> 6) * ENVS_PER_WAVE); }

// The new observation of a lane's env, output columns 21 g .. 21 g + 20 (g: the lane's part), into
// fresh[e * OBS_PIX + o]: the boot observation right after a reset, else INTER_AREA of the last frame,
// max-pooled with its partner frame (fastmario.cpp:377-386); `bits` as step_lane returns them; the output rows of
// NP row periods from p0 (7 rows from 20 source rows each). k_step runs it for all 12 periods once the wave's
// frame loop is over, on the frames the wave has just drawn, except in the waves that finish last, whose envs
// k_obs_late takes with a wave per period. The 4 lanes of an env take the 4
// column periods of the tables (AreaPeriod), so every lane runs the same code with constant taps and weights,
// and the wave reads every frame byte once: a load takes word 16 g + i of a source row for the 16 envs of each
// part (4 x 64 contiguous bytes). The loads of the next source row are in flight while a row is summed. The
// float operations and their order are area_pixel's. Not inlined, so that its registers stay out of the frame
// loop's allocation.
typedef __attribute__((address_space(1))) uint8_t gbyte;       // global memory, addressed as such
constexpr int kBufferWord3 = 0x00020000;   // buffer resource word 3 on gfx9: 32-bit raw (untyped) accesses
// a wave-uniform 64-bit value, as such (the builtin returns a signed int: each half is taken as unsigned before
// it is widened, so that the low half's bit 31 does not spread into the high half)
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (uint64_t)lo | (uint64_t)hi << 32;
}
template <int NP>
__device__ __attribute__((noinline)) void obs_tail(const uint8_t* gray_, uint32_t np_, uint8_t* fresh_,
                                                   const uint8_t* boot_obs, uint32_t e, uint32_t g, uint32_t bits,
                                                   int p0) {
    // The frames were stored by the env's lanes of this wave (streaming stores, and read-modify-writes whose loads
    // may have left lines in this CU's L1): wait for the stores, and drop the L1's lines, before reading them.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // the arguments a call passes in vector registers: the buffers and np are the kernel's, the same in every lane
    const gbyte* gray = (const gbyte*)uniform64((uint64_t)gray_);
    gbyte* fresh = (gbyte*)uniform64((uint64_t)fresh_);
    const uint32_t np = __builtin_amdgcn_readfirstlane(np_);
    p0 = __builtin_amdgcn_readfirstlane(p0);          // the same in every lane of both callers' waves
    gbyte* out = fresh + (size_t)e * OBS_PIX + 21 * g;
    if (bits & 4) {
        const uint8_t* b = boot_obs + (size_t)(bits >> 8) * OBS_PIX + 21 * g;
        for (int d = 7 * p0; d < 7 * (p0 + NP); d++)
            for (int q = 0; q < 21; q++) out[d * 84 + q] = b[d * 84 + q];
        return;
    }
    const bool pool = (bits & 1) != 0, swap = (bits & 2) != 0, all_pool = __all(pool);
    const size_t fb = (size_t)GRAY_PIX * np, rowb = (size_t)256 * np;   // bytes per frame buffer, per source row
    const uint32_t lo = (16 * g * np + e) * 4, step = 4 * np;           // word 16 g of the row, the next word
    uint32_t a0[16], b0[16], a1[16], b1[16];
    // Source row sy of both frame buffers as buffer resources (base: the row, size: the row's 256 np bytes, so
    // that no offset reaches past it), loaded with the lane's 32-bit word offsets: no 64-bit address per lane
    // and word. The loads are streaming (cache policy nt, aux bit 1): the frames are read once, and the
    // console state of the waves still in their frame loops stays in the L2.
    auto load = [&](int sy, uint32_t (&a)[16], uint32_t (&b)[16]) {
        const __amdgpu_buffer_rsrc_t r0 =
            __builtin_amdgcn_make_buffer_rsrc((void*)(gray + (size_t)sy * rowb), 0, (int)rowb, kBufferWord3);
        const __amdgpu_buffer_rsrc_t r1 =
            __builtin_amdgcn_make_buffer_rsrc((void*)(gray + fb + (size_t)sy * rowb), 0, (int)rowb, kBufferWord3);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            a[i] = __builtin_amdgcn_raw_buffer_load_b32(r0, (int)(lo + (uint32_t)i * step), 0, 2);
            b[i] = __builtin_amdgcn_raw_buffer_load_b32(r1, (int)(lo + (uint32_t)i * step), 0, 2);
        }
    };
    float acc[21];
#pragma unroll
    for (int q = 0; q < 21; q++) acc[q] = 0.f;
    auto row = [&](int sy, const uint32_t (&a)[16], const uint32_t (&b)[16]) {
        uint32_t ev[16], od[16];
        if (all_pool) {
#pragma unroll
            for (int i = 0; i < 16; i++) { ev[i] = max_even_bytes(a[i], b[i]); od[i] = max_odd_bytes(a[i], b[i]); }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t w = swap ? b[i] : a[i];
                ev[i] = pool ? max_even_bytes(a[i], b[i]) : w;
                od[i] = pool ? max_odd_bytes(a[i], b[i]) : w;
            }
        }
        float rs[21];
        obs_period_sums(ev, od, rs);
        obs_period_take(sy, rs, acc, [&](int dy, const float (&v)[21]) {
            gbyte* o = out + dy * 84;
#pragma unroll
            for (int q = 0; q < 21; q++) o[q] = round_sat(v[q]);
        });
    };
    // the 20 source rows of each of periods p0 .. p0 + NP - 1 (output rows 7 p .. 7 p + 6); acc is +0 at every
    // period's start
    for (int pi = 0; pi < NP; pi++) {
        const int sy0 = 20 * (p0 + pi);
        load(sy0, a0, b0);
#pragma nounroll
        for (int r = 0; r < 20; r += 2) {
            load(sy0 + r + 1, a1, b1);
            row(sy0 + r, a0, b0);
            if (r + 2 < 20) load(sy0 + r + 2, a0, b0);
            row(sy0 + r + 1, a1, b1);
        }
    }
}

__global__ void EMU_BOUNDS k_boot(BootArgs A) {
    ROM_LDS
    stage_rom(A.R, s_rom, s_lut, s_dec);
    const int slot = lane_slot();
    const int l = (int)(block_base() + slot);
    if (l < A.nl) boot_lane(A, lane_ctx(A.R, s_rom, s_lut, s_dec, s_sp, s_gp, slot), l);
}

__global__ void EMU_BOUNDS k_cache(CacheArgs A) {
    ROM_LDS
    stage_rom(A.R, s_rom, s_lut, s_dec);
    const int slot = lane_slot();
    const int ci = (int)(block_base() + slot);
    if (ci < A.nc) cache_lane(A, lane_ctx(A.R, s_rom, s_lut, s_dec, s_sp, s_gp, slot), ci);
}

// k_step's launch order for the next step. When k_step has more blocks than the GPU has CUs (past 32,768 envs on
// 256 CUs), a block that starts late and runs long holds the kernel's end, and a block holds its CU until its slowest
// env is done. A group's busy run (an area transition, a death, a level load) lasts several steps, so the last step's
// work predicts the next one's: the groups run in order of their slowest env's executed 6502 instructions in the
// last step, most first, and the cheap ones fill the CUs they free (longest-first list scheduling).
// k_work: each group's slowest env's executed instructions since the last call, from the env counters.
__global__ __launch_bounds__(LDS_LANES) void k_work(const uint32_t* ev, uint32_t np, int n, uint64_t* prev,
                                                    uint32_t* work) {
    const uint32_t e = blockIdx.x * LDS_LANES + threadIdx.x;
    uint32_t w = 0;
    if (e < (uint32_t)n) {
        auto counter = [&](int lo) {
            return (uint64_t)ev[(size_t)lo * np + e] | (uint64_t)ev[(size_t)(lo + 1) * np + e] << 32;
        };
        const uint64_t c = counter(E_INSTR_LO) - counter(E_FF_LO);
        const uint64_t d = c - prev[e];
        w = d > 0xffffffffull ? 0xffffffffu : (uint32_t)d;
        prev[e] = c;
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)w, off);
        w = o > w ? o : w;
    }
    __shared__ uint32_t wmax[LDS_LANES / 64];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = w;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < LDS_LANES / 64; k++) w = wmax[k] > w ? wmax[k] : w;
        work[blockIdx.x] = w;
    }
}
// k_order: one block; a bitonic sort of (work, ~index) keys in LDS (ties: the lower index first).
constexpr int ORDER_MAX = 8192;   // groups: MAX_ENVS / LDS_LANES fits
__global__ __launch_bounds__(1024) void k_order(const uint32_t* work, uint32_t* perm, int ng) {
    __shared__ uint64_t key[ORDER_MAX];
    int P = 1;
    while (P < ng) P <<= 1;
    for (int i = threadIdx.x; i < P; i += blockDim.x)
        key[i] = i < ng ? ((uint64_t)work[i] << 32 | (uint32_t)~(uint32_t)i) : 0ull;   // padding sorts last
    __syncthreads();
    for (int k = 2; k <= P; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < P; i += blockDim.x) {
                const int l = i ^ j;
                if (l > i) {
                    const uint64_t a = key[i], b = key[l];
                    if ((i & k) == 0 ? a < b : a > b) { key[i] = b; key[l] = a; }   // descending overall
                }
            }
            __syncthreads();
        }
    for (int i = threadIdx.x; i < ng; i += blockDim.x) perm[i] = ~(uint32_t)key[i];
}
static_assert(MAX_ENVS / LDS_LANES <= ORDER_MAX, "k_order holds every group");

__device__ __forceinline__ void step_block(const StepArgs& A, uint32_t base) {
    ROM_LDS
    stage_rom(A.R, s_rom, s_lut, s_dec);
    // The frame loop issues ahead of the observations of the waves that have finished it (on a SIMD, the two
    // waves' instructions are arbitrated by this priority first).
    __builtin_amdgcn_s_setprio(2);
    const int slot = lane_slot();
    const uint32_t e = base + (uint32_t)slot;
    const bool live = e < (uint32_t)A.n;
    uint32_t bits = 0;
    if (live) bits = step_lane(A, lane_ctx(A.R, s_rom, s_lut, s_dec, s_sp, s_gp, slot), e);
    if (!__any(live)) return;
    // The wave's ticket: its place in the order in which the waves finish their frame loops (a vector atomic
    // from one lane). The waves that finish last would hold the kernel's end with their observations; they
    // leave them to k_obs_late, which spreads an env's rows over 12 waves.
    uint32_t ticket = 0;
    if (__lane_id() == 0) ticket = atomicAdd(A.obs_order, 1u);
    ticket = (uint32_t)__builtin_amdgcn_readfirstlane(ticket);
    if (ticket >= A.obs_late_from && ticket < A.obs_late_to) {
        if (__lane_id() == 0) A.obs_order[1 + ticket - A.obs_late_from] = e;   // lane 0 holds the wave's first slot
    } else if (live) {
        __builtin_amdgcn_s_setprio(0);
        obs_tail<12>(A.gray, A.np, A.fresh, A.boot_obs, e, lane_part(), bits, 0);
    }
}

// base: the first env slot of the block's group (blocks of blockDim.x / 64 waves)
__global__ void EMU_BOUNDS k_step(StepArgs A) { step_block(A, block_base()); }
// k_step in the launch order of k_order: block b runs group perm[b]
__global__ void EMU_BOUNDS k_step_ordered(StepArgs A, const uint32_t* perm) {
    step_block(A, perm[blockIdx.x] * ((blockDim.x >> 6) * ENVS_PER_WAVE));
}

// The observations of the envs of the waves that finished k_step's frame loop last (obs_tail, one wave per
// (deferred wave, row period): 12 waves per env group instead of one), then k_step's counter back to 0.
struct ObsLateArgs {
    int n; uint32_t np; int waves;       // deferred waves (their first slots at order[1 ..])
    const uint32_t* ev;
    const uint8_t* gray; uint8_t* fresh; const uint8_t* boot_obs;
    uint32_t* order;
};
constexpr int OBS_LATE_MAX = 64;         // waves that may defer
__global__ void __launch_bounds__(256) k_obs_late(ObsLateArgs A) {
    if (blockIdx.x == 0 && threadIdx.x == 0) A.order[0] = 0;   // k_step is over: no ticket is taken any more
    const int u = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));   // (deferred wave u / 12, row period u % 12)
    if (u >= A.waves * 12) return;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t e = A.order[1 + u / 12] + (lane & (ENVS_PER_WAVE - 1));   // k_step's lanes: env slot, part
    if (e >= (uint32_t)A.n) return;
    const uint32_t pw = A.ev[(size_t)E_POOLED * A.np + e];
    const uint32_t bits = (pw & 3u) | (A.ev[(size_t)E_SHOWS_BOOT * A.np + e] ? 4u : 0u) |
                          A.ev[(size_t)E_LEVEL * A.np + e] << 8;
    obs_tail<1>(A.gray, A.np, A.fresh, A.boot_obs, e, lane / ENVS_PER_WAVE, bits, u % 12);
}

// A wave carries A.cpw consoles (raw_launch): its lanes l, l + 16, l + 32, l + 48 with l < cpw run console
// wave * cpw + l of the block; the others idle.
__global__ void EMU_BOUNDS k_raw(RawArgs A) {
    ROM_LDS
    stage_rom(A.R, s_rom, s_lut, s_dec);
    const int in_wave = (int)(threadIdx.x & (ENVS_PER_WAVE - 1));
    const int slot = (int)(threadIdx.x >> 6) * A.cpw + in_wave;
    const uint32_t e = blockIdx.x * ((blockDim.x >> 6) * (uint32_t)A.cpw) + (uint32_t)slot;
    if (in_wave < A.cpw && e < (uint32_t)A.n) raw_lane(A, lane_ctx(A.R, s_rom, s_lut, s_dec, s_sp, s_gp, slot), e);
}

// One wave of 64 envs per block: each lane draws its env's reset, then the wave copies the chosen cache
// consoles one env at a time with all 64 lanes.
__global__ void __launch_bounds__(64) k_reset(ResetArgs A) {
    const uint32_t e = blockIdx.x * 64 + threadIdx.x;
    const int ci = e < (uint32_t)A.n ? reset_lane(A, e) : -1;
    uint64_t m = __ballot(ci >= 0);
    while (m) {
        const int l = __builtin_ctzll(m);
        m &= m - 1;
        const uint32_t el = (uint32_t)__shfl((int)e, l);
        const int cl = __shfl(ci, l);
        copy_console_wave(Region{A.mem, A.sc, A.np, el}, Region{(uint8_t*)A.cmem, (uint32_t*)A.csc, A.ncp, (uint32_t)cl},
                          threadIdx.x, 64);
    }
}

// Observation of a reset-cache entry or a boot state: the boot observation, or the resized last frame.
struct SmallObsArgs {
    const uint8_t* gray; uint32_t stride;     // frame buffer of `stride` lanes, entry i in lane i
    const uint8_t* use_boot;                  // per entry (nullable): take boot_obs[level(i)]
    const uint8_t* boot_obs; int nk;          // boot observations [level * OBS_PIX]
    uint8_t* out; int count;                  // [i * OBS_PIX + o]
    const AreaTables* T;
};
__global__ void k_small_obs(SmallObsArgs A) {
    const int i = blockIdx.y;
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= A.count || o >= OBS_PIX) return;
    uint8_t v;
    if (A.use_boot && A.use_boot[i]) v = A.boot_obs[(size_t)(i / A.nk) * OBS_PIX + o];
    else v = area_pixel(Image{A.gray, A.stride, (uint32_t)i}, Image{}, false, o, A.T);
    A.out[(size_t)i * OBS_PIX + o] = v;
}

struct StackArgs {
    int n; uint32_t np; int K;
    uint8_t* obs; uint8_t* fin;   // [env][K][OBS_PIX]
    const int32_t* slot_env;      // env of each console slot
    const uint8_t* fresh;         // new observation of slot e at [e * OBS_PIX + o]
    const uint32_t* ev;
    const uint8_t* cobs;          // [ci * OBS_PIX + o]
    int mode;                     // 0 step, 1 reset
};
// Frame stack, final_obs, reset observation (fastmario.cpp:477-504). Block: 64 envs x 64 words of one
// frame; consecutive threads take consecutive words of one env.
__global__ void __launch_bounds__(256) k_stack(StackArgs A) {
    const uint32_t e0 = blockIdx.x * 64;   // env groups vary fastest: neighbouring workgroups read adjacent envs
    const int w0 = blockIdx.y * 64;        // word index within a frame (OBS_PIX / 4 = 1764 words)
    const int nw = OBS_PIX / 4;
    const size_t fw = (size_t)nw * A.K;   // words per env stack
    for (int idx = threadIdx.x; idx < 64 * 64; idx += 256) {
        const int j = idx >> 6, wl = idx & 63;
        const uint32_t e = e0 + j;
        const int w = w0 + wl;
        if (w >= nw || e >= (uint32_t)A.n) continue;
        const size_t env = (size_t)A.slot_env[e];
        uint32_t* st = (uint32_t*)A.obs + env * fw;
        const uint32_t ri = A.ev[(size_t)E_RESET_IDX * A.np + e];
        if (A.mode == 1) {
            for (int s = 0; s < A.K - 1; s++) st[(size_t)s * nw + w] = 0;
            st[(size_t)(A.K - 1) * nw + w] = ((const uint32_t*)A.cobs)[(size_t)ri * nw + w];
            continue;
        }
        const uint32_t fresh = ((const uint32_t*)A.fresh)[(size_t)e * nw + w];
        if (ri != 0xffffffffu) {
            uint32_t* fo = (uint32_t*)A.fin + env * fw;
            for (int s = 0; s < A.K - 1; s++) { fo[(size_t)s * nw + w] = st[(size_t)(s + 1) * nw + w]; st[(size_t)s * nw + w] = 0; }
            fo[(size_t)(A.K - 1) * nw + w] = fresh;
            st[(size_t)(A.K - 1) * nw + w] = ((const uint32_t*)A.cobs)[(size_t)ri * nw + w];
        } else {
            for (int s = 0; s < A.K - 1; s++) st[(size_t)s * nw + w] = st[(size_t)(s + 1) * nw + w];
            st[(size_t)(A.K - 1) * nw + w] = fresh;
        }
    }
}

// k_stack with 16-byte accesses, for obs / fin buffers (and the reset cache) 16-byte aligned: the same block
// (64 envs x 64 words of a frame), but a thread moves 4 consecutive words of one env per access (16 threads per
// env, 16 envs per pass, 4 passes), and reads the env's slot and reset index once per pass.
__global__ void __launch_bounds__(256) k_stack4(StackArgs A) {
    const uint32_t e0 = blockIdx.x * 64;
    const int w0 = blockIdx.y * 64;
    const int nw = OBS_PIX / 4;
    const size_t fw = (size_t)nw * A.K;   // words per env stack
    const int g = threadIdx.x & 15, w = w0 + 4 * g;   // this thread's 4 words: w .. w + 3 (nw is a multiple of 4)
    for (int pass = 0; pass < 4; pass++) {
        const int j = 16 * pass + (threadIdx.x >> 4);
        const uint32_t e = e0 + j;
        if (w >= nw || e >= (uint32_t)A.n) continue;
        const size_t env = (size_t)A.slot_env[e];
        uint4* st = (uint4*)((uint32_t*)A.obs + env * fw + w);          // frame s of the stack at st + s * nw / 4
        const uint32_t ri = A.ev[(size_t)E_RESET_IDX * A.np + e];
        const size_t fq = (size_t)nw / 4;
        if (A.mode == 1) {
            for (int s = 0; s < A.K - 1; s++) st[s * fq] = make_uint4(0, 0, 0, 0);
            st[(A.K - 1) * fq] = *(const uint4*)((const uint32_t*)A.cobs + (size_t)ri * nw + w);
            continue;
        }
        const uint4 fresh = *(const uint4*)((const uint32_t*)A.fresh + (size_t)e * nw + w);
        if (ri != 0xffffffffu) {
            uint4* fo = (uint4*)((uint32_t*)A.fin + env * fw + w);
            for (int s = 0; s < A.K - 1; s++) { fo[s * fq] = st[(s + 1) * fq]; st[s * fq] = make_uint4(0, 0, 0, 0); }
            fo[(A.K - 1) * fq] = fresh;
            st[(A.K - 1) * fq] = *(const uint4*)((const uint32_t*)A.cobs + (size_t)ri * nw + w);
        } else {
            // streaming stores: the stacks are read next by the caller, not by a kernel of this step
            // (0.453 -> 0.422 ms at 32,768 envs)
            typedef uint32_t v4u __attribute__((ext_vector_type(4)));
            v4u* sv = (v4u*)st;
            for (int s = 0; s < A.K - 1; s++) __builtin_nontemporal_store(sv[(s + 1) * fq], &sv[s * fq]);
            __builtin_nontemporal_store(*(const v4u*)&fresh, &sv[(A.K - 1) * fq]);
        }
    }
}

// slot_env (nullable): the output row of each console slot
__global__ void k_canon(const uint8_t* mem, const uint32_t* sc, uint32_t np, int n, const int32_t* slot_env, uint8_t* out) {
    const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < (uint32_t)n) canon_lane(mem, sc, np, e, out + (size_t)(slot_env ? slot_env[e] : (int32_t)e) * MH_CANON_BYTES);
}

// Lane-interleaved rows -> env-major (n x rows), slot e to row slot_env[e] (identity if null). Threads: x = slot,
// y = row.
__global__ void k_rows_out(const uint8_t* src, uint32_t np, int n, uint32_t rows, const int32_t* slot_env, uint8_t* out) {
    const uint32_t e = blockIdx.x * 64 + (threadIdx.x & 63);
    const uint32_t r = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (e >= (uint32_t)n || r >= rows) return;
    out[(size_t)(slot_env ? slot_env[e] : (int32_t)e) * rows + r] = src[(size_t)r * np + e];
}

// Frame buffer (4-pixel words, lane-interleaved) -> env-major 240x256 frames. Threads: x = env, y = word.
__global__ void k_frames_out(const uint8_t* src, uint32_t np, int n, uint8_t* out) {
    const uint32_t e = blockIdx.x * 64 + (threadIdx.x & 63);
    const uint32_t w = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (e >= (uint32_t)n || w >= GRAY_PIX / 4) return;
    const uint32_t v = ((const uint32_t*)src)[(size_t)w * np + e];
    for (int b = 0; b < 4; b++) out[(size_t)e * GRAY_PIX + 4 * w + b] = (uint8_t)(v >> (8 * b));
}

// Frame buffer of palette values -> env-major 240x256x3 RGB24 through a 64-entry RGB table (a palette value
// is taken & 63, as nes-py's screen). Threads: x = env, y = word of 4 pixels.
__global__ void k_frames_rgb(const uint8_t* src, uint32_t np, int n, const uint8_t* rgb64, uint8_t* out) {
    __shared__ uint8_t tab[64 * 3];
    for (int i = threadIdx.x; i < 64 * 3; i += blockDim.x) tab[i] = rgb64[i];
    __syncthreads();
    const uint32_t e = blockIdx.x * 64 + (threadIdx.x & 63);
    const uint32_t w = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (e >= (uint32_t)n || w >= GRAY_PIX / 4) return;
    const uint32_t v = ((const uint32_t*)src)[(size_t)w * np + e];
    uint8_t* o = out + ((size_t)e * GRAY_PIX + 4 * w) * 3;
    for (int b = 0; b < 4; b++) {
        const uint32_t c = (v >> (8 * b)) & 63u;
        o[3 * b] = tab[3 * c]; o[3 * b + 1] = tab[3 * c + 1]; o[3 * b + 2] = tab[3 * c + 2];
    }
}

// 240x256 gray images (env-major) -> 84x84.
__global__ void k_resize_images(const uint8_t* src, uint8_t* dst, int n, const AreaTables* T) {
    const int i = blockIdx.y;
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n || o >= OBS_PIX) return;
    dst[(size_t)i * OBS_PIX + o] = area_pixel(Image{src + (size_t)i * GRAY_PIX, 0, 0}, Image{}, false, o, T);
}

// ------------------------------------------------------------------ host side
thread_local std::string g_err;

static bool ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    g_err = std::string(what) + ": " + hipGetErrorString(e);
    return false;
}
#define CK(expr) do { if (!ok((expr), #expr)) return -1; } while (0)
#define CKN(expr) do { if (!ok((expr), #expr)) { return nullptr; } } while (0)

static uint32_t pad64(int n) { return (uint32_t)((n + 63) / 64 * 64); }

struct DevBufs {
    std::vector<void*> ptrs;
    template <class T> T* alloc(size_t count, bool& good) {
        void* p = nullptr;
        if (hipMalloc(&p, count * sizeof(T) + 16) != hipSuccess) { good = false; g_err = "hipMalloc failed"; return nullptr; }
        if (hipMemset(p, 0, count * sizeof(T) + 16) != hipSuccess) { good = false; g_err = "hipMemset failed"; }
        ptrs.push_back(p);
        return (T*)p;
    }
    ~DevBufs() { for (void* p : ptrs) (void)hipFree(p); }
};

// iNES NROM image -> 0x8000 PRG (16 KB mirrored) + 0x2000 CHR and name-table offsets (nes_core.hpp:66-87).
static bool load_cart(const uint8_t* d, int64_t n, std::vector<uint8_t>& img, uint16_t nt[4]) {
    if (!d || n < 16 || d[0] != 'N' || d[1] != 'E' || d[2] != 'S' || d[3] != 0x1a) { g_err = "not an iNES image"; return false; }
    int mapper = ((d[6] >> 4) & 0xf) | (d[7] & 0xf0);
    if (mapper != 0 || (d[6] & 0x6)) { g_err = "unsupported ROM (mapper / PRG-RAM / trainer)"; return false; }
    int banks = d[4];
    if (banks < 1 || banks > 2 || d[5] != 1) { g_err = "unsupported ROM (PRG/CHR size)"; return false; }
    if (n < 16 + 0x4000LL * banks + 0x2000) { g_err = "truncated ROM"; return false; }
    img.assign(0xa000, 0);
    for (int i = 0; i < 0x8000; i++) img[i] = d[16 + (i % (0x4000 * banks))];
    memcpy(img.data() + 0x8000, d + 16 + 0x4000 * banks, 0x2000);
    switch (d[6] & 0xB) {
        case 0: nt[0] = 0; nt[1] = 0; nt[2] = 0x400; nt[3] = 0x400; break;
        case 1: nt[0] = 0; nt[1] = 0x400; nt[2] = 0; nt[3] = 0x400; break;
        default: nt[0] = nt[1] = nt[2] = nt[3] = 0; break;
    }
    return true;
}

// ---- the PPO policy's input (the rollout harness's observation -> bf16 channels-last scaling)
// Observation stacks (n, k, 84, 84) u8 -> the bf16 (n, k, 84, 84) tensor in channels-last memory, i.e. element
// (b, c, h, w) at ((b * 84 + h) * 84 + w) * k + c, of value bf16(float(v) * float(1 / 255)) rounded to nearest
// even: what torch's float32 scaling followed by the bf16 cast gives. Thread: 4 consecutive pixels of one row of
// one image, all k channels (k u32 loads of 4 pixels, then 4 k bf16 values stored as 32-bit pairs).
__device__ __forceinline__ uint32_t bf16_rne(float f) {   // f finite and >= 0
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
template <int K>
__global__ void __launch_bounds__(256) k_policy_input(const uint8_t* obs, uint32_t* out, int64_t groups) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= groups) return;
    const int64_t b = t / (OBS_PIX / 4);
    const int r = (int)(t - b * (OBS_PIX / 4));          // pixel group in the image: pixels 4 r .. 4 r + 3
    const float s = (float)(1.0 / 255.0);
    uint32_t v[K];
#pragma unroll
    for (int c = 0; c < K; c++) v[c] = ((const uint32_t*)obs)[(b * K + c) * (OBS_PIX / 4) + r];
    // pixel q of the group: its K channels at out halves (4 r + q) * K .. + K - 1 of image b
    uint32_t* o = out + (b * OBS_PIX + 4 * r) * K / 2;
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
        for (int c = 0; c < K; c += 2) {
            const uint32_t lo = bf16_rne((float)((v[c] >> (8 * q)) & 0xffu) * s);
            const uint32_t hi = c + 1 < K ? bf16_rne((float)((v[c + 1] >> (8 * q)) & 0xffu) * s) : 0u;
            o[(q * K + c) / 2] = lo | hi << 16;
        }
    }
}

__global__ void __launch_bounds__(256) k_policy_input_k1(const uint8_t* obs, uint32_t* out, int64_t groups) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= groups) return;
    const float s = (float)(1.0 / 255.0);
    const uint32_t v = ((const uint32_t*)obs)[t];
    out[2 * t] = bf16_rne((float)(v & 0xffu) * s) | bf16_rne((float)((v >> 8) & 0xffu) * s) << 16;
    out[2 * t + 1] = bf16_rne((float)((v >> 16) & 0xffu) * s) | bf16_rne((float)(v >> 24) * s) << 16;
}

// ---- the PPO policy's first convolution (Nature CNN: 4 -> 32 channels, 8x8 kernel, stride 4, 84x84 -> 20x20)
// fused with the input scaling, the bias and the ReLU, on the matrix cores: relu(conv(bf16(obs / 255), W) + b)
// as an implicit GEMM, M = output pixels, N = 32 channels, K = 4 x 8 x 8 = 256 in the weight's own (ci, kh, kw)
// order, one v_mfma_f32_32x32x16_bf16 per 16 of K with float32 accumulation.
// A wave holds the whole weight matrix in registers (lane l: output channel l % 32, k = 16 s + 8 (l / 32) ..
// + 7 of step s) and walks tiles of 32 output pixels: lane l's A operand of step s is input row 4 oy + kh of
// channel ci, columns 4 ox .. 4 ox + 7 (two aligned u32 loads of 4 pixels) for pixel l % 32 of the tile,
// scaled to bf16 as mh_policy_input scales it. Output: the (n, 32, 20, 20) bf16 tensor in channels-last memory
// (pixel m's 32 channels at m * 32 ..), written as bf16(relu(acc + b)).
typedef __bf16 mh_bf16x8 __attribute__((ext_vector_type(8)));
typedef float mh_f32x16 __attribute__((ext_vector_type(16)));
constexpr int CONV1_OUT = 20 * 20;   // output pixels per image
__global__ void __launch_bounds__(256) k_policy_conv1(const uint8_t* obs, const uint16_t* w, const uint16_t* bias,
                                                      uint16_t* out, int64_t n) {
    const int l = threadIdx.x & 63;
    const int j = l & 31, kg = l >> 5;
    // B operand of the 16 steps: W[j][16 s + 8 kg .. + 7] (OIHW, K = ci * 64 + kh * 8 + kw)
    mh_bf16x8 wb[16];
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const uint4 q = *(const uint4*)(w + (size_t)j * 256 + 16 * s + 8 * kg);
        const uint32_t q4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 8; e++) wb[s][e] = __builtin_bit_cast(__bf16, (uint16_t)(q4[e >> 1] >> (16 * (e & 1))));
    }
    const float bj = __uint_as_float((uint32_t)bias[j] << 16);
    const float sc = (float)(1.0 / 255.0);
    const int64_t M = n * CONV1_OUT, tiles = (M + 31) / 32;
    const int64_t wave = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6, waves = (int64_t)gridDim.x * 4;
    for (int64_t t = wave; t < tiles; t += waves) {
        // this lane's A pixel: row l % 32 of the tile (clamped to the last pixel past the end; not stored)
        int64_t m = t * 32 + j;
        if (m >= M) m = M - 1;
        const int64_t b = m / CONV1_OUT;
        const int p = (int)(m - b * CONV1_OUT), oy = p / 20, ox = p - oy * 20;
        const uint8_t* img = obs + (size_t)b * 4 * OBS_PIX + (size_t)(4 * oy) * 84 + 4 * ox;
        uint32_t raw[16][2];
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const int k0 = 16 * s + 8 * kg, ci = k0 >> 6, kh = (k0 >> 3) & 7;
            const uint32_t* r = (const uint32_t*)(img + (size_t)ci * OBS_PIX + kh * 84);
            raw[s][0] = r[0];
            raw[s][1] = r[1];
        }
        mh_f32x16 acc = {};
#pragma unroll
        for (int s = 0; s < 16; s++) {
            mh_bf16x8 a;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t v = (raw[s][e >> 2] >> (8 * (e & 3))) & 0xffu;
                a[e] = __builtin_bit_cast(__bf16, (uint16_t)bf16_rne((float)v * sc));
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, wb[s], acc, 0, 0, 0);
        }
        // D: register v holds output pixel 8 (v / 4) + 4 kg + v % 4 of the tile, channel j
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int64_t mo = t * 32 + 8 * (v >> 2) + 4 * kg + (v & 3);
            if (mo < M) {
                const float y = acc[v] + bj;
                out[(size_t)mo * 32 + j] = (uint16_t)bf16_rne(y > 0.f ? y : 0.f);
            }
        }
    }
}

// ---- the PPO policy's second and third convolutions (Nature CNN: 32 -> 64 channels 4x4 stride 2, 20x20 -> 9x9;
// 64 -> 64 channels 3x3 stride 1, 9x9 -> 7x7), each fused with its bias and ReLU, on the matrix cores. Input and
// output are bf16 in channels-last memory (pixel m's channels at m * C ..), the weight is (CO, KS, KS, CI)
// (channels last), so K = (kh, kw, ci) and lane l's A operand of a step is 8 consecutive input channels of one
// input pixel (one 16-byte load). A wave holds one half of the output channels' weights in registers (lane l:
// channel 32 h + l % 32, K = 16 s + 8 (l / 32) .. + 7 of step s) and walks tiles of 32 output pixels; the two
// halves are the block's even and odd waves. Output: bf16(relu(sum + b)) with float32 accumulation.
template <int CI, int CO, int KS, int ST, int HI, int HO>
__global__ void __launch_bounds__(256) k_policy_conv(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                                     uint16_t* y, int64_t n) {
    static_assert(CI % 8 == 0 && CO == 64, "8-channel loads, two 32-channel halves");
    constexpr int K = KS * KS * CI, STEPS = K / 16, PIX = HO * HO;
    static_assert(K % 16 == 0, "whole MFMA steps");
    const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int j = l & 31, kg = l >> 5, half = wv & 1;
    const int ch = 32 * half + j;
    mh_bf16x8 wb[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; s++) {
        const uint4 q = *(const uint4*)(w + (size_t)ch * K + 16 * s + 8 * kg);
        const uint32_t q4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 8; e++) wb[s][e] = __builtin_bit_cast(__bf16, (uint16_t)(q4[e >> 1] >> (16 * (e & 1))));
    }
    const float bj = __uint_as_float((uint32_t)bias[ch] << 16);
    const int64_t M = n * PIX, tiles = (M + 31) / 32;
    const int64_t pair = (int64_t)blockIdx.x * 2 + (wv >> 1), pairs = (int64_t)gridDim.x * 2;
    // this lane's input pixel of tile t (past the end: a valid pixel, not stored)
    auto pixel = [&](int64_t t) {
        int64_t m = t * 32 + j;
        if (m >= M) m = M - 1;
        const int64_t b = m / PIX;
        const int p = (int)(m - b * PIX), oy = p / HO, ox = p - oy * HO;
        return x + ((size_t)(b * HI + ST * oy) * HI + ST * ox) * CI;
    };
    // the A operands of steps c .. c + CH - 1: 16-byte loads issued a chunk ahead of their MFMAs
    constexpr int CH = STEPS % 8 == 0 ? 8 : 6, NCH = STEPS / CH;
    static_assert(STEPS % CH == 0, "whole chunks");
    auto load_chunk = [&](const uint16_t* px, int c, uint4 (&q)[CH]) {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int k0 = 16 * (CH * c + i) + 8 * kg, kh = k0 / (KS * CI), kw = (k0 / CI) % KS, ci = k0 % CI;
            q[i] = *(const uint4*)(px + ((size_t)kh * HI + kw) * CI + ci);
        }
    };
    uint4 qa[CH], qb[CH];
    const uint16_t* px = pixel(pair);
    if (pair < tiles) load_chunk(px, 0, qa);
    for (int64_t t = pair; t < tiles; t += pairs) {
        mh_f32x16 acc = {};
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            uint4 (&cur)[CH] = (c & 1) ? qb : qa;
            uint4 (&nxt)[CH] = (c & 1) ? qa : qb;
            if (c + 1 < NCH) load_chunk(px, c + 1, nxt);
            else if (t + pairs < tiles) load_chunk(pixel(t + pairs), 0, nxt);   // the next tile's first chunk
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const uint32_t q4[4] = {cur[i].x, cur[i].y, cur[i].z, cur[i].w};
                mh_bf16x8 a;
#pragma unroll
                for (int e = 0; e < 8; e++) a[e] = __builtin_bit_cast(__bf16, (uint16_t)(q4[e >> 1] >> (16 * (e & 1))));
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, wb[CH * c + i], acc, 0, 0, 0);
            }
        }
        if constexpr (NCH & 1) {   // the next tile's first chunk landed in qb: move it to qa
#pragma unroll
            for (int i = 0; i < CH; i++) qa[i] = qb[i];
        }
        if (t + pairs < tiles) px = pixel(t + pairs);
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int64_t mo = t * 32 + 8 * (v >> 2) + 4 * kg + (v & 3);
            if (mo < M) {
                const float r = acc[v] + bj;
                y[(size_t)mo * CO + ch] = (uint16_t)bf16_rne(r > 0.f ? r : 0.f);
            }
        }
    }
}

}  // namespace

// compute units of a device (the emulator kernels' launch shape depends on it)
static int device_cus(int device) {
    hipDeviceProp_t prop;
    return hipGetDeviceProperties(&prop, device) == hipSuccess ? prop.multiProcessorCount : 0;
}

struct MhEnv {
    int n = 0, K = 4, nl = 0, nk = 1, nc = 0, device = 0, cus = 0;
    uint32_t np = 0, nlp = 0, ncp = 0;
    Cfg cfg{};
    DevBufs B;
    RomArgs R{};
    AreaTables* T = nullptr;
    uint8_t *mem = nullptr, *gray = nullptr, *fresh = nullptr;
    uint32_t* obs_order = nullptr;     // k_step's finish counter and the deferred waves (k_obs_late)
    // k_step's launch order (k_work, k_order), when it has more blocks than the GPU has CUs: null otherwise
    uint32_t *grp_work = nullptr, *grp_perm = nullptr;
    uint64_t* grp_prev = nullptr;      // each env's executed-instruction count at the last k_work
    int n_groups = 0;
    uint32_t *sc = nullptr, *ev = nullptr;
    uint8_t* snap_mem = nullptr;     // 2 snapshot slots of the live consoles (early-termination re-emulation)
    uint32_t* snap_sc = nullptr;
    uint8_t *boot_mem = nullptr, *boot_gray = nullptr, *boot_obs = nullptr;
    uint32_t* boot_sc = nullptr;
    int64_t *x0 = nullptr, *t0 = nullptr;
    uint8_t *cmem = nullptr, *cgray = nullptr, *cobs = nullptr, *cboot = nullptr;
    uint8_t* key_bank = nullptr;     // CHR bank of each (level, ROM) key
    int32_t* slot_env = nullptr;     // env of each console slot (slots grouped by (level, ROM) key)
    uint32_t *csc = nullptr;
    uint8_t* csnap_mem = nullptr;    // 2 snapshot slots of the cache consoles
    uint32_t* csnap_sc = nullptr;
    int64_t *cx = nullptr, *ct = nullptr;
    int32_t *clives = nullptr, *cdraws = nullptr;
    uint64_t *cframes = nullptr, *cinstr = nullptr, *cff = nullptr;
    uint32_t* cbad = nullptr;
    uint8_t *obs = nullptr, *fin = nullptr, *term = nullptr, *trunc = nullptr;
    float* rew = nullptr;
    int32_t *info = nullptr, *ep_len = nullptr;
    double* ep_ret = nullptr;
    // per-stage HIP event timing of mh_step_async (mh_timing / mh_timing_read)
    bool timing = false;
    std::vector<hipEvent_t> events;    // MH_STAGES + 1 events per timed step
    size_t timed_steps = 0;
    ~MhEnv() { for (hipEvent_t e : events) (void)hipEventDestroy(e); }

    ResetArgs reset_args(int all) const {
        return ResetArgs{n, np, cfg, nk, ncp, mem, sc, ev, cmem, csc, cx, ct, clives, cdraws, cboot,
                         cframes, cinstr, cff, cbad, all};
    }
    StackArgs stack_args(int mode) const { return StackArgs{n, np, K, obs, fin, slot_env, fresh, ev, cobs, mode}; }
};

// k_stack4 when the stacks (and the reset cache) allow 16-byte accesses, else k_stack
static void launch_stack(const MhEnv* h, hipStream_t s, int mode) {
    const dim3 grid(h->np / 64, (OBS_PIX / 4 + 63) / 64);
    const bool al = ((((uintptr_t)h->obs) | ((uintptr_t)h->fin) | ((uintptr_t)h->cobs)) & 15) == 0;
    if (al) hipLaunchKernelGGL(k_stack4, grid, dim3(256), 0, s, h->stack_args(mode));
    else hipLaunchKernelGGL(k_stack, grid, dim3(256), 0, s, h->stack_args(mode));
}

struct MhRaw {
    int n = 0, device = 0, cus = 0, cpw = 0;
    EmuLaunch lr{};                // k_raw's launch shape, with cpw consoles per wave (raw_launch)
    uint32_t np = 0;
    DevBufs B;
    RomArgs R{};
    uint8_t *mem = nullptr, *screen = nullptr, *bk_mem = nullptr;
    uint32_t *sc = nullptr, *bk_sc = nullptr, *bad = nullptr, *instr = nullptr, *ff = nullptr;
};

extern "C" {

const char* mh_last_error(void) { return g_err.c_str(); }

MhEnv* mh_create(const uint8_t* rom, int64_t rom_len, int n, const int* levels, const uint8_t* lut,
                 int skip, int max_steps, double sticky, int noop_max, int maxpool, int frame_stack,
                 const uint64_t* rng, int device) {
    return mh_create_roms(rom, &rom_len, 1, nullptr, n, levels, lut, skip, max_steps, sticky, noop_max, maxpool,
                          frame_stack, rng, device);
}

MhEnv* mh_create_roms(const uint8_t* roms, const int64_t* rom_lens, int n_roms, const int32_t* env_rom, int n,
                      const int* levels, const uint8_t* lut, int skip, int max_steps, double sticky, int noop_max,
                      int maxpool, int frame_stack, const uint64_t* rng, int device) {
    g_err.clear();
    if (n < 1 || skip < 1 || skip > MAX_SKIP || frame_stack < 1 || frame_stack > 16 || noop_max < 0 ||
        max_steps < 1 || !(sticky >= 0.0 && sticky <= 1.0) || !levels || !lut || !rng || !roms || !rom_lens ||
        n_roms < 1 || n_roms > MAX_CHR_BANKS || (n_roms > 1 && !env_rom)) {
        g_err = "invalid arguments";
        return nullptr;
    }
    if ((uint32_t)n > MAX_ENVS) { g_err = "too many envs (at most 979,648: console memory takes 32-bit offsets)"; return nullptr; }
    // the cartridge image: ROM 0's PRG, then the CHR of every ROM; the ROMs must agree on PRG and mirroring
    std::vector<uint8_t> img;
    uint16_t nt[4];
    int64_t off = 0;
    for (int r = 0; r < n_roms; r++) {
        std::vector<uint8_t> one;
        uint16_t ntr[4];
        if (!load_cart(roms + off, rom_lens[r], one, ntr)) return nullptr;
        off += rom_lens[r];
        if (r == 0) {
            img.assign(one.begin(), one.begin() + 0x8000);
            memcpy(nt, ntr, sizeof(nt));
        } else if (memcmp(img.data(), one.data(), 0x8000) != 0 || memcmp(nt, ntr, sizeof(nt)) != 0) {
            g_err = "per-env ROMs must share PRG and mirroring (rom_mode variants differ in CHR only)";
            return nullptr;
        }
        img.insert(img.end(), one.begin() + 0x8000, one.begin() + 0xa000);
    }
    for (int i = 0; i < n && env_rom; i++)
        if (env_rom[i] < 0 || env_rom[i] >= n_roms) { g_err = "env ROM index out of range"; return nullptr; }
    CKN(hipSetDevice(device));
    MhEnv* h = new MhEnv();
    auto fail = [&]() -> MhEnv* { delete h; return nullptr; };
    bool good = true;
    h->n = n; h->K = frame_stack; h->device = device; h->np = pad64(n); h->cus = device_cus(device);
    h->cfg = Cfg{skip, max_steps, noop_max, maxpool ? 1 : 0, sticky};
    // distinct (level, ROM) keys in order of first appearance (levels: fastmario.cpp:584-593); a key has its
    // own boot state and reset-cache entries
    std::vector<int> lv, env_level(n);
    std::vector<uint8_t> key_bank;
    for (int i = 0; i < n; i++) {
        const int ri = env_rom ? env_rom[i] : 0;
        int li = -1;
        for (size_t k = 0; k < key_bank.size(); k++)
            if (lv[3 * k] == levels[3 * i] && lv[3 * k + 1] == levels[3 * i + 1] && lv[3 * k + 2] == levels[3 * i + 2] &&
                key_bank[k] == ri) li = (int)k;
        if (li < 0) {
            li = (int)key_bank.size();
            lv.insert(lv.end(), levels + 3 * i, levels + 3 * i + 3);
            key_bank.push_back((uint8_t)ri);
        }
        env_level[i] = li;
    }
    h->nl = (int)lv.size() / 3; h->nlp = pad64(h->nl);
    // Console slots grouped by key, ordered by (world, stage, area, ROM), envs of a key in index order: a wave then
    // holds envs of one level (one game code path) wherever the batch mixes levels, so its lanes diverge less.
    // State lives in slot order; actions, outputs, RAM and state dumps stay in env order (slot_env).
    std::vector<int32_t> slot_env(h->np, 0), env_slot(n);
    {
        std::vector<int> order(n);
        for (int i = 0; i < n; i++) order[i] = i;
        auto key_of = [&](int i) {
            const int k = env_level[i];
            return std::make_tuple(lv[3 * k], lv[3 * k + 1], lv[3 * k + 2], (int)key_bank[k], i);
        };
        std::sort(order.begin(), order.end(), [&](int a, int b) { return key_of(a) < key_of(b); });
        for (int s = 0; s < n; s++) { slot_env[s] = order[s]; env_slot[order[s]] = s; }
        for (uint32_t s = (uint32_t)n; s < h->np; s++) slot_env[s] = (int32_t)s;   // padding slots: never used
    }
    h->nk = noop_max + 1; h->nc = h->nl * h->nk; h->ncp = pad64(h->nc);
    auto& B = h->B;
    uint8_t* d_rom = B.alloc<uint8_t>(img.size(), good);
    uint8_t* d_lut = B.alloc<uint8_t>(256, good);
    h->T = B.alloc<AreaTables>(1, good);
    int* d_levels = B.alloc<int>(lv.size(), good);
    h->key_bank = B.alloc<uint8_t>(key_bank.size(), good);
    h->slot_env = B.alloc<int32_t>(h->np, good);
    h->mem = B.alloc<uint8_t>((size_t)MEM_ROWS * h->np, good);
    h->sc = B.alloc<uint32_t>((size_t)S_COUNT * h->np, good);
    h->ev = B.alloc<uint32_t>((size_t)E_COUNT * h->np, good);
    h->gray = B.alloc<uint8_t>((size_t)2 * GRAY_PIX * h->np, good);
    h->snap_mem = B.alloc<uint8_t>((size_t)2 * MEM_ROWS * h->np, good);
    h->snap_sc = B.alloc<uint32_t>((size_t)2 * S_COUNT * h->np, good);
    h->fresh = B.alloc<uint8_t>((size_t)OBS_PIX * h->np, good);
    h->obs_order = B.alloc<uint32_t>(1 + OBS_LATE_MAX, good);
    {
        const EmuLaunch ls = emu_launch(h->n, h->cus);
        if ((int)ls.grid.x > h->cus) {   // more than one block per CU: the launch order decides what runs last
            h->n_groups = (int)ls.grid.x;
            h->grp_work = B.alloc<uint32_t>(h->n_groups, good);
            h->grp_perm = B.alloc<uint32_t>(h->n_groups, good);
            h->grp_prev = B.alloc<uint64_t>(h->np, good);
        }
    }
    h->boot_mem = B.alloc<uint8_t>((size_t)MEM_ROWS * h->nlp, good);
    h->boot_sc = B.alloc<uint32_t>((size_t)S_COUNT * h->nlp, good);
    h->boot_gray = B.alloc<uint8_t>((size_t)GRAY_PIX * h->nlp, good);
    h->boot_obs = B.alloc<uint8_t>((size_t)OBS_PIX * h->nl, good);
    h->x0 = B.alloc<int64_t>(h->nl, good); h->t0 = B.alloc<int64_t>(h->nl, good);
    h->cmem = B.alloc<uint8_t>((size_t)MEM_ROWS * h->ncp, good);
    h->csc = B.alloc<uint32_t>((size_t)S_COUNT * h->ncp, good);
    h->cgray = B.alloc<uint8_t>((size_t)2 * GRAY_PIX * h->ncp, good);
    h->csnap_mem = B.alloc<uint8_t>((size_t)2 * MEM_ROWS * h->ncp, good);
    h->csnap_sc = B.alloc<uint32_t>((size_t)2 * S_COUNT * h->ncp, good);
    h->cobs = B.alloc<uint8_t>((size_t)OBS_PIX * h->nc, good);
    h->cboot = B.alloc<uint8_t>(h->nc, good);
    h->cx = B.alloc<int64_t>(h->nc, good); h->ct = B.alloc<int64_t>(h->nc, good);
    h->clives = B.alloc<int32_t>(h->nc, good); h->cdraws = B.alloc<int32_t>(h->nc, good);
    h->cframes = B.alloc<uint64_t>(h->nc, good); h->cinstr = B.alloc<uint64_t>(h->nc, good);
    h->cff = B.alloc<uint64_t>(h->nc, good);
    h->cbad = B.alloc<uint32_t>(h->nc, good);
    uint32_t* d_err = B.alloc<uint32_t>(1, good);
    if (!good) return fail();
    AreaTables T;
    area_tables(&T);
    if (!area_period_match(T)) { g_err = "INTER_AREA tables differ from the compiled-in periods"; return fail(); }
    // per-env words: level, RNG, lives = -1 (reset() installs the real start state)
    std::vector<uint32_t> ev((size_t)E_COUNT * h->np, 0);
    for (int i = 0; i < n; i++) {
        const size_t slot = (size_t)env_slot[i];
        auto w = [&](int k) -> uint32_t& { return ev[(size_t)k * h->np + slot]; };
        w(E_LEVEL) = (uint32_t)env_level[i];
        const uint64_t* r = rng + 6 * i;
        w(E_RNG_S3) = (uint32_t)(r[0] >> 32); w(E_RNG_S2) = (uint32_t)r[0];
        w(E_RNG_S1) = (uint32_t)(r[1] >> 32); w(E_RNG_S0) = (uint32_t)r[1];
        w(E_RNG_I3) = (uint32_t)(r[2] >> 32); w(E_RNG_I2) = (uint32_t)r[2];
        w(E_RNG_I1) = (uint32_t)(r[3] >> 32); w(E_RNG_I0) = (uint32_t)r[3];
        w(E_RNG_HAS32) = (uint32_t)r[4]; w(E_RNG_HALF) = (uint32_t)r[5];
        w(E_LIVES) = 0xffffffffu; w(E_SHOWS_BOOT) = 1; w(E_RESET_IDX) = 0xffffffffu;
    }
    if (!ok(hipMemcpy(d_rom, img.data(), img.size(), hipMemcpyHostToDevice), "upload rom") ||
        !ok(hipMemcpy(h->key_bank, key_bank.data(), key_bank.size(), hipMemcpyHostToDevice), "upload key banks") ||
        !ok(hipMemcpy(h->slot_env, slot_env.data(), slot_env.size() * 4, hipMemcpyHostToDevice), "upload slot map") ||
        !ok(hipMemcpy(d_lut, lut, 256, hipMemcpyHostToDevice), "upload lut") ||
        !ok(hipMemcpy(h->T, &T, sizeof(T), hipMemcpyHostToDevice), "upload tables") ||
        !ok(hipMemcpy(d_levels, lv.data(), lv.size() * sizeof(int), hipMemcpyHostToDevice), "upload levels") ||
        !ok(hipMemcpy(h->ev, ev.data(), ev.size() * 4, hipMemcpyHostToDevice), "upload env words"))
        return fail();
    h->R.rom = d_rom; h->R.lut = d_lut; h->R.n_chr = n_roms;
    h->R.nt_bits = 0;
    for (int i = 0; i < 4; i++) h->R.nt_bits |= (nt[i] ? 1u : 0u) << i;
    // boot every level, build the reset cache
    BootArgs ba{h->R, h->nl, h->nlp, d_levels, h->key_bank, h->boot_mem, h->boot_sc, h->boot_gray, h->x0, h->t0, d_err};
    const EmuLaunch lb = emu_launch(h->nl, h->cus);
    hipLaunchKernelGGL(k_boot, lb.grid, lb.block, 0, 0, ba);
    if (!ok(hipGetLastError(), "k_boot launch")) return fail();
    SmallObsArgs so{h->boot_gray, h->nlp, nullptr, nullptr, 1, h->boot_obs, h->nl, h->T};
    hipLaunchKernelGGL(k_small_obs, dim3((OBS_PIX + 255) / 256, h->nl), dim3(256), 0, 0, so);
    CacheArgs ca{h->R, h->cfg, h->key_bank, h->nl, h->nk, h->nc, h->nlp, h->ncp, h->boot_mem, h->boot_sc, h->x0, h->t0,
                 h->cmem, h->csc, h->cgray, h->csnap_mem, h->csnap_sc, h->cx, h->ct, h->clives, h->cdraws, h->cboot,
                 h->cframes, h->cinstr, h->cff, h->cbad};
    const EmuLaunch lc = emu_launch(h->nc, h->cus);
    hipLaunchKernelGGL(k_cache, lc.grid, lc.block, 0, 0, ca);
    if (!ok(hipGetLastError(), "k_cache launch")) return fail();
    SmallObsArgs co{h->cgray, h->ncp, h->cboot, h->boot_obs, h->nk, h->cobs, h->nc, h->T};
    hipLaunchKernelGGL(k_small_obs, dim3((OBS_PIX + 255) / 256, h->nc), dim3(256), 0, 0, co);
    if (!ok(hipDeviceSynchronize(), "boot / reset cache")) return fail();
    uint32_t err = 0;
    if (!ok(hipMemcpy(&err, d_err, 4, hipMemcpyDeviceToHost), "boot status")) return fail();
    if (err) { g_err = "level boot did not finish (the ROM never started a level)"; return fail(); }
    return h;
}

// A buffer the kernels may write: device memory of the env's GPU or pinned host memory, aligned to `align`.
static bool kernel_writable(const MhEnv* h, const void* p, uintptr_t align, const char* name) {
    if (((uintptr_t)p & (align - 1)) != 0) {
        g_err = std::string(name) + ": not aligned to " + std::to_string(align) + " bytes";
        return false;
    }
    hipPointerAttribute_t at;
    const hipError_t e = hipPointerGetAttributes(&at, p);
    (void)hipGetLastError();   // a refused host pointer must not surface as the error of a later launch
    const bool dev = e == hipSuccess && at.type == hipMemoryTypeDevice && at.device == h->device;
    const bool pinned = e == hipSuccess && (at.type == hipMemoryTypeHost || at.type == hipMemoryTypeManaged);
    if (!dev && !pinned) {
        g_err = std::string(name) + ": neither device memory of GPU " + std::to_string(h->device) +
                " nor pinned host memory (pageable host memory cannot be written by the kernels)";
        return false;
    }
    return true;
}

int mh_set_buffers(MhEnv* h, uint8_t* obs, uint8_t* fin, float* rew, uint8_t* term, uint8_t* trunc,
                   int32_t* info, double* ep_ret, int32_t* ep_len) {
    if (!h || !obs || !fin || !rew || !term || !trunc || !info || !ep_ret || !ep_len) { g_err = "null buffer"; return -1; }
    if (!ok(hipSetDevice(h->device), "hipSetDevice")) return -1;
    if (!kernel_writable(h, obs, 4, "obs") || !kernel_writable(h, fin, 4, "final_obs") ||
        !kernel_writable(h, rew, 4, "rew") || !kernel_writable(h, term, 1, "term") ||
        !kernel_writable(h, trunc, 1, "trunc") || !kernel_writable(h, info, 4, "info") ||
        !kernel_writable(h, ep_ret, 8, "ep_ret") || !kernel_writable(h, ep_len, 4, "ep_len"))
        return -1;
    h->obs = obs; h->fin = fin; h->rew = rew; h->term = term; h->trunc = trunc; h->info = info;
    h->ep_ret = ep_ret; h->ep_len = ep_len;
    return 0;
}

int mh_reset(MhEnv* h, void* stream) {
    if (!h || !h->obs) { g_err = "buffers not set"; return -1; }
    CK(hipSetDevice(h->device));
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_reset, dim3(h->np / 64), dim3(64), 0, s, h->reset_args(1));
    CK(hipGetLastError());
    launch_stack(h, s, 1);
    CK(hipGetLastError());
    return 0;
}

// Records event k of the current timed step (k = 0 .. MH_STAGES).
static int mark(MhEnv* h, hipStream_t s, int k) {
    if (!h->timing) return 0;
    size_t idx = h->timed_steps * (MH_STAGES + 1) + k;
    while (h->events.size() <= idx) {
        hipEvent_t e;
        CK(hipEventCreate(&e));
        h->events.push_back(e);
    }
    CK(hipEventRecord(h->events[idx], s));
    return 0;
}

int mh_step_async(MhEnv* h, const int64_t* d_actions, void* stream) {
    if (!h || !h->obs || !d_actions) { g_err = "buffers or actions not set"; return -1; }
    CK(hipSetDevice(h->device));
    hipStream_t s = (hipStream_t)stream;
    if (mark(h, s, 0)) return -1;
    // waves with live envs, and how many of the last to finish defer their observations
    const int waves = (h->n + ENVS_PER_WAVE - 1) / ENVS_PER_WAVE, late = std::min(waves, OBS_LATE_MAX);
    StepArgs sa{h->R, h->cfg, h->n, h->np, h->mem, h->sc, h->ev, h->gray, h->snap_mem, h->snap_sc, d_actions,
                h->rew, h->term, h->trunc, h->info, h->ep_ret, h->ep_len, h->key_bank, h->slot_env, h->fresh,
                h->boot_obs, h->obs_order, (uint32_t)(waves - late), (uint32_t)waves};
    const EmuLaunch ls = emu_launch(h->n, h->cus);
    if (h->grp_perm) {   // this step's launch order, from the last step's work
        hipLaunchKernelGGL(k_work, dim3((unsigned)h->n_groups), dim3(LDS_LANES), 0, s, h->ev, h->np, h->n,
                           h->grp_prev, h->grp_work);
        hipLaunchKernelGGL(k_order, dim3(1), dim3(1024), 0, s, h->grp_work, h->grp_perm, h->n_groups);
        hipLaunchKernelGGL(k_step_ordered, ls.grid, ls.block, 0, s, sa, (const uint32_t*)h->grp_perm);
    } else {
        hipLaunchKernelGGL(k_step, ls.grid, ls.block, 0, s, sa);
    }
    CK(hipGetLastError());
    if (mark(h, s, 1)) return -1;
    const ObsLateArgs la{h->n, h->np, late, h->ev, h->gray, h->fresh, h->boot_obs, h->obs_order};
    hipLaunchKernelGGL(k_obs_late, dim3((unsigned)((late * 12 + 3) / 4)), dim3(256), 0, s, la);
    CK(hipGetLastError());
    if (mark(h, s, 2)) return -1;
    hipLaunchKernelGGL(k_reset, dim3(h->np / 64), dim3(64), 0, s, h->reset_args(0));
    CK(hipGetLastError());
    if (mark(h, s, 3)) return -1;
    launch_stack(h, s, 0);
    CK(hipGetLastError());
    if (mark(h, s, 4)) return -1;
    if (h->timing) h->timed_steps++;
    return 0;
}

int mh_timing(MhEnv* h, int enable) {
    if (!h) return -1;
    h->timing = enable != 0;
    h->timed_steps = 0;
    // events for the first 128 timed steps now rather than inside the steps being timed: creating them
    // there cost ~1.5 ms per step of wall time in a 100-step run
    while (h->timing && h->events.size() < (size_t)128 * (MH_STAGES + 1)) {
        hipEvent_t e;
        CK(hipEventCreate(&e));
        h->events.push_back(e);
    }
    return 0;
}

int mh_timing_read(MhEnv* h, double* ms, int64_t* steps) {
    if (!h || !ms) return -1;
    CK(hipDeviceSynchronize());
    for (int k = 0; k < MH_STAGES; k++) ms[k] = 0.0;
    for (size_t t = 0; t < h->timed_steps; t++)
        for (int k = 0; k < MH_STAGES; k++) {
            float f = 0.f;
            CK(hipEventElapsedTime(&f, h->events[t * (MH_STAGES + 1) + k], h->events[t * (MH_STAGES + 1) + k + 1]));
            ms[k] += f;
        }
    if (steps) *steps = (int64_t)h->timed_steps;
    return 0;
}

int mh_step_wait(MhEnv* h, void* stream) {
    if (!h) return -1;
    CK(hipStreamSynchronize((hipStream_t)stream));
    return 0;
}

void mh_destroy(MhEnv* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    (void)hipDeviceSynchronize();
    delete h;
}

static int64_t sum_words(const MhEnv* h, int lo_word, bool wide) {
    std::vector<uint32_t> lo(h->np), hi(h->np, 0);
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    if (hipMemcpy(lo.data(), h->ev + (size_t)lo_word * h->np, h->np * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (wide && hipMemcpy(hi.data(), h->ev + (size_t)(lo_word + 1) * h->np, h->np * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    int64_t s = 0;
    for (int i = 0; i < h->n; i++) s += (int64_t)(lo[i] | ((uint64_t)hi[i] << 32));
    return s;
}
int64_t mh_frames(MhEnv* h) { return h ? sum_words(h, E_FRAMES_LO, true) : -1; }
int64_t mh_bad_ops(MhEnv* h) { return h ? sum_words(h, E_BAD, false) : -1; }
int64_t mh_instructions(MhEnv* h) { return h ? sum_words(h, E_INSTR_LO, true) : -1; }
int64_t mh_ff_instructions(MhEnv* h) { return h ? sum_words(h, E_FF_LO, true) : -1; }
int64_t mh_hack_redraws(MhEnv* h) { return h ? sum_words(h, E_HACK_REDRAWS, false) : -1; }
int mh_reemulations(MhEnv* h, int64_t* out) {
    if (!h || !out) { g_err = "null handle or buffer"; return -1; }
    for (int k = 0; k < 3; k++)
        if ((out[k] = sum_words(h, E_REEMU_ONE + k, false)) < 0) { g_err = "counter read failed"; return -1; }
    return 0;
}

int mh_env_ram(MhEnv* h, uint8_t* d_out, void* stream) {
    if (!h || !d_out) return -1;
    hipLaunchKernelGGL(k_rows_out, dim3(h->np / 64, 2048 / 4), dim3(256), 0, (hipStream_t)stream, h->mem, h->np, h->n,
                       2048u, (const int32_t*)h->slot_env, d_out);
    CK(hipGetLastError());
    return 0;
}
int mh_env_canon(MhEnv* h, uint8_t* d_out, void* stream) {
    if (!h || !d_out) return -1;
    hipLaunchKernelGGL(k_canon, dim3(h->np / 64), dim3(64), 0, (hipStream_t)stream, h->mem, h->sc, h->np, h->n,
                       (const int32_t*)h->slot_env, d_out);
    CK(hipGetLastError());
    return 0;
}
int mh_level_canon(MhEnv* h, uint8_t* d_out, void* stream) {
    if (!h || !d_out) return -1;
    hipLaunchKernelGGL(k_canon, dim3(h->nlp / 64), dim3(64), 0, (hipStream_t)stream, h->boot_mem, h->boot_sc, h->nlp, h->nl,
                       nullptr, d_out);
    CK(hipGetLastError());
    return 0;
}
int mh_level_obs(MhEnv* h, uint8_t* d_out, void* stream) {
    if (!h || !d_out) return -1;
    CK(hipMemcpyAsync(d_out, h->boot_obs, (size_t)OBS_PIX * h->nl, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return 0;
}
int mh_num_levels(MhEnv* h) { return h ? h->nl : -1; }

int64_t mh_state_bytes(void) { return (int64_t)MEM_ROWS + 4LL * S_COUNT; }
int64_t mh_env_bytes(MhEnv* h) {
    if (!h) return -1;
    int64_t per = 3LL * (MEM_ROWS + 4LL * S_COUNT) + 4LL * E_COUNT + 2LL * GRAY_PIX + OBS_PIX;
    return per * h->np / h->n;
}

MhRaw* mh_raw_create(const uint8_t* rom, int64_t rom_len, int n, int device) {
    g_err.clear();
    if (n < 1) { g_err = "invalid arguments"; return nullptr; }
    if ((uint32_t)n > MAX_ENVS) { g_err = "too many consoles (at most 979,648: console memory takes 32-bit offsets)"; return nullptr; }
    int force = 0;
    if (const char* f = getenv("MH_RAW_CONSOLES_PER_WAVE"); f && *f) {
        force = atoi(f);
        if (force != 1 && force != 2 && force != 4 && force != 8 && force != ENVS_PER_WAVE) {
            g_err = "MH_RAW_CONSOLES_PER_WAVE must be 1, 2, 4, 8 or 16";
            return nullptr;
        }
    }
    std::vector<uint8_t> img;
    uint16_t nt[4];
    if (!load_cart(rom, rom_len, img, nt)) return nullptr;
    CKN(hipSetDevice(device));
    MhRaw* h = new MhRaw();
    bool good = true;
    h->n = n; h->np = pad64(n); h->device = device; h->cus = device_cus(device);
    h->lr = raw_launch(n, h->cus, force, h->cpw);
    auto& B = h->B;
    uint8_t* d_rom = B.alloc<uint8_t>(0xa000, good);
    uint8_t* d_lut = B.alloc<uint8_t>(256, good);
    h->mem = B.alloc<uint8_t>((size_t)MEM_ROWS * h->np, good);
    h->bk_mem = B.alloc<uint8_t>((size_t)MEM_ROWS * h->np, good);
    h->sc = B.alloc<uint32_t>((size_t)S_COUNT * h->np, good);
    h->bk_sc = B.alloc<uint32_t>((size_t)S_COUNT * h->np, good);
    h->screen = B.alloc<uint8_t>((size_t)GRAY_PIX * h->np, good);
    h->bad = B.alloc<uint32_t>(h->np, good);
    h->instr = B.alloc<uint32_t>(h->np, good);
    h->ff = B.alloc<uint32_t>(h->np, good);
    if (!good) { delete h; return nullptr; }
    uint8_t ident[256];
    for (int i = 0; i < 256; i++) ident[i] = (uint8_t)i;
    if (!ok(hipMemcpy(d_rom, img.data(), 0xa000, hipMemcpyHostToDevice), "upload rom") ||
        !ok(hipMemcpy(d_lut, ident, 256, hipMemcpyHostToDevice), "upload lut")) { delete h; return nullptr; }
    h->R.rom = d_rom; h->R.lut = d_lut; h->R.n_chr = 1;
    h->R.nt_bits = 0;
    for (int i = 0; i < 4; i++) h->R.nt_bits |= (nt[i] ? 1u : 0u) << i;
    RawArgs ra{h->R, h->n, h->np, h->mem, h->sc, h->screen, nullptr, 0, h->bad, h->instr, h->ff, 1, h->cpw};
    hipLaunchKernelGGL(k_raw, h->lr.grid, h->lr.block, 0, 0, ra);
    if (!ok(hipDeviceSynchronize(), "raw power-on")) { delete h; return nullptr; }
    return h;
}
int mh_raw_frame(MhRaw* h, const uint8_t* d_buttons, int render, void* stream) {
    if (!h || !d_buttons) return -1;
    RawArgs ra{h->R, h->n, h->np, h->mem, h->sc, h->screen, d_buttons, render, h->bad, h->instr, h->ff, 0, h->cpw};
    hipLaunchKernelGGL(k_raw, h->lr.grid, h->lr.block, 0, (hipStream_t)stream, ra);
    CK(hipGetLastError());
    return 0;
}
int mh_raw_ram(MhRaw* h, uint8_t* d_out, void* stream) {
    if (!h || !d_out) return -1;
    hipLaunchKernelGGL(k_rows_out, dim3(h->np / 64, 2048 / 4), dim3(256), 0, (hipStream_t)stream, h->mem, h->np, h->n,
                       2048u, nullptr, d_out);
    CK(hipGetLastError());
    return 0;
}
int mh_raw_screen(MhRaw* h, uint8_t* d_out, void* stream) {
    if (!h || !d_out) return -1;
    hipLaunchKernelGGL(k_frames_out, dim3(h->np / 64, GRAY_PIX / 16), dim3(256), 0, (hipStream_t)stream, h->screen,
                       h->np, h->n, d_out);
    CK(hipGetLastError());
    return 0;
}
int mh_raw_screen_rgb(MhRaw* h, const uint8_t* d_rgb64, uint8_t* d_out, void* stream) {
    if (!h || !d_rgb64 || !d_out) { g_err = "null handle or buffer"; return -1; }
    hipLaunchKernelGGL(k_frames_rgb, dim3(h->np / 64, GRAY_PIX / 16), dim3(256), 0, (hipStream_t)stream, h->screen,
                       h->np, h->n, d_rgb64, d_out);
    CK(hipGetLastError());
    return 0;
}
int mh_raw_canon(MhRaw* h, uint8_t* d_out, void* stream) {
    if (!h || !d_out) return -1;
    hipLaunchKernelGGL(k_canon, dim3(h->np / 64), dim3(64), 0, (hipStream_t)stream, h->mem, h->sc, h->np, h->n, nullptr,
                       d_out);
    CK(hipGetLastError());
    return 0;
}
int mh_raw_backup(MhRaw* h, void* stream) {
    if (!h) return -1;
    CK(hipMemcpyAsync(h->bk_mem, h->mem, (size_t)MEM_ROWS * h->np, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    CK(hipMemcpyAsync(h->bk_sc, h->sc, (size_t)S_COUNT * h->np * 4, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return 0;
}
int mh_raw_restore(MhRaw* h, void* stream) {
    if (!h) return -1;
    CK(hipMemcpyAsync(h->mem, h->bk_mem, (size_t)MEM_ROWS * h->np, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    CK(hipMemcpyAsync(h->sc, h->bk_sc, (size_t)S_COUNT * h->np * 4, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return 0;
}
static int64_t raw_sum(MhRaw* h, uint32_t* d) {
    std::vector<uint32_t> v(h->np);
    if (hipDeviceSynchronize() != hipSuccess) return -1;
    if (hipMemcpy(v.data(), d, h->np * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    int64_t s = 0;
    for (int i = 0; i < h->n; i++) s += v[i];
    return s;
}
int64_t mh_raw_bad_ops(MhRaw* h) { return h ? raw_sum(h, h->bad) : -1; }
int64_t mh_raw_instructions(MhRaw* h) { return h ? raw_sum(h, h->instr) : -1; }
int64_t mh_raw_ff_instructions(MhRaw* h) { return h ? raw_sum(h, h->ff) : -1; }
void mh_raw_destroy(MhRaw* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    (void)hipDeviceSynchronize();
    delete h;
}

// mh_resize's tables: one copy per device, allocated on the device's first call and kept until the process ends.
static std::mutex g_tables_mu;
static std::map<int, AreaTables*> g_tables;

int mh_resize(const uint8_t* d_src, uint8_t* d_dst, int n, void* stream) {
    if (!d_src || !d_dst || n < 1 || n > MH_RESIZE_MAX_IMAGES) { g_err = "invalid arguments (n must be 1..65535)"; return -1; }
    int dev = 0;
    CK(hipGetDevice(&dev));
    AreaTables* d_T = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_tables_mu);
        auto it = g_tables.find(dev);
        if (it == g_tables.end()) {
            AreaTables T;
            area_tables(&T);
            CK(hipMalloc(&d_T, sizeof(T)));
            if (!ok(hipMemcpy(d_T, &T, sizeof(T), hipMemcpyHostToDevice), "upload tables")) { (void)hipFree(d_T); return -1; }
            g_tables[dev] = d_T;
        } else {
            d_T = it->second;
        }
    }
    hipLaunchKernelGGL(k_resize_images, dim3((OBS_PIX + 255) / 256, n), dim3(256), 0, (hipStream_t)stream, d_src, d_dst, n, d_T);
    CK(hipGetLastError());
    return 0;
}

// The policy entry points' buffers: memory of the current GPU (device, or pinned host memory it maps); anything
// else (pageable host memory, another GPU's memory) is refused before a kernel could fault on it.
static bool on_gpu(const void* p, const char* name) {
    int dev = 0;
    if (!ok(hipGetDevice(&dev), "hipGetDevice")) return false;
    hipPointerAttribute_t at;
    const hipError_t e = hipPointerGetAttributes(&at, p);
    (void)hipGetLastError();   // a refused pointer must not surface as the error of a later launch
    const bool good = e == hipSuccess && ((at.type == hipMemoryTypeDevice && at.device == dev) ||
                                          at.type == hipMemoryTypeHost || at.type == hipMemoryTypeManaged);
    if (!good) g_err = std::string(name) + ": not memory of GPU " + std::to_string(dev);
    return good;
}

int mh_policy_conv1(const uint8_t* d_obs, const void* d_w, const void* d_b, void* d_out, int64_t n, void* stream) {
    if (!d_obs || !d_w || !d_b || !d_out || n < 1) { g_err = "invalid arguments (n >= 1)"; return -1; }
    if ((((uintptr_t)d_obs) & 3) || (((uintptr_t)d_w) & 15) || (((uintptr_t)d_out) & 1) || (((uintptr_t)d_b) & 1)) {
        g_err = "obs must be 4-byte, weight 16-byte and bias / out 2-byte aligned";
        return -1;
    }
    if (!on_gpu(d_obs, "obs") || !on_gpu(d_w, "weight") || !on_gpu(d_b, "bias") || !on_gpu(d_out, "out")) return -1;
    int dev = 0, cus = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int64_t tiles = (n * CONV1_OUT + 31) / 32;
    const int64_t blocks = std::min<int64_t>((tiles + 3) / 4, (int64_t)cus * 8);   // persistent: tiles per wave
    hipLaunchKernelGGL(k_policy_conv1, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, d_obs,
                       (const uint16_t*)d_w, (const uint16_t*)d_b, (uint16_t*)d_out, n);
    CK(hipGetLastError());
    return 0;
}

int mh_policy_conv(const void* d_x, const void* d_w, const void* d_b, void* d_out, int64_t n, int layer, void* stream) {
    if (!d_x || !d_w || !d_b || !d_out || n < 1 || (layer != 2 && layer != 3)) {
        g_err = "invalid arguments (n >= 1, layer 2 or 3)";
        return -1;
    }
    if ((((uintptr_t)d_x) & 15) || (((uintptr_t)d_w) & 15) || (((uintptr_t)d_out) & 1) || (((uintptr_t)d_b) & 1)) {
        g_err = "input and weight must be 16-byte, bias and out 2-byte aligned";
        return -1;
    }
    if (!on_gpu(d_x, "input") || !on_gpu(d_w, "weight") || !on_gpu(d_b, "bias") || !on_gpu(d_out, "out")) return -1;
    int dev = 0, cus = 0;
    CK(hipGetDevice(&dev));
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int64_t pix = layer == 2 ? 81 : 49, tiles = (n * pix + 31) / 32;
    const int64_t blocks = std::min<int64_t>((tiles + 1) / 2, (int64_t)cus * 8);   // 2 tiles in flight per block
    hipStream_t s = (hipStream_t)stream;
    const uint16_t *x = (const uint16_t*)d_x, *w = (const uint16_t*)d_w, *b = (const uint16_t*)d_b;
    uint16_t* y = (uint16_t*)d_out;
    if (layer == 2) hipLaunchKernelGGL((k_policy_conv<32, 64, 4, 2, 20, 9>), dim3((unsigned)blocks), dim3(256), 0, s, x, w, b, y, n);
    else hipLaunchKernelGGL((k_policy_conv<64, 64, 3, 1, 9, 7>), dim3((unsigned)blocks), dim3(256), 0, s, x, w, b, y, n);
    CK(hipGetLastError());
    return 0;
}

int mh_policy_input(const uint8_t* d_obs, void* d_out, int64_t n, int k, void* stream) {
    if (!d_obs || !d_out || n < 1 || (k != 1 && k != 2 && k != 4 && k != 8)) {
        g_err = "invalid arguments (n >= 1, k in 1, 2, 4, 8)";
        return -1;
    }
    if ((((uintptr_t)d_obs) & 3) || (((uintptr_t)d_out) & 3)) { g_err = "obs and out must be 4-byte aligned"; return -1; }
    if (!on_gpu(d_obs, "obs") || !on_gpu(d_out, "out")) return -1;
    const int64_t groups = n * (OBS_PIX / 4);
    const dim3 grid((unsigned)((groups + 255) / 256));
    hipStream_t s = (hipStream_t)stream;
    uint32_t* o = (uint32_t*)d_out;
    if (k == 1) {   // one channel: two pixels per 32-bit word
        hipLaunchKernelGGL(k_policy_input_k1, grid, dim3(256), 0, s, d_obs, o, groups);
    } else if (k == 2) {
        hipLaunchKernelGGL(k_policy_input<2>, grid, dim3(256), 0, s, d_obs, o, groups);
    } else if (k == 4) {
        hipLaunchKernelGGL(k_policy_input<4>, grid, dim3(256), 0, s, d_obs, o, groups);
    } else {
        hipLaunchKernelGGL(k_policy_input<8>, grid, dim3(256), 0, s, d_obs, o, groups);
    }
    CK(hipGetLastError());
    return 0;
}

// ---- the allocation-free resize (mh_resize_noalloc)
// Its filter tables live in `scratch`, a file-scope device array statically initialised with the tables the
// compiler computes (kAreaTables, area_taps's double operations at compile time): every GPU the library runs on
// holds one copy, loaded with the code object, at its own address, until the process ends. No kernel writes it
// and every call only reads it, so calls on one GPU never race over it and a first call under stream capture
// records nothing but the resize. The first call on a device looks up that device's address of the array
// (hipGetSymbolAddress; the array's name in host code is only a host-side stand-in, not a device address); the
// first call in the process checks once that the compile-time tables are, bit for bit, the run-time tables that
// mh_resize copies to the device (area_tables()).
static_assert(sizeof(AreaTables) == 8736, "the scratch array holds 8,736 B on every GPU");
static __device__ __align__(256) AreaTables scratch[1] = {kAreaTables};
constexpr int MH_MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static int g_scratch_checked;                          // 0 not yet, 1 the tables match, -1 they differ
static AreaTables* g_scratch_tables[MH_MAX_DEVICES];   // the device address of `scratch`, per device

static AreaTables* scratch_tables() {
    int dev = 0;
    if (!ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= MH_MAX_DEVICES) { g_err = "device index beyond the allocation-free path's table"; return nullptr; }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_checked) {
        AreaTables host;
        area_tables(&host);
        g_scratch_checked = area_tables_equal(host, kAreaTables) ? 1 : -1;
    }
    if (g_scratch_checked < 0) { g_err = "compile-time INTER_AREA tables differ from the run-time ones"; return nullptr; }
    if (!g_scratch_tables[dev]) {
        void* p = nullptr;
        if (!ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return nullptr;
        g_scratch_tables[dev] = (AreaTables*)p;
    }
    return g_scratch_tables[dev];
}

int mh_resize_noalloc(const uint8_t* d_src, uint8_t* d_dst, int n, void* stream) {
    if (!d_src || !d_dst) { g_err = "null image buffer"; return -1; }
    if (n < 1 || n > MH_RESIZE_MAX_IMAGES) {
        g_err = "mh_resize_noalloc: n = " + std::to_string(n) + " images; one call takes 1 .. 65535";
        return -1;
    }
    hipStream_t s = (hipStream_t)stream;
    AreaTables* T = scratch_tables();
    if (!T) return -1;
    hipLaunchKernelGGL(k_resize_images, dim3((OBS_PIX + 255) / 256, n), dim3(256), 0, s, d_src, d_dst, n, (const AreaTables*)T);
    CK(hipGetLastError());
    return 0;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int mh_replay_add(uint8_t* frames, uint8_t* age, int16_t* act, float* rew, uint8_t* flags, int64_t* ptr,
                  uint8_t* new_ep, int n_envs, int capacity, int frame_bytes, int k, const uint8_t* obs,
                  const uint8_t* next_obs, const int64_t* action, const float* reward, const uint8_t* done,
                  const uint8_t* truncated, void* stream) {
    if (!frames || !age || !act || !rew || !flags || !ptr || !new_ep || !obs || !next_obs || !action || !reward ||
        !done || !truncated || n_envs < 1 || capacity < 2 || k < 1 || frame_bytes < 16 || frame_bytes % 16) {
        g_err = "invalid arguments"; return -1;
    }
    if (k > capacity) { g_err = "stack depth k exceeds the ring capacity"; return -1; }
    if (!aligned16(frames) || !aligned16(obs) || !aligned16(next_obs)) { g_err = "frame buffers must be 16-byte aligned"; return -1; }
    ReplayAddArgs A{ReplayRing{frames, age, act, rew, flags, ptr, new_ep, n_envs, capacity, (uint32_t)frame_bytes},
                    obs, next_obs, k, action, reward, done, truncated};
    hipLaunchKernelGGL(k_replay_add, dim3(n_envs), dim3(256), 0, (hipStream_t)stream, A);
    CK(hipGetLastError());
    return 0;
}

int mh_replay_gather(const uint8_t* frames, const uint8_t* age, const int16_t* act, const float* rew,
                     const uint8_t* flags, int n_envs, int capacity, int frame_bytes, int k, const int64_t* env,
                     const int64_t* pos, int batch, int n_step, const float* gamma_pow, uint8_t* obs,
                     uint8_t* next_obs, int64_t* action, float* reward, float* discount, float* terminal,
                     int64_t* steps, int32_t* err, void* stream) {
    if (!frames || !age || !act || !rew || !flags || !env || !pos || !gamma_pow || !obs || !next_obs || !action ||
        !reward || !discount || !terminal || !steps || !err || n_envs < 1 || capacity < 2 || k < 1 ||
        frame_bytes < 16 || frame_bytes % 16 || batch < 0 || n_step < 0) {
        g_err = "invalid arguments"; return -1;
    }
    // a stack reaches k - 1 slots back from its newest one: deeper than the ring it would wrap onto itself
    if (k > capacity) { g_err = "stack depth k exceeds the ring capacity"; return -1; }
    if (!aligned16(frames) || !aligned16(obs) || !aligned16(next_obs)) { g_err = "frame buffers must be 16-byte aligned"; return -1; }
    if (batch == 0) return 0;
    ReplayGatherArgs A{ReplayRing{(uint8_t*)frames, (uint8_t*)age, (int16_t*)act, (float*)rew, (uint8_t*)flags,
                                  nullptr, nullptr, n_envs, capacity, (uint32_t)frame_bytes},
                       k, n_step, batch, env, pos, gamma_pow, obs, next_obs, action, reward, discount, terminal,
                       steps, err};
    hipLaunchKernelGGL(k_replay_gather, dim3(batch), dim3(REPLAY_GATHER_THREADS), 0, (hipStream_t)stream, A);
    CK(hipGetLastError());
    return 0;
}

}  // extern "C"
