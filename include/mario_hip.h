/* mario_hip: batched Super Mario Bros env stepping on one AMD MI355X (gfx950) — C ABI.
 *
 * This is the drop-in boundary for the hot path. It replaces the reference's CPU C-ABI
 * (csrc/fastmario.cpp:562-674, bound by ctypes in src/fast_mario_env/_native.py:30-60) and its GPU
 * launch path (src/fast_mario_env/cuda/vec_env.py:350-393 + cuda/cujit.py:157-178) with one library:
 * the same create / set_buffers / reset / step_async / step_wait / destroy life cycle, but every
 * per-env buffer lives in HBM and every call is queued on the caller's HIP stream.
 *
 * Conventions
 *   - Plain C types only. `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *   - Output buffers are device pointers owned by the caller (e.g. torch tensors); the library
 *     writes them in place. Internal state (consoles, frame buffers, reset cache) is owned by the library.
 *   - Functions returning int return 0 on success and -1 on failure; creators return NULL on
 *     failure. mh_last_error() then returns a message (thread-local, valid until the next call).
 *   - One host thread drives one handle. Calls on one stream are ordered; no call blocks except
 *     mh_step_wait and the query functions that copy results to the host.
 */
#ifndef MARIO_HIP_H
#define MARIO_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct MhEnv MhEnv;
typedef struct MhRaw MhRaw;

#define MH_OBS_HW 84
#define MH_INFO_FIELDS 10   /* x_pos flag_get life score time world stage coins y_pos status */
#define MH_CANON_BYTES 4464 /* canonical console-state dump, layout shared with the CPU checker */

/* Last error message of this thread ("" if none). */
const char* mh_last_error(void);

/* Creates N envs and boots every distinct level on the GPU (power-on + title sequence), then
 * builds the no-op reset cache (one console per (level, k), k = 0..noop_max).
 * Replaces fm_create (fastmario.cpp:566-601) and CudaVecEnv.__init__ (vec_env.py:247-347).
 *   rom/rom_len   iNES image (NROM only), host memory
 *   levels        3*n ints (world, stage, area) per env, host memory
 *   lut           256 bytes, palette value -> gray, host memory
 *   rng           6*n u64 per env: numpy PCG64 (state_hi, state_lo, inc_hi, inc_lo, has_uint32, uinteger)
 *   skip 1..16, frame_stack 1..16, maxpool 0/1, sticky in [0, 1], noop_max >= 0, max_steps >= 1,
 *   1 <= n <= 979648 (the console memory is addressed with 32-bit offsets).
 * Blocks until construction is finished. */
MhEnv* mh_create(const uint8_t* rom, int64_t rom_len, int n, const int* levels, const uint8_t* lut,
                 int skip, int max_steps, double sticky, int noop_max, int maxpool, int frame_stack,
                 const uint64_t* rng, int device);

/* mh_create with a ROM per env: the per-env rom_mode that CudaVecEnv refuses (vec_env.py:250-269) and
 * FastVecEnv takes once per instance (env.py:113-160, rom.py:46-61). The ROMs are the rom_mode variants
 * of one game: they must share PRG and mirroring (their CHR differs), at most 4.
 *   roms          the n_roms iNES images back to back, host memory; rom_lens their sizes
 *   env_rom       n ints, the ROM index of each env (NULL: every env on ROM 0)
 * Each distinct (level, ROM) gets its own boot state and reset-cache entries. */
MhEnv* mh_create_roms(const uint8_t* roms, const int64_t* rom_lens, int n_roms, const int32_t* env_rom, int n,
                      const int* levels, const uint8_t* lut, int skip, int max_steps, double sticky, int noop_max,
                      int maxpool, int frame_stack, const uint64_t* rng, int device);

/* Output buffers (caller-owned). Replaces fm_set_buffers (fastmario.cpp:603-609).
 *   obs, fin  n * frame_stack * 84 * 84 u8 (stacked observations; final stack of finished episodes)
 *   rew       n f32;  term, trunc  n u8 (0/1);  info  n * 10 i32
 *   ep_ret    n f64;  ep_len  n i32 (written only for envs whose episode ended this step)
 * Each must be device memory of the env's GPU (or pinned / managed host memory) and aligned to its element
 * size, obs and fin to 4 bytes (the frame stack is written in 32-bit words). Pageable host memory, memory
 * of another GPU and misaligned buffers are refused (-1), where the reference's CPU path takes host arrays. */
int mh_set_buffers(MhEnv* h, uint8_t* obs, uint8_t* fin, float* rew, uint8_t* term, uint8_t* trunc,
                   int32_t* info, double* ep_ret, int32_t* ep_len);

/* Reset every env (no-op starts drawn from each env's PCG64 stream). Replaces fm_reset. */
int mh_reset(MhEnv* h, void* stream);

/* Queue one agent step of every env; d_actions: n i64 device pointer (values 0..6).
 * Replaces fm_step_async (fastmario.cpp:611-616) / CudaVecEnv.step (vec_env.py:367-373). */
int mh_step_async(MhEnv* h, const int64_t* d_actions, void* stream);

/* Wait for queued work on `stream`. Replaces fm_step_wait (fastmario.cpp:617). */
int mh_step_wait(MhEnv* h, void* stream);

void mh_destroy(MhEnv* h);

/* Per-stage timing of mh_step_async with HIP events recorded on the step's own stream (no counterpart
 * in the reference; used by the benchmark). Stages: 0 k_step (emulation, render, and the max-pool +
 * INTER_AREA observation of most envs), 1 k_obs_late (the observation of the envs of the waves that finish
 * k_step last), 2 k_reset, 3 k_stack. mh_timing(h, 1) clears and starts
 * recording; mh_timing_read synchronizes and returns the summed milliseconds per stage and the number
 * of timed steps. */
#define MH_STAGES 4
int mh_timing(MhEnv* h, int enable);
int mh_timing_read(MhEnv* h, double* ms, int64_t* steps);

/* Counters summed over envs (synchronizing). Replace fm_frames / fm_bad_ops (fastmario.cpp:619-628).
 * frames counts every emulated NES frame the reference CPU path emulates (hack frames and
 * early-termination re-renders included); instructions counts retired 6502 instructions. */
int64_t mh_frames(MhEnv* h);
int64_t mh_bad_ops(MhEnv* h);
int64_t mh_instructions(MhEnv* h);
/* Of mh_instructions, those the exact sprite-0 poll-loop fast-forward retired without executing them (the
 * reference executes each; its FM_PROF counter prof_cpu_instr, nes_core.hpp:1195, counts both kinds). */
int64_t mh_ff_instructions(MhEnv* h);
/* Early-termination re-emulations so far, by kind (synchronizing): out[0] an episode end at frame
 * last < K-1 re-ran frame last alone, out[1] it re-ran the max-pool partner last-1 as well (the two
 * branches of fastmario.cpp:351-362), out[2] of all of these, the ends at frame K-2 under max-pool. */
int mh_reemulations(MhEnv* h, int64_t* out);
/* Hack frames run a second time so far (synchronizing). The hack frames after a drawn agent frame
 * (fastmario.cpp:297-308 with render on) run undrawn, each from a snapshot; the one that ends the busy run
 * runs again from its snapshot, drawn. Frames and instructions count it once, as the reference does.
 * No counterpart in the reference (it draws every hack frame): a measure of how often this path runs. */
int64_t mh_hack_redraws(MhEnv* h);

/* RAM of every env into d_out (n * 2048 u8, device). Replaces fm_env_ram (fastmario.cpp:630). */
int mh_env_ram(MhEnv* h, uint8_t* d_out, void* stream);
/* Canonical console state of every env (n * MH_CANON_BYTES u8, device); level boot states
 * (n_levels * MH_CANON_BYTES) and boot observations (n_levels * 84 * 84). */
int mh_env_canon(MhEnv* h, uint8_t* d_out, void* stream);
int mh_level_canon(MhEnv* h, uint8_t* d_out, void* stream);
int mh_level_obs(MhEnv* h, uint8_t* d_out, void* stream);
int mh_num_levels(MhEnv* h);

/* Bytes of console state per env (replaces fm_state_bytes) and device bytes per env. */
int64_t mh_state_bytes(void);
int64_t mh_env_bytes(MhEnv* h);

/* ---- raw consoles: frame stepping without the env layer (replaces fm_raw_*, fastmario.cpp:651-673) */
/* 1 <= n <= 979648 consoles (32-bit offsets into the console memory). The consoles run 1 to 16 per wave (the
   most that still give every SIMD two waves); MH_RAW_CONSOLES_PER_WAVE=1|2|4|8|16 in the environment at this
   call sets it instead (any other value: NULL, with mh_last_error()). Results do not depend on it. */
MhRaw*  mh_raw_create(const uint8_t* rom, int64_t rom_len, int n, int device);
/* one frame of every console; d_buttons: n u8 device pointer; render != 0 draws the screen */
int     mh_raw_frame(MhRaw* h, const uint8_t* d_buttons, int render, void* stream);
int     mh_raw_ram(MhRaw* h, uint8_t* d_out, void* stream);        /* n * 2048 */
int     mh_raw_screen(MhRaw* h, uint8_t* d_out, void* stream);     /* n * 240 * 256 palette values */
/* The screen as RGB24, n * 240 * 256 * 3 bytes, through the 64-entry RGB table d_rgb64 (device, 192 bytes;
   palette values taken & 63). Replaces reading fm_raw_screen (fastmario.cpp:665) and mapping it through
   the palette table of fm_palette (fastmario.cpp:632) on the host, which nes-py's RGB screen is. */
int     mh_raw_screen_rgb(MhRaw* h, const uint8_t* d_rgb64, uint8_t* d_out, void* stream);
int     mh_raw_canon(MhRaw* h, uint8_t* d_out, void* stream);      /* n * MH_CANON_BYTES */
int     mh_raw_backup(MhRaw* h, void* stream);
int     mh_raw_restore(MhRaw* h, void* stream);
int64_t mh_raw_bad_ops(MhRaw* h);
int64_t mh_raw_instructions(MhRaw* h);
int64_t mh_raw_ff_instructions(MhRaw* h);   /* of those, poll-loop fast-forwards (see mh_ff_instructions) */
void    mh_raw_destroy(MhRaw* h);

/* ---- helpers */
/* 240x256 gray images -> 84x84 INTER_AREA on the device (n images, device pointers, n <= 65535).
 * Replaces fm_resize_fast (fastmario.cpp:641-649). The first call on a device allocates that device's
 * filter tables (kept until the process ends). */
#define MH_RESIZE_MAX_IMAGES 65535
int mh_resize(const uint8_t* d_src, uint8_t* d_dst, int n, void* stream);

/* mh_resize without any device allocation: no counterpart in the reference. For callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The same
 * kernel and results as mh_resize; its filter tables (8,736 B) sit in a file-scope device array that is
 * statically initialised with them, which the library holds on every GPU it runs on until the process ends.
 * No call writes the array, so calls on one GPU, overlapping or not, never race over it, and a first call
 * made under stream capture enqueues nothing but the resize itself. At most MH_RESIZE_MAX_IMAGES images per
 * call; more, fewer than 1, or a null buffer is refused (-1). */
int mh_resize_noalloc(const uint8_t* d_src, uint8_t* d_dst, int n, void* stream);

/* ---- the PPO rollout harness's policy input
 * No counterpart in the reference's C ABI: the device step of its PPO trainer scales the observation with torch
 * (ppo/backends.py:127-162, ppo/model.py:13-38: obs.float() / 255 feeding a Nature CNN); this is that scaling
 * written for the bf16 channels-last input the harness's convolutions take.
 * d_obs: (n, k, 84, 84) uint8 stacks, contiguous; d_out: the (n, k, 84, 84) bf16 tensor in channels-last
 * memory (element (b, c, h, w) at ((b * 84 + h) * 84 + w) * k + c), of value bf16(float(v) * float(1 / 255))
 * rounded to nearest even. k in 1, 2, 4, 8; both pointers 4-byte aligned and memory of the current GPU (device
 * memory, or pinned host memory); -1 otherwise. The two layer entry points below check their pointers alike. */
int mh_policy_input(const uint8_t* d_obs, void* d_out, int64_t n, int k, void* stream);

/* The harness's first policy layer fused with that scaling: relu(conv(bf16(obs / 255), W) + b) for the Nature
 * CNN's first convolution (ppo/model.py:13-27: 4 -> 32 channels, 8x8 kernel, stride 4), on the matrix cores
 * with float32 accumulation. d_obs: (n, 4, 84, 84) uint8 stacks, contiguous, 4-byte aligned; d_w: the bf16
 * weight (32, 4, 8, 8) contiguous, 16-byte aligned; d_b: the bf16 bias (32); d_out: the (n, 32, 20, 20) bf16
 * tensor in channels-last memory (pixel m's 32 channels at m * 32 ..), each value bf16(relu(sum + b)). */
int mh_policy_conv1(const uint8_t* d_obs, const void* d_w, const void* d_b, void* d_out, int64_t n, void* stream);

/* The Nature CNN's second (layer 2: 32 -> 64 channels, 4x4 kernel, stride 2, 20x20 -> 9x9) or third (layer 3:
 * 64 -> 64 channels, 3x3, stride 1, 9x9 -> 7x7) convolution with its bias and ReLU (ppo/model.py:13-27), on the
 * matrix cores with float32 accumulation: d_x the bf16 (n, CI, H, H) input in channels-last memory and d_out the
 * bf16 (n, 64, HO, HO) output likewise, each value bf16(relu(sum + b)); d_w the bf16 weight as (64, KS, KS, CI)
 * (channels last), d_b the bf16 bias (64). d_x and d_w 16-byte aligned. */
int mh_policy_conv(const void* d_x, const void* d_w, const void* d_b, void* d_out, int64_t n, int layer, void* stream);

/* ---- frame-deduplicating replay ring (device storage owned by the caller)
 * The ring of FrameReplay (src/fast_mario_env/replay.py:43-60) for n_envs envs and `capacity` slots each,
 * all device memory, slot s of env e at index e * capacity + s:
 *   frames  u8  [n_envs][capacity][frame_bytes]   (16-byte aligned, frame_bytes a multiple of 16)
 *   age     u8  [n_envs][capacity]   frames since the episode start, saturating at 255
 *   act     i16 [n_envs][capacity]   rew f32 [n_envs][capacity]
 *   flags   u8  [n_envs][capacity]   1 valid transition start, 2 done, 4 terminal (done and not truncated)
 *   ptr     i64 [n_envs]             slots written so far
 *   new_ep  u8  [n_envs]             the next add starts an episode (1 initially) */

/* Both replay entry points require 2 <= capacity and 1 <= k <= capacity (-1 otherwise).
 * FrameReplay.add (replay.py:76-95): obs / next_obs are (n_envs, k, frame_bytes) stacks, of which only
 * the newest frame is stored (obs's only when new_ep is set); action i64, reward f32, done and truncated
 * u8, n_envs each. Updates ptr and new_ep on the device. */
int mh_replay_add(uint8_t* frames, uint8_t* age, int16_t* act, float* rew, uint8_t* flags, int64_t* ptr,
                  uint8_t* new_ep, int n_envs, int capacity, int frame_bytes, int k, const uint8_t* obs,
                  const uint8_t* next_obs, const int64_t* action, const float* reward, const uint8_t* done,
                  const uint8_t* truncated, void* stream);

/* Batch assembly of FrameReplay.sample (replay.py:99-106, 131-145) for `batch` sampled (env, pos): the
 * n-step return (gamma_pow[i] = float32(gamma ** i), i = 0..n_step), steps m, terminal, discount
 * gamma_pow[m] * (1 - terminal), the action at pos, and the zero-padded (k, frame_bytes) stacks ending at
 * pos (obs) and pos + m (next_obs). An (env, pos) outside the ring sets *err = 1 and yields zeros. */
int mh_replay_gather(const uint8_t* frames, const uint8_t* age, const int16_t* act, const float* rew,
                     const uint8_t* flags, int n_envs, int capacity, int frame_bytes, int k, const int64_t* env,
                     const int64_t* pos, int batch, int n_step, const float* gamma_pow, uint8_t* obs,
                     uint8_t* next_obs, int64_t* action, float* reward, float* discount, float* terminal,
                     int64_t* steps, int32_t* err, void* stream);

#ifdef __cplusplus
}
#endif
#endif
