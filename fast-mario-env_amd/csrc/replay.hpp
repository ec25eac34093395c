// Frame-deduplicating replay ring on the device: the storage and batch assembly of the reference's
// FrameReplay (src/fast_mario_env/replay.py:43-145), for frame-stacked observations.
//
// Per env e a ring of C frame slots (E x C x FB bytes) with per-slot age (frames since the episode
// start, saturating at 255), action (int16), reward (f32) and flags (1 valid start, 2 done, 4 terminal).
// ptr[e] counts the slots ever written. Both kernels are HBM copies: one workgroup per env (add) or per
// output frame (gather), 16-byte accesses.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mh {

struct ReplayRing {
    uint8_t* frames;     // [e][slot][FB]
    uint8_t* age;        // [e][slot]
    int16_t* act;
    float* rew;
    uint8_t* flags;
    int64_t* ptr;        // [e]: slots written
    uint8_t* new_ep;     // [e]: the next add starts an episode (its obs frame is stored first)
    int E, C;
    uint32_t fb;         // bytes per frame, a multiple of 16
};

__device__ __forceinline__ int64_t ring_slot(int64_t q, int64_t C) { return ((q % C) + C) % C; }

struct ReplayAddArgs {
    ReplayRing R;
    const uint8_t* obs;        // (E, k, FB): the newest frame of env e at obs + (e k + k - 1) FB
    const uint8_t* next_obs;
    int k;
    const int64_t* action;
    const float* reward;
    const uint8_t* done;       // terminated | truncated
    const uint8_t* trunc;      // time-limit ends
};

// FrameReplay.add for env blockIdx.x (replay.py:62-95): a new episode first stores its obs frame (age 0),
// then the transition's action, reward and flags go to the slot of the frame it starts from, and its
// next frame is stored with that slot's age + 1.
__global__ void __launch_bounds__(256) k_replay_add(ReplayAddArgs A) {
    const ReplayRing& R = A.R;
    const int e = blockIdx.x;
    if (e >= R.E) return;
    const int64_t C = R.C, p0 = R.ptr[e];
    const bool ne = R.new_ep[e] != 0;
    const int64_t pn = p0 + (ne ? 1 : 0);                 // slot of the next frame
    const size_t fb = R.fb, env_row = (size_t)e * (size_t)C;
    const size_t src = ((size_t)e * A.k + (A.k - 1)) * fb;
    const uint4* so = (const uint4*)(A.obs + src);
    const uint4* sn = (const uint4*)(A.next_obs + src);
    uint4* dn = (uint4*)(R.frames + (env_row + ring_slot(pn, C)) * fb);
    uint4* dob = (uint4*)(R.frames + (env_row + ring_slot(p0, C)) * fb);
    for (uint32_t i = threadIdx.x; i < fb / 16; i += blockDim.x) {
        if (ne) dob[i] = so[i];
        dn[i] = sn[i];
    }
    __syncthreads();                                      // every thread has read ptr and new_ep
    if (threadIdx.x != 0) return;
    if (ne) { R.age[env_row + ring_slot(p0, C)] = 0; R.flags[env_row + ring_slot(p0, C)] = 0; }
    const size_t s = env_row + ring_slot(pn - 1, C);      // the slot the transition starts from
    const bool d = A.done[e] != 0, t = A.trunc[e] != 0;
    R.act[s] = (int16_t)A.action[e];
    R.rew[s] = A.reward[e];
    R.flags[s] = (uint8_t)(1 | (d ? 2 : 0) | ((d && !t) ? 4 : 0));
    const int a1 = (int)R.age[s] + 1;
    const size_t sn_slot = env_row + ring_slot(pn, C);
    R.age[sn_slot] = (uint8_t)(a1 < 255 ? a1 : 255);
    R.flags[sn_slot] = 0;
    R.ptr[e] = pn + 1;
    R.new_ep[e] = d ? 1 : 0;
}

struct ReplayGatherArgs {
    ReplayRing R;
    int k, n_step, B;
    const int64_t* env;        // (B) sampled env
    const int64_t* pos;        // (B) sampled absolute slot
    const float* gpow;         // gpow[i] = float32(gamma ** i), i = 0..n_step
    uint8_t* obs;              // (B, k, FB)
    uint8_t* next_obs;         // (B, k, FB)
    int64_t* action; float* reward; float* discount; float* terminal; int64_t* steps;
    int32_t* err;              // set to 1 when a sampled (env, pos) is out of range
};

// The n-step return of a sampled transition (replay.py:131-141), in the reference's float32 order:
// R += (alive * gamma^i) * rew, m += alive, term = max(term, alive * terminal), alive *= !done.
struct NStep { float R, term; int m; };
__device__ __forceinline__ NStep n_step_return(const ReplayRing& R, const ReplayGatherArgs& A, int64_t e, int64_t p) {
    float ret = 0.0f, alive = 1.0f, term = 0.0f;
    int m = 0;
    const size_t row = (size_t)e * (size_t)R.C;
    for (int i = 0; i < A.n_step; i++) {
        const size_t s = row + ring_slot(p + i, R.C);
        const uint8_t f = R.flags[s];
        ret = __fadd_rn(ret, __fmul_rn(__fmul_rn(alive, A.gpow[i]), R.rew[s]));
        m += alive != 0.0f;
        const float tv = __fmul_rn(alive, (f & 4) ? 1.0f : 0.0f);
        term = term > tv ? term : tv;
        alive = __fmul_rn(alive, (f & 2) ? 0.0f : 1.0f);
    }
    return NStep{ret, term, m};
}

// Batch assembly (replay.py:99-106 and 143-145): workgroup (b, j) writes frame j of obs (j < k) or of
// next_obs (j >= k) of sample b: the ring frame (q - off) mod C, or zeros where off exceeds the age of the
// stack's newest slot (before the episode start). q = pos (obs) or pos + m (next_obs), off = k-1 .. 0.
__global__ void __launch_bounds__(128) k_replay_gather(ReplayGatherArgs A) {
    const ReplayRing& R = A.R;
    const int b = blockIdx.x, j = blockIdx.y;
    if (b >= A.B || j >= 2 * A.k) return;
    const int64_t e = A.env[b], p = A.pos[b];
    const bool bad = e < 0 || e >= R.E || p < 0;
    const NStep ns = bad ? NStep{0.0f, 0.0f, 0} : n_step_return(R, A, e, p);
    const bool nxt = j >= A.k;
    const int jj = nxt ? j - A.k : j, off = A.k - 1 - jj;
    const int64_t q = p + (nxt ? ns.m : 0);
    const size_t fb = R.fb, row = bad ? 0 : (size_t)e * (size_t)R.C;
    const bool keep = !bad && off <= (int)R.age[row + ring_slot(q, R.C)];
    const uint4* src = (const uint4*)(R.frames + (row + ring_slot(q - off, R.C)) * fb);
    uint4* dst = (uint4*)((nxt ? A.next_obs : A.obs) + ((size_t)b * A.k + jj) * fb);
    const uint4 z = make_uint4(0, 0, 0, 0);
    for (uint32_t i = threadIdx.x; i < fb / 16; i += blockDim.x) dst[i] = keep ? src[i] : z;
    if (j != 0 || threadIdx.x != 0) return;
    if (bad) *A.err = 1;                                  // every writer stores 1
    A.action[b] = bad ? 0 : (int64_t)R.act[row + ring_slot(p, R.C)];
    A.reward[b] = ns.R;
    A.steps[b] = ns.m;
    A.terminal[b] = ns.term;
    A.discount[b] = __fmul_rn(A.gpow[ns.m], 1.0f - ns.term);
}

}  // namespace mh
