// Frame-deduplicating replay ring on the device: the storage and batch assembly of the reference's
// FrameReplay (src/fast_mario_env/replay.py:43-145), for frame-stacked observations.
//
// Per env e a ring of C frame slots (E x C x FB bytes) with per-slot age (frames since the episode
// start, saturating at 255), action (int16), reward (f32) and flags (1 valid start, 2 done, 4 terminal).
// ptr[e] counts the slots ever written. Both kernels are HBM copies in 16-byte accesses.
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

// 16-byte word i of a sample's 2k output frames (obs stack, then next_obs stack): where it comes from in
// the env's ring (frame (q - off) mod C, or zeros before the episode start) and where it goes.
struct GatherView {
    const uint4* ring;     // the env's ring, frame s at ring + s nv
    uint4* obs; uint4* nxt;  // the sample's output stacks
    uint32_t nv, total, k, C, qo, qn;   // words per frame, 2k nv, stack depth, ring size, newest slots
    int age_o, age_n;      // ages of the newest slots
    __device__ __forceinline__ uint4 load(uint32_t i) const {
        const uint32_t ic = i < total ? i : 0u;                // past the end: an in-range word, not stored
        const uint32_t f = ic / nv, o = ic - f * nv;
        const bool second = f >= k;
        const uint32_t jj = second ? f - k : f, off = k - 1u - jj, qs = second ? qn : qo;
        const uint32_t slot = qs >= off ? qs - off : qs + C - off;   // (q - off) mod C, off < k <= C
        const uint4 w = ring[(size_t)slot * nv + o];
        return (int)off <= (second ? age_n : age_o) ? w : make_uint4(0, 0, 0, 0);
    }
    __device__ __forceinline__ void store(uint32_t i, uint4 w) const {
        if (i >= total) return;
        const uint32_t f = i / nv, o = i - f * nv;
        if (f >= k) nxt[(size_t)(f - k) * nv + o] = w;
        else obs[(size_t)f * nv + o] = w;
    }
};

// Batch assembly (replay.py:99-106 and 143-145), one 256-thread workgroup per sample b: every thread
// computes the sample's n-step return and the ages it needs (the same few addresses for all of them), then
// the workgroup copies the 2k frames, obs stack (q = pos) then next_obs stack (q = pos + m): frame j is the
// ring frame (q - off) mod C, off = k-1-j, or zeros where off exceeds the age of the stack's newest slot
// (before the episode start). Eight 16-byte loads are in flight per thread.
constexpr int REPLAY_GATHER_THREADS = 256;
__global__ void __launch_bounds__(REPLAY_GATHER_THREADS) k_replay_gather(ReplayGatherArgs A) {
    const ReplayRing& R = A.R;
    const int b = blockIdx.x;
    if (b >= A.B) return;
    const int64_t e = A.env[b], p = A.pos[b];
    const bool bad = e < 0 || e >= R.E || p < 0;
    const NStep ns = bad ? NStep{0.0f, 0.0f, 0} : n_step_return(R, A, e, p);
    const size_t fb = R.fb, row = bad ? 0 : (size_t)e * (size_t)R.C;
    const uint32_t C = (uint32_t)R.C;
    const uint32_t qo = bad ? 0u : (uint32_t)ring_slot(p, R.C), qn = bad ? 0u : (uint32_t)ring_slot(p + ns.m, R.C);
    const int age_o = bad ? -1 : (int)R.age[row + qo], age_n = bad ? -1 : (int)R.age[row + qn];
    const uint32_t nv = (uint32_t)(fb / 16), total = 2u * (uint32_t)A.k * nv;
    const GatherView G{(const uint4*)(R.frames + row * fb), (uint4*)A.obs + (size_t)b * A.k * nv,
                       (uint4*)A.next_obs + (size_t)b * A.k * nv, nv, total, (uint32_t)A.k, C, qo, qn, age_o, age_n};
    for (uint32_t i0 = threadIdx.x; i0 < total; i0 += 8 * REPLAY_GATHER_THREADS) {
        constexpr uint32_t T = REPLAY_GATHER_THREADS;
        const uint4 t0 = G.load(i0), t1 = G.load(i0 + T), t2 = G.load(i0 + 2 * T), t3 = G.load(i0 + 3 * T);
        const uint4 t4 = G.load(i0 + 4 * T), t5 = G.load(i0 + 5 * T), t6 = G.load(i0 + 6 * T), t7 = G.load(i0 + 7 * T);
        G.store(i0, t0); G.store(i0 + T, t1); G.store(i0 + 2 * T, t2); G.store(i0 + 3 * T, t3);
        G.store(i0 + 4 * T, t4); G.store(i0 + 5 * T, t5); G.store(i0 + 6 * T, t6); G.store(i0 + 7 * T, t7);
    }
    if (threadIdx.x != 0) return;
    if (bad) *A.err = 1;                                  // every writer stores 1
    A.action[b] = bad ? 0 : (int64_t)R.act[row + qo];
    A.reward[b] = ns.R;
    A.steps[b] = ns.m;
    A.terminal[b] = ns.term;
    A.discount[b] = __fmul_rn(A.gpow[ns.m], 1.0f - ns.term);
}

}  // namespace mh
