// Host build of the device sources (test infrastructure only; see tests/hostbuild/host_driver.cpp).
//
// The device headers (fast-mario-env_amd/csrc/{nes_device,env_device,lane_kernels}.hpp) include
// <hip/hip_runtime.h>; with -I tests/hostbuild this file is found instead, so the same source compiles as
// plain x86 C++ for a wave of ONE lane per env (MH_LANES_PER_ENV=1): a wave vote over one lane is the lane's
// own value, the wave barrier and fences order nothing, and the two AMDGPU byte instructions the code uses
// are written out from their ISA definitions. It exists so that the device code can run under
// AddressSanitizer and UndefinedBehaviorSanitizer against the golden traces.
#pragma once
#include <stdint.h>
#include <string.h>

#define __device__
#define __host__
#define __global__
#define __constant__
#define __forceinline__ inline __attribute__((always_inline))
// host memory has one address space
#define MH_SCALAR_CONST
#define MH_GLOBAL

// a one-lane wave
static inline unsigned __lane_id() { return 0u; }
static inline uint64_t __ballot(int p) { return p ? 1ull : 0ull; }
static inline int __any(int p) { return p != 0; }
static inline int __all(int p) { return p != 0; }
static inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
// a one-lane wave's first active lane is the lane itself; like the device builtin, it takes and returns a
// signed int (widening its result to 64 bits sign-extends it, on the host as on the device)
static inline int __builtin_amdgcn_readfirstlane(int v) { return v; }
#define __builtin_amdgcn_wave_barrier() ((void)0)
// a wave's issue priority orders nothing on the host
#define __builtin_amdgcn_s_setprio(p) ((void)(p))
#define __builtin_amdgcn_fence(order, scope) ((void)0)
// the optimization barrier of Console::in_register, with a host register constraint
#define MH_REG_BARRIER(x) asm volatile("" : "+r"(x))

static inline uint32_t __umul24(uint32_t a, uint32_t b) { return (a & 0xffffffu) * (b & 0xffffffu); }

// v_alignbyte_b32: the 32 bits of {hi, lo} starting at byte (sel & 3)
static inline uint32_t mh_host_alignbyte(uint32_t hi, uint32_t lo, uint32_t sel) {
    return (uint32_t)((((uint64_t)hi << 32) | lo) >> (8u * (sel & 3u)));
}
#define __builtin_amdgcn_alignbyte mh_host_alignbyte

// v_perm_b32: byte i of the result is selected by byte i of sel from the 8 bytes {hi, lo} (0..7), or is
// the sign of byte 1/3/5/7 replicated (8..11), zero (12) or 0xff (13..)
static inline uint32_t mh_host_perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    const uint64_t v = ((uint64_t)hi << 32) | lo;
    uint32_t out = 0;
    for (int i = 0; i < 4; i++) {
        const uint32_t s = (sel >> (8 * i)) & 0xffu;
        uint32_t b;
        if (s < 8) b = (uint32_t)(v >> (8 * s)) & 0xffu;
        else if (s < 12) b = ((v >> (16 * (s - 8) + 15)) & 1u) ? 0xffu : 0u;
        else if (s == 12) b = 0u;
        else b = 0xffu;
        out |= b << (8 * i);
    }
    return out;
}
#define __builtin_amdgcn_perm mh_host_perm

static inline long long __double_as_longlong(double d) { long long r; memcpy(&r, &d, 8); return r; }
static inline double __longlong_as_double(long long x) { double r; memcpy(&r, &x, 8); return r; }
static inline uint32_t atomicOr(uint32_t* p, uint32_t v) { const uint32_t o = *p; *p = o | v; return o; }
