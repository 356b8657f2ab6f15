// Wave64 helpers for gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace vdttfs {

constexpr float kInfTime = 9999.0f;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Orders LDS traffic between lanes of one wave (LDS ops of a wave execute in
// program order; this keeps the compiler from reordering across the point).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint64_t lanemask_lt() {
    return (1ull << lane_id()) - 1ull;
}

// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = lane_id();
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        int u = __shfl_up(v, off, 64);
        if (lane >= off) v += u;
    }
    return v;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// A zero made in a VGPR where it is used: a plain 0 stored to LDS is often
// hoisted by the compiler into a register that stays live for the whole
// kernel.
__device__ __forceinline__ int vzero() {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// x + 1 in the lanes whose bit of `mask` is set, x elsewhere: one
// v_addc_co_u32 with the mask as its carry-in (the compiler would spend a
// v_cndmask and a v_add).
__device__ __forceinline__ int add_lane_bit(int x, uint64_t mask) {
    int r;
    uint64_t carry_out;
    asm("v_addc_co_u32_e64 %0, %1, 0, %2, %3" : "=v"(r), "=s"(carry_out) : "v"(x), "s"(mask));
    return r;
}

// Division of 0 <= n < 2^31 by a fixed divisor d >= 1 with a precomputed
// multiplier (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994, the round-up method): l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (umulhi(n, m) + n) >> l (the
// sum stays below 2^32 because n < 2^31).  Wave-uniform n keeps it in
// scalar instructions.
struct FastDiv {
    unsigned m;
    int l, d;
};
inline FastDiv make_fastdiv(int d) {
    FastDiv f{0u, 0, d};
    while ((1ll << f.l) < (long long)d) ++f.l;
    f.m = (unsigned)((((unsigned long long)1 << 32) * ((1ull << f.l) - (unsigned long long)d)) / (unsigned)d + 1);
    return f;
}
__device__ __forceinline__ int fdiv(int n, const FastDiv& f) {
    return (int)((__umulhi((unsigned)n, f.m) + (unsigned)n) >> f.l);
}

// Arrival bin of a spike (T1V:58-59 / T2V:59-60): -1 if no spike or outside
// the window.
__device__ __forceinline__ int arrival_bin(float t, float tfs, int T) {
    if (!(t < kInfTime)) return -1;
    int tb = (int)floorf(t - tfs);
    if (tb < 0) tb = 0;
    return tb < T ? tb : -1;
}

// Decay-LUT index of an event: tb (T1V:128,144) or clamp((int)t,0,T)
// (T2V:132,150).
__device__ __forceinline__ int alpha_index(float t, int tb, int alpha_by_time, int T) {
    if (!alpha_by_time) return tb;
    int ti = (int)t;
    return ti < 0 ? 0 : (ti > T ? T : ti);
}

}  // namespace vdttfs
