// Synthetic workload generator: counter-mode splitmix64 (the mixing step of
// Steele, Lea & Flood, "Fast splittable pseudorandom number generators",
// OOPSLA 2014), uniform floats from the top 24 bits, normals by Box-Muller
// in fp64.  Host-only; the same arrays feed the GPU engine and the CPU
// baseline, so results never depend on where a number was drawn.
#include <cmath>

#include "common.h"

using namespace vdttfs;

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t draw(uint64_t seed, uint64_t stream, uint64_t i) {
    return mix64(seed + kGamma * ((stream << 40) + i + 1));
}

}  // namespace

extern "C" {

int vdttfs_synth_uniform(uint64_t seed, uint64_t stream, float* out, int64_t n) {
    if (n < 0 || (n > 0 && !out)) return set_error(VDTTFS_E_INVALID, "synth: bad args");
    if (n >= (INT64_C(1) << 40)) return set_error(VDTTFS_E_INVALID, "synth: n >= 2^40");
    for (int64_t i = 0; i < n; ++i)
        out[i] = (float)((double)(draw(seed, stream, (uint64_t)i) >> 40) * 0x1.0p-24);
    return VDTTFS_OK;
}

int vdttfs_synth_normal(uint64_t seed, uint64_t stream, float* out, int64_t n, double sigma) {
    if (n < 0 || (n > 0 && !out)) return set_error(VDTTFS_E_INVALID, "synth: bad args");
    if (n >= (INT64_C(1) << 39)) return set_error(VDTTFS_E_INVALID, "synth: n >= 2^39");
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        const uint64_t z1 = draw(seed, stream, (uint64_t)i);
        const uint64_t z2 = draw(seed, stream, (uint64_t)i + 1);
        const double u1 = ((double)(z1 >> 11) + 1.0) * 0x1.0p-53;  // (0, 1]
        const double u2 = (double)(z2 >> 11) * 0x1.0p-53;          // [0, 1)
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = (float)(sigma * r * std::cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(sigma * r * std::sin(two_pi * u2));
    }
    return VDTTFS_OK;
}

}  // extern "C"
