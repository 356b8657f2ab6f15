// Synthetic workload generator: counter-mode splitmix64 (the mixing step of
// Steele, Lea & Flood, "Fast splittable pseudorandom number generators",
// OOPSLA 2014), uniform floats from the top 24 bits, normals by Box-Muller
// in fp64.  Host-only; the same arrays feed the GPU engine and the CPU
// baseline, so results never depend on where a number was drawn.
#include <cmath>
#include <vector>

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

int vdttfs_synth_dvs(uint64_t seed, int N, int C, int H, int W, int T, double density, double sigma,
                     double vmax, float* out, double* scales) {
    if (N <= 0 || C <= 0 || H <= 0 || W <= 0 || T <= 0 || !out || !(sigma > 0.0) || !(density > 0.0))
        return set_error(VDTTFS_E_INVALID, "synth_dvs: bad args");
    const int64_t per = (int64_t)C * H * W * T;
    if (per >= (INT64_C(1) << 40)) return set_error(VDTTFS_E_INVALID, "synth_dvs: sample too large");
    std::vector<double> g((size_t)H * W * T);
    for (int n = 0; n < N; ++n) {
        auto u = [&](int k) { return (double)(draw(seed, 3000 + (uint64_t)n, (uint64_t)k) >> 40) * 0x1.0p-24; };
        const double cx0 = W * (0.25 + 0.5 * u(0)), cy0 = H * (0.25 + 0.5 * u(1));
        const double vx = vmax * (2.0 * u(2) - 1.0), vy = vmax * (2.0 * u(3) - 1.0);
        double sum = 0.0;
        for (int y = 0; y < H; ++y)
            for (int x = 0; x < W; ++x)
                for (int t = 0; t < T; ++t) {
                    const double dx = x - (cx0 + vx * t), dy = y - (cy0 + vy * t);
                    const double v = std::exp(-(dx * dx + dy * dy) / (2.0 * sigma * sigma));
                    g[((size_t)y * W + x) * T + t] = v;
                    sum += v;
                }
        const double scale = sum > 0.0 ? density * (double)H * W * T / sum : 0.0;
        if (scales) scales[n] = scale;
        float* o = out + (int64_t)n * per;
        for (int c = 0; c < C; ++c)
            for (int64_t k = 0; k < (int64_t)H * W * T; ++k) {
                const double p = std::fmin(1.0, scale * g[(size_t)k]);
                const int64_t idx = (int64_t)c * H * W * T + k;
                const double r = (double)(draw(seed, 2000 + (uint64_t)n, (uint64_t)idx) >> 40) * 0x1.0p-24;
                o[idx] = r < p ? 1.0f : 0.0f;
            }
    }
    return VDTTFS_OK;
}

}  // extern "C"
