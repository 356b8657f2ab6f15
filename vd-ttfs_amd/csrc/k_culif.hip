// CuLIF kernels (T3V, config 4): the current-based LIF neuron
//   I = fma(I, decay, in_t);  V = V + I;  fire at the first t with V >= th
// over one arrival-ordered pass per layer.  The reference processes Delta-wide
// chunks and stops at the chunk that fires; with Delta | T this equals the
// per-step recurrence above, so every kernel here steps bins in time order
// and leaves at the first crossing (results are Delta-invariant).
//
//  k_culif_conv1_tile  conv1_raw_early (T3V:30-65) for C_in <= 4: row tiles of
//                      16 pixels with the input neighbourhood staged in LDS;
//  k_culif_conv1_lane  the same for any C_in, one wave per pixel, time
//                      vectors broadcast with readlane.  Lanes are c_out;
//                      output layout by strides (NCHW for the drop-in, NHWC
//                      for the engine).
//  k_culif_bucketize   k_bucketize_conv / k_bucketize_fc (T3V:70-106) in the
//                      reference layout: one thread per site, counters in LDS
//                      (k_culif_bucketize_wave: a wave per site, for few sites).
//  k_culif_generic     conv_bucketed_early / fc2_bucketed_early (T3V:109-143,
//                      203-225) over the reference layout, one thread per
//                      neuron (the drop-in path and the engine's small FC).
//  k_culif_pool        pool_chunk_early (T3V:146-168), layouts by strides.
//  k_culif_fc_rec      fc1_bucketed_recurrent (T3V:171-200): one block per
//                      sample; fired-last-step neurons as a bitmask in LDS.
//  k_fc_currents       the engine's per-step feed-forward input of that layer,
//                      computed per (sample, step group) from the dense input.
//  k_nhwc_to_nchw      flattening order for an FC layer after a spatial map.
#include <type_traits>

#include "common.h"
#include "wave.h"

namespace vdttfs {
namespace {

constexpr int kRawChunk = 32;  // steps per register chunk in conv1_raw (any T)

// ---------------------------------------------------------------------------
struct RawArgs {
    const float* data;  // [N][C_in][H][W][T]
    float* out;
    const float* W;     // OIHW [C_out][C_in][3][3]
    int64_t n_pix;      // N*H*W
    int C_in, C_out, H, Wd, T, n_cblk;
    int64_t sN, sC, sY, sX;  // output strides
    float decay, th;
    uint8_t* fired;     // k_culif_conv1_mask, one c_out block: per pixel, 1 when some neuron fired (or null)
};

// Tiled variant for few input channels (C_in <= kTileMaxCin): a block of 4
// waves owns kTileX consecutive output pixels of one row and one 64-wide
// c_out block.  Per 32-step chunk the block stages the 3 x (kTileX + 2)
// input neighbourhood (C_in channels, 32 steps each: coalesced 128-byte
// segments) in LDS; each wave then integrates its pixels with the time
// vectors read as LDS broadcasts.  The per-step fma order is conv1_raw's
// (c_in, ky, kx), out-of-bounds taps skipped.  The block stops once no lane
// of any pixel is alive.
constexpr int kTileX = 16;
constexpr int kTileMaxCin = 4;
constexpr int kTilePix = kTileX / 4;  // pixels per wave

__global__ __launch_bounds__(256) void k_culif_conv1_tile(RawArgs a) {
    __shared__ float4 tile4[kTileMaxCin * 3 * (kTileX + 2) * (kRawChunk / 4)];
    float* tile = reinterpret_cast<float*>(tile4);
    const int wave = uniform(threadIdx.x >> 6);
    const int n_xt = (a.Wd + kTileX - 1) / kTileX;
    int64_t b = blockIdx.x;
    const int cb = (int)(b % a.n_cblk);
    b /= a.n_cblk;
    const int xt = (int)(b % n_xt);
    b /= n_xt;
    const int y = (int)(b % a.H);
    const int64_t n = b / a.H;
    const int x0 = xt * kTileX;
    const int c = cb * 64 + lane_id();
    const bool ok = c < a.C_out;
    const int segs = a.C_in * 3 * (kTileX + 2);  // (ci, r, cx) time vectors
    float I[kTilePix], V[kTilePix], res[kTilePix];
    bool alive[kTilePix];
#pragma unroll
    for (int q = 0; q < kTilePix; ++q) {
        const int x = x0 + wave + 4 * q;
        I[q] = 0.0f;
        V[q] = 0.0f;
        res[q] = kInfTime;
        alive[q] = ok && x < a.Wd;
    }
    for (int t0 = 0; t0 < a.T; t0 += kRawChunk) {
        __syncthreads();  // previous chunk's readers are done
        for (int idx = threadIdx.x; idx < segs * kRawChunk; idx += blockDim.x) {
            const int t = idx % kRawChunk, sg = idx / kRawChunk;
            const int cx = sg % (kTileX + 2), r = (sg / (kTileX + 2)) % 3, ci = sg / (3 * (kTileX + 2));
            const int iy = y + r - 1, ix = x0 + cx - 1;
            float v = 0.0f;
            if (iy >= 0 && iy < a.H && ix >= 0 && ix < a.Wd && t0 + t < a.T)
                v = a.data[(((n * a.C_in + ci) * a.H + iy) * a.Wd + ix) * (int64_t)a.T + t0 + t];
            tile[idx] = v;
        }
        __syncthreads();
        bool any = false;
#pragma unroll
        for (int q = 0; q < kTilePix; ++q) {
            const int x = x0 + wave + 4 * q;
            if (x >= a.Wd || __ballot(alive[q]) == 0) continue;  // uniform per wave
            float in[kRawChunk];
#pragma unroll
            for (int t = 0; t < kRawChunk; ++t) in[t] = 0.0f;
            for (int ci = 0; ci < a.C_in; ++ci)
                for (int ky = 0; ky < 3; ++ky) {
                    const int iy = y + ky - 1;
                    if (iy < 0 || iy >= a.H) continue;
                    for (int kx = 0; kx < 3; ++kx) {
                        const int ix = x + kx - 1;
                        if (ix < 0 || ix >= a.Wd) continue;
                        const float w = ok ? a.W[(((int64_t)c * a.C_in + ci) * 3 + ky) * 3 + kx] : 0.0f;
                        const float4* v4 = tile4 + ((ci * 3 + ky) * (kTileX + 2) + (ix - x0 + 1)) * (kRawChunk / 4);
#pragma unroll
                        for (int t4 = 0; t4 < kRawChunk / 4; ++t4) {
                            const float4 v = v4[t4];
                            in[4 * t4 + 0] = __builtin_fmaf(w, v.x, in[4 * t4 + 0]);
                            in[4 * t4 + 1] = __builtin_fmaf(w, v.y, in[4 * t4 + 1]);
                            in[4 * t4 + 2] = __builtin_fmaf(w, v.z, in[4 * t4 + 2]);
                            in[4 * t4 + 3] = __builtin_fmaf(w, v.w, in[4 * t4 + 3]);
                        }
                    }
                }
#pragma unroll
            for (int t = 0; t < kRawChunk; ++t) {
                if (t0 + t < a.T) {
                    I[q] = __builtin_fmaf(I[q], a.decay, in[t]);
                    V[q] = V[q] + I[q];
                    if (alive[q] && V[q] >= a.th) {
                        res[q] = (float)(t0 + t);
                        alive[q] = false;
                    }
                }
            }
            any = any || alive[q];
        }
        if (!__syncthreads_or(any)) break;
    }
#pragma unroll
    for (int q = 0; q < kTilePix; ++q) {
        const int x = x0 + wave + 4 * q;
        if (ok && x < a.Wd)
            a.out[n * a.sN + (int64_t)c * a.sC + (int64_t)y * a.sY + (int64_t)x * a.sX] = res[q];
    }
}

// Any C_in (the tiled kernel takes C_in <= 4): one wave per output pixel and
// 64-wide c_out block (lanes = c_out), time in blocks of 64 steps.  For each
// tap one coalesced vector load fetches 64 steps (lane i = step i) and
// v_readlane hands step t's value to every lane as a scalar fma operand (8
// readlanes into distinct SGPRs, then 8 fmas).  Taps run in the reference's
// (c_in, ky, kx) order, out-of-bounds taps skipped.  Measured on the 2-channel
// layer of config 4: 4.8 ms against 3.9 ms for the tiled kernel and 6.9 ms for
// per-tap scalar loads of the time vectors.
__global__ __launch_bounds__(256) void k_culif_conv1_lane(RawArgs a) {
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t b = blockIdx.x;
    const int cb = (int)(b % a.n_cblk);
    const int64_t pix0 = (b / a.n_cblk) * 4 + wave;
    if (pix0 >= a.n_pix) return;  // uniform per wave
    const int64_t pix = ((int64_t)uniform((int)(pix0 >> 32)) << 32) | (uint32_t)uniform((int)pix0);
    const int x = (int)(pix % a.Wd);
    const int y = (int)((pix / a.Wd) % a.H);
    const int64_t n = pix / ((int64_t)a.Wd * a.H);
    const int lane = lane_id();
    const int c = cb * 64 + lane;
    const bool ok = c < a.C_out;
    const int cin = a.C_in;
    float I = 0.0f, V = 0.0f, res = kInfTime;
    bool alive = ok;
    auto tap_ok = [&](int k) {
        const int iy = y + (k % 9) / 3 - 1, ix = x + k % 3 - 1;
        return iy >= 0 && iy < a.H && ix >= 0 && ix < a.Wd;
    };
    auto tap_base = [&](int k, int t0) {
        const int ci = k / 9, iy = y + (k % 9) / 3 - 1, ix = x + k % 3 - 1;
        return (((n * cin + ci) * a.H + iy) * a.Wd + ix) * (int64_t)a.T + t0;
    };
    auto accumulate = [&](float (&in)[64], float w, float v) {
        const int vi = __float_as_int(v);
#pragma unroll
        for (int t = 0; t < 64; t += 8) {
            // 8 readlanes into distinct SGPRs, then 8 fmas: one SGPR
            // write-to-read wait per 8 instead of per fma
            int sv[8];
#pragma unroll
            for (int g = 0; g < 8; ++g) sv[g] = __builtin_amdgcn_readlane(vi, t + g);
            asm volatile("" ::"s"(sv[0]), "s"(sv[1]), "s"(sv[2]), "s"(sv[3]), "s"(sv[4]), "s"(sv[5]),
                         "s"(sv[6]), "s"(sv[7]));
#pragma unroll
            for (int g = 0; g < 8; ++g) in[t + g] = __builtin_fmaf(w, __int_as_float(sv[g]), in[t + g]);
        }
    };
    for (int t0 = 0; t0 < a.T; t0 += 64) {
        const bool tin = t0 + lane < a.T;
        float in[64];
#pragma unroll
        for (int t = 0; t < 64; ++t) in[t] = 0.0f;
        for (int k = 0; k < cin * 9; ++k) {
            if (!tap_ok(k)) continue;  // uniform
            const float w = ok ? a.W[(int64_t)c * cin * 9 + k] : 0.0f;
            accumulate(in, w, tin ? a.data[tap_base(k, t0) + lane] : 0.0f);
        }
#pragma unroll
        for (int t = 0; t < 64; ++t) {
            if (t0 + t < a.T) {
                I = __builtin_fmaf(I, a.decay, in[t]);
                V = V + I;
                if (alive && V >= a.th) {
                    res = (float)(t0 + t);
                    alive = false;
                }
            }
        }
        if (__ballot(alive) == 0) break;
    }
    if (ok) a.out[n * a.sN + (int64_t)c * a.sC + (int64_t)y * a.sY + (int64_t)x * a.sX] = res;
}

// ---------------------------------------------------------------------------
// conv1_raw from event masks (the engine's path when every weight is finite).
// k_culif_event_masks reads the dense [N][C][H][W][T] input once and keeps,
// per site and 64-step block, the mask of nonzero steps and a flag set when
// a nonzero value is not exactly 1.0.  k_culif_conv1_mask then integrates
// from the masks: a step's input current is the fma chain over the taps whose
// bit is set, in the reference's (c_in, ky, kx) order, with v = 1.0 (or the
// value itself under the flag).  Skipping the zero taps is exact for finite
// weights: the chain starts at +0.0f and fma(w, 0, acc) = acc + (+-0) = acc
// for every acc the chain can hold (it is never -0), so only the taps with a
// nonzero input change it.  A non-finite weight turns w * 0 into NaN, so such
// layers keep the dense kernels above.
struct MaskArgs {
    const float* data;
    uint64_t* mask;    // [site][nblk]
    uint32_t* nonbin;  // [site][nblk]
    int64_t units;     // sites * nblk
    int T, nblk;
};

constexpr int kMaskUnitsPerWave = 8;
constexpr int kMaskPixPerWave = 16;  // consecutive output pixels per wave
constexpr int kMaskMaxCin = 3;  // taps held in registers and in 32-bit step masks: C_in * 9 <= 27

__global__ __launch_bounds__(256) void k_culif_event_masks(MaskArgs a) {
    const int lane = lane_id();
    const int64_t u0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kMaskUnitsPerWave;
    if (u0 >= a.units) return;  // uniform per wave
    float v[kMaskUnitsPerWave];
#pragma unroll
    for (int q = 0; q < kMaskUnitsPerWave; ++q) {
        const int64_t u = u0 + q;
        const int64_t site = u / a.nblk;
        const int t = (int)(u - site * a.nblk) * 64 + lane;
        v[q] = (u < a.units && t < a.T) ? a.data[site * a.T + t] : 0.0f;
    }
    uint64_t my_m = 0;
    uint32_t my_nb = 0;
#pragma unroll
    for (int q = 0; q < kMaskUnitsPerWave; ++q) {
        const uint64_t m = __ballot(v[q] != 0.0f);
        const uint64_t nb = __ballot(v[q] != 0.0f && v[q] != 1.0f);
        if (lane == q) {
            my_m = m;
            my_nb = nb != 0;
        }
    }
    if (lane < kMaskUnitsPerWave && u0 + lane < a.units) {
        a.mask[u0 + lane] = my_m;
        a.nonbin[u0 + lane] = my_nb;
    }
}

// One wave per kMaskPixPerWave consecutive output pixels and a 64-wide c_out
// block (lanes = c_out), four waves of one c_out block per workgroup; NK =
// C_in * 9 taps, the lane's NK weights in registers.  Per 64-step block the
// tap masks are transposed so that lane t holds the taps with input at step t
// (NK <= 32 bits); a step with input then visits only its set taps, in
// ascending k, one add each (fma(w, 1, in) is exactly in + w).  All T steps
// run the neuron update (a step without input still decays I and adds it to
// V).  The wave's live neurons are an SGPR lane mask and each lane counts the
// steps it has lived through, which is its spike step once it fires; steps
// are tested eight at a time against one byte of the block's input mask.
template <int NK>
__global__ __launch_bounds__(256) void k_culif_conv1_mask(RawArgs a, const uint64_t* __restrict__ mask,
                                                          const uint32_t* __restrict__ nonbin, int nblk) {
    static_assert(NK <= 32, "tap masks are 32-bit");
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t b = blockIdx.x;
    const int cb = (int)(b % a.n_cblk);
    const int lane = lane_id();
    const int c = cb * 64 + lane;
    const bool ok = c < a.C_out;
    float w[NK];
#pragma unroll
    for (int k = 0; k < NK; ++k) w[k] = ok ? a.W[(int64_t)c * NK + k] : 0.0f;
    // lane k < NK: tap k = (ci, ky, kx) in the reference's order, as a site
    // offset from (n, ci = 0, y, x)
    const int tk = lane < NK ? lane : 0;
    const int tdy = (tk % 9) / 3 - 1, tdx = tk % 3 - 1;
    const int64_t toff = ((int64_t)(tk / 9) * a.H + tdy) * a.Wd + tdx;
    const int pix0 = uniform((int)((b / a.n_cblk) * 4 + wave)) * kMaskPixPerWave;  // < 2^31 (host check)
    for (int pq = 0; pq < kMaskPixPerWave; ++pq) {
        const int pix = pix0 + pq;
        if (pix >= a.n_pix) return;  // uniform per wave
        const int x = pix % a.Wd;
        const int y = (pix / a.Wd) % a.H;
        const int n = pix / (a.Wd * a.H);
        // this lane's tap site, or none out of bounds (skipped, as the
        // reference does)
        const int iy = y + tdy, ix = x + tdx;
        const bool tap_in = lane < NK && iy >= 0 && iy < a.H && ix >= 0 && ix < a.Wd;
        const int64_t site = ((int64_t)n * a.C_in * a.H + y) * a.Wd + x + toff;
        auto tap_site = [&](int k) -> int64_t {  // wave-uniform, for a tap with input
            const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)site, k);
            const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)site >> 32), k);
            return (int64_t)(lo | (hi << 32));
        };
        float I = 0.0f, V = 0.0f;
        int lived = 0;  // steps survived: the spike step once the lane fired
        const uint64_t all = __ballot(ok);
        uint64_t alive = all;
        for (int tb = 0; tb < nblk && alive; ++tb) {
            // lane k's tap: its mask of steps with input, and whether a
            // nonzero input is not 1.0
            uint64_t mk = 0;
            bool nbk = false;
            if (tap_in) {
                mk = mask[site * nblk + tb];
                nbk = nonbin[site * nblk + tb] != 0;
            }
            const uint32_t nbm = (uint32_t)__ballot(nbk);  // bit k: tap k (NK <= 32)
            uint32_t tapm = 0;  // lane t: taps with input at step t0 + t
            if (__ballot(mk != 0)) {  // the transpose, for a block with any input
                const int mlo = (int)(uint32_t)mk, mhi = (int)(uint32_t)(mk >> 32);
#pragma unroll
                for (int k = 0; k < NK; ++k) {
                    const uint64_t m = (uint64_t)(uint32_t)__builtin_amdgcn_readlane(mlo, k) |
                                       ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(mhi, k) << 32);
                    tapm |= (__builtin_amdgcn_inverse_ballot_w64(m) ? 1u : 0u) << k;
                }
            }
            const uint64_t any = __ballot(tapm != 0);  // steps with input (none at t >= T)
            const int t0 = tb * 64;
            const int tn = (a.T - t0) < 64 ? (a.T - t0) : 64;
            // the input current of step t0 + t, which has input in some tap
            // (so tm != 0); NB: some tap's values are not all 1.0
            auto input = [&](int t, auto nb) -> float {
                uint32_t tm = (uint32_t)__builtin_amdgcn_readlane((int)tapm, t);
                float in = 0.0f;
                if (decltype(nb)::value && (tm & nbm)) {
                    // an input value other than 1.0 at this step (rare)
                    do {
                        const int k = __builtin_ctz(tm);
                        tm &= tm - 1;
                        const float v = ((nbm >> k) & 1) ? a.data[(int64_t)tap_site(k) * a.T + t0 + t] : 1.0f;
                        in = __builtin_fmaf(w[k], v, in);
                    } while (tm);
                } else {
                    do {
                        const int k = __builtin_ctz(tm);
                        tm &= tm - 1;
                        in = in + w[k];
                    } while (tm);
                }
                return in;
            };
            auto neuron = [&](float in) {
                I = __builtin_fmaf(I, a.decay, in);
                V = V + I;
                alive &= ~__builtin_amdgcn_ballot_w64(V >= a.th);
                lived = add_lane_bit(lived, alive);
            };
            auto run = [&](auto nb) {
                // whole groups of 8 steps, then the last, partial group of T
                int t8 = 0;
                int first = t0 == 0 ? 1 : 0;  // the group holding step 0 never skips
                for (; t8 + 8 <= tn; t8 += 8) {
                    const uint32_t a8 = (uint32_t)(any >> t8) & 0xffu;
                    // steps without input while every lane's current is zero
                    // change nothing: I stays 0, V stays V (the threshold is
                    // fixed), and a lane with V >= th would have fired at the
                    // step before (none precedes step 0); its live lanes live
                    // through them
                    const int key = (int)a8 | first;
                    first = 0;
                    if (key == 0) {
                        if (__builtin_amdgcn_ballot_w64(I != 0.0f) == 0) {
                            lived += __builtin_amdgcn_inverse_ballot_w64(alive) ? 8 : 0;
                            continue;
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) neuron((a8 & (1u << u)) ? input(t8 + u, nb) : 0.0f);
                    if (alive == 0) return;
                }
                if (t8 < tn) {
                    const uint32_t a8 = (uint32_t)(any >> t8) & 0xffu;
                    for (int u = 0; u < tn - t8; ++u) neuron((a8 & (1u << u)) ? input(t8 + u, nb) : 0.0f);
                }
            };
            if (nbm) run(std::true_type{});
            else run(std::false_type{});
        }
        if (ok)
            a.out[(int64_t)n * a.sN + (int64_t)c * a.sC + (int64_t)y * a.sY + (int64_t)x * a.sX] =
                __builtin_amdgcn_inverse_ballot_w64(alive) ? kInfTime : (float)lived;
        if (a.fired && lane == 0) a.fired[pix] = (all & ~alive) != 0 ? 1 : 0;
    }
}

// ---------------------------------------------------------------------------
// Reference-layout bucketize (T3V:70-106).  Site s = (n, hw): element c at
// (n*C + c)*HW + hw; an FC input is HW = 1, C = F.  tb = (int)t, kept if
// 0 <= tb < T; chunks of D; events in ascending c within a chunk.
constexpr int kCBktThreads = 64;
constexpr int kCBktMaxChunks = 64;

struct CBktArgs {
    const float* in;
    int32_t* cin;
    float* tin;
    int32_t* off;
    int64_t n_sites;
    int C, HW, T, D, NC;
};

__device__ __forceinline__ int culif_bin(float tf, int T) {
    if (!(tf < kInfTime)) return -1;
    const int tb = (int)tf;
    return (tb >= 0 && tb < T) ? tb : -1;
}

__global__ __launch_bounds__(kCBktThreads) void k_culif_bucketize(CBktArgs a) {
    __shared__ int cnt[kCBktMaxChunks * kCBktThreads];  // [chunk][lane]
    const int lane = threadIdx.x;
    const int64_t s = (int64_t)blockIdx.x * kCBktThreads + lane;
    if (s >= a.n_sites) return;  // no barriers below
    int* my = cnt + lane;
    for (int k = 0; k < a.NC; ++k) my[k * kCBktThreads] = 0;
    const int64_t base = (s / a.HW) * (int64_t)a.C * a.HW + s % a.HW;
    for (int c = 0; c < a.C; ++c) {
        const int tb = culif_bin(a.in[base + (int64_t)c * a.HW], a.T);
        if (tb >= 0) my[(tb / a.D) * kCBktThreads] += 1;
    }
    const int OS = a.NC + 1;
    int run = 0;
    for (int k = 0; k < a.NC; ++k) {
        a.off[s * OS + k] = run;
        const int v = my[k * kCBktThreads];
        my[k * kCBktThreads] = run;
        run += v;
    }
    a.off[s * OS + a.NC] = run;
    int32_t* dc = a.cin + s * a.C;
    float* dt = a.tin + s * a.C;
    for (int c = 0; c < a.C; ++c) {
        const float tf = a.in[base + (int64_t)c * a.HW];
        const int tb = culif_bin(tf, a.T);
        if (tb >= 0) {
            const int p = my[(tb / a.D) * kCBktThreads]++;
            dc[p] = c;
            dt[p] = tf;
        }
    }
}

// Few sites (an FC layer's sites are its samples, one thread each above):
// one wave per site, 64 elements a step.  Ranks within a chunk come from one
// ballot per chunk the step holds, lane k keeps chunk k's count (NC <= 64);
// the elements are read twice (count, then place).  Same output as
// k_culif_bucketize.
constexpr int64_t kCBktWaveMaxSites = 4096;

__global__ __launch_bounds__(256) void k_culif_bucketize_wave(CBktArgs a) {
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t s = (int64_t)blockIdx.x * 4 + wave;
    if (s >= a.n_sites) return;  // uniform per wave; no barriers below
    const int lane = lane_id();
    const int64_t base = (s / a.HW) * (int64_t)a.C * a.HW + s % a.HW;
    const uint64_t lt = lanemask_lt();
    auto chunk_of = [&](int c, float& tf) {
        tf = c < a.C ? a.in[base + (int64_t)c * a.HW] : kInfTime;
        const int tb = culif_bin(tf, a.T);
        return tb >= 0 ? tb / a.D : -1;
    };
    int cnt = 0;  // lane k: events of chunk k
    for (int c0 = 0; c0 < a.C; c0 += 64) {
        float tf;
        const int k = chunk_of(c0 + lane, tf);
        uint64_t pending = __ballot(k >= 0);
        while (pending) {
            const int kk = __builtin_amdgcn_readlane(k, __builtin_ctzll(pending));
            const uint64_t m = __ballot(k == kk);
            if (lane == kk) cnt += __popcll(m);
            pending &= ~m;
        }
    }
    const int OS = a.NC + 1;
    const int incl = wave_incl_scan(cnt);  // lanes >= NC hold 0
    int pos = incl - cnt;                  // lane k < NC: chunk k's first position
    if (lane < a.NC) a.off[s * OS + lane] = pos;
    if (lane == a.NC - 1) a.off[s * OS + a.NC] = incl;
    int32_t* dc = a.cin + s * a.C;
    float* dt = a.tin + s * a.C;
    for (int c0 = 0; c0 < a.C; c0 += 64) {
        float tf;
        const int k = chunk_of(c0 + lane, tf);
        uint64_t pending = __ballot(k >= 0);
        while (pending) {
            const int kk = __builtin_amdgcn_readlane(k, __builtin_ctzll(pending));
            const uint64_t m = __ballot(k == kk);
            const int start = __builtin_amdgcn_readlane(pos, kk);
            if (k == kk) {
                const int p = start + __popcll(m & lt);
                dc[p] = c0 + lane;
                dt[p] = tf;
            }
            if (lane == kk) pos += __popcll(m);
            pending &= ~m;
        }
    }
}

// ---------------------------------------------------------------------------
struct CGenArgs {
    const int32_t* cin;
    const float* tin;
    const int32_t* off;
    float* out;
    const float* W;   // conv OIHW [C_out][C_in][3][3]; fc [out][in]
    int64_t total;
    int C_in, C_out, H, Wd, T, D, NC;
    float decay, th;
};

// One thread per neuron; in_val[] of a chunk in private memory.
template <bool FC, int DMAX>
__global__ __launch_bounds__(256) void k_culif_generic(CGenArgs a) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        int64_t n;
        int c_out, y = 0, x = 0;
        if (FC) {
            n = idx / a.C_out;
            c_out = (int)(idx % a.C_out);
        } else {  // NCHW, x fastest (T3V:112-114)
            const int64_t hw = (int64_t)a.H * a.Wd;
            n = idx / (a.C_out * hw);
            const int64_t rem = idx % (a.C_out * hw);
            c_out = (int)(rem / hw);
            y = (int)((rem / a.Wd) % a.H);
            x = (int)(rem % a.Wd);
        }
        const int OS = a.NC + 1;
        float I = 0.0f, V = 0.0f, res = kInfTime;
        for (int ch = 0; ch < a.NC && res == kInfTime; ++ch) {
            const int base_t = ch * a.D;
            float in_val[DMAX];
            for (int t = 0; t < a.D; ++t) in_val[t] = 0.0f;
            const int ntap = FC ? 1 : 9;
            for (int k = 0; k < ntap; ++k) {
                int64_t site;
                int64_t wk;
                if (FC) {
                    site = n;
                    wk = (int64_t)c_out * a.C_in;  // + j
                } else {
                    const int ky = k / 3, kx = k % 3;
                    const int iy = y + ky - 1, ix = x + kx - 1;
                    if (iy < 0 || iy >= a.H || ix < 0 || ix >= a.Wd) continue;
                    site = (n * a.H + iy) * a.Wd + ix;
                    wk = (int64_t)c_out * a.C_in * 9 + ky * 3 + kx;  // + cin*9
                }
                // offsets and indices are the caller's: keep every access in bounds
                const int s = max(a.off[site * OS + ch], 0), e = min(a.off[site * OS + ch + 1], a.C_in);
                const int32_t* sc = a.cin + site * a.C_in;
                const float* st = a.tin + site * a.C_in;
                for (int p = s; p < e; ++p) {
                    const int j = sc[p];
                    const int dt = (int)st[p] - base_t;
                    if ((unsigned)dt < (unsigned)a.D && (unsigned)j < (unsigned)a.C_in)
                        in_val[dt] = in_val[dt] + a.W[wk + (int64_t)j * (FC ? 1 : 9)];
                }
            }
            for (int t = 0; t < a.D; ++t) {
                I = __builtin_fmaf(I, a.decay, in_val[t]);
                V = V + I;
                if (V >= a.th) {
                    res = (float)(base_t + t);
                    break;
                }
            }
        }
        a.out[idx] = res;
    }
}

// ---------------------------------------------------------------------------
struct CPoolArgs {
    const float* in;
    float* out;
    int64_t total;
    int C, H_in, W_in, T;
    int nhwc;                       // flat output order: 1 = NHWC, 0 = NCHW
    int64_t iN, iC, iY, iX;         // input strides
    int64_t oN, oC, oY, oX;         // output strides
    float decay, th;
    FastDiv div_c, div_w, div_h;    // C, W_out, H_out (flat indices below 2^31)
};

// T3V:146-168.  in_t = 1.0 when one of the 4 inputs has floor(tf) == t
// (the reference sets in_val[(int)tf - chunk] for chunk <= tf < chunk+D).
// I32: flat indices below 2^31, split with precomputed multipliers instead
// of 64-bit divisions.  Before a neuron's first input step I and V are +0,
// so it fires there only if th <= 0, at step 0.
template <bool I32>
__global__ __launch_bounds__(256) void k_culif_pool(CPoolArgs a) {
    const int H_out = a.H_in / 2, W_out = a.W_in / 2;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        int64_t n;
        int c, yo, xo;
        if constexpr (I32) {
            const int i = (int)idx;
            if (a.nhwc) {
                const int p = fdiv(i, a.div_c), q = fdiv(p, a.div_w), r = fdiv(q, a.div_h);
                c = i - p * a.C;
                xo = p - q * W_out;
                yo = q - r * H_out;
                n = r;
            } else {
                const int p = fdiv(i, a.div_w), q = fdiv(p, a.div_h), r = fdiv(q, a.div_c);
                xo = i - p * W_out;
                yo = p - q * H_out;
                c = q - r * a.C;
                n = r;
            }
        } else if (a.nhwc) {
            c = (int)(idx % a.C);
            xo = (int)((idx / a.C) % W_out);
            yo = (int)((idx / a.C / W_out) % H_out);
            n = idx / ((int64_t)a.C * W_out * H_out);
        } else {
            xo = (int)(idx % W_out);
            yo = (int)((idx / W_out) % H_out);
            c = (int)((idx / W_out / H_out) % a.C);
            n = idx / ((int64_t)a.C * W_out * H_out);
        }
        int tf[4];
        int t_first = a.T;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float v = a.in[n * a.iN + c * a.iC + (int64_t)(yo * 2 + (k >> 1)) * a.iY +
                                 (int64_t)(xo * 2 + (k & 1)) * a.iX];
            // arrival step, or -1: only 0 <= tf < T can ever set in_t
            tf[k] = (v >= 0.0f && v < (float)a.T) ? (int)v : -1;
            t_first = (tf[k] >= 0 && tf[k] < t_first) ? tf[k] : t_first;
        }
        float res = kInfTime;
        if (0.0f >= a.th) {
            res = 0.0f;  // V = +0 reaches th at step 0, input or not
        } else {
            float I = 0.0f, V = 0.0f;
            for (int t = t_first; t < a.T; ++t) {
                const float in = (tf[0] == t || tf[1] == t || tf[2] == t || tf[3] == t) ? 1.0f : 0.0f;
                I = __builtin_fmaf(I, a.decay, in);
                V = V + I;
                if (V >= a.th) {
                    res = (float)t;
                    break;
                }
            }
        }
        a.out[n * a.oN + c * a.oC + (int64_t)yo * a.oY + (int64_t)xo * a.oX] = res;
    }
}

// ---------------------------------------------------------------------------
struct CRecArgs {
    const int32_t* cin;  // drop-in: reference buckets
    const float* tin;
    const int32_t* off;
    const float* cur;    // engine: feed-forward input per step [N][T][out_f]
    float* out;
    const float* W;      // drop-in: [out][in]
    const float* Wrec;   // drop-in [i][j]; engine [j][i]
    int in_f, out_f, out_pad, T, D, NC;
    float decay, th;
};

// T3V:171-200: block per sample, thread i = neuron i.  The feed-forward
// input of step t is either accumulated per chunk in LDS from the reference
// buckets (drop-in, in bucket order) or read from k_bin_currents' output
// (engine).  Every step then adds the recurrent input of the neurons that
// fired on the previous step (ascending j), between two barriers as the
// reference does.
template <bool CURRENTS>
__global__ __launch_bounds__(1024) void k_culif_fc_rec(CRecArgs a) {
    extern __shared__ float in_ff[];              // drop-in: [D][out_pad]
    __shared__ unsigned long long fmask[16];      // fired on the previous step
    const int n = blockIdx.x;
    const int i = threadIdx.x;
    const bool ok = i < a.out_f;
    const int nwords = a.out_pad >> 6;
    if (i < 16) fmask[i] = 0ull;
    float I = 0.0f, V = 0.0f, my_fire = kInfTime;
    bool has_fired = false;
    const int OS = a.NC + 1;
    for (int ch = 0; ch < a.NC; ++ch) {
        const int base_t = ch * a.D;
        if (!CURRENTS) {
            const int32_t* sc = a.cin + (int64_t)n * a.in_f;
            const float* st = a.tin + (int64_t)n * a.in_f;
            for (int t = 0; t < a.D; ++t) in_ff[t * a.out_pad + i] = 0.0f;
            const int s = max(a.off[(int64_t)n * OS + ch], 0);
            const int e = min(a.off[(int64_t)n * OS + ch + 1], a.in_f);
            for (int p = s; p < e; ++p) {
                const int j = sc[p];
                const int dt = (int)st[p] - base_t;
                if (ok && (unsigned)dt < (unsigned)a.D && (unsigned)j < (unsigned)a.in_f)
                    in_ff[dt * a.out_pad + i] = in_ff[dt * a.out_pad + i] + a.W[(int64_t)i * a.in_f + j];
            }
        }
        for (int t = 0; t < a.D; ++t) {
            __syncthreads();
            float in_rec = 0.0f;
            for (int wd = 0; wd < nwords; ++wd) {
                unsigned long long m = fmask[wd];
                while (m) {
                    const int j = wd * 64 + __builtin_ctzll(m);
                    m &= m - 1;
                    if (ok)
                        in_rec = in_rec + (CURRENTS ? a.Wrec[(int64_t)j * a.out_f + i]
                                                    : a.Wrec[(int64_t)i * a.out_f + j]);
                }
            }
            float ff = 0.0f;
            if (CURRENTS)
                ff = ok ? a.cur[((int64_t)n * a.T + base_t + t) * a.out_f + i] : 0.0f;
            else
                ff = in_ff[t * a.out_pad + i];
            I = __builtin_fmaf(I, a.decay, ff) + in_rec;
            V = V + I;
            bool fire_now = false;
            if (ok && V >= a.th && !has_fired) {
                fire_now = true;
                has_fired = true;
                my_fire = (float)(base_t + t);
                V = -10000.0f;
            }
            __syncthreads();
            const unsigned long long b = __ballot(fire_now);
            if ((i & 63) == 0) fmask[i >> 6] = b;
        }
    }
    if (ok) a.out[(int64_t)n * a.out_f + i] = my_fire;
}

// Engine feed-forward currents of an FC layer:
//   cur[n][t][o] = sum over inputs j ascending with step(x[n][j]) == t of W_t[j][o]
// (T3V:78 arrival rule; W_t is the [in][out] transpose, so each term is one
// coalesced row segment), summed in the reference's bucket order.  The
// inputs of each sample are first counting-sorted by arrival step, stably in
// j, by three small kernels over segments of kFcSeg inputs (one wave each):
//   k_fcsort_count    per-segment step histogram (LDS atomics);
//   k_fcsort_offsets  per-sample offsets, step-major then segment order;
//   k_fcsort_scatter  each input's j to its step's list, ranked within a
//                     64-input chunk by a bit-ballot multisplit.
// k_fc_currents then gives each (sample, step, 64 outputs) wave its list:
// 32 rows gathered at a time with the next 32 in flight (entries read 64 at a time, a window ahead), added in list
// (= ascending j) order; the waves run step-major, so the long lists of the dense early steps start first.  Scanning
// every input per step group instead left each wave about one gather per
// 64-input chunk, a memory latency each.
constexpr int kFcSeg = 2048;    // inputs per sort segment
constexpr int kFcGroup = 32;    // rows gathered together
constexpr int kFcListPad = 6 * kFcGroup;  // list entries readable past the end (k_fc_currents' windows)

__global__ __launch_bounds__(256) void k_fcsort_count(const float* __restrict__ x, int32_t* __restrict__ counts,
                                                      int N, int F, int T, int S) {
    __shared__ int cnt_all[4][256];
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t u = (int64_t)blockIdx.x * 4 + wave;  // (n, segment)
    if (u >= (int64_t)N * S) return;                   // uniform per wave
    const int lane = lane_id();
    int* cnt = cnt_all[wave];
    for (int t = lane; t < T; t += 64) cnt[t] = 0;
    wave_sync();
    const int64_t n = u / S;
    const int j0 = (int)(u - n * S) * kFcSeg;
    const int j1 = (F - j0) < kFcSeg ? F : j0 + kFcSeg;
    const float* __restrict__ X = x + n * F;
    for (int jb = j0; jb < j1; jb += 64 * 4) {
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int j = jb + 64 * r + lane;
            v[r] = j < j1 ? X[j] : kInfTime;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int b = culif_bin(v[r], T);
            if (b >= 0) atomicAdd(&cnt[b], 1);
        }
    }
    wave_sync();
    for (int t = lane; t < T; t += 64) counts[u * T + t] = cnt[t];
}

// One block per sample, thread t = step (T <= 255 < blockDim).
__global__ __launch_bounds__(256) void k_fcsort_offsets(const int32_t* __restrict__ counts,
                                                        int32_t* __restrict__ offs,
                                                        int32_t* __restrict__ binstart, int T, int S) {
    __shared__ int base[257];
    const int64_t n = blockIdx.x;
    const int t = threadIdx.x;
    const int32_t* __restrict__ C = counts + n * S * T;
    int tot = 0;
    if (t < T)
        for (int s = 0; s < S; ++s) tot += C[(int64_t)s * T + t];
    if (t < T) base[t] = tot;
    __syncthreads();
    if (t == 0) {
        int run = 0;
        for (int k = 0; k < T; ++k) {
            const int v = base[k];
            base[k] = run;
            run += v;
        }
        base[T] = run;
    }
    __syncthreads();
    if (t <= T) binstart[n * (T + 1) + t] = base[t];
    if (t < T) {
        int run = base[t];
        for (int s = 0; s < S; ++s) {
            offs[(n * S + s) * T + t] = run;
            run += C[(int64_t)s * T + t];
        }
    }
}

__global__ __launch_bounds__(256) void k_fcsort_scatter(const float* __restrict__ x,
                                                        const int32_t* __restrict__ offs,
                                                        int32_t* __restrict__ list, int N, int F, int T,
                                                        int S, int nbits) {
    __shared__ int cur_all[4][256];
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t u = (int64_t)blockIdx.x * 4 + wave;
    if (u >= (int64_t)N * S) return;  // uniform per wave
    const int lane = lane_id();
    int* cur = cur_all[wave];
    for (int t = lane; t < T; t += 64) cur[t] = offs[u * T + t];
    wave_sync();
    const int64_t n = u / S;
    const int j0 = (int)(u - n * S) * kFcSeg;
    const int j1 = (F - j0) < kFcSeg ? F : j0 + kFcSeg;
    const float* __restrict__ X = x + n * F;
    int32_t* __restrict__ Ln = list + n * F;
    const uint64_t lt = lanemask_lt();
    float v_next = j0 + lane < j1 ? X[j0 + lane] : kInfTime;
    for (int jb = j0; jb < j1; jb += 64) {
        const float v = v_next;
        v_next = jb + 64 + lane < j1 ? X[jb + 64 + lane] : kInfTime;  // next chunk in flight
        const int b = culif_bin(v, T);
        const bool valid = b >= 0;
        uint64_t m = __ballot(valid);
        if (m == 0) continue;  // uniform
        for (int bit = 0; bit < nbits; ++bit) {
            const bool set = valid && ((b >> bit) & 1);
            const uint64_t bb = __ballot(set);
            m &= set ? bb : ~bb;
        }
        if (valid) Ln[cur[b] + __popcll(m & lt)] = jb + lane;
        wave_sync();
        if (valid && (m & lt) == 0) cur[b] += __popcll(m);
        wave_sync();
    }
}

__global__ __launch_bounds__(256) void k_fc_currents(const int32_t* __restrict__ list,
                                                     const int32_t* __restrict__ binstart,
                                                     const float* __restrict__ W, float* __restrict__ cur,
                                                     int N, int T, int F, int out_f, int n_oblk, int w_bytes) {
    const int wave = uniform(threadIdx.x >> 6);
    // step-major: the dense early steps, whose lists are the longest (and
    // bound the kernel's time), start first
    const int64_t u = (int64_t)blockIdx.x * 4 + wave;  // (t, n, oblk)
    if (u >= (int64_t)N * T * n_oblk) return;          // uniform per wave
    const int ob = (int)(u % n_oblk);
    const int64_t n = (u / n_oblk) % N;
    const int t = (int)(u / ((int64_t)n_oblk * N));
    const int lane = lane_id();
    const int o = ob * 64 + lane;
    const bool ok = o < out_f;
    const int32_t* __restrict__ L = list + n * F;
    const int beg = binstart[n * (T + 1) + t], end = binstart[n * (T + 1) + t + 1];
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, w_bytes, 0x00020000);
    const int voff = (ok ? o : 0) * 4;
    const int rowb = out_f * 4;
    float acc = 0.0f;
    // two groups of gathers in flight: the next group's are issued before
    // this group's are added.  List entries come 64 at a time, one per lane
    // (a window, read one window ahead), and v_readlane hands each gather its
    // row; the list is padded, so entries past `end` are read but never used
    // (the last window read starts below end + 96)
    static_assert(kFcGroup == 32, "two groups per 64-entry window");
    int wcur = L[beg + lane];       // entries beg + 64k .. beg + 64k + 63
    int wnxt = L[beg + 64 + lane];  // the window after it
    auto issue = [&](int i, int win, int half, float (&w)[kFcGroup]) {
#pragma unroll
        for (int g = 0; g < kFcGroup; ++g) {
            const int j = __builtin_amdgcn_readlane(win, 32 * half + g);
            w[g] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, (i + g < end ? j : 0) * rowb, 0));
        }
    };
    auto add = [&](int i, const float (&w)[kFcGroup]) {
        if (i + kFcGroup <= end) {
#pragma unroll
            for (int g = 0; g < kFcGroup; ++g) acc = acc + w[g];
        } else {
#pragma unroll
            for (int g = 0; g < kFcGroup; ++g)
                if (i + g < end) acc = acc + w[g];
        }
    };
    float w0[kFcGroup], w1[kFcGroup];
    if (beg < end) issue(beg, wcur, 0, w0);
    for (int i = beg; i < end; i += 2 * kFcGroup) {
        issue(i + kFcGroup, wcur, 1, w1);
        __builtin_amdgcn_sched_barrier(0);
        add(i, w0);
        if (i + kFcGroup >= end) break;
        issue(i + 2 * kFcGroup, wnxt, 0, w0);
        __builtin_amdgcn_sched_barrier(0);
        add(i + kFcGroup, w1);
        wcur = wnxt;
        wnxt = L[i + 128 + lane];
    }
    if (ok) cur[(n * T + t) * out_f + o] = acc;
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_nhwc_to_nchw(const float* __restrict__ in,
                                                      float* __restrict__ out, int64_t total, int C,
                                                      int H, int W) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int x = (int)(idx % W);
        const int y = (int)((idx / W) % H);
        const int c = (int)((idx / ((int64_t)W * H)) % C);
        const int64_t n = idx / ((int64_t)W * H * C);
        out[idx] = in[((n * H + y) * W + x) * C + c];
    }
}

unsigned flat_grid(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b > (1 << 20)) b = 1 << 20;
    return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

int check_culif_consts(const vdttfs_ctx* ctx) {
    if (ctx->c.T % ctx->c.delta != 0)
        return set_error(VDTTFS_E_UNSUPPORTED,
                         "CuLIF layers need delta to divide T (the reference chunk loop has no t < T guard)");
    return VDTTFS_OK;
}

namespace {

RawArgs raw_args(vdttfs_ctx* ctx, const float* data, float* out, const float* W, int N, int C_in,
                 int C_out, int H, int Wd, int nhwc_out, float decay, float th) {
    RawArgs a{};
    a.data = data;
    a.out = out;
    a.W = W;
    a.n_pix = (int64_t)N * H * Wd;
    a.C_in = C_in;
    a.C_out = C_out;
    a.H = H;
    a.Wd = Wd;
    a.T = ctx->c.T;
    a.n_cblk = (C_out + 63) / 64;
    if (nhwc_out) {
        a.sX = C_out;
        a.sY = (int64_t)Wd * C_out;
        a.sN = (int64_t)H * Wd * C_out;
        a.sC = 1;
    } else {
        a.sX = 1;
        a.sY = Wd;
        a.sC = (int64_t)H * Wd;
        a.sN = (int64_t)C_out * H * Wd;
    }
    a.decay = decay;
    a.th = th;
    return a;
}

}  // namespace

int launch_culif_conv1_raw(vdttfs_ctx* ctx, const float* data, float* out, const float* W, int N,
                           int C_in, int C_out, int H, int Wd, int nhwc_out, float decay, float th) {
    VD_TRY(check_culif_consts(ctx));
    if (N <= 0 || C_in <= 0 || C_out <= 0 || H <= 0 || Wd <= 0)
        return set_error(VDTTFS_E_INVALID, "culif_conv1_raw: non-positive shape");
    const RawArgs a = raw_args(ctx, data, out, W, N, C_in, C_out, H, Wd, nhwc_out, decay, th);
    if (C_in <= kTileMaxCin) {
        const int64_t blocks = (int64_t)N * H * ((Wd + kTileX - 1) / kTileX) * a.n_cblk;
        if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "culif_conv1_raw: grid too large");
        hipLaunchKernelGGL(k_culif_conv1_tile, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a);
        VD_HIP(hipGetLastError());
        return VDTTFS_OK;
    }
    const int64_t blocks = ((a.n_pix + 3) / 4) * a.n_cblk;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "culif_conv1_raw: grid too large");
    hipLaunchKernelGGL(k_culif_conv1_lane, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

bool culif_conv1_mask_ok(int C_in) { return C_in >= 1 && C_in <= kMaskMaxCin; }

int launch_culif_conv1_mask(vdttfs_ctx* ctx, const float* data, float* out, const float* W, int N, int C_in,
                            int C_out, int H, int Wd, int nhwc_out, float decay, float th, uint64_t* mask,
                            uint32_t* nonbin, uint8_t* fired) {
    VD_TRY(check_culif_consts(ctx));
    if (N <= 0 || C_in <= 0 || C_out <= 0 || H <= 0 || Wd <= 0)
        return set_error(VDTTFS_E_INVALID, "culif_conv1_mask: non-positive shape");
    if (!culif_conv1_mask_ok(C_in))
        return set_error(VDTTFS_E_UNSUPPORTED, "culif_conv1_mask: C_in %d > %d", C_in, kMaskMaxCin);
    RawArgs a = raw_args(ctx, data, out, W, N, C_in, C_out, H, Wd, nhwc_out, decay, th);
    if (fired && a.n_cblk != 1) return set_error(VDTTFS_E_INVALID, "culif_conv1_mask: fired flags need C_out <= 64");
    a.fired = fired;
    const int nblk = (a.T + 63) / 64;
    const int64_t sites = (int64_t)N * C_in * H * Wd;
    if (a.n_pix >= (INT64_C(1) << 31) || sites >= (INT64_C(1) << 31))
        return set_error(VDTTFS_E_UNSUPPORTED, "culif_conv1_mask: more than 2^31 sites");
    MaskArgs m{data, mask, nonbin, sites * nblk, a.T, nblk};
    const int64_t mwaves = (m.units + kMaskUnitsPerWave - 1) / kMaskUnitsPerWave;
    const int64_t mblocks = (mwaves + 3) / 4;
    if (mblocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "culif_conv1_mask: grid too large");
    hipLaunchKernelGGL(k_culif_event_masks, dim3((unsigned)mblocks), dim3(256), 0, ctx->stream, m);
    VD_HIP(hipGetLastError());
    const int64_t blocks = ((a.n_pix + 4 * kMaskPixPerWave - 1) / (4 * kMaskPixPerWave)) * a.n_cblk;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "culif_conv1_mask: grid too large");
    switch (C_in) {
        case 1:
            hipLaunchKernelGGL(k_culif_conv1_mask<9>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a,
                               mask, nonbin, nblk);
            break;
        case 2:
            hipLaunchKernelGGL(k_culif_conv1_mask<18>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a,
                               mask, nonbin, nblk);
            break;
        default:
            hipLaunchKernelGGL(k_culif_conv1_mask<27>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a,
                               mask, nonbin, nblk);
            break;
    }
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_culif_bucketize(vdttfs_ctx* ctx, const float* in, int64_t n_sites, int C, int HW,
                           int32_t* cin, float* tin, int32_t* off) {
    VD_TRY(check_culif_consts(ctx));
    const int NC = ctx->c.T / ctx->c.delta;
    if (NC > kCBktMaxChunks)
        return set_error(VDTTFS_E_UNSUPPORTED, "culif bucketize: T/delta = %d chunks > %d", NC,
                         kCBktMaxChunks);
    if (n_sites <= 0 || C <= 0 || HW <= 0) return set_error(VDTTFS_E_INVALID, "culif bucketize: bad shape");
    CBktArgs a{in, cin, tin, off, n_sites, C, HW, ctx->c.T, ctx->c.delta, NC};
    if (n_sites <= kCBktWaveMaxSites) {  // a thread per site would leave the device idle
        hipLaunchKernelGGL(k_culif_bucketize_wave, dim3((unsigned)((n_sites + 3) / 4)), dim3(256), 0, ctx->stream, a);
        VD_HIP(hipGetLastError());
        return VDTTFS_OK;
    }
    const int64_t blocks = (n_sites + kCBktThreads - 1) / kCBktThreads;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "culif bucketize: grid too large");
    hipLaunchKernelGGL(k_culif_bucketize, dim3((unsigned)blocks), dim3(kCBktThreads), 0, ctx->stream, a);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_culif_generic(vdttfs_ctx* ctx, const int32_t* cin, const float* tin, const int32_t* off,
                         float* out, const float* W, int N, int C_in, int C_out, int H, int Wd,
                         int is_fc, float decay, float th) {
    VD_TRY(check_culif_consts(ctx));
    CGenArgs a{};
    a.cin = cin;
    a.tin = tin;
    a.off = off;
    a.out = out;
    a.W = W;
    a.C_in = C_in;
    a.C_out = C_out;
    a.H = is_fc ? 1 : H;
    a.Wd = is_fc ? 1 : Wd;
    a.T = ctx->c.T;
    a.D = ctx->c.delta;
    a.NC = a.T / a.D;
    a.decay = decay;
    a.th = th;
    a.total = (int64_t)N * C_out * a.H * a.Wd;
    if (a.total <= 0) return set_error(VDTTFS_E_INVALID, "culif integrate: bad shape");
    const unsigned g = flat_grid(a.total);
#define VD_CG(FC, DM) hipLaunchKernelGGL((k_culif_generic<FC, DM>), dim3(g), dim3(256), 0, ctx->stream, a)
    if (a.D <= 32) {
        if (is_fc) VD_CG(true, 32); else VD_CG(false, 32);
    } else if (a.D <= 64) {
        if (is_fc) VD_CG(true, 64); else VD_CG(false, 64);
    } else {
        if (is_fc) VD_CG(true, 256); else VD_CG(false, 256);
    }
#undef VD_CG
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_culif_pool(vdttfs_ctx* ctx, const float* in, float* out, int N, int C, int H_in, int W_in,
                      int nhwc_in, int nhwc_out, float decay, float th) {
    VD_TRY(check_culif_consts(ctx));
    if (N <= 0 || C <= 0 || H_in < 2 || W_in < 2)
        return set_error(VDTTFS_E_INVALID, "culif_pool: bad shape");
    const int H_out = H_in / 2, W_out = W_in / 2;
    CPoolArgs a{};
    a.in = in;
    a.out = out;
    a.total = (int64_t)N * C * H_out * W_out;
    a.C = C;
    a.H_in = H_in;
    a.W_in = W_in;
    a.T = ctx->c.T;
    a.nhwc = nhwc_out;
    if (nhwc_in) {
        a.iC = 1; a.iX = C; a.iY = (int64_t)W_in * C; a.iN = (int64_t)H_in * W_in * C;
    } else {
        a.iX = 1; a.iY = W_in; a.iC = (int64_t)H_in * W_in; a.iN = (int64_t)C * H_in * W_in;
    }
    if (nhwc_out) {
        a.oC = 1; a.oX = C; a.oY = (int64_t)W_out * C; a.oN = (int64_t)H_out * W_out * C;
    } else {
        a.oX = 1; a.oY = W_out; a.oC = (int64_t)H_out * W_out; a.oN = (int64_t)C * H_out * W_out;
    }
    a.decay = decay;
    a.th = th;
    a.div_c = make_fastdiv(C);
    a.div_w = make_fastdiv(W_out > 0 ? W_out : 1);
    a.div_h = make_fastdiv(H_out > 0 ? H_out : 1);
    if (a.total < (INT64_C(1) << 31))
        hipLaunchKernelGGL(k_culif_pool<true>, dim3(flat_grid(a.total)), dim3(256), 0, ctx->stream, a);
    else
        hipLaunchKernelGGL(k_culif_pool<false>, dim3(flat_grid(a.total)), dim3(256), 0, ctx->stream, a);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_culif_fc_rec(vdttfs_ctx* ctx, const int32_t* cin, const float* tin, const int32_t* off,
                        const float* cur, float* out, const float* W, const float* Wrec, int N,
                        int in_f, int out_f, float decay, float th) {
    VD_TRY(check_culif_consts(ctx));
    if (N <= 0 || in_f <= 0 || out_f <= 0 || out_f > 1024)
        return set_error(VDTTFS_E_UNSUPPORTED, "culif_fc_recurrent: needs 1 <= out_f <= 1024");
    CRecArgs a{};
    a.cin = cin;
    a.tin = tin;
    a.off = off;
    a.cur = cur;
    a.out = out;
    a.W = W;
    a.Wrec = Wrec;
    a.in_f = in_f;
    a.out_f = out_f;
    a.out_pad = (out_f + 63) / 64 * 64;
    a.T = ctx->c.T;
    a.D = ctx->c.delta;
    a.NC = a.T / a.D;
    a.decay = decay;
    a.th = th;
    if (cur) {
        hipLaunchKernelGGL(k_culif_fc_rec<true>, dim3(N), dim3(a.out_pad), 0, ctx->stream, a);
    } else {
        const size_t lds = (size_t)a.D * a.out_pad * sizeof(float);
        if (lds > 64 * 1024)
            return set_error(VDTTFS_E_UNSUPPORTED, "culif_fc_recurrent: delta*out_f*4 = %zu B > 64 KB", lds);
        hipLaunchKernelGGL(k_culif_fc_rec<false>, dim3(N), dim3(a.out_pad), lds, ctx->stream, a);
    }
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

FcSortSizes fc_sort_sizes(int N, int F, int T) {
    FcSortSizes z;
    z.segments = (F + kFcSeg - 1) / kFcSeg;
    z.counts = (int64_t)N * z.segments * T;
    z.binstart = (int64_t)N * (T + 1);
    z.list = (int64_t)N * F + kFcListPad;
    return z;
}

int launch_fc_currents(vdttfs_ctx* ctx, const float* x, const float* W_t, float* cur, int N, int F, int out_f,
                       const FcSortScratch& sc) {
    const int T = ctx->c.T;
    if (N <= 0 || F <= 0 || out_f <= 0) return set_error(VDTTFS_E_INVALID, "fc currents: bad shape");
    if ((int64_t)F * out_f * 4 >= (INT64_C(1) << 31) || (int64_t)N * F >= (INT64_C(1) << 31))
        return set_error(VDTTFS_E_UNSUPPORTED, "fc currents: weights or inputs beyond 2^31");
    const FcSortSizes z = fc_sort_sizes(N, F, T);
    const int S = z.segments;
    int nbits = 0;
    while ((1 << nbits) < T) ++nbits;
    const int64_t sblocks = ((int64_t)N * S + 3) / 4;
    hipLaunchKernelGGL(k_fcsort_count, dim3((unsigned)sblocks), dim3(256), 0, ctx->stream, x, sc.counts, N, F,
                       T, S);
    hipLaunchKernelGGL(k_fcsort_offsets, dim3((unsigned)N), dim3(256), 0, ctx->stream, sc.counts, sc.offs,
                       sc.binstart, T, S);
    hipLaunchKernelGGL(k_fcsort_scatter, dim3((unsigned)sblocks), dim3(256), 0, ctx->stream, x, sc.offs, sc.list,
                       N, F, T, S, nbits);
    const int n_oblk = (out_f + 63) / 64;
    const int64_t waves = (int64_t)N * T * n_oblk;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "fc currents: grid too large");
    hipLaunchKernelGGL(k_fc_currents, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, sc.list, sc.binstart,
                       W_t, cur, N, T, F, out_f, n_oblk, (int)((int64_t)F * out_f * 4));
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_nhwc_to_nchw(vdttfs_ctx* ctx, const float* in, float* out, int N, int C, int H, int W) {
    const int64_t total = (int64_t)N * C * H * W;
    hipLaunchKernelGGL(k_nhwc_to_nchw, dim3(flat_grid(total)), dim3(256), 0, ctx->stream, in, out,
                       total, C, H, W);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

}  // namespace vdttfs
