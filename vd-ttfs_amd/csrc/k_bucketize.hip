// Arrival-time counting sort of each input column's spikes (the reference's
// k_bucketize, T1V:45-80 / T2V:45-81), rebuilt for wave64:
//  * a wave owns 64/SEG columns, SEG = next_pow2(C_in) capped at 64, so even
//    C_in = 1 or 3 keeps every lane busy and reads stay coalesced;
//  * pass 1 builds a wave-private histogram in LDS (order-free atomics);
//  * a wave prefix scan turns it into bucket offsets, written coalesced;
//  * pass 2 scatters stably: lanes sharing a bucket are ranked in lane
//    (= ascending cin) order by a bitwise multisplit (one ballot per bit of
//    the bucket index), so the output order is exactly the reference's
//    serial loop.
// Two output layouts share the code:
//  * REF  - buckets are Delta-wide chunks, events (cin, raw t): bit-exact
//           reference layout (off[col*(NC+1)+c], cin/tin[col*C_in+pos]);
//  * BINS - buckets are single arrival bins (T+1 offsets per column), events
//           packed as (cin | bin<<24, alpha[idx]) for the engine's integrator.
#include "common.h"
#include "wave.h"

namespace vdttfs {
namespace {

struct BktParams {
    int T;
    float tfs;
    int delta;
    int alpha_by_time;
};

template <bool BINS>
__global__ __launch_bounds__(256) void k_bucketize(
    const float* __restrict__ in, int64_t n_cols, int c_in, int seg_log2, BktParams p, int nb,
    int32_t* __restrict__ out_cin, float* __restrict__ out_tin, vd_event* __restrict__ out_ev,
    const float* __restrict__ alpha, int32_t* __restrict__ out_off,
    unsigned long long* __restrict__ n_ev_counter) {
    extern __shared__ int lds[];
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int seg_size = 1 << seg_log2;
    const int cpw = 64 >> seg_log2;  // columns per wave
    const int OS = nb + 1;
    int* cur = lds + wave * cpw * OS;
    const int64_t col0 = ((int64_t)blockIdx.x * (blockDim.x >> 6) + wave) * cpw;
    if (col0 >= n_cols) return;  // uniform per wave
    const int seg = lane >> seg_log2;
    const int l = lane & (seg_size - 1);
    const int64_t col = col0 + seg;
    const bool col_ok = col < n_cols;
    const uint64_t segmask =
        (seg_size == 64) ? ~0ull : (((1ull << seg_size) - 1ull) << (seg * seg_size));
    const uint64_t lt = lanemask_lt();

    for (int i = lane; i < cpw * OS; i += 64) cur[i] = 0;
    wave_sync();
    const float* src = in + (col_ok ? col : col0) * (int64_t)c_in;

    // pass 1: per-column histogram
    for (int base = 0; base < c_in; base += seg_size) {
        const int i = base + l;
        if (col_ok && i < c_in) {
            const int tb = arrival_bin(src[i], p.tfs, p.T);
            if (tb >= 0) atomicAdd(&cur[seg * OS + (BINS ? tb : tb / p.delta)], 1);
        }
    }
    wave_sync();

    // exclusive scan of each column's counts; slot nb receives the total
    if (cpw == 1) {
        int run = 0;
        for (int b0 = 0; b0 < OS; b0 += 64) {
            const int b = b0 + lane;
            const int v = (b < nb) ? cur[b] : 0;
            const int incl = wave_incl_scan(v);
            if (b < OS) cur[b] = run + incl - v;
            run += __shfl(incl, 63, 64);
        }
    } else if (l == 0 && col_ok) {
        int run = 0;
        for (int b = 0; b < nb; ++b) {
            const int v = cur[seg * OS + b];
            cur[seg * OS + b] = run;
            run += v;
        }
        cur[seg * OS + nb] = run;
    }
    wave_sync();

    // offsets of the wave's columns are one contiguous block
    {
        const int64_t ncol_here = (n_cols - col0) < cpw ? (n_cols - col0) : cpw;
        const int total = (int)ncol_here * OS;
        for (int i = lane; i < total; i += 64) out_off[col0 * OS + i] = cur[i];
        if (n_ev_counter != nullptr) {
            int mine = (l == 0 && col_ok) ? cur[seg * OS + nb] : 0;
            for (int off = 32; off > 0; off >>= 1) mine += __shfl_xor(mine, off, 64);
            if (lane == 0) atomicAdd(counter_stripe(n_ev_counter), (unsigned long long)mine);
        }
    }
    wave_sync();

    // pass 2: stable scatter; a lane's rank in its bucket is the number of
    // lower lanes of its column with the same bucket (multisplit over the
    // ceil(log2 nb) bits of the bucket index), so one pass per chunk
    const int nbits = nb > 1 ? 32 - __clz(nb - 1) : 0;
    for (int base = 0; base < c_in; base += seg_size) {
        const int i = base + l;
        float t = 0.0f;
        int tb = -1;
        if (col_ok && i < c_in) {
            t = src[i];
            tb = arrival_bin(t, p.tfs, p.T);
        }
        const int b = (tb < 0) ? -1 : (BINS ? tb : tb / p.delta);
        const bool active = b >= 0;
        // lanes of this column in the same bucket: AND of per-bit ballots
        uint64_t same = __ballot(active) & segmask;
        for (int k = 0; k < nbits; ++k) {
            const uint64_t ones = __ballot(active && ((b >> k) & 1));
            same &= ((b >> k) & 1) ? ones : ~ones;
        }
        if (active) {
            const int pos = cur[seg * OS + b] + __popcll(same & lt);
            const int64_t dst = col * (int64_t)c_in + pos;
            if (BINS) {
                vd_event e;
                e.key = (uint32_t)i | ((uint32_t)tb << 24);
                e.alpha = alpha[alpha_index(t, tb, p.alpha_by_time, p.T)];
                out_ev[dst] = e;
            } else {
                out_cin[dst] = i;
                out_tin[dst] = t;
            }
        }
        wave_sync();
        if (active && (same & lt) == 0) cur[seg * OS + b] += __popcll(same);
        wave_sync();
    }
}

// Long columns on a narrow grid (an FC layer's inputs: a few hundred columns
// of thousands of inputs each) would leave most of the chip idle with one
// wave per column walking its chunks one load at a time.  k_bucketize_wide
// gives each column a workgroup of W waves: wave w takes a contiguous range of
// 64-input chunks, counts it into its own LDS histogram, then wave 0 turns the
// W histograms into the column's bucket offsets and each wave's starting
// cursor per bucket (buckets in order, waves in order within a bucket), and
// every wave places its chunks as k_bucketize does.  Waves hold consecutive
// cin ranges, so the placement is the same stable (bucket, cin) order.
// Loads are issued 8 chunks at a time.
constexpr int kWideWaves = 8;
constexpr int kWideBatch = 8;

template <bool BINS>
__global__ __launch_bounds__(64 * kWideWaves) void k_bucketize_wide(
    const float* __restrict__ in, int c_in, BktParams p, int nb, int32_t* __restrict__ out_cin,
    float* __restrict__ out_tin, vd_event* __restrict__ out_ev, const float* __restrict__ alpha,
    int32_t* __restrict__ out_off, unsigned long long* __restrict__ n_ev_counter) {
    extern __shared__ int lds[];
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t col = blockIdx.x;
    const int OS = nb + 1;
    int* cur = lds + wave * OS;  // this wave's counts, then its cursors
    const float* src = in + col * (int64_t)c_in;
    const int n_chunks = (c_in + 63) >> 6;
    const int per = (n_chunks + kWideWaves - 1) / kWideWaves;
    const int c_begin = wave * per;
    const int c_end = c_begin + per < n_chunks ? c_begin + per : n_chunks;
    for (int i = lane; i < OS; i += 64) cur[i] = 0;
    wave_sync();
    // element `lane` of chunks c0 .. c0+kWideBatch-1 (past the range: no event)
    auto load_batch = [&](int c0, float (&x)[kWideBatch]) {
#pragma unroll
        for (int k = 0; k < kWideBatch; ++k) {
            const int i = (c0 + k) * 64 + lane;
            const bool ok = c0 + k < c_end && i < c_in;
            const float v = src[ok ? i : 0];
            x[k] = ok ? v : kInfTime;
        }
    };
    // pass 1: this wave's histogram
    for (int c0 = c_begin; c0 < c_end; c0 += kWideBatch) {
        float x[kWideBatch];
        load_batch(c0, x);
#pragma unroll
        for (int k = 0; k < kWideBatch; ++k) {
            const int tb = arrival_bin(x[k], p.tfs, p.T);
            if (tb >= 0) atomicAdd(&cur[BINS ? tb : tb / p.delta], 1);
        }
    }
    __syncthreads();
    // wave 0: the column's bucket offsets; every wave's cursor per bucket
    if (wave == 0) {
        int run = 0;
        for (int b0 = 0; b0 < nb; b0 += 64) {
            const int b = b0 + lane;
            int tot = 0;
            if (b < nb)
                for (int w = 0; w < kWideWaves; ++w) tot += lds[w * OS + b];
            const int incl = wave_incl_scan(tot);
            if (b < nb) {
                int s = run + incl - tot;
                out_off[col * OS + b] = s;
                for (int w = 0; w < kWideWaves; ++w) {
                    const int c = lds[w * OS + b];
                    lds[w * OS + b] = s;
                    s += c;
                }
            }
            run += __shfl(incl, 63, 64);
        }
        if (lane == 0) {
            out_off[col * OS + nb] = run;
            if (n_ev_counter != nullptr) atomicAdd(counter_stripe(n_ev_counter), (unsigned long long)run);
        }
    }
    __syncthreads();
    // pass 2: stable scatter of this wave's chunks (multisplit ranks, as k_bucketize)
    const uint64_t lt = lanemask_lt();
    const int nbits = nb > 1 ? 32 - __clz(nb - 1) : 0;
    for (int c0 = c_begin; c0 < c_end; c0 += kWideBatch) {
        float x[kWideBatch];
        load_batch(c0, x);
#pragma unroll
        for (int k = 0; k < kWideBatch; ++k) {
            if (c0 + k >= c_end) break;  // uniform
            const int i = (c0 + k) * 64 + lane;
            const float t = x[k];
            const int tb = arrival_bin(t, p.tfs, p.T);
            const int b = (tb < 0) ? -1 : (BINS ? tb : tb / p.delta);
            const bool active = b >= 0;
            uint64_t same = __ballot(active);
            for (int bit = 0; bit < nbits; ++bit) {
                const uint64_t ones = __ballot(active && ((b >> bit) & 1));
                same &= ((b >> bit) & 1) ? ones : ~ones;
            }
            if (active) {
                const int pos = cur[b] + __popcll(same & lt);
                const int64_t dst = col * (int64_t)c_in + pos;
                if (BINS) {
                    vd_event e;
                    e.key = (uint32_t)i | ((uint32_t)tb << 24);
                    e.alpha = alpha[alpha_index(t, tb, p.alpha_by_time, p.T)];
                    out_ev[dst] = e;
                } else {
                    out_cin[dst] = i;
                    out_tin[dst] = t;
                }
            }
            wave_sync();
            if (active && (same & lt) == 0) cur[b] += __popcll(same);
            wave_sync();
        }
    }
}

int seg_log2_for(int c_in) {
    int s = 0;
    while ((1 << s) < c_in && s < 6) ++s;
    return s;
}

template <bool BINS>
int launch_bucketize(vdttfs_ctx* ctx, const float* in, int64_t n_cols, int c_in, int nb,
                     int32_t* out_cin, float* out_tin, vd_event* out_ev, const float* alpha,
                     int32_t* out_off, unsigned long long* n_ev_counter) {
    if (n_cols <= 0 || c_in <= 0) return VDTTFS_OK;
    BktParams p{ctx->c.T, ctx->c.tfs, ctx->c.delta, ctx->c.alpha_by_time};
    // few long columns: a workgroup per column (fewer columns than 2 waves per
    // SIMD of a 256-CU device, at least 8 chunks each)
    if (c_in >= 64 * kWideWaves && n_cols < 2048 && (size_t)kWideWaves * (nb + 1) * sizeof(int) <= 64 * 1024) {
        hipLaunchKernelGGL(k_bucketize_wide<BINS>, dim3((unsigned)n_cols), dim3(64 * kWideWaves),
                           (size_t)kWideWaves * (nb + 1) * sizeof(int), ctx->stream, in, c_in, p, nb, out_cin,
                           out_tin, out_ev, alpha, out_off, n_ev_counter);
        VD_HIP(hipGetLastError());
        return VDTTFS_OK;
    }
    // one segment per column; widen segments (fewer columns per wave) until
    // the wave's bucket counters fit 16 KB, so 4 waves stay within 64 KB
    int sl = seg_log2_for(c_in);
    while (sl < 6 && (size_t)(64 >> sl) * (nb + 1) * sizeof(int) > 16 * 1024) ++sl;
    const int cpw = 64 >> sl;
    const size_t wave_lds = (size_t)cpw * (nb + 1) * sizeof(int);
    const int waves = 4;
    if (wave_lds * waves > 64 * 1024)
        return set_error(VDTTFS_E_UNSUPPORTED, "bucketize: %d buckets exceed LDS", nb);
    const int64_t n_waves = (n_cols + cpw - 1) / cpw;
    const int64_t blocks = (n_waves + waves - 1) / waves;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "bucketize: grid too large");
    hipLaunchKernelGGL(k_bucketize<BINS>, dim3((unsigned)blocks), dim3(64 * waves),
                       wave_lds * waves, ctx->stream, in, n_cols, c_in, sl, p, nb, out_cin,
                       out_tin, out_ev, alpha, out_off, n_ev_counter);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

}  // namespace

int launch_bucketize_ref(vdttfs_ctx* ctx, const float* in, int64_t n_cols, int c_in,
                         int32_t* out_cin, float* out_tin, int32_t* out_off) {
    return launch_bucketize<false>(ctx, in, n_cols, c_in, ctx->NC, out_cin, out_tin, nullptr,
                                   nullptr, out_off, nullptr);
}

int launch_bucketize_bins(vdttfs_ctx* ctx, const float* in, int64_t n_cols, int c_in,
                          const float* alpha, vd_event* out_ev, int32_t* out_off,
                          unsigned long long* n_ev_counter) {
    if (c_in >= (1 << 24))
        return set_error(VDTTFS_E_UNSUPPORTED, "bucketize: C_in %d >= 2^24", c_in);
    return launch_bucketize<true>(ctx, in, n_cols, c_in, ctx->c.T, nullptr, nullptr, out_ev,
                                  alpha, out_off, n_ev_counter);
}

}  // namespace vdttfs
