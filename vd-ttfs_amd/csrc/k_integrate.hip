// Chunked early-exit integrator (the reference's k_conv_bucketed,
// T1V:83-162 / T2V:84-170) for gfx950.
//
// Per neuron the result is fixed by the reference's arithmetic: for every
// arrival bin t, delta_t = fma-chain over the bin's events in (kh, kw) order,
// then ascending cin, starting from 0.0f; then carry += delta_t and the neuron
// fires at the first t >= t_min with carry >= theta[t] >= 1e-5f.  Both kernels
// below keep exactly that per-bin order, so their output is bit-identical to
// the reference for every chunk width (chunking only regroups whole bins).
//
// Engine path, two kernels per layer:
//  k_merge  - one wave per output pixel: the in-bounds receptive columns'
//             bin-sorted event lists are merged into (bin, column, cin)
//             order with a closed-form position table and written to HBM as
//             {weight-row byte offset, alpha} pairs plus T+1 bin starts.
//  k_stream - one wave64 per (output pixel, c_out block); lanes are c_out, so
//             each event is wave-uniform: the list is read through the scalar
//             cache 8 events at a time and every weight gather is one
//             coalesced row segment (dword or dwordx4 per lane); with one
//             c_out per lane two groups of 8 gathers are in flight.  Bins are
//             closed between fmas; lanes that fired stop fetching and the wave
//             leaves once its ballot of live lanes is empty.
//
// k_integrate_generic: one thread per neuron, the reference loop nest over
// either the reference bucket layout (drop-in) or the engine's bin layout
// (narrow layers), with the chunk's delta[] in private memory.
#include <atomic>
#include <type_traits>

#include "common.h"
#include "wave.h"

namespace vdttfs {
namespace {

constexpr int kBlockBins = 64;  // arrival bins handled per table / per VGPR of bin starts
constexpr int kListPad = 32;    // zeroed entries after each pixel's merged list (four groups)
constexpr int kMergeWaves = 4;
// most waves per workgroup of k_stream_quad.  Each wave has its own LDS
// region and pixels, so a workgroup is only the unit its LDS is freed in;
// the launcher picks 1 or 4 (see launch_integrate_dense).
constexpr int kQuadWaves = 4;

// ---------------------------------------------------------------------------
// k_merge: one wave per output pixel.  The in-bounds receptive columns' bin
// lists are merged into (bin, column, cin) order -- the per-bin fma order of
// the reference -- with a closed-form position table: event i of column k in
// bin t lands at D[k][t] + i, D[k][t] = sum_{k'<k} O_k'[t+1] + sum_{k'>k} O_k'[t]
// (O_k = the column's bin offsets).  Entries are (weight-row byte offset,
// alpha bits); bstart[pix][t] is the merged start of bin t.  The list is read
// by every c_out block of the pixel, so it is built once.
struct MergeArgs {
    int2* list;            // [n_pix][cap]
    int32_t* bstart;       // [n_pix][T+1]
    const vd_event* ev;    // bin layout [n_cols][C_in]
    const int32_t* off;    // [n_cols][T+1]
    int64_t n_pix;
    int64_t cap;
    int T;
    int H_in, W_in, C_in, H_out, W_out, K_h, K_w, pad_h, pad_w, is_fc;
    int rowbytes;          // C_out * 4
    FastDiv div_w, div_h;  // by W_out, H_out (n_pix < 2^31)
};

template <int KMAX>
__global__ __launch_bounds__(64 * kMergeWaves) void k_merge(MergeArgs a) {
    __shared__ int dtab_all[kMergeWaves][KMAX * kBlockBins];
    __shared__ int kinfo_all[kMergeWaves][2 * KMAX];
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t pix = (int64_t)blockIdx.x * kMergeWaves + wave;
    if (pix >= a.n_pix) return;  // uniform per wave
    int* dtab = dtab_all[wave];
    int* kinfo = kinfo_all[wave];

    int img, h_out = 0, w_out = 0;
    if (a.is_fc) {
        img = (int)pix;
    } else {
        const int q = fdiv((int)pix, a.div_w);
        w_out = (int)pix - q * a.W_out;
        img = fdiv(q, a.div_h);
        h_out = q - img * a.H_out;
    }
    // in-bounds receptive columns, compacted in (kh, kw) order
    int nk;
    if (a.is_fc) {
        nk = 1;
        if (lane == 0) {
            kinfo[0] = img;
            kinfo[KMAX] = 0;
        }
    } else {
        bool v = false;
        int col = 0;
        if (lane < a.K_h * a.K_w) {
            const int kh = lane / a.K_w, kw = lane - kh * a.K_w;
            const int hi = h_out - a.pad_h + kh, wi = w_out - a.pad_w + kw;
            v = hi >= 0 && hi < a.H_in && wi >= 0 && wi < a.W_in;
            col = (img * a.H_in + hi) * a.W_in + wi;
        }
        const uint64_t m = __ballot(v);
        nk = __popcll(m);
        if (v) {
            const int slot = __popcll(m & lanemask_lt());
            kinfo[slot] = col;
            kinfo[KMAX + slot] = lane * a.C_in * a.rowbytes;
        }
    }
    wave_sync();
    int colk[KMAX], krow[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        colk[k] = (k < nk) ? uniform(kinfo[k]) : 0;
        krow[k] = (k < nk) ? uniform(kinfo[KMAX + k]) : 0;
    }

    int2* out = a.list + pix * a.cap;
    int32_t* bs = a.bstart + pix * (int64_t)(a.T + 1);
    const int osb = a.T + 1;
    int base = 0;  // merged position of the current block's first event
    for (int t0 = 0; t0 < a.T; t0 += kBlockBins) {
        const int nb = (a.T - t0) < kBlockBins ? (a.T - t0) : kBlockBins;
        int o[KMAX], on[KMAX];
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            o[k] = 0;
            on[k] = 0;
            if (k < nk && lane < nb) {
                const int32_t* ob = a.off + (int64_t)colk[k] * osb + t0 + lane;
                o[k] = ob[0];
                on[k] = ob[1];
            }
        }
        int S = 0;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) S += o[k];
        const int C0 = uniform(S);
        int A = 0, P = 0;
        int st[KMAX], cnt[KMAX];  // per column: first event of the block, events in the block
        int total = 0;            // events of the block
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            st[k] = 0;
            cnt[k] = 0;
            if (k < nk) {
                P += o[k];
                if (lane < nb) dtab[k * kBlockBins + lane] = A + (S - P) - C0;
                A += on[k];
                st[k] = __builtin_amdgcn_readlane(o[k], 0);
                cnt[k] = __builtin_amdgcn_readlane(on[k], nb - 1) - st[k];
                total += cnt[k];
            }
        }
        if (lane < nb) bs[t0 + lane] = base + S - C0;
        wave_sync();
        // column by column, lanes over the column's events (the column and
        // its weight-row base stay wave-uniform)
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            if (k < nk) {  // uniform
                const vd_event* evk = a.ev + (int64_t)colk[k] * a.C_in + st[k];
                const int* dk = dtab + k * kBlockBins - t0;
                for (int f = lane; f < cnt[k]; f += 64) {
                    const vd_event e = evk[f];
                    const int pos = dk[(int)(e.key >> 24)] + st[k] + f;
                    out[base + pos] = make_int2(krow[k] + (int)(e.key & 0xFFFFFFu) * a.rowbytes,
                                                __float_as_int(e.alpha));
                }
            }
        }
        base += total;
        wave_sync();
    }
    if (lane == 0) bs[a.T] = base;
    // zeroed tail: the stream kernel reads whole groups of 8 entries
    if (lane < kListPad) out[base + lane] = make_int2(0, 0);
}

// ---------------------------------------------------------------------------
// k_merge_dense: the same merged list built straight from the dense NHWC
// spike map, for conv layers with C_in <= 64, so they need no separate
// bucketize pass.  One wave per output pixel counting-sorts the pixel's
// receptive events by arrival bin in LDS.  The pixel's (tap, cin) elements,
// flattened in (kh, kw, cin) order, are taken 64 per chunk (a 3-channel
// layer's 27 elements are one chunk): pass 1 counts every bin, a wave scan
// gives the bin starts, pass 2 (re-reading the chunk, now in cache) places
// each event at its bin's
// cursor plus its rank among the chunk's lanes of the same bin.  The rank
// comes from the bin's LDS bit mask of the chunk's lanes (k_merge_dense), or
// from a multisplit of bit ballots (same-bin mask = AND over the bin's bits
// of the matching ballot; k_stream_dense), so the order within a bin is
// (kh, kw, cin) -- the reference's per-bin fma order.  Neighbouring pixels
// read the same columns, which stay in L2.
struct DenseMergeArgs {
    int2* list;            // [n_pix][cap]
    int32_t* bstart;       // [n_pix][T+1]
    const float* in;       // [n_cols][C_in] spike times
    const float* alpha;    // decay LUT, T+1 entries
    int64_t n_pix;
    int64_t cap;
    int T;
    float tfs;
    int alpha_by_time;
    int nbits;             // bits of a bin index (ceil(log2 T))
    int H_in, W_in, C_in, H_out, W_out, K_h, K_w, pad_h, pad_w;
    int rowbytes;          // C_out * 4
    float inv_cin;         // 1 / C_in
    const uint8_t* fired;  // CuLIF: per input site, nonzero where a channel spiked (or null)
    FastDiv div_w, div_h;  // by W_out, H_out (n_pix < 2^31)
    int in_bytes;          // bytes of `in` (k_stream_quad: below 2^31), else 0
    // A 2x2 min pool fused into the list build (k_stream_quad<..., POOL>):
    // `in` is then the pool's input [B][H_u][W_u][C_in], and the map the
    // layer reads at (hi, wi, ci) is its min over rows 2hi, 2hi+1 and columns
    // 2wi, 2wi+1 (in_bytes covers the pool's input); pdx and pdy are the byte
    // steps to a window's next column and next row.
    int H_u, W_u, pdx, pdy;
};

constexpr int kDenseMaxBins = 256;
constexpr int kDenseMaxCin = 64;
constexpr int kQuadMaxCin = 128;  // k_stream_quad's list build: 18 chunks of 64 per 3x3 pixel
// quad_build packs an event's weight row (tap * C_in + cin < 9 * kQuadMaxCin)
// into bits 21..31 of its register
static_assert(9 * kQuadMaxCin <= (1 << 11), "quad_build's 11-bit weight-row field");

// Spike time of one element of the map a list build reads, at byte offset
// off of `in`.  POOL: off addresses the first element of the element's 2x2
// window in the pool's input, and the time is k_pool_min4's: m = t where
// t < m, from kInfTime, over (0,0), (0,1), (1,0), (1,1) (T2V:192-209).  The
// four loads are issued together, their offsets in scalar registers.
template <bool POOL>
__device__ __forceinline__ float map_time(__amdgpu_buffer_rsrc_t rin, int off, const DenseMergeArgs& a) {
    if constexpr (!POOL) {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, off, 0, 0));
    } else {
        const float t0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, off, 0, 0));
        const float t1 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, off, a.pdx, 0));
        const float t2 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, off, a.pdy, 0));
        const float t3 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, off, a.pdx + a.pdy, 0));
        float m = kInfTime;
        if (t0 < m) m = t0;
        if (t1 < m) m = t1;
        if (t2 < m) m = t2;
        if (t3 < m) m = t3;
        return m;
    }
}

// Input column of tap (hi, wi) of image img (in bounds): the map's, or with
// POOL the first column of its 2x2 window in the pool's input.
template <bool POOL>
__device__ __forceinline__ int map_col(const DenseMergeArgs& a, int img, int hi, int wi) {
    if constexpr (POOL)
        return (img * a.H_u + 2 * hi) * a.W_u + 2 * wi;
    else
        return (img * a.H_in + hi) * a.W_in + wi;
}
constexpr size_t kFusedMaxLds = 64 * 1024;  // LDS of one k_stream_dense block

// Builds pixel `pix`'s merged list into `out` (total + kListPad entries, the
// tail zeroed) and its T+1 bin starts into `bs`, and returns the list length.
// `cur` (T ints) and `kinfo` (2 * KMAX ints) are the wave's LDS scratch.  The
// outputs are HBM (k_merge_dense) or the wave's LDS (k_stream_dense).
// `msk` (2T words, or null): LDS bit masks for the ranks in pass 2; without
// them the ranks come from a bit-ballot multisplit.
template <int KMAX, int NB, class ListPtr, class BinPtr>
__device__ __forceinline__ int dense_build(const DenseMergeArgs& a, int64_t pix, int* cur, int* kinfo,
                                           ListPtr out, BinPtr bs, unsigned* msk = nullptr) {
    const int lane = lane_id();
    const int q = fdiv((int)pix, a.div_w);
    const int w_out = (int)pix - q * a.W_out;
    const int img = fdiv(q, a.div_h);
    const int h_out = q - img * a.H_out;
    // in-bounds receptive columns, compacted in (kh, kw) order
    int nk;
    {
        bool v = false;
        int col = 0;
        if (lane < a.K_h * a.K_w) {
            const int kh = lane / a.K_w, kw = lane - kh * a.K_w;
            const int hi = h_out - a.pad_h + kh, wi = w_out - a.pad_w + kw;
            v = hi >= 0 && hi < a.H_in && wi >= 0 && wi < a.W_in;
            col = (img * a.H_in + hi) * a.W_in + wi;
        }
        const uint64_t m = __ballot(v);
        nk = uniform(__popcll(m));
        if (v) {
            const int slot = __popcll(m & lanemask_lt());
            kinfo[slot] = col;
            kinfo[KMAX + slot] = lane * a.C_in;  // first weight row of the tap
        }
    }
    for (int t = lane; t < a.T; t += 64) {
        cur[t] = 0;
        if (msk) {
            msk[2 * t] = 0;
            msk[2 * t + 1] = 0;
        }
    }
    wave_sync();
    const int nel = nk * a.C_in;  // <= KMAX * 64 (C_in <= 64)
    // Elements f = chunk * 64 + lane are loaded a batch of NB chunks at a
    // time, every load of a batch issued together, so the wave waits for one
    // round of loads per batch rather than one per chunk.  Each element
    // packs into one register: weight row (bits 16..), decay-LUT index (bits
    // 8..15) and arrival bin (bits 0..7, 0xFF: no event; T <= 255 keeps bins
    // and indices below 0xFF).  A pixel of at most NB chunks (every 3x3
    // layer at NB = 9) keeps its batch in registers for pass 2; wider ones
    // reload it.  NB = 1 serves pixels of at most 64 elements with the
    // fewest registers.
    static_assert(NB >= 1 && NB <= 9, "NB chunks per batch");
    const int n_chunks = (nel + 63) >> 6;
    int pk[NB];
    auto load_batch = [&](int c0) {
        float xs[NB];
        int rows[NB];
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            xs[c] = kInfTime;
            rows[c] = 0;
            if (c0 + c < n_chunks) {  // uniform
                // tap k = f / C_in (the quotient's fractional part is >=
                // 0.5 / 64, so the float product rounds it correctly), cin ci
                const int f = (c0 + c) * 64 + lane;
                const bool in = f < nel;
                const int k = in ? (int)(((float)f + 0.5f) * a.inv_cin) : 0;
                const int ci = f - k * a.C_in;
                rows[c] = kinfo[KMAX + k] + ci;
                const float v = a.in[in ? (int64_t)kinfo[k] * a.C_in + ci : 0];
                xs[c] = in ? v : kInfTime;
            }
        }
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const int b = arrival_bin(xs[c], a.tfs, a.T);
            const int ai = b >= 0 ? alpha_index(xs[c], b, a.alpha_by_time, a.T) : 0;
            pk[c] = (rows[c] << 16) | (ai << 8) | (b & 0xFF);
        }
    };
    // pass 1: events per bin
    for (int c0 = 0; c0 < n_chunks; c0 += NB) {
        load_batch(c0);
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const int b = pk[c] & 0xFF;
            if (c0 + c < n_chunks && b != 0xFF) atomicAdd(&cur[b], 1);
        }
    }
    wave_sync();
    // bin starts: lane l scans bins 4l .. 4l+3
    int v4[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * lane + i;
        v4[i] = t < a.T ? cur[t] : 0;
        sum += v4[i];
    }
    const int incl = wave_incl_scan(sum);
    int run = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * lane + i;
        if (t < a.T) {
            cur[t] = run;
            bs[t] = run;
        }
        run += v4[i];
    }
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (lane == 0) bs[a.T] = total;
    wave_sync();
    // pass 2: stable placement, chunk by chunk in (kh, kw, cin) order
    const uint64_t lt = lanemask_lt();
    for (int c0 = 0; c0 < n_chunks; c0 += NB) {
        if (n_chunks > NB) load_batch(c0);  // uniform; else the batch is still in registers
        float al[NB];
#pragma unroll
        for (int c = 0; c < NB; ++c) al[c] = a.alpha[(pk[c] >> 8) & 0xFF];
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const int b = pk[c] & 0xFF;
            const bool valid = c0 + c < n_chunks && b != 0xFF;
            uint64_t m = __ballot(valid);
            if (m != 0) {  // uniform (also false for chunks past the end)
                if (msk) {
                    // the lanes of the chunk in bin b: each ORs its lane bit
                    // into the bin's 64-bit mask (OR commutes, so the order the
                    // LDS serves same-address lanes in does not matter) and
                    // reads the mask back; the bin's first lane clears it
                    // after the cursor update below
                    if (valid) atomicOr(&msk[2 * b + (lane >> 5)], 1u << (lane & 31));
                    wave_sync();
                    m = valid ? *reinterpret_cast<const uint64_t*>(&msk[2 * b]) : 0ull;
                } else {
                    for (int bit = 0; bit < a.nbits; ++bit) {
                        const bool set = valid && ((b >> bit) & 1);
                        const uint64_t bb = __ballot(set);
                        m &= set ? bb : ~bb;
                    }
                }
                if (valid) {
                    const int pos = cur[b] + __popcll(m & lt);
                    out[pos] = make_int2((pk[c] >> 16) * a.rowbytes, __float_as_int(al[c]));
                }
                wave_sync();
                if (valid && (m & lt) == 0) {
                    cur[b] += __popcll(m);
                    if (msk) *reinterpret_cast<uint64_t*>(&msk[2 * b]) = 0ull;
                }
                wave_sync();
            }
        }
    }
    // zeroed tail: the stream kernel reads whole groups of 8 entries
    for (int i = lane; i < kListPad; i += 64) out[total + i] = make_int2(0, 0);
    return total;
}

template <int KMAX>
__global__ __launch_bounds__(64 * kMergeWaves) void k_merge_dense(DenseMergeArgs a) {
    __shared__ int cur_all[kMergeWaves][kDenseMaxBins];
    __shared__ __align__(8) unsigned msk_all[kMergeWaves][2 * kDenseMaxBins];
    __shared__ int kinfo_all[kMergeWaves][2 * KMAX];
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t pix = (int64_t)blockIdx.x * kMergeWaves + wave;
    if (pix >= a.n_pix) return;  // uniform per wave
    (void)dense_build<KMAX, 9>(a, pix, cur_all[wave], kinfo_all[wave], a.list + pix * a.cap,
                            a.bstart + pix * (int64_t)(a.T + 1), msk_all[wave]);
}

// ---------------------------------------------------------------------------
// k_stream: one wave64 per (output pixel, 64-wide c_out block); lanes are
// c_out.  The merged list is read through the scalar cache 8 events at a time
// (one s_load_dwordx16), each event costs one buffer_load (the weight row's
// byte offset goes in soffset, so no per-lane address arithmetic) and one fma
// with alpha as a scalar operand.  Gathers are batched across bin boundaries;
// bins are closed between fmas, in order, so every bin's fma chain is the
// reference's.  Lanes that fired stop fetching; the wave leaves when its
// ballot of live lanes is empty.
struct StreamArgs {
    float* out;
    const int2* list;
    const int32_t* bstart;
    const float* W;
    const float* bias;
    const float* theta;
    unsigned long long* counters;
    int64_t n_pix;
    int64_t cap;
    int T, D, t_min, C_out, n_cblk;
    int ppw;               // consecutive output pixels per wave
    int w_bytes;
    float decay, th;  // CuLIF neuron (T3V:62-63): I = I*decay + in; V += I; fire at V >= th
    // windowed merge (k_stream_window): the bin layout and its row scale
    const vd_event* bev;
    int b_cin, b_rowbytes;
};

// Block -> (c_out block, group of 4 output pixels).  Workgroups are dealt to
// the 8 XCDs round-robin, so when C_out spans a multiple of 8 blocks of 64,
// XCD x only ever integrates c_out blocks x, x+8, ...: its L2 then holds
// 1/8 of the layer's weights (the 3x3x512x512 planes are 9.4 MB, an XCD's L2
// is 4 MB).  With 1, 2 or 4 blocks, b % n_cblk already pins XCD x to block
// x % n_cblk.  Past 8 blocks, XCD x takes its blocks x, x + 8, ... one
// after the other, each over every pixel group (the grid is n_pg pixel
// groups x n_cblk blocks, dealt in order), so its L2 holds one block's
// weights at a time.
__device__ __forceinline__ void map_block(int n_cblk, int& cb, int64_t& pg) {
    const int64_t b = blockIdx.x;
    if ((n_cblk & 7) == 0) {
        const int64_t n_pg = (int64_t)gridDim.x / n_cblk;
        const int64_t q = b >> 3;
        cb = (int)(b & 7) + 8 * (int)(q / n_pg);
        pg = q % n_pg;
    } else {
        cb = (int)(b % n_cblk);
        pg = b / n_cblk;
    }
}

struct Group8 {
    int2 v[8];
};

// VEC consecutive c_out per lane (1, or 4 with dwordx4 gathers: a 64-lane
// dword gather and a dwordx4 gather cost the same texture-unit time, so four
// c_out per lane quadruple the bytes per gather).  A c_out block is 64*VEC.
template <int VEC>
struct Vf {
    float v[VEC];
};

template <int VEC>
__device__ __forceinline__ Vf<VEC> gather(const __amdgpu_buffer_rsrc_t r, int voff, int row) {
    Vf<VEC> o;
    if constexpr (VEC == 1) {
        o.v[0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, row, 0));
    } else {
        typedef unsigned int u4 __attribute__((ext_vector_type(4)));
        const u4 x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, row, 0);
        o.v[0] = __uint_as_float(x.x);
        o.v[1] = __uint_as_float(x.y);
        o.v[2] = __uint_as_float(x.z);
        o.v[3] = __uint_as_float(x.w);
    }
    return o;
}

// Weight gathers of a group of 8 events.  A gather type fixes which c_out a
// lane owns (c0(cb, lane) .. + OWN - 1) and fills w[g] with those c_out's
// weights for event g.
//
// GlobalGather<VEC>: one buffer_load per event, the row offset in soffset;
// lane owns VEC consecutive c_out of a 64*VEC block.  Lanes whose neurons
// all fired skip their loads (exec-masked).  Measured: the gather cost
// follows the active lanes, so masked lanes are free, while an out-of-range
// address for them (to keep the loads unconditional and pipeline the next
// group's gathers) made narrow layers slower.
template <int VEC>
struct GlobalGather {
    static constexpr int OWN = VEC;
    __amdgpu_buffer_rsrc_t r;
    int voff;
    __device__ static int c0(int cb, int lane) { return (cb * 64 + lane) * VEC; }
    __device__ __forceinline__ void group(const int2 (&e)[8], Vf<VEC> (&w)[8], bool live) const {
        if (live) {
#pragma unroll
            for (int g = 0; g < 8; ++g) w[g] = gather<VEC>(r, voff, e[g].x);
        }
    }
};

// PairGather: a 128-wide c_out block per wave (512 B of each row), one
// dwordx4 load fetches two events at once -- the lower half-wave loads event
// 2i's row, the upper half event 2i+1's, 4 c_out per lane -- and two
// v_permlane32_swap exchange the halves' (2,3) and (0,1) components, so that
// lane (h, r) ends owning c_out 128cb+4r+2h, +1 with both events' weights.
// Every load then carries 1 KB with all 64 lanes busy (a 4-c_out-per-lane
// load would leave half the wave idle); lanes load for each other, so loads
// are not skipped per lane.  Against four c_out per lane (one event, 256
// c_out per load) it moves the same bytes per instruction with half the
// c_out per wave: twice the waves per pixel, for layers too small to fill
// the device, and each XCD's share of the weights halves.  Loads past the
// last c_out (C_out not a multiple of 128) read the next row or, past the
// buffer, zero; those lanes' results are not stored.
struct PairGather {
    static constexpr int OWN = 2;
    __amdgpu_buffer_rsrc_t r;
    int lane_off;  // 16 * (lane % 32) + 512 * cb
    int h;         // lane / 32: which event of a load this lane fetches
    __device__ static int c0(int cb, int lane) { return 128 * cb + 4 * (lane & 31) + 2 * (lane >> 5); }
    __device__ __forceinline__ void group(const int2 (&e)[8], Vf<2> (&w)[8], bool) const {
        typedef unsigned int u4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = h == 0 ? e[2 * i].x : e[2 * i + 1].x;
            const u4 x = __builtin_amdgcn_raw_buffer_load_b128(r, row + lane_off, 0, 0);
            unsigned c0 = x.x, c1 = x.y, c2 = x.z, c3 = x.w;
            // permlane32_swap(a, b) exchanges a's upper 32 lanes with b's lower 32
            auto p = __builtin_amdgcn_permlane32_swap(c0, c2, false, false);
            c0 = p[0];
            c2 = p[1];
            p = __builtin_amdgcn_permlane32_swap(c1, c3, false, false);
            c1 = p[0];
            c3 = p[1];
            w[2 * i].v[0] = __uint_as_float(c0);
            w[2 * i].v[1] = __uint_as_float(c1);
            w[2 * i + 1].v[0] = __uint_as_float(c2);
            w[2 * i + 1].v[1] = __uint_as_float(c3);
        }
    }
};


// List reader: groups of 8 merged events (row, alpha) as wave-uniform
// SGPRs, one s_load_dwordx16 per group, read NA groups ahead; take() is
// called for consecutive groups (j, j + 8, ...) until the next start().  The
// list is zero-padded by four groups, so reads stay in the pixel's region.
template <int NA>
struct ScalarListN {
    const int2* L;
    Group8 ahead[NA];
    __device__ __forceinline__ void start(const void* L_, int j, const StreamArgs&) {
        L = static_cast<const int2*>(L_);
#pragma unroll
        for (int q = 0; q < NA; ++q) ahead[q] = *reinterpret_cast<const Group8*>(L + j + 8 * q);
    }
    __device__ __forceinline__ Group8 take(int j) {
        const Group8 g = ahead[0];
#pragma unroll
        for (int q = 0; q + 1 < NA; ++q) ahead[q] = ahead[q + 1];
        ahead[NA - 1] = *reinterpret_cast<const Group8*>(L + j + 8 * NA);
        return g;
    }
};
using ScalarList = ScalarListN<1>;

// Integrates one output pixel for one c_out block (lane = VEC c_out) from its
// merged event list and writes the first-spike times.  CULIF selects the
// neuron that closes each bin: the LUT-threshold neuron of T1V/T2V (carry +=
// delta_t, fire at carry >= theta[t] >= 1e-5, t >= t_min) or the CuLIF neuron
// of T3V (I = fma(I, decay, in_t); V += I; fire at V >= th).  CuLIF events
// carry alpha = 1, so fma(w, 1, acc) is exactly the reference's acc + w.
template <bool COUNT, bool CULIF, class G, class LR = ScalarList, int NG = 1, int VEC = G::OWN>
__device__ __forceinline__ void stream_pixel(const StreamArgs& a, float* __restrict__ out,
                                             const void* __restrict__ L,
                                             const int32_t* __restrict__ BS,
                                             const float* __restrict__ theta, int64_t pix, int cb,
                                             const G& gather_w, unsigned long long& cnt_proc,
                                             unsigned long long& cnt_bin) {
    const int lane = lane_id();
    const int c0 = G::c0(cb, lane);  // first c_out of this lane
    bool ok[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) ok[v] = c0 + v < a.C_out;

    // carry: membrane (V for CuLIF); cur: CuLIF current I; res: spike time.
    // The CuLIF neuron tests "alive" as res == kInfTime (lanes past C_out
    // start at -1): a bool array there is packed into bytes and cost about
    // ten more VALU per bin closing (CuLIF conv2 8.5 -> 8.2 ms).  The same
    // change made the T1V/T2V kernels slower (VGG-16 30.5K -> 27.9K
    // images/s), so they keep the flags.
    float carry[VEC], cur[VEC], res[VEC];
    bool alive[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
        carry[v] = (ok[v] && !CULIF) ? a.bias[c0 + v] : 0.0f;
        cur[v] = 0.0f;
        res[v] = (CULIF && !ok[v]) ? -1.0f : kInfTime;
        alive[v] = ok[v];
    }
#define VD_ALIVE(v) (CULIF ? res[v] == kInfTime : alive[v])
    bool live = ok[0];  // any neuron of the lane still integrating
    int live_chunk_n = 0;
    if (COUNT) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) live_chunk_n += __popcll(__ballot(VD_ALIVE(v)));
    }
    const int T = a.T, D = a.D;
    bool done = false;
    int j = 0;  // next merged event

    for (int t0 = 0; t0 < T && !done; t0 += kBlockBins) {
        const int nb = (T - t0) < kBlockBins ? (T - t0) : kBlockBins;
        // lane d keeps bin t0+d's merged start and threshold
        const int v_bs = lane < nb ? BS[t0 + lane] : 0;
        const float v_th = (!CULIF && lane < nb) ? theta[t0 + lane] : 0.0f;
        const int blk_end = BS[t0 + nb];
        asm volatile("" ::"v"(v_bs), "v"(v_th));  // complete these loads before streaming
        // Empty bin runs in O(1) (the LUT neuron without counters): a bin with
        // no event adds +0 to carry, which changes no comparison, so across
        // a run of empty bins carry is constant.  With theta non-increasing
        // over the block (checked here; NaN fails the check), "carry >=
        // theta[t]" holds on a suffix of the run and "theta[t] >= 1e-5" on a
        // prefix of the block (bins below th_end), so a neuron fires in the
        // run iff it clears theta at the run's last bin it may fire in, and
        // then at the first such bin -- a per-lane lower bound over the run.
        // Otherwise the bins are closed one by one as before.  Only the
        // one-c_out-per-lane streams take it: their layers are the sparse
        // ones (VGG-16 L0: 27 events over 64 bins), while in the pair and
        // dwordx4 streams empty bins are rare and the extra scalar registers
        // cost a wave per SIMD (pair stream: 8 -> 7; VGG L2/L3 +15%).
        constexpr bool FAST = !COUNT && !CULIF && VEC == 1;
        bool mono = false;
        int th_end = 0;
        if (FAST) {
            const float nxt = __shfl_down(v_th, 1, 64);
            mono = __ballot(lane + 1 < nb && !(v_th >= nxt)) == 0;
            const uint64_t low = __ballot(lane < nb && !(v_th >= 1e-5f));
            th_end = low ? (int)__builtin_ctzll(low) : nb;
        }

#define VD_BIN_START(b) ((b) < nb ? __builtin_amdgcn_readlane(v_bs, (b)) : blk_end)
#define VD_FINALIZE(b, acc_)                                                            \
    do {                                                                                \
        const int t_ = t0 + (b);                                                        \
        if (COUNT) {                                                                    \
            const int n_ = VD_BIN_START((b) + 1) - VD_BIN_START(b);                     \
            int nl_ = 0;                                                                \
            _Pragma("unroll") for (int v = 0; v < VEC; ++v) nl_ += __popcll(__ballot(VD_ALIVE(v))); \
            cnt_bin += (unsigned long long)n_ * nl_;                                    \
            cnt_proc += (unsigned long long)n_ * live_chunk_n;                          \
        }                                                                               \
        if (CULIF) {                                                                    \
            _Pragma("unroll") for (int v = 0; v < VEC; ++v) {                           \
                cur[v] = __builtin_fmaf(cur[v], a.decay, (acc_)[v]);                    \
                carry[v] = carry[v] + cur[v];                                           \
                const bool f_ = VD_ALIVE(v) && carry[v] >= a.th;                        \
                res[v] = f_ ? (float)t_ : res[v];                                       \
            }                                                                           \
        } else {                                                                        \
            const float th_ = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_th), (b))); \
            const bool can_ = t_ >= a.t_min && th_ >= 1e-5f;                            \
            _Pragma("unroll") for (int v = 0; v < VEC; ++v) {                           \
                carry[v] = carry[v] + (acc_)[v];                                        \
                if (can_ && alive[v] && carry[v] >= th_) {                              \
                    res[v] = (float)t_;                                                 \
                    alive[v] = false;                                                   \
                }                                                                       \
            }                                                                           \
        }                                                                               \
        live = VD_ALIVE(0);                                                             \
        _Pragma("unroll") for (int v = 1; v < VEC; ++v) live = live || VD_ALIVE(v);     \
        const bool chunk_end_ = ((t_ + 1) % D) == 0;                                    \
        if (COUNT && chunk_end_) {                                                      \
            live_chunk_n = 0;                                                           \
            _Pragma("unroll") for (int v = 0; v < VEC; ++v) live_chunk_n += __popcll(__ballot(VD_ALIVE(v))); \
        }                                                                               \
        if (__ballot(live) == 0 && (!COUNT || chunk_end_)) done = true;                 \
    } while (0)

        // bins [r0, r1) of the block are empty and every earlier bin is
        // closed: fire the neurons that cross in the run (see FAST above)
        auto skip_empty = [&](int r0, int r1) {
            const int ta = r0 > a.t_min - t0 ? r0 : a.t_min - t0;
            const int tb = r1 < th_end ? r1 : th_end;
            if (ta >= tb) return;
            const float th_last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_th), tb - 1));
            bool any = false;
#pragma unroll
            for (int v = 0; v < VEC; ++v) any = any || (alive[v] && carry[v] >= th_last);
            if (__ballot(any) == 0) return;
            int n_it = 0;
            while ((1 << n_it) < tb - ta) ++n_it;
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                // first t in [ta, tb) with theta[t] <= carry (it exists where
                // carry >= th_last); every lane runs the search, as
                // ds_bpermute reads the source lanes' registers
                int lo = ta, hi = tb - 1;
                for (int it = 0; it < n_it; ++it) {
                    const int mid = (lo + hi) >> 1;
                    const float thm =
                        __int_as_float(__builtin_amdgcn_ds_bpermute(mid << 2, __float_as_int(v_th)));
                    const bool le = thm <= carry[v];
                    hi = le ? mid : hi;
                    lo = le ? lo : mid + 1;
                }
                if (alive[v] && carry[v] >= th_last) {
                    res[v] = (float)(t0 + lo);
                    alive[v] = false;
                }
            }
            live = alive[0];
#pragma unroll
            for (int v = 1; v < VEC; ++v) live = live || alive[v];
            if (__ballot(live) == 0) done = true;
        };
        // the block-relative bin holding merged event idx (blk_end > idx):
        // the last bin whose start is at most idx
        auto bin_of = [&](int idx) { return __popcll(__ballot(lane < nb && v_bs <= idx)) - 1; };

        int bcur = 0;                    // open bin of this block
        int bend = VD_BIN_START(1);      // merged end of the open bin
        float acc[VEC];
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
        // groups of 8 (row, alpha) pairs, read one group (chunk) ahead
        LR lr;
        lr.start(L, j, a);
        // NG groups of 8 per step: their gathers are issued together
        constexpr int GE = 8 * NG;
        while (j < blk_end) {
            const int n = (blk_end - j) < GE ? (blk_end - j) : GE;
            Group8 grp[NG];
#pragma unroll
            for (int q = 0; q < NG; ++q) grp[q] = lr.take(j + 8 * q);
#pragma unroll
            for (int q = 0; q < NG; ++q)
#pragma unroll
                for (int g = 0; g < 8; ++g) asm volatile("" ::"s"(grp[q].v[g].x), "s"(grp[q].v[g].y));
            Vf<VEC> w[NG][8];
#pragma unroll
            for (int q = 0; q < NG; ++q)
#pragma unroll
                for (int g = 0; g < 8; ++g)
#pragma unroll
                    for (int v = 0; v < VEC; ++v) w[q][g].v[v] = 0.0f;
#pragma unroll
            for (int q = 0; q < NG; ++q) gather_w.group(grp[q].v, w[q], live);
#define VD_EV(i) grp[(i) / 8].v[(i) % 8]
#define VD_W(i) w[(i) / 8][(i) % 8]
            if (bend >= j + n) {
                // the whole step belongs to the open bin
                if (n == GE) {
#pragma unroll
                    for (int i = 0; i < GE; ++i)
#pragma unroll
                        for (int v = 0; v < VEC; ++v)
                            acc[v] = __builtin_fmaf(VD_W(i).v[v], __int_as_float(VD_EV(i).y), acc[v]);
                } else {
#pragma unroll
                    for (int i = 0; i < GE; ++i)
                        if (i < n)
#pragma unroll
                            for (int v = 0; v < VEC; ++v)
                                acc[v] = __builtin_fmaf(VD_W(i).v[v], __int_as_float(VD_EV(i).y), acc[v]);
                }
            } else {
#pragma unroll
                for (int q = 0; q < NG; ++q) {
#pragma unroll
                    for (int g = 0; g < 8; ++g) {
                        if (8 * q + g >= n) break;
                        while (bend <= j + 8 * q + g) {
                            VD_FINALIZE(bcur, acc);
                            if (done) goto stream_done;
#pragma unroll
                            for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
                            ++bcur;
                            bend = VD_BIN_START(bcur + 1);
                            if (FAST && mono && bend <= j + 8 * q + g) {
                                const int bn = bin_of(j + 8 * q + g);
                                skip_empty(bcur, bn);
                                if (done) goto stream_done;
                                bcur = bn;
                                bend = VD_BIN_START(bcur + 1);
                            }
                        }
#pragma unroll
                        for (int v = 0; v < VEC; ++v)
                            acc[v] = __builtin_fmaf(w[q][g].v[v], __int_as_float(grp[q].v[g].y), acc[v]);
                    }
                }
            }
#undef VD_EV
#undef VD_W
            j += n;
        }
        // close the block's remaining bins (the open one and trailing empty ones)
        while (bcur < nb) {
            VD_FINALIZE(bcur, acc);
            if (done) break;
#pragma unroll
            for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
            ++bcur;
            if (FAST && mono && bcur < nb) {  // every bin after the last event is empty
                skip_empty(bcur, nb);
                break;
            }
        }
#undef VD_FINALIZE
#undef VD_BIN_START
    }
stream_done:
#pragma unroll
    for (int v = 0; v < VEC; ++v)
        if (ok[v]) out[pix * a.C_out + c0 + v] = res[v];
#undef VD_ALIVE
}

// One (pixel, c_out block) with the gather type of EPI = events per load:
// 1 (GlobalGather<VEC>) or 2 (PairGather, VEC = 2, 128-wide c_out blocks).  L and BS
// are the pixel's merged list and bin starts; LR reads the list.
template <bool COUNT, int VEC, bool CULIF, int EPI, class LR>
__device__ __forceinline__ void stream_one(const StreamArgs& a, float* __restrict__ out,
                                           const void* __restrict__ L, const int32_t* __restrict__ BS,
                                           const float* __restrict__ theta, int64_t pix, int cb) {
    const int lane = lane_id();
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.w_bytes, 0x00020000);
    unsigned long long cnt_proc = 0, cnt_bin = 0;
    if constexpr (EPI == 1) {
        GlobalGather<VEC> g;
        g.r = rsrc;
        const int c0 = GlobalGather<VEC>::c0(cb, lane);
        g.voff = (c0 < a.C_out ? c0 : 0) * 4;  // C_out is a multiple of VEC
        // one c_out per lane: two groups of gathers in flight (16 events),
        // the scalar list read two groups ahead
        constexpr int NG = VEC == 1 ? 2 : 1;
        using LRN = typename std::conditional<NG == 2 && std::is_same<LR, ScalarList>::value, ScalarListN<2>,
                                              LR>::type;
        stream_pixel<COUNT, CULIF, GlobalGather<VEC>, LRN, NG>(a, out, L, BS, theta, pix, cb, g, cnt_proc,
                                                               cnt_bin);
    } else {
        static_assert(VEC == 2 && EPI == 2, "PairGather owns 2 c_out per lane");
        PairGather g;
        g.r = rsrc;
        g.lane_off = 16 * (lane & 31) + 512 * cb;
        g.h = lane >> 5;
        stream_pixel<COUNT, CULIF, PairGather, LR>(a, out, L, BS, theta, pix, cb, g, cnt_proc, cnt_bin);
    }
    if (COUNT && lane == 0) {
        unsigned long long* c = counter_stripe(a.counters);
        atomicAdd(&c[0], cnt_proc);
        atomicAdd(&c[1], cnt_bin);
    }
}

template <bool COUNT, int VEC, bool CULIF, int EPI>
__global__ __launch_bounds__(256) void k_stream(StreamArgs a, float* __restrict__ out,
                                                const int2* __restrict__ list,
                                                const int32_t* __restrict__ bstart,
                                                const float* __restrict__ theta) {
    const int wave = uniform(threadIdx.x >> 6);
    int cb;
    int64_t pg;
    map_block(a.n_cblk, cb, pg);
    const int64_t pix0 = (pg * 4 + wave) * a.ppw;
    for (int q = 0; q < a.ppw; ++q) {
        const int64_t pix = pix0 + q;
        if (pix >= a.n_pix) return;  // uniform per wave
        stream_one<COUNT, VEC, CULIF, EPI, ScalarList>(a, out, list + pix * a.cap,
                                                       bstart + pix * (int64_t)(a.T + 1), theta, pix, cb);
    }
}

// k_stream_lean: k_stream without counters and T <= 64 (the LUT-threshold
// neuron, or the CuLIF neuron, which steps every bin, empty ones with an
// input of 0), with k_stream_quad's bin closing: the wave's live neurons are SGPR
// lane masks (one per c_out a lane owns), a bin where no spike may occur has
// a NaN threshold, so a bin closes with one compare, one v_cndmask and two
// mask operations per owned c_out, and a run of empty bins up to the next
// event costs one ballot to find.  GEO 4: four c_out per lane (256 per wave),
// one event per dwordx4 load with the row in soffset; GEO 2: the pair gather
// (128 c_out per wave, two events per load, permlane32 exchange).  The list
// is read through the scalar cache a group of 8 events ahead.
template <int GEO, bool CULIF>
__global__ __launch_bounds__(256) void k_stream_lean(StreamArgs a, float* __restrict__ out,
                                                     const int2* __restrict__ list,
                                                     const int32_t* __restrict__ bstart,
                                                     const float* __restrict__ theta) {
    static_assert(GEO == 4 || GEO == 2, "four c_out per lane or the pair gather");
    constexpr int OWN = GEO == 4 ? 4 : 2;  // c_out per lane
    constexpr int LPG = GEO == 4 ? 8 : 4;  // loads per group of 8 events
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    const int wave = uniform(threadIdx.x >> 6);
    int cb;
    int64_t pg;
    map_block(a.n_cblk, cb, pg);
    const int lane = lane_id();
    const int h = lane >> 5;  // GEO 2: which event of a load this lane fetches
    const int hmask = -h;
    const int co = GEO == 4 ? 256 * cb + 4 * lane : 128 * cb + 4 * (lane & 31) + 2 * h;
    const int voff = GEO == 4 ? co * 4 : 16 * (lane & 31) + 512 * cb;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.w_bytes, 0x00020000);
    const int T = a.T;
    const float th_d = lane < T ? theta[lane] : 0.0f;
    const float v_th = (lane < T && lane >= a.t_min && th_d >= 1e-5f) ? th_d : __builtin_nanf("");
    bool ok[OWN];
    float bias[OWN];
#pragma unroll
    for (int v = 0; v < OWN; ++v) {
        ok[v] = co + v < a.C_out;
        bias[v] = (ok[v] && !CULIF) ? a.bias[co + v] : 0.0f;  // the CuLIF neuron starts at V = 0
    }
    const int vsafe = GEO == 4 && !ok[0] ? 0 : voff;  // C_out is a multiple of 4
    const int64_t pix0 = (pg * 4 + wave) * a.ppw;
    for (int pq = 0; pq < a.ppw; ++pq) {
        const int64_t pix = pix0 + pq;
        if (pix >= a.n_pix) return;  // uniform per wave
        const int2* L = list + pix * a.cap;
        const int32_t* BS = bstart + pix * (int64_t)(T + 1);
        const int v_end = lane < T ? BS[lane + 1] : INT_MAX;  // end of bin `lane`
        float carry[OWN], acc[OWN], cur[OWN];  // cur: the CuLIF current I
        int res[OWN];  // bins closed with the neuron still alive: its spike bin once it fired
        uint64_t alive[OWN];
#pragma unroll
        for (int v = 0; v < OWN; ++v) {
            carry[v] = bias[v];
            acc[v] = 0.0f;
            cur[v] = 0.0f;
            res[v] = 0;
            alive[v] = __ballot(ok[v]);
        }
        int b = 0;
        int bend = __builtin_amdgcn_readlane(v_end, 0);
        auto close_to = [&](int p) -> bool {
            if constexpr (!CULIF) {
#pragma unroll
                for (int v = 0; v < OWN; ++v) {
                    carry[v] = carry[v] + acc[v];
                    acc[v] = 0.0f;
                }
            }
            const int stop = __popcll(__builtin_amdgcn_ballot_w64(v_end <= p));  // > b (lanes >= T: INT_MAX)
            if constexpr (CULIF) {
                do {
                    // I = fma(I, decay, in_b); V += I; fire at V >= th (T3V:50-62);
                    // every bin steps the neuron, empty ones with in_b = 0
#pragma unroll
                    for (int v = 0; v < OWN; ++v) {
                        cur[v] = __builtin_fmaf(cur[v], a.decay, acc[v]);
                        acc[v] = 0.0f;
                        carry[v] = carry[v] + cur[v];
                        alive[v] &= ~__ballot(carry[v] >= a.th);
                        res[v] = add_lane_bit(res[v], alive[v]);
                    }
                } while (++b < stop);
            } else {
                auto close_bin = [&]() {
                    const float th = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_th), b));
#pragma unroll
                    for (int v = 0; v < OWN; ++v) {
                        alive[v] &= ~__ballot(carry[v] >= th);
                        res[v] = add_lane_bit(res[v], alive[v]);
                    }
                };
                do close_bin();
                while (++b < stop);
            }
            uint64_t any = alive[0];
#pragma unroll
            for (int v = 1; v < OWN; ++v) any |= alive[v];
            if (b >= T || any == 0) return true;
            bend = __builtin_amdgcn_readlane(v_end, b);
            return false;
        };
        ScalarList lr;
        lr.start(L, 0, a);
        for (int j = 0;; j += 8) {
            const Group8 e = lr.take(j);
#pragma unroll
            for (int g = 0; g < 8; ++g) asm volatile("" ::"s"(e.v[g].x), "s"(e.v[g].y));
            float w[8][OWN];
#pragma unroll
            for (int k = 0; k < LPG; ++k) {
                if constexpr (GEO == 4) {
                    const u4 x = __builtin_amdgcn_raw_buffer_load_b128(rsrc, vsafe, e.v[k].x, 0);
                    w[k][0] = __uint_as_float(x.x);
                    w[k][1 % OWN] = __uint_as_float(x.y);
                    w[k][2 % OWN] = __uint_as_float(x.z);
                    w[k][3 % OWN] = __uint_as_float(x.w);
                } else {
                    // lower half: event 2k's row, upper half: 2k+1's (a mask,
                    // not a select, keeps the entries in SGPRs)
                    const int d = e.v[2 * k + 1].x - e.v[2 * k].x;
                    const u4 x = __builtin_amdgcn_raw_buffer_load_b128(rsrc, e.v[2 * k].x + (d & hmask) + voff, 0, 0);
                    unsigned c0 = x.x, c1 = x.y, c2 = x.z, c3 = x.w;
                    auto p = __builtin_amdgcn_permlane32_swap(c0, c2, false, false);
                    c0 = p[0];
                    c2 = p[1];
                    p = __builtin_amdgcn_permlane32_swap(c1, c3, false, false);
                    c1 = p[0];
                    c3 = p[1];
                    w[2 * k][0] = __uint_as_float(c0);
                    w[2 * k][1 % OWN] = __uint_as_float(c1);
                    w[2 * k + 1][0] = __uint_as_float(c2);
                    w[2 * k + 1][1 % OWN] = __uint_as_float(c3);
                }
            }
            // integrates positions j .. j+7; true when the stream is over
            auto consume = [&]() -> bool {
                if (bend >= j + 8) {  // all eight in the open bin
#pragma unroll
                    for (int i = 0; i < 8; ++i)
#pragma unroll
                        for (int v = 0; v < OWN; ++v)
                            acc[v] = __builtin_fmaf(w[i][v], __int_as_float(e.v[i].y), acc[v]);
                    return false;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    if (bend <= j + i && close_to(j + i)) return true;
#pragma unroll
                    for (int v = 0; v < OWN; ++v)
                        acc[v] = __builtin_fmaf(w[i][v], __int_as_float(e.v[i].y), acc[v]);
                }
                return false;
            };
            if (consume()) break;
        }
#pragma unroll
        for (int v = 0; v < OWN; ++v)
            if (ok[v]) out[pix * a.C_out + co + v] = __builtin_amdgcn_inverse_ballot_w64(alive[v]) ? kInfTime : (float)res[v];
    }
}

// ---------------------------------------------------------------------------
// k_stream_dense: k_merge_dense and k_stream fused for layers whose pixel is
// one wave of dword gathers (C_out <= 64) and T <= 64.  Each wave builds its
// pixel's merged list and bin starts in its own LDS region, then streams the
// list from there, so the list never reaches HBM.  The list is read 64
// entries per LDS load (lane i holds entry base + i) with the next 64
// prefetched; v_readlane turns a group's 8 entries into the wave-uniform
// SGPRs that the gathers and fmas take.  Groups start at multiples of 8 (one
// bin block), so a group never straddles two windows.
// Measured on VGG-16 B=256: L0 (3->64) 659 us against 716 us for the two
// kernels, L1 (64->64) 1958 against 1981.  With two events per load
// (64 < C_out <= 128) it lost (848 against 734 us at L2; 9.22 against 8.53 ms
// at the 2^20-pixel CuLIF conv2), and 4-byte packed
// entries (alpha by LUT index) lost on every layer, so neither is used.
struct LdsList {
    const int2* L;
    int base;
    int2 w0, w1;  // entries base + lane and base + 64 + lane
    __device__ __forceinline__ void start(const void* L_, int j, const StreamArgs&) {
        L = static_cast<const int2*>(L_);
        base = j;
        const int lane = lane_id();
        w0 = L[base + lane];
        w1 = L[base + 64 + lane];
    }
    __device__ __forceinline__ Group8 take(int j) {
        if (j - base >= 64) {  // uniform
            base += 64;
            w0 = w1;
            w1 = L[base + 64 + lane_id()];
        }
        const int k = j - base;
        Group8 g;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            g.v[i].x = __builtin_amdgcn_readlane(w0.x, k + i);
            g.v[i].y = __builtin_amdgcn_readlane(w0.y, k + i);
        }
        return g;
    }
};

// LDS words of one wave's region: the list (rounded up to whole 64-entry
// windows plus the prefetched one), T + 1 bin starts, T cursors, the tap
// table; a multiple of 4 so every region stays 16-byte aligned.
__host__ __device__ inline int fused_list_entries(int nel_max) {
    return ((nel_max + kListPad + 63) / 64) * 64 + 64;
}
__host__ __device__ inline int fused_wave_words(int nel_max, int T) {
    const int w = 2 * fused_list_entries(nel_max) + (T + 1) + T + 2 * 9;
    return (w + 3) & ~3;
}

template <bool COUNT, int VEC, bool CULIF, int EPI, int NB>
__global__ __launch_bounds__(256) void k_stream_dense(DenseMergeArgs m, StreamArgs a,
                                                      float* __restrict__ out,
                                                      const float* __restrict__ theta, int nel_max) {
    extern __shared__ int lds_words[];
    const int wave = uniform(threadIdx.x >> 6);
    int* region = lds_words + wave * fused_wave_words(nel_max, a.T);
    int2* L = reinterpret_cast<int2*>(region);
    int* bs = region + 2 * fused_list_entries(nel_max);
    int* cur = bs + a.T + 1;
    int* kinfo = cur + a.T;
    const int64_t pix0 = ((int64_t)blockIdx.x * 4 + wave) * a.ppw;
    for (int q = 0; q < a.ppw; ++q) {
        const int64_t pix = pix0 + q;
        if (pix >= a.n_pix) return;  // uniform per wave
        (void)dense_build<9, NB>(m, pix, cur, kinfo, L, bs);
        wave_sync();
        stream_one<COUNT, VEC, CULIF, EPI, LdsList>(a, out, L, bs, theta, pix, 0);
        wave_sync();  // this pixel's list reads precede the next pixel's build
    }
}

// ---------------------------------------------------------------------------
// k_stream_quad: the fused dense path without counters (C_out <= 128,
// T <= 64), built for the fewest instructions per event and per bin, for
// the LUT-threshold neuron or (CULIF) the CuLIF neuron; counting forwards
// take k_stream_dense (C_out <= 64) or k_merge_dense + k_stream.
//
// Gathers: one dwordx4 load fetches four events at once -- lane (q, r)
// (q = lane / 16, r = lane % 16) loads c_out 4r .. 4r+3 of event q's row --
// and a 4x4 transpose across lanes r, r+16, r+32, r+48 (v_permlane32_swap
// on components (0,2), (1,3), then v_permlane16_swap on (0,1), (2,3)) leaves
// lane (q, r) owning c_out 4r+q with all four events' weights.  A dwordx4
// load costs the texture unit about 2.3x a dword load and carries 4x the
// bytes.  The list lives in LDS as two arrays; each lane group reads its
// event's row (one ds_read_b32 per four events) and every lane the four
// alphas (one broadcast ds_read_b128), so no v_readlane per event.
//
// Bins: the neuron's state is carry, the open bin's delta (acc) and the
// spike bin; "alive" is a wave mask in SGPRs and a bin where no spike may
// occur (b < t_min or theta[b] < 1e-5) takes a NaN threshold, so closing a
// bin is one compare, two mask operations and one v_cndmask.  Positions at
// or past the list's end close every remaining bin, which ends the stream.
//
// List build (quad_build): as dense_build, but the rank of an event among
// its chunk's lanes of the same bin comes from LDS bit masks instead of a
// multisplit of bit ballots: each lane ORs its lane bit into its bin's
// 64-bit mask (OR commutes, so the order the LDS serves same-address lanes
// in does not matter), reads the mask back and counts the bits below its
// own; the bin's last lane adds the chunk's count to the bin and clears the
// mask.  Pass 1 keeps each event's rank in its packed register, so pass 2
// places it at cursor + rank with no second ranking.
//
// LDS words of one wave: list rows and alphas (the list, its zeroed tail and
// a multiple of 4 so the alpha array stays 16-byte aligned; the bin masks,
// 2T words, use the start of this region during pass 1), T + 1 bin starts,
// T cursors, the tap table.
__host__ __device__ inline int quad_list_entries(int nel_max, int T) {
    const int e = nel_max + kListPad > T ? nel_max + kListPad : T;
    return (e + 7) & ~7;
}
// LDS words of one k_stream_quad wave: the list, bin starts, cursors, tap
// table.  With alphas an entry is a 16-bit row index and an alpha (6 bytes);
// the CuLIF neuron's inputs are unscaled, so its entries are row byte offsets
// (4 bytes).  Either way the list region holds pass 1's 2T mask words before
// the cursors (entries >= T).
__host__ __device__ inline int quad_list_words(int nel_max, int T, bool alphas) {
    const int E = quad_list_entries(nel_max, T);
    return alphas ? E / 2 + E : E;
}
__host__ __device__ inline int quad_wave_words(int nel_max, int T, bool alphas = true) {
    return (quad_list_words(nel_max, T, alphas) + (T + 1) + T + 2 * 9 + 3) & ~3;
}

// Packed event of quad_build: bin (bits 0..6, 0x7F: no event), decay-LUT
// index (7..13), rank in its chunk's bin (14..19), last of the chunk's bin
// (20), weight row (21..31).  T <= 64 and at most 9 x 128 rows.
// OPAQUE: the lane index is made opaque per pixel, so that nothing derived
// from it (per-chunk element indices and offsets) is hoisted out of the
// pixel loop into registers held through the stream.  The CuLIF kernel
// takes it (k_stream_quad<2, 9, true>: 91 -> 67 VGPRs, 5 -> 7 waves per
// SIMD, CuLIF-7 conv2 4.46 -> 4.08 ms), and so do the 18-chunk builds (120
// -> 79 VGPRs); the VALU-bound 9-chunk LUT kernels keep the hoisted values
// (VGG-16 conv 1 +0.7% with it).  ALPHA: entries are 16-bit rows beside
// alphas (the LUT neuron); without, row byte offsets (the CuLIF neuron), and
// a field without events returns 0 before the passes.
template <int NB, bool OPAQUE, bool ALPHA, bool POOL = false>
__device__ __forceinline__ int quad_build(const DenseMergeArgs& a, int64_t pix, int* cur, int* kinfo, int* rows,
                                          int* alph, int* bs) {
    static_assert(!(POOL && !ALPHA), "the pool is fused into LUT-neuron builds only");
    constexpr int KMAX = 9;
    int lane = lane_id();
    if constexpr (OPAQUE) asm volatile("" : "+v"(lane));
    const int qd = fdiv((int)pix, a.div_w);
    const int w_out = (int)pix - qd * a.W_out;
    const int img = fdiv(qd, a.div_h);
    const int h_out = qd - img * a.H_out;
    int nk;
    {
        bool v = false;
        int col = 0;
        if (lane < a.K_h * a.K_w) {
            const int kh = lane / a.K_w, kw = lane - kh * a.K_w;
            const int hi = h_out - a.pad_h + kh, wi = w_out - a.pad_w + kw;
            v = hi >= 0 && hi < a.H_in && wi >= 0 && wi < a.W_in;
            col = map_col<POOL>(a, img, hi, wi);
        }
        const uint64_t m = __ballot(v);
        if constexpr (!ALPHA) {
            // the producer's per-site flags: a field of silent sites has no
            // event, and the CuLIF kernel skips the pixel's stream
            if (a.fired && __ballot(v && a.fired[col] != 0) == 0) return 0;
        }
        nk = uniform(__popcll(m));
        if (v) {
            const int slot = __popcll(m & lanemask_lt());
            kinfo[slot] = col * a.C_in;
            kinfo[KMAX + slot] = lane * a.C_in;
        }
    }
    unsigned* msk = reinterpret_cast<unsigned*>(rows);  // 2 words per bin during pass 1
    if (lane < a.T) {
        const int z = vzero();
        cur[lane] = z;
        msk[2 * lane] = z;
        msk[2 * lane + 1] = z;
    }
    wave_sync();
    const int nel = nk * a.C_in;       // <= 9 * 128
    const int n_chunks = (nel + 63) >> 6;  // <= NB
    int pk[NB];
    {
        // element f = c * 64 + lane: tap k = f / C_in (the quotient's
        // fractional part is >= 0.5 / C_in >= 0.5 / 128, far above the
        // product's rounding error, so it rounds down correctly), cin ci.  Every chunk's load is issued before any is
        // used, with no branch (elements past the end load the map's first
        // word; their row and tap fields are never read).
        const __amdgpu_buffer_rsrc_t rin =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, a.in_bytes, 0x00020000);
        float xs[NB];
        int rw[NB];
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const int f = c * 64 + lane;
            const bool in = f < nel;
            const int k = in ? (int)(((float)f + 0.5f) * a.inv_cin) : 0;
            const int ci = f - (int)__umul24((unsigned)k, (unsigned)a.C_in);  // k <= 8, C_in <= 128
            rw[c] = kinfo[KMAX + k] + ci;
            const int off = (kinfo[k] + ci) * 4;
            xs[c] = map_time<POOL>(rin, in ? off : 0, a);
        }
        // arrival_bin and alpha_index without branches: bin floor(t - tfs)
        // clamped below at 0 (floor commutes with the clamp), -1 for no
        // spike (t >= kInfTime or NaN) or a bin past the window; the LUT
        // index is the bin, or clamp((int)t, 0, T) by spike time
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            const float t = xs[c];
            const int tb = (int)floorf(fmaxf(t - a.tfs, 0.0f));  // t < kInfTime keeps it in range
            const bool ev = c * 64 + lane < nel && t < kInfTime && tb < a.T;
            int ai = tb;
            // clamp(t, 0, T) in one med3 (NaN or t >= kInfTime: no event)
            if (a.alpha_by_time) ai = (int)__builtin_amdgcn_fmed3f(t, 0.0f, (float)a.T);
            pk[c] = ev ? (rw[c] << 21) | (ai << 7) | tb : 0x7F;
            __builtin_amdgcn_sched_barrier(0);  // one chunk at a time: fewer live registers
        }
    }
    if constexpr (!ALPHA) {
        // the CuLIF kernel skips the stream of a pixel without events, so a
        // silent field returns here, before the passes (bs and the list are
        // not written)
        bool any = false;
#pragma unroll
        for (int c = 0; c < NB; ++c) any |= (pk[c] & 0x7F) != 0x7F;
        if (__ballot(any) == 0) return 0;
    }
    // pass 1: ranks within each chunk's bins, counts per bin
    const uint64_t lt = lanemask_lt();
    const unsigned bit = 1u << (lane & 31);
#pragma unroll
    for (int c = 0; c < NB; ++c) {
        if (c < n_chunks) {  // uniform
            const int b = pk[c] & 0x7F;
            const bool valid = b != 0x7F;
            if (valid) atomicOr(&msk[2 * b + (lane >> 5)], bit);
            wave_sync();
            uint64_t mm = 0;
            if (valid) mm = *reinterpret_cast<const uint64_t*>(&msk[2 * b]);
            wave_sync();
            const int rank = __popcll(mm & lt);
            const bool last = valid && (mm >> lane) == 1ull;
            if (last) {
                cur[b] += rank + 1;
                const int z = vzero();
                *reinterpret_cast<int2*>(&msk[2 * b]) = make_int2(z, z);
            }
            wave_sync();
            pk[c] |= (rank << 14) | ((last ? 1 : 0) << 20);
        }
    }
    // bin starts: lane l scans bins 4l .. 4l+3 (T <= 64: lane l < 16)
    int v4[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * lane + i;
        v4[i] = t < a.T ? cur[t] : 0;
        sum += v4[i];
    }
    const int incl = wave_incl_scan(sum);
    int run = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * lane + i;
        if (t < a.T) {
            cur[t] = run;
            bs[t] = run;
        }
        run += v4[i];
    }
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (lane == 0) bs[a.T] = total;
    wave_sync();
    // pass 2: event (chunk c, rank) of bin b goes to cur[b] + rank
    float al[NB];
    if constexpr (ALPHA) {
#pragma unroll
        for (int c = 0; c < NB; ++c) al[c] = a.alpha[(pk[c] >> 7) & 0x7F];  // index 0 where no event
    }
#pragma unroll
    for (int c = 0; c < NB; ++c) {
        if (c < n_chunks) {  // uniform
            const int b = pk[c] & 0x7F;
            const int rank = (pk[c] >> 14) & 0x3F;
            if (b != 0x7F) {
                const int pos = cur[b] + rank;
                if constexpr (ALPHA)
                    reinterpret_cast<unsigned short*>(rows)[pos] = (unsigned short)((unsigned)pk[c] >> 21);  // < 2^11
                else
                    rows[pos] = (int)__umul24((unsigned)pk[c] >> 21, (unsigned)a.rowbytes);  // row < 2^11, <= 512 B
                if constexpr (ALPHA) alph[pos] = __float_as_int(al[c]);
            }
            wave_sync();
            if ((pk[c] >> 20) & 1) cur[b] += rank + 1;
            wave_sync();
        }
    }
    // zeroed tail: the stream reads up to 16 entries past the end
    if (lane < kListPad) {
        const int z = vzero();
        if constexpr (ALPHA)
            reinterpret_cast<unsigned short*>(rows)[total + lane] = (unsigned short)z;
        else
            rows[total + lane] = z;
        if constexpr (ALPHA) alph[total + lane] = z;
    }
    return total;
}

// ---------------------------------------------------------------------------
// Shared-list build (k_stream_quad<GEO, 0, CULIF>).  Past the per-wave
// kernels' limits -- more than 128 inputs per tap (a 3x3 pixel of 512 inputs
// has 4,608 receptive elements, 72 chunks of 64) or more c_out than one wave
// gathers -- one workgroup of W waves takes one output pixel: the W waves
// build the pixel's merged list together in the workgroup's LDS, then each
// streams it for its own c_out block.  The build is quad_build's stable
// counting sort of the receptive elements in (kh, kw, cin) order, with the
// chunks split over the waves in contiguous ranges, so that a bin's events
// stay in element order across waves:
//  pass 1  each wave counts its chunks' events per bin: bin 0, where the fire
//          start (T2V:59-60) puts most events, from ballots, the others with
//          LDS atomics;
//  scan    lane b sums bin b's counts over the waves, and a wave scan gives
//          the bin ends (the stream's v_end) and each wave's cursor: the bin's
//          start plus the counts of the lower waves;
//  pass 2  each wave reloads its chunks (L1/L2 hits) and places every event
//          at its bin's cursor plus its rank among the chunk's lanes of the
//          same bin: a ballot for bin 0 (its cursor stays in a scalar), the
//          LDS bit masks of quad_build for the other bins.
// Entries are as in k_stream_quad's per-wave lists: 16-bit weight rows and
// alphas (the LUT neuron), or row byte offsets (the CuLIF neuron).  LDS of a
// workgroup: the list (quad_list_words, rounded up to 4 words), then per
// wave 64 counts, 64 cursors, 128 mask words and the tap table.
constexpr int kSharedMaxWaves = 4;
constexpr int kSharedWaveWords = 64 + 64 + 128 + 32;
constexpr int kSharedBatch = 8;  // chunk loads a wave issues before using any
constexpr int kSharedKeep = 16;  // chunks per wave whose pass-1 results pass 2 takes from registers

__host__ __device__ inline int shared_list_words(int nel_max, int T, bool alphas) {
    return (quad_list_words(nel_max, T, alphas) + 3) & ~3;
}
__host__ __device__ inline int shared_block_words(int nel_max, int T, bool alphas, int waves) {
    return shared_list_words(nel_max, T, alphas) + kSharedWaveWords * waves;
}

// Builds pixel `pix`'s list with the W waves of the workgroup (every wave
// calls it; it ends with a workgroup barrier) and returns its length; v_end
// gets, in lane b < T, the end of bin b, INT_MAX elsewhere.  al_lane holds
// alpha[lane] for lane <= T and al_64 alpha[64] (T = 64); ALPHA selects the
// entry form.
// Keeps the compiler from moving LDS accesses across this point without
// making the wave wait: a wave's LDS instructions execute in program order,
// so a read issued after a write or atomic of the same wave sees its effect.
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

// Receptive element f = 64 c + lane of the shared-list build: tap k =
// f / C_in (the float quotient's fractional part is >= 0.5 / C_in, far above
// its rounding error for the C_in this kernel takes), cin ci; its spike time
// t and weight row.  With C_in a multiple of 64 a chunk lies in one tap,
// whose table entries are scalars (readlane); a chunk of a layer with
// C_in >= 64 (or one tap) spans at most two taps, k0 = the tap of its first
// element and k0 + 1, chosen per lane; otherwise the entries come from the
// wave's LDS tap table.  Elements past the end load the map's first word and
// are no event.
template <bool POOL>
__device__ __forceinline__ void shared_element(const DenseMergeArgs& a, int c, int nel, int nk, int tcol, int trow,
                                               const int* ktab, float& t, int& row) {
    const int lane = lane_id();
    const int f = c * 64 + lane;
    const bool in = f < nel;
    const __amdgpu_buffer_rsrc_t rin =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, a.in_bytes, 0x00020000);
    if ((a.C_in & 63) == 0) {  // uniform: the chunk lies in one tap, k0 = 64 c / C_in
        const int k0 = __builtin_amdgcn_readfirstlane((int)(((float)(c * 64) + 0.5f) * a.inv_cin));
        const int ci = c * 64 - k0 * a.C_in + lane;
        row = __builtin_amdgcn_readlane(trow, k0) + ci;
        t = map_time<POOL>(rin, (__builtin_amdgcn_readlane(tcol, k0) + ci) * 4, a);
        return;  // f < nel: nel is a multiple of 64
    }
    const int k = in ? (int)(((float)f + 0.5f) * a.inv_cin) : 0;
    const int ci = f - k * a.C_in;
    int co, ro;
    if (a.C_in >= 64 || nk == 1) {  // uniform
        const int k0 = __builtin_amdgcn_readfirstlane(k);  // lane 0's element 64 c is in the field
        const int k1 = k0 + 1 < nk ? k0 + 1 : k0;
        const bool lo = k == k0;
        co = lo ? __builtin_amdgcn_readlane(tcol, k0) : __builtin_amdgcn_readlane(tcol, k1);
        ro = lo ? __builtin_amdgcn_readlane(trow, k0) : __builtin_amdgcn_readlane(trow, k1);
    } else {
        co = ktab[k];
        ro = ktab[16 + k];
    }
    row = ro + ci;
    t = map_time<POOL>(rin, in ? (co + ci) * 4 : 0, a);
    if (!in) t = kInfTime;
}

// Arrival bin floor(max(t - tfs, 0)), -1 for no spike or past the window.
__device__ __forceinline__ int shared_bin(const DenseMergeArgs& a, float t) {
    const int tb = (int)floorf(fmaxf(t - a.tfs, 0.0f));
    return (t < kInfTime && tb < a.T) ? tb : -1;
}

// The first KEEP chunks of a wave's range, as pass 1 found them, held in
// registers for pass 2 (which then neither reloads nor re-bins them): bin
// (bits 0..6, 0x7F: no event), decay-LUT index (7..13), weight row (14..29).
template <int KEEP>
struct SharedKeep {
    int v[KEEP > 0 ? KEEP : 1];
};
__device__ __forceinline__ int keep_pack(int b, int ai, int row) { return (row << 14) | (ai << 7) | (b & 0x7F); }

// Decay-LUT index of an event at time t in bin b >= 0: the bin, or
// clamp((int)t, 0, T) by spike time; 0 for no event.
__device__ __forceinline__ int shared_alpha_index(const DenseMergeArgs& a, float t, int b) {
    return b < 0 ? 0 : (a.alpha_by_time ? (int)fminf(fmaxf(t, 0.0f), (float)a.T) : b);
}

// Pass 1 and the scan of the shared-list build, with every wave of the
// workgroup (it ends with a workgroup barrier).  Returns the pixel's list
// length; v_end gets, in lane b < T, the end of bin b (INT_MAX elsewhere);
// nk, tcol and trow describe the in-bounds taps for shared_place: lane
// s < nk holds tap s's input element offset col * C_in and first weight row
// tap * C_in (taps compacted in (kh, kw) order).
template <bool POOL, int KEEP>
__device__ __forceinline__ int shared_count(const DenseMergeArgs& a, int pix, int W, int wave, int* tables,
                                            int& v_end, int& nk, int& tcol, int& trow, SharedKeep<KEEP>& keep) {
    const int lane = lane_id();
    const int T = a.T;
    int* mine = tables + kSharedWaveWords * wave;
    int* cnt = mine;                                         // events per bin
    unsigned* msk = reinterpret_cast<unsigned*>(mine + 128);  // rank masks, two words per bin
    int* ktab = mine + 256;                                  // tap table: offsets [0, 9), rows [16, 25)
    const int qd = fdiv(pix, a.div_w);
    const int w_out = pix - qd * a.W_out;
    const int img = fdiv(qd, a.div_h);
    const int h_out = qd - img * a.H_out;
    {
        bool v = false;
        int col = 0;
        if (lane < a.K_h * a.K_w) {
            const int kh = lane / a.K_w, kx = lane - kh * a.K_w;
            const int hi = h_out - a.pad_h + kh, wi = w_out - a.pad_w + kx;
            v = hi >= 0 && hi < a.H_in && wi >= 0 && wi < a.W_in;
            col = map_col<POOL>(a, img, hi, wi);
        }
        const uint64_t m = __ballot(v);
        nk = uniform(__popcll(m));
        if (v) {
            const int slot = __popcll(m & lanemask_lt());
            ktab[slot] = col * a.C_in;
            ktab[16 + slot] = lane * a.C_in;
        }
        const int z = vzero();
        cnt[lane] = z;
        msk[lane] = z;
        msk[64 + lane] = z;
    }
    wave_sync();
    tcol = lane < nk ? ktab[lane] : 0;
    trow = lane < nk ? ktab[16 + lane] : 0;
    const int nel = nk * a.C_in;
    const int n_chunks = (nel + 63) >> 6;
    const int c_lo = (int)((unsigned)(n_chunks * wave) / (unsigned)W);
    const int c_hi = (int)((unsigned)(n_chunks * (wave + 1)) / (unsigned)W);
    // pass 1: this wave's events per bin (bin 0 from ballots; the counting
    // atomics return nothing, so nothing waits on them); the first KEEP
    // chunks are kept in registers
    static_assert(KEEP % kSharedBatch == 0, "whole batches are kept");
    int n0 = 0;
#pragma unroll
    for (int bt = 0; bt < KEEP / kSharedBatch; ++bt) {
        const int c0 = c_lo + bt * kSharedBatch;
        if (c0 < c_hi) {  // uniform
            float t[kSharedBatch];
            int rw[kSharedBatch];
#pragma unroll
            for (int i = 0; i < kSharedBatch; ++i) {
                t[i] = kInfTime;
                rw[i] = 0;
                if (c0 + i < c_hi) shared_element<POOL>(a, c0 + i, nel, nk, tcol, trow, ktab, t[i], rw[i]);
            }
#pragma unroll
            for (int i = 0; i < kSharedBatch; ++i) {
                const int b = c0 + i < c_hi ? shared_bin(a, t[i]) : -1;
                n0 += __popcll(__ballot(b == 0));
                if (b > 0) atomicAdd(&cnt[b], 1);
                keep.v[bt * kSharedBatch + i] = keep_pack(b, shared_alpha_index(a, t[i], b), rw[i]);
            }
        }
    }
    for (int c0 = c_lo + KEEP; c0 < c_hi; c0 += kSharedBatch) {  // uniform
        float t[kSharedBatch];
        int rw[kSharedBatch];
#pragma unroll
        for (int i = 0; i < kSharedBatch; ++i) {
            t[i] = kInfTime;
            rw[i] = 0;
            if (c0 + i < c_hi) shared_element<POOL>(a, c0 + i, nel, nk, tcol, trow, ktab, t[i], rw[i]);
        }
#pragma unroll
        for (int i = 0; i < kSharedBatch; ++i) {
            if (c0 + i < c_hi) {
                const int b = shared_bin(a, t[i]);
                n0 += __popcll(__ballot(b == 0));
                if (b > 0) atomicAdd(&cnt[b], 1);
            }
        }
    }
    lds_order();
    if (lane == 0) cnt[0] = n0;
    __syncthreads();
    int tot = 0;
    for (int w2 = 0; w2 < W; ++w2) tot += lane < T ? tables[kSharedWaveWords * w2 + lane] : 0;
    const int incl = wave_incl_scan(tot);
    v_end = lane < T ? incl : INT_MAX;
    return __builtin_amdgcn_readlane(incl, 63);
}

// Pass 2 of the shared-list build for the list window [P0, P0 + cap): every
// wave places its chunks' events whose list position falls in the window at
// position - P0 (16-bit weight rows and alphas, or row byte offsets), and
// the positions from the window's end (or the list's) get 32 zeroed
// entries.  Every wave of the workgroup calls it; it ends with a workgroup
// barrier.  The cursors restart from the counts of pass 1, so a window's
// positions do not depend on the windows before it.  NBAT chunk loads are
// issued together.
template <bool ALPHA, int NBAT, bool POOL, int KEEP>
__device__ __forceinline__ void shared_place(const DenseMergeArgs& a, int W, int wave, int* rows, int* alph,
                                             int* tables, int P0, int cap, int total, int nk, int tcol,
                                             int trow, float al_lane, float al_64, const SharedKeep<KEEP>& keep) {
    const int lane = lane_id();
    const int T = a.T;
    int* mine = tables + kSharedWaveWords * wave;
    int* cur = mine + 64;                                    // cursors
    unsigned* msk = reinterpret_cast<unsigned*>(mine + 128);  // rank masks, two words per bin (clear)
    int* ktab = mine + 256;
    // this wave's cursor in bin b: the bin's start plus the lower waves' counts
    int tot = 0, below = 0;
    for (int w2 = 0; w2 < W; ++w2) {
        const int x = lane < T ? tables[kSharedWaveWords * w2 + lane] : 0;
        tot += x;
        below += w2 < wave ? x : 0;
    }
    const int incl = wave_incl_scan(tot);
    cur[lane] = incl - tot + below;
    int cur0 = __builtin_amdgcn_readfirstlane(incl - tot + below);  // bin 0's cursor
    const int n_w = total - P0 < cap ? total - P0 : cap;
    if (wave == 0 && lane < kListPad) {
        const int z = vzero();
        if constexpr (ALPHA) {
            reinterpret_cast<unsigned short*>(rows)[n_w + lane] = (unsigned short)z;
            alph[n_w + lane] = z;
        } else {
            rows[n_w + lane] = z;
        }
    }
    lds_order();
    const int nel = nk * a.C_in;
    const int n_chunks = (nel + 63) >> 6;
    const int c_lo = (int)((unsigned)(n_chunks * wave) / (unsigned)W);
    const int c_hi = (int)((unsigned)(n_chunks * (wave + 1)) / (unsigned)W);
    // Per chunk with events past bin 0 one round trip: OR the lane bits into
    // the bins' masks, read the masks and the cursors back; the bin's last
    // lane in the chunk then advances the cursor and clears the mask (no
    // result, no wait).
    const uint64_t lt = lanemask_lt();
    const unsigned bit = 1u << (lane & 31);
    // one chunk's events: bin b (-1: none), weight row rw, decay-LUT index ai
    auto place = [&](int b, int rw, int ai) {
        float al = 0.0f;
        if constexpr (ALPHA) al = __shfl(al_lane, ai & 63, 64);
        const uint64_t z0 = __ballot(b == 0);
        int pos = cur0 + __popcll(z0 & lt);
        cur0 += __popcll(z0);
        const bool oth = b > 0;
        if (__ballot(oth) != 0) {  // uniform
            if (oth) atomicOr(&msk[2 * b + (lane >> 5)], bit);
            lds_order();
            uint64_t mm = 0;
            int cb = 0;
            if (oth) {
                mm = *reinterpret_cast<const uint64_t*>(&msk[2 * b]);
                cb = cur[b];
            }
            lds_order();
            if (oth) pos = cb + __popcll(mm & lt);
            if (oth && (mm >> lane) == 1ull) {  // the bin's last lane in this chunk
                atomicAdd(&cur[b], __popcll(mm));
                const int z = vzero();
                *reinterpret_cast<int2*>(&msk[2 * b]) = make_int2(z, z);
            }
            lds_order();
        }
        const int q = pos - P0;
        if (b >= 0 && q >= 0 && q < cap) {
            if constexpr (ALPHA) {
                reinterpret_cast<unsigned short*>(rows)[q] = (unsigned short)rw;
                alph[q] = __float_as_int(ai == 64 ? al_64 : al);
            } else {
                rows[q] = (int)__umul24((unsigned)rw, (unsigned)a.rowbytes);
            }
        }
    };
#pragma unroll
    for (int j = 0; j < KEEP; ++j) {
        if (c_lo + j < c_hi) {  // uniform
            const unsigned pk = (unsigned)keep.v[j];
            const int b7 = (int)(pk & 0x7F);
            place(b7 == 0x7F ? -1 : b7, (int)(pk >> 14), (int)((pk >> 7) & 0x7F));
        }
    }
    for (int c0 = c_lo + KEEP; c0 < c_hi; c0 += NBAT) {  // uniform
        float t[NBAT];
        int rw[NBAT];
#pragma unroll
        for (int i = 0; i < NBAT; ++i) {
            t[i] = kInfTime;
            rw[i] = 0;
            if (c0 + i < c_hi) shared_element<POOL>(a, c0 + i, nel, nk, tcol, trow, ktab, t[i], rw[i]);
        }
#pragma unroll
        for (int i = 0; i < NBAT; ++i) {
            if (c0 + i < c_hi) {  // uniform
                const int b = shared_bin(a, t[i]);
                place(b, rw[i], ALPHA ? shared_alpha_index(a, t[i], b) : 0);
            }
        }
    }
    __syncthreads();
}

// POOL: a 2x2 min pool runs inside the list build, from the pool's input
// (DenseMergeArgs::H_u, W_u, pdx, pdy), so the pooled map is never written.
template <int GEO, int NB, bool CULIF, bool POOL = false>
// The CuLIF pair kernel with 9 chunks (CuLIF-7 conv2, VALU-bound) is held to
// 8 waves per SIMD: its 104 scalar registers would allow 7, and the 27 it
// spills to VGPR lanes cost less than the wave (A/B on one box: 2.38 -> 2.29
// ms).  The other instantiations keep the compiler's own choice.
__global__ __launch_bounds__(64 * kQuadWaves)
__attribute__((amdgpu_waves_per_eu(CULIF && GEO == 2 && NB == 9 ? 8 : 1))) void k_stream_quad(
    DenseMergeArgs m, StreamArgs a, float* __restrict__ out, const float* __restrict__ theta, int nel_max) {
    static_assert(GEO == 4 || GEO == 2 || (GEO == 1 && NB <= 0),
                  "four events per load (64 c_out), two (128 c_out), or one (256 c_out, shared lists)");
    static_assert(!(POOL && CULIF), "the pool is fused into LUT-neuron builds only");
    constexpr int OWN = 4 / GEO;  // c_out per lane
    constexpr int LPG = 8 / GEO;  // loads per group of 8 events
    // NB <= 0: one pixel per workgroup, its list shared by the workgroup's
    // waves (shared_count, shared_place), wave w streaming c_out block
    // grp * W + w
    constexpr bool SHARED = NB <= 0;
    // NB = -1: the list may exceed the workgroup's capacity (nel_max entries)
    // and then comes in windows (below); NB = 0: it always fits
    constexpr bool WINDOWS = NB < 0;
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) int lds_words[];
    const int wave = uniform(threadIdx.x >> 6);
    // entries: 16-bit row indices and alphas; the CuLIF neuron adds its
    // weights unscaled (alpha = 1, the reference's acc + w), so its lists
    // hold row byte offsets only
    const int E = quad_list_entries(nel_max, a.T);
    int* region = SHARED ? lds_words : lds_words + wave * quad_wave_words(nel_max, a.T, !CULIF);
    int* rows = region;
    const unsigned short* rows16 = reinterpret_cast<const unsigned short*>(region);
    int* alph = region + E / 2;  // not used by the CuLIF neuron
    int* bs = region + quad_list_words(nel_max, a.T, !CULIF);
    int* cur = bs + a.T + 1;
    int* kinfo = cur + a.T;
    const int lane = lane_id();
    // GEO 4: lane (q, r) = (lane / 16, lane % 16) loads c_out 4r..4r+3 of
    // event q and owns c_out 4r+q; GEO 2: lane (q, r) = (lane / 32, lane % 32)
    // loads c_out 4r..4r+3 of event q and owns c_out 4r+2q, 4r+2q+1; GEO 1:
    // lane r loads and owns c_out 4r..4r+3 of every event (no exchange)
    const int q = GEO == 4 ? lane >> 4 : (GEO == 2 ? lane >> 5 : 0);
    const int r = GEO == 4 ? (lane & 15) : (GEO == 2 ? (lane & 31) : lane);
    int cb = 0;           // SHARED: this wave's c_out block (64 or 128 wide)
    int64_t spix = 0;     // SHARED: the workgroup's pixel
    if constexpr (SHARED) {
        // Workgroups are dealt to the 8 XCDs round-robin.  Block bi takes
        // c_out group bi % n_grp, so where n_grp divides 8 every XCD
        // integrates one group and its L2 holds only that group's share of
        // the weights.  The S = 8 / n_grp XCDs of a group each take a
        // contiguous range of pixels, so the input columns that neighbouring
        // pixels share meet in one L2.
        const int W = blockDim.x >> 6;
        const int n_grp = (a.n_cblk + W - 1) / W;
        const int bi = blockIdx.x;
        const int j = bi / n_grp;
        const int n = (int)a.n_pix;
        const int S = (8 % n_grp == 0) ? 8 / n_grp : 1;
        const int mbr = j % S, per = n / S, rem = n - per * S;
        spix = mbr * per + (mbr < rem ? mbr : rem) + j / S;
        cb = (bi - j * n_grp) * W + wave;
    }
    const int co = (GEO == 4 ? 4 * r + q : (GEO == 2 ? 4 * r + 2 * q : 4 * r)) +
                   cb * (64 * (4 / GEO));  // first c_out of the lane
    const int voff = 16 * r + cb * (256 * (4 / GEO));
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.w_bytes, 0x00020000);
    const int T = a.T;
    // lane d: theta[d] where a spike may occur in bin d (d >= t_min,
    // theta[d] >= 1e-5), else NaN, which no carry compares >= to
    const float th_d = lane < T ? theta[lane] : 0.0f;
    const float v_th = (lane < T && lane >= a.t_min && th_d >= 1e-5f) ? th_d : __builtin_nanf("");
    bool ok[OWN];
    float bias[OWN];
#pragma unroll
    for (int v = 0; v < OWN; ++v) {
        ok[v] = co + v < a.C_out;
        bias[v] = (ok[v] && !CULIF) ? a.bias[co + v] : 0.0f;  // the CuLIF neuron starts at V = 0
    }
    float al_lane = 0.0f, al_64 = 0.0f;  // SHARED: the decay LUT, alpha[lane] and alpha[64]
    if constexpr (SHARED && !CULIF) {
        if (lane <= T) al_lane = m.alpha[lane];
        if (T == 64) al_64 = m.alpha[64];
    }
    const int64_t pix0 = SHARED ? spix : ((int64_t)blockIdx.x * (blockDim.x >> 6) + wave) * a.ppw;
    for (int pq = 0; pq < (SHARED ? 1 : a.ppw); ++pq) {
        const int64_t pix = pix0 + pq;
        if (pix >= a.n_pix) return;  // uniform per wave (SHARED: per workgroup)
        int total, sv_end = 0;
        int snk = 0, stcol = 0, strow = 0;  // SHARED: the pixel's taps
        int* tables = lds_words + shared_list_words(nel_max, T, !CULIF);
        if constexpr (SHARED) {
            SharedKeep<kSharedKeep> keep;
            total = shared_count<POOL>(m, (int)pix, blockDim.x >> 6, wave, tables, sv_end, snk, stcol, strow, keep);
            shared_place<!CULIF, kSharedBatch, POOL>(m, blockDim.x >> 6, wave, rows, alph, tables, 0, nel_max, total,
                                                     snk, stcol, strow, al_lane, al_64, keep);
        } else {
            total = quad_build<NB, (CULIF || NB > 9), !CULIF, POOL>(m, pix, cur, kinfo, rows, alph, bs);
            wave_sync();
        }
        if (CULIF && total == 0) {  // uniform
            // no input: I and V stay 0, so a neuron fires at step 0 when
            // 0 >= th (T3V:50-62) and never otherwise; the 64 steps are skipped
            const float o = 0.0f >= a.th ? 0.0f : kInfTime;
#pragma unroll
            for (int v = 0; v < OWN; ++v)
                if (ok[v]) out[pix * a.C_out + co + v] = o;
            continue;
        }
        int v_end = SHARED ? sv_end : (lane < T ? bs[lane + 1] : INT_MAX);  // end of bin `lane`
        float carry[OWN], acc[OWN], cur[OWN];  // cur: the CuLIF current I
        int res[OWN];  // bins closed with the neuron still alive: its spike bin once it fired
        uint64_t alive[OWN];
#pragma unroll
        for (int v = 0; v < OWN; ++v) {
            carry[v] = bias[v];
            acc[v] = 0.0f;
            cur[v] = 0.0f;
            res[v] = 0;
            alive[v] = __ballot(ok[v]);
        }
        int b = 0;
        int bend = __builtin_amdgcn_readlane(v_end, 0);
        // GEO 2 reads a group's alphas when it consumes the group rather than
        // with its loads: 8 fewer registers in flight (5 waves per SIMD, not 4)
        constexpr bool AL_AHEAD = GEO == 4 && !CULIF;
        struct Raw {
            u4 x[LPG];
            f4 al[AL_AHEAD ? 2 : 1];
        };
        auto load = [&](int j, Raw& g) {
            if constexpr (GEO == 1) {
                // one event per load, its row wave-uniform: the eight rows
                // come with one or two broadcast LDS reads, and each row's
                // byte offset goes to the load's scalar offset
                unsigned so[8];
                if constexpr (CULIF) {
                    const u4 ra = *reinterpret_cast<const u4*>(rows + j);
                    const u4 rb = *reinterpret_cast<const u4*>(rows + j + 4);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        so[k] = __builtin_amdgcn_readfirstlane(ra[k]);
                        so[4 + k] = __builtin_amdgcn_readfirstlane(rb[k]);
                    }
                } else {
                    const u4 rr = *reinterpret_cast<const u4*>(rows16 + j);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const unsigned pr = __builtin_amdgcn_readfirstlane(rr[k]);
                        so[2 * k] = (pr & 0xFFFFu) * (unsigned)m.rowbytes;
                        so[2 * k + 1] = (pr >> 16) * (unsigned)m.rowbytes;
                    }
                }
#pragma unroll
                for (int k = 0; k < LPG; ++k) g.x[k] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, (int)so[k], 0);
            } else {
#pragma unroll
                for (int k = 0; k < LPG; ++k) {
                    const int off = CULIF ? rows[j + GEO * k + q] + voff
                                          : (int)__umul24((unsigned)rows16[j + GEO * k + q], (unsigned)m.rowbytes) + voff;
                    g.x[k] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
                }
            }
            if constexpr (AL_AHEAD) {
                g.al[0] = *reinterpret_cast<const f4*>(alph + j);
                g.al[1] = *reinterpret_cast<const f4*>(alph + j + 4);
            }
        };
        // close bin b and the empty bins after it that end by position p (bin
        // ends do not decrease, so they are the first `stop` bins); true when
        // the stream is over
        auto close_to = [&](int p) -> bool {
            if constexpr (!CULIF) {
#pragma unroll
                for (int v = 0; v < OWN; ++v) {
                    carry[v] = carry[v] + acc[v];
                    acc[v] = 0.0f;
                }
            }
            const int stop = __popcll(__builtin_amdgcn_ballot_w64(v_end <= p));  // > b (lanes >= T: INT_MAX)
            if constexpr (CULIF) {
                do {
                    // I = fma(I, decay, in_b); V += I; fire at V >= th (T3V:50-62);
                    // every bin steps the neuron, empty ones with in_b = 0
#pragma unroll
                    for (int v = 0; v < OWN; ++v) {
                        cur[v] = __builtin_fmaf(cur[v], a.decay, acc[v]);
                        acc[v] = 0.0f;
                        carry[v] = carry[v] + cur[v];
                        alive[v] &= ~__ballot(carry[v] >= a.th);
                        res[v] = add_lane_bit(res[v], alive[v]);
                    }
                } while (++b < stop);
            } else {
                auto close_bin = [&]() {
                    const float th = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_th), b));
#pragma unroll
                    for (int v = 0; v < OWN; ++v) {
                        alive[v] &= ~__ballot(carry[v] >= th);
                        res[v] = add_lane_bit(res[v], alive[v]);
                    }
                };
                do close_bin();
                while (++b < stop);
            }
            uint64_t any = alive[0];
#pragma unroll
            for (int v = 1; v < OWN; ++v) any |= alive[v];
            if (b >= T || any == 0) return true;
            bend = __builtin_amdgcn_readlane(v_end, b);
            return false;
        };
        // integrates positions j .. j+7; true when the stream is over
        auto consume = [&](int j, Raw& g) -> bool {
            float w[8][OWN], al[8];
#pragma unroll
            for (int k = 0; k < LPG; ++k) {
                if constexpr (GEO == 1) {  // the lane's own four c_out of event k
                    w[k][0] = __uint_as_float(g.x[k].x);
                    w[k][1 % OWN] = __uint_as_float(g.x[k].y);
                    w[k][2 % OWN] = __uint_as_float(g.x[k].z);
                    w[k][3 % OWN] = __uint_as_float(g.x[k].w);
                    continue;
                }
                unsigned c0 = g.x[k].x, c1 = g.x[k].y, c2 = g.x[k].z, c3 = g.x[k].w;
                // permlane32_swap(x, y): x's lanes 32..63 <-> y's lanes 0..31
                auto p = __builtin_amdgcn_permlane32_swap(c0, c2, false, false);
                c0 = p[0];
                c2 = p[1];
                p = __builtin_amdgcn_permlane32_swap(c1, c3, false, false);
                c1 = p[0];
                c3 = p[1];
                if constexpr (GEO == 4) {
                    // permlane16_swap(x, y): x's lanes 16..31, 48..63 <-> y's 0..15, 32..47
                    p = __builtin_amdgcn_permlane16_swap(c0, c1, false, false);
                    c0 = p[0];
                    c1 = p[1];
                    p = __builtin_amdgcn_permlane16_swap(c2, c3, false, false);
                    c2 = p[0];
                    c3 = p[1];
                    w[4 * k + 0][0] = __uint_as_float(c0);
                    w[4 * k + 1][0] = __uint_as_float(c1);
                    w[4 * k + 2][0] = __uint_as_float(c2);
                    w[4 * k + 3][0] = __uint_as_float(c3);
                } else {
                    w[2 * k + 0][0] = __uint_as_float(c0);
                    w[2 * k + 0][OWN - 1] = __uint_as_float(c1);
                    w[2 * k + 1][0] = __uint_as_float(c2);
                    w[2 * k + 1][OWN - 1] = __uint_as_float(c3);
                }
            }
            if constexpr (!CULIF) {
                f4 a0, a1;
                if constexpr (AL_AHEAD) {
                    a0 = g.al[0];
                    a1 = g.al[AL_AHEAD ? 1 : 0];
                } else {
                    a0 = *reinterpret_cast<const f4*>(alph + j);
                    a1 = *reinterpret_cast<const f4*>(alph + j + 4);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    al[i] = a0[i];
                    al[4 + i] = a1[i];
                }
            }
            // event i: fma(w, alpha, acc); the CuLIF neuron's acc + w
            auto integ = [&](int i) {
#pragma unroll
                for (int v = 0; v < OWN; ++v)
                    acc[v] = CULIF ? acc[v] + w[i][v] : __builtin_fmaf(w[i][v], al[i], acc[v]);
            };
            if (bend >= j + 8) {  // all eight in the open bin
#pragma unroll
                for (int i = 0; i < 8; ++i) integ(i);
                return false;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (bend <= j + i && close_to(j + i)) return true;
                integ(i);
            }
            return false;
        };
        // the next group's loads are issued before this group's wait
        Raw g0, g1;
        if constexpr (!WINDOWS) {
            if (SHARED && cb >= a.n_cblk) continue;  // a wave past the last c_out block only helps build
            load(0, g0);
            for (int j = 0;; j += 16) {
                load(j + 8, g1);
                __builtin_amdgcn_sched_barrier(0);
                if (consume(j, g0)) break;
                load(j + 16, g0);
                __builtin_amdgcn_sched_barrier(0);
                if (consume(j + 8, g1)) break;
            }
        } else {
            // Windows of at most nel_max list entries: positions are window-
            // relative (v_end shifted by the window's start P0), and a window
            // that more follow stops its stream at its end (jlim) with the
            // open bin and the neuron state kept; the next window then goes
            // on from its first entry.  Waves past the last c_out block only
            // help build.  Later windows place one chunk at a time: their
            // placement runs beside the live neuron state, and a batch of
            // loads there cost the kernel its eighth wave per SIMD.
            bool live = cb < a.n_cblk;
            int P0 = 0;
            for (;;) {
                const int jlim = total - P0 > nel_max ? nel_max : INT_MAX;
                if (live) {
                    load(0, g0);
                    for (int j = 0;; j += 16) {
                        if (j >= jlim) break;
                        load(j + 8, g1);
                        __builtin_amdgcn_sched_barrier(0);
                        if (consume(j, g0)) {
                            live = false;
                            break;
                        }
                        if (j + 8 >= jlim) break;
                        load(j + 16, g0);
                        __builtin_amdgcn_sched_barrier(0);
                        if (consume(j + 8, g1)) {
                            live = false;
                            break;
                        }
                    }
                }
                if (jlim == INT_MAX) break;  // uniform: the last window
                P0 += nel_max;
                __syncthreads();  // every wave is done with this window
                shared_place<!CULIF, 1, POOL>(m, blockDim.x >> 6, wave, rows, alph, tables, P0, nel_max, total, snk,
                                              stcol, strow, al_lane, al_64, SharedKeep<0>{});
                if (lane < T) v_end = sv_end - P0;
                if (live) bend = __builtin_amdgcn_readlane(v_end, b);
            }
        }
#pragma unroll
        for (int v = 0; v < OWN; ++v)
            if (ok[v]) out[pix * a.C_out + co + v] = __builtin_amdgcn_inverse_ballot_w64(alive[v]) ? kInfTime : (float)res[v];
        wave_sync();  // this pixel's list reads precede the next pixel's build
    }
}

// ---------------------------------------------------------------------------
// k_stream_multi: weight rows reused across images.  One wave integrates one
// output position of kMultiImages = 4 consecutive images over a block of 256
// c_out (four per lane, one 16-byte load per weight row, no transposes), so a
// weight row gathered once serves every image that holds the same (tap, cin)
// event in the same bin.  The fire start (T2V:59-60) puts most events in bin
// 0, where the images' events coincide often: at a bin-0 density d0 an
// element is a bin-0 event of at least one of the four images with
// probability 1 - (1 - d0)^4, against 4 d0 events (d0 = 0.35: 1.7 events per
// row load).
//  bin 0   the wave walks the receptive elements in (kh, kw, cin) order, 64
//          per chunk, lane = element: a lane reads the element's spike time
//          in the four images and forms the mask of images whose event falls
//          in bin 0 and their alphas; the chunk's elements with a nonzero
//          mask go, in element order, to a ring in LDS (row and mask, four
//          alphas), and the stream takes the ring four entries at a time:
//          one row load, then for each image of the entry's mask (a
//          wave-uniform branch) four fmas into that image's bin sum.  An
//          image absent from an entry is never touched, so each image's
//          bin-0 chain is its own events in (kh, kw, cin) order, the
//          reference's per-bin order (T2V:135-152);
//  counts  the same pass counts every image's events of the later bins
//          (LDS atomics that return nothing); a scan gives the bin ends;
//  later   a second pass over the chunks places the later events, stable in
//          (chunk, image, lane) order, at the bin's cursor plus the rank
//          among the lanes of the same bin (shared_place's LDS bit masks), so
//          within a bin each image's events stay in element order; entries
//          hold the 16-bit row, the image (one-hot) and the alpha index.
//          The stream closes bins in time order between entries as the
//          per-wave kernels do, each entry's fmas going to its image.
// A later list longer than the wave's capacity streams in windows (as the
// shared-list kernel's NB = -1): the second pass runs once per window.
// Measured on VGG-16 (per-layer HIP events, bit-identical maps): slower than
// the shared-list kernel on every layer it takes.  B=256: the 8x8 layers
// 0.39/0.56/0.56 -> 0.59/0.89/0.91 ms, the 4x4 layers 0.36/0.53/0.53 ->
// 0.62/0.91/1.04, the 2x2 layers 4-5x, the FC 9x: a wave holds four images
// x 256 c_out, so the 4x4 layers have 2,048 waves (two per SIMD) and the
// FC 128, and each wave's entries wait on an LDS read, a readfirstlane and
// the row's scalar offset before its load.  B=1024 (16,384 waves on the 8x8
// layers): about even on conv 4, 5-15% slower on conv 5-6, 20-45% on the
// 4x4 layers.  The union saves row loads (0.68 per event at input density
// 0.48); each entry pays instead an LDS read of its row and mask, a
// readfirstlane, four alphas and a branch per image.  So it is a plan the
// caller may select (VDTTFS_PATH_FUSED, gather 4, 4 pixels per wave), not
// the built-in one.
constexpr int kMultiImages = 4;
constexpr int kMultiRing = 128;  // bin-0 ring entries (a chunk adds at most 64 past the 8 ahead)
constexpr int kMultiFixedWords = kMultiRing * 5 + 64 + 64 + 128 + 32;  // ring, counts, cursors, masks, taps

__host__ __device__ inline int multi_wave_words(int cap) { return kMultiFixedWords + cap + kListPad; }

// Three waves per SIMD: its LDS (about 12 KB per wave) allows about as many,
// and the compiler then keeps the sixteen neurons' state in registers.
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3, 3))) void k_stream_multi(
    DenseMergeArgs m, StreamArgs a, float* __restrict__ out,
                                                     const float* __restrict__ theta, int cap, int n_pos,
                                                     int n_img) {
    constexpr int NI = kMultiImages;
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    typedef float f4 __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) int lds_words[];
    f4* al4 = reinterpret_cast<f4*>(lds_words);             // ring alphas, one f4 per entry
    unsigned* rm = reinterpret_cast<unsigned*>(lds_words + 4 * kMultiRing);  // ring (row << 4) | mask
    int* cnt = lds_words + 5 * kMultiRing;                   // later events per bin
    int* cur = cnt + 64;                                     // later-bin cursors
    unsigned* msk = reinterpret_cast<unsigned*>(cur + 64);   // rank masks, two words per bin
    int* ktab = reinterpret_cast<int*>(msk + 128);           // tap table: offsets [0, 9), rows [16, 25)
    unsigned* list = reinterpret_cast<unsigned*>(ktab + 32);  // later entries of the window
    const int lane = lane_id();
    const int T = a.T;
    // block -> (c_out block, problem): blocks are dealt to the 8 XCDs
    // round-robin, so block b's c_out block b % n_cblk pins each XCD to one
    // block where n_cblk divides 8; the S = 8 / n_cblk XCDs of a block take
    // contiguous ranges of problems (consecutive positions of one image
    // group share input columns)
    const int n_cblk = a.n_cblk;
    const int n_prob = ((n_img + NI - 1) / NI) * n_pos;
    const int bi = blockIdx.x;
    const int cb = bi % n_cblk;
    const int j0 = bi / n_cblk;
    const int S = (8 % n_cblk == 0) ? 8 / n_cblk : 1;
    const int mbr = j0 % S, per = n_prob / S, rem = n_prob - per * S;
    const int prob = mbr * per + (mbr < rem ? mbr : rem) + j0 / S;
    if (prob >= n_prob) return;
    const int grp = prob / n_pos;
    const int pos = prob - grp * n_pos;
    const int img0 = grp * NI;
    const int n_live = (n_img - img0) < NI ? (n_img - img0) : NI;  // images of this group
    const int h_out = pos / m.W_out;
    const int w_out = pos - h_out * m.W_out;
    const int istride = m.H_in * m.W_in * m.C_in;  // one image's map (elements)
    const int co = 4 * lane + cb * 256;
    const int voff = 16 * lane + cb * 1024;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.w_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rin =
        __builtin_amdgcn_make_buffer_rsrc((void*)m.in, (short)0, m.in_bytes, 0x00020000);
    // lane d: theta[d] where a spike may occur in bin d (d >= t_min,
    // theta[d] >= 1e-5), else NaN, which no carry compares >= to
    const float th_d = lane < T ? theta[lane] : 0.0f;
    const float v_th = (lane < T && lane >= a.t_min && th_d >= 1e-5f) ? th_d : __builtin_nanf("");
    const float al_lane = lane <= T ? m.alpha[lane] : 0.0f;  // the decay LUT: alpha[lane], alpha[64]
    const float al_64 = T == 64 ? m.alpha[64] : 0.0f;
    const bool ok = co < a.C_out;  // C_out % 4 == 0: the lane's four c_out are all in or all out
    float bias[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) bias[v] = ok ? a.bias[co + v] : 0.0f;
    // taps of the position (the same in every image): lane s < nk holds tap
    // s's input element offset in image img0 and its first weight row
    int nk, tcol, trow;
    {
        bool vt = false;
        int col = 0;
        if (lane < m.K_h * m.K_w) {
            const int kh = lane / m.K_w, kx = lane - kh * m.K_w;
            const int hi = h_out - m.pad_h + kh, wi = w_out - m.pad_w + kx;
            vt = hi >= 0 && hi < m.H_in && wi >= 0 && wi < m.W_in;
            col = (img0 * m.H_in + hi) * m.W_in + wi;
        }
        const uint64_t mt = __ballot(vt);
        nk = uniform(__popcll(mt));
        if (vt) {
            const int slot = __popcll(mt & lanemask_lt());
            ktab[slot] = col * m.C_in;
            ktab[16 + slot] = lane * m.C_in;
        }
        const int z = vzero();
        cnt[lane] = z;
        msk[lane] = z;
        msk[64 + lane] = z;
        wave_sync();
        tcol = lane < nk ? ktab[lane] : 0;
        trow = lane < nk ? ktab[16 + lane] : 0;
    }
    const int nel = nk * m.C_in;
    const int n_chunks = (nel + 63) >> 6;
    // chunk c's element per lane: its offset in image img0's map (-1 past
    // the field) and its weight row (as shared_element)
    auto element = [&](int c, int& eo, int& row) {
        const int f = c * 64 + lane;
        if ((m.C_in & 63) == 0) {  // uniform: the chunk lies in one tap
            const int k0 = __builtin_amdgcn_readfirstlane((int)(((float)(c * 64) + 0.5f) * m.inv_cin));
            const int ci = c * 64 - k0 * m.C_in + lane;
            row = __builtin_amdgcn_readlane(trow, k0) + ci;
            eo = __builtin_amdgcn_readlane(tcol, k0) + ci;
            return;
        }
        const bool in = f < nel;
        const int k = in ? (int)(((float)f + 0.5f) * m.inv_cin) : 0;
        const int ci = f - k * m.C_in;
        int c0, r0;
        if (m.C_in >= 64 || nk == 1) {  // uniform
            const int k0 = __builtin_amdgcn_readfirstlane(k);
            const int k1 = k0 + 1 < nk ? k0 + 1 : k0;
            const bool lo = k == k0;
            c0 = lo ? __builtin_amdgcn_readlane(tcol, k0) : __builtin_amdgcn_readlane(tcol, k1);
            r0 = lo ? __builtin_amdgcn_readlane(trow, k0) : __builtin_amdgcn_readlane(trow, k1);
        } else {
            c0 = ktab[k];
            r0 = ktab[16 + k];
        }
        row = r0 + ci;
        eo = in ? c0 + ci : -1;
    };
    // the element's spike times in the group's images (no event: kInfTime)
    auto times = [&](int eo, float (&t)[NI]) {
#pragma unroll
        for (int p = 0; p < NI; ++p) {
            const bool v = eo >= 0 && p < n_live;
            t[p] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, v ? (eo + p * istride) * 4 : 0, 0, 0));
            if (!v) t[p] = kInfTime;
        }
    };
    auto alpha_of = [&](float t, int b) -> int {
        return m.alpha_by_time ? (int)fminf(fmaxf(t, 0.0f), (float)T) : b;
    };
    // neuron state per (image, c_out of the lane): V (carry), the open bin's
    // sum, the spike bin (kNoSpike while it has not fired; -1 for no neuron).
    // The spike bins live in VGPRs, not as SGPR masks: sixteen 64-bit masks
    // would take a third of the wave's scalar registers.
    constexpr int kNoSpike = 0x7F;
    float carry[NI][4], acc[NI][4];
    int fb[NI][4];
#pragma unroll
    for (int p = 0; p < NI; ++p) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            carry[p][v] = bias[v];
            acc[p][v] = 0.0f;
            fb[p][v] = (p < n_live && ok) ? kNoSpike : -1;
        }
    }
    // ---- bin 0: produce ring entries from the chunks, stream them ----
    int tail = 0;  // ring entries produced
    int c = 0;     // next chunk to produce
    int eo_n = -1, row_n = 0;
    float t_n[NI];
    const uint64_t lt = lanemask_lt();
    if (n_chunks > 0) {
        element(0, eo_n, row_n);
        times(eo_n, t_n);
    }
    auto produce = [&]() {
        float t[NI];
#pragma unroll
        for (int p = 0; p < NI; ++p) t[p] = t_n[p];
        const int row = row_n;
        if (c + 1 < n_chunks) {  // uniform: the next chunk's loads go out first
            element(c + 1, eo_n, row_n);
            times(eo_n, t_n);
        }
        ++c;
        unsigned mk = 0;
        f4 al;
#pragma unroll
        for (int p = 0; p < NI; ++p) {
            const int b = shared_bin(m, t[p]);
            if (b > 0) atomicAdd(&cnt[b], 1);
            const int ai = b == 0 ? alpha_of(t[p], 0) : 0;
            const float x = __shfl(al_lane, ai & 63, 64);
            al[p] = ai == 64 ? al_64 : x;
            mk |= (b == 0 ? 1u : 0u) << p;
        }
        const uint64_t any = __ballot(mk != 0);
        const int q = (tail + __popcll(any & lt)) & (kMultiRing - 1);
        if (mk != 0) {
            rm[q] = ((unsigned)row << 4) | mk;
            al4[q] = al;
        }
        lds_order();
        tail += __popcll(any);
    };
    auto ensure = [&](int upto) {
        while (c < n_chunks && tail < upto) produce();  // uniform
    };
    struct Raw {
        u4 x[4];
        unsigned mk;  // four 4-bit image masks
    };
    auto load0 = [&](int j, Raw& g) {
        const u4 e = *reinterpret_cast<const u4*>(rm + (j & (kMultiRing - 1)));
        g.mk = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned s = __builtin_amdgcn_readfirstlane(e[i]);
            const bool in = j + i < tail;
            g.mk |= (in ? (s & 15u) : 0u) << (4 * i);
            const int so = in ? (int)((s >> 4) * (unsigned)m.rowbytes) : 0;
            g.x[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, so, 0);
        }
    };
    auto consume0 = [&](int j, Raw& g) {
        f4 A[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) A[i] = al4[(j + i) & (kMultiRing - 1)];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float w[4] = {__uint_as_float(g.x[i].x), __uint_as_float(g.x[i].y), __uint_as_float(g.x[i].z),
                                __uint_as_float(g.x[i].w)};
#pragma unroll
            for (int p = 0; p < NI; ++p) {
                if ((g.mk >> (4 * i + p)) & 1u) {  // uniform
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[p][v] = __builtin_fmaf(w[v], A[i][p], acc[p][v]);
                }
            }
        }
    };
    {
        Raw g0, g1;
        ensure(8);
        int j = 0;
        if (tail > 0) {
            load0(0, g0);
            for (;;) {
                ensure(j + 8);
                load0(j + 4, g1);
                __builtin_amdgcn_sched_barrier(0);
                consume0(j, g0);
                j += 4;
                if (j >= tail) break;  // uniform: every chunk is produced (ensure)
                ensure(j + 8);
                load0(j + 4, g0);
                __builtin_amdgcn_sched_barrier(0);
                consume0(j, g1);
                j += 4;
                if (j >= tail) break;
            }
        }
        while (c < n_chunks) produce();  // chunks without bin-0 events still count
    }
    // ---- later bins: ends, close bin 0, place and stream ----
    lds_order();
    const int tot = (lane >= 1 && lane < T) ? cnt[lane] : 0;
    const int incl = wave_incl_scan(tot);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    int v_end = lane < T ? incl : INT_MAX;  // end of bin `lane` in the later list (bin 0: 0)
    int b = 0;
    int bend = 0;
    // close bin b and the empty bins after it that end by position p; true
    // when the stream is over
    auto close_to = [&](int p) -> bool {
#pragma unroll
        for (int q = 0; q < NI; ++q)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                carry[q][v] = carry[q][v] + acc[q][v];
                acc[q][v] = 0.0f;
            }
        const int stop = __popcll(__builtin_amdgcn_ballot_w64(v_end <= p));
        uint64_t any;
        do {
            const float th = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_th), b));
            any = 0;
#pragma unroll
            for (int q = 0; q < NI; ++q)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const uint64_t fire = __ballot(carry[q][v] >= th);
                    const uint64_t live = __ballot(fb[q][v] == kNoSpike);
                    fb[q][v] = __builtin_amdgcn_inverse_ballot_w64(fire & live) ? b : fb[q][v];
                    any |= live & ~fire;
                }
        } while (++b < stop);
        if (b >= T || any == 0) return true;
        bend = __builtin_amdgcn_readlane(v_end, b);
        return false;
    };
    bool done = close_to(0);
    // pass 2: place the later events of window [P0, P0 + cap)
    auto place = [&](int P0) {
        cur[lane] = incl - tot;
        const int n_w = total - P0 < cap ? total - P0 : cap;
        if (lane < kListPad) list[n_w + lane] = (unsigned)vzero();
        lds_order();
        const unsigned bit = 1u << (lane & 31);
        for (int cc = 0; cc < n_chunks; ++cc) {  // uniform
            int eo, row;
            float t[NI];
            element(cc, eo, row);
            times(eo, t);
#pragma unroll
            for (int p = 0; p < NI; ++p) {
                const int bb = shared_bin(m, t[p]);
                const bool oth = bb > 0;
                if (__ballot(oth) == 0) continue;  // uniform
                if (oth) atomicOr(&msk[2 * bb + (lane >> 5)], bit);
                lds_order();
                uint64_t mm = 0;
                int cbin = 0;
                if (oth) {
                    mm = *reinterpret_cast<const uint64_t*>(&msk[2 * bb]);
                    cbin = cur[bb];
                }
                lds_order();
                const int q = cbin + __popcll(mm & lt) - P0;
                if (oth && (mm >> lane) == 1ull) {  // the bin's last lane in this chunk
                    atomicAdd(&cur[bb], __popcll(mm));
                    const int z = vzero();
                    *reinterpret_cast<int2*>(&msk[2 * bb]) = make_int2(z, z);
                }
                lds_order();
                if (oth && q >= 0 && q < cap)
                    list[q] = (unsigned)row | (1u << (16 + p)) | ((unsigned)alpha_of(t[p], bb) << 20);
            }
        }
        lds_order();
    };
    if (!done) {
        const float al_64s = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(al_64)));
        struct RawL {
            u4 x[4];
            unsigned s[4];
        };
        auto loadL = [&](int j, RawL& g) {
            const u4 e = *reinterpret_cast<const u4*>(list + j);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                g.s[i] = __builtin_amdgcn_readfirstlane(e[i]);
                g.x[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, (int)((g.s[i] & 0xFFFFu) * (unsigned)m.rowbytes),
                                                               0);
            }
        };
        // integrates positions j .. j+3; true when the stream is over
        auto consumeL = [&](int j, RawL& g) -> bool {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (bend <= j + i && close_to(j + i)) return true;
                const unsigned s = g.s[i];
                const int ai = (int)(s >> 20);
                const float al = ai == 64 ? al_64s : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(al_lane), ai));
                const float w[4] = {__uint_as_float(g.x[i].x), __uint_as_float(g.x[i].y), __uint_as_float(g.x[i].z),
                                    __uint_as_float(g.x[i].w)};
                // the entry's image as a one-hot mask, tested bit by bit: a
                // test on the image's index would let the compiler index the
                // state arrays by it, which puts them in scratch memory
#pragma unroll
                for (int q = 0; q < NI; ++q) {
                    if ((s >> (16 + q)) & 1u) {  // uniform
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[q][v] = __builtin_fmaf(w[v], al, acc[q][v]);
                    }
                }
            }
            return false;
        };
        RawL g0, g1;
        int P0 = 0;
        for (;;) {
            place(P0);
            if (lane < T) v_end = incl - P0;
            bend = __builtin_amdgcn_readlane(v_end, b);
            const int jlim = total - P0 > cap ? cap : INT_MAX;
            bool over = false;
            loadL(0, g0);
            for (int j = 0;; j += 8) {
                if (j >= jlim) break;
                loadL(j + 4, g1);
                __builtin_amdgcn_sched_barrier(0);
                if (consumeL(j, g0)) {
                    over = true;
                    break;
                }
                if (j + 4 >= jlim) break;
                loadL(j + 8, g0);
                __builtin_amdgcn_sched_barrier(0);
                if (consumeL(j + 4, g1)) {
                    over = true;
                    break;
                }
            }
            if (over || jlim == INT_MAX) break;  // uniform
            P0 += cap;
        }
    }
#pragma unroll
    for (int p = 0; p < NI; ++p) {
        if (p < n_live && ok) {
            const int64_t pix = (int64_t)(img0 + p) * n_pos + pos;
#pragma unroll
            for (int v = 0; v < 4; ++v) out[pix * a.C_out + co + v] = fb[p][v] == kNoSpike ? kInfTime : (float)fb[p][v];
        }
    }
}

// ---------------------------------------------------------------------------
// k_stream_window: k_merge and k_stream in one kernel for the bins path (the
// layers whose columns were bucketized: conv with C_in > 64, FC), T <= 64.
// Whole merged lists in LDS would cost occupancy (a 3x3 pixel of 512 inputs
// is up to 37 KB), so each wave streams its pixel's merged list through a
// window of 64 entries held one per lane in registers, with the next window
// in a second register: when the stream passes a window, the following one
// is built straight from the columns' bin-layout lists.  Merged position p
// of event i of column k in bin t is D[k][t] + i with D[k][t] =
// sum_{k'<k} O_k'[t+1] + sum_{k'>k} O_k'[t] (O_k = the column's bin offsets,
// as in k_merge), so within a column positions increase with i and a window
// [P0, P0 + 64) takes from each column one contiguous index range: from
// where the previous window stopped to the index whose position reaches
// P0 + 64, which the bin holding P0 + 64 and the closed form give.  Lane f
// loads the window's f-th event (column-major), computes its position and
// ds_permute moves the entry to lane p - P0.  Nothing goes through HBM but
// the bucketize output; the per-pixel tables live in LDS.
// Measured on VGG-16 B=256 against bucketize + k_merge + k_stream (layer
// times include the bucketize): slower on every bins layer -- 128 -> 128 at
// 16x16 0.92 -> 1.16 ms, the 8x8 and 4x4 layers +3..7%, the 2x2 layers and
// the FC +5..10% -- as building a window costs the wave about as many
// instructions as streaming it, where k_merge's work ran in a kernel of its
// own with every lane busy.  So the built-in plan keeps the two kernels, and
// this path is a plan the caller may select (VDTTFS_PATH_WINDOW).
template <int KMAX>
struct WinCtx {
    int dtab[KMAX][kBlockBins];   // D[k][t]
    int o[KMAX][kBlockBins + 1];  // O_k[t], t in [0, T]
    int S[kBlockBins + 1];        // merged start of bin t, S[T] = list length
    int col[KMAX], krow[KMAX];    // in-bounds columns in (kh, kw) order; first weight-row byte offset
    int lo[KMAX];                 // first index of column k not yet windowed
    int nk, total;
};

// Per pixel: the in-bounds columns, their bin offsets, D and S.  T <= 64.
template <int KMAX>
__device__ __forceinline__ void win_setup(const MergeArgs& m, int64_t pix, WinCtx<KMAX>& w) {
    const int lane = lane_id();
    int img, h_out = 0, w_out = 0;
    if (m.is_fc) {
        img = (int)pix;
    } else {
        const int q = fdiv((int)pix, m.div_w);
        w_out = (int)pix - q * m.W_out;
        img = fdiv(q, m.div_h);
        h_out = q - img * m.H_out;
    }
    int nk;
    if (m.is_fc) {
        nk = 1;
        if (lane == 0) {
            w.col[0] = img;
            w.krow[0] = 0;
        }
    } else {
        bool v = false;
        int col = 0;
        if (lane < m.K_h * m.K_w) {
            const int kh = lane / m.K_w, kw = lane - kh * m.K_w;
            const int hi = h_out - m.pad_h + kh, wi = w_out - m.pad_w + kw;
            v = hi >= 0 && hi < m.H_in && wi >= 0 && wi < m.W_in;
            col = (img * m.H_in + hi) * m.W_in + wi;
        }
        const uint64_t mk = __ballot(v);
        nk = __popcll(mk);
        if (v) {
            const int slot = __popcll(mk & lanemask_lt());
            w.col[slot] = col;
            w.krow[slot] = lane * m.C_in * m.rowbytes;
        }
    }
    wave_sync();
    const int T = m.T, osb = T + 1;
    int lo[KMAX], hi[KMAX];
    int S = 0, total = 0;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        lo[k] = hi[k] = 0;
        if (k < nk) {
            const int32_t* ob = m.off + (int64_t)uniform(w.col[k]) * osb;
            if (lane < T) {
                lo[k] = ob[lane];
                hi[k] = ob[lane + 1];
            }
            const int tk = ob[T];
            total += tk;
            S += lo[k];
            if (lane < T) w.o[k][lane] = lo[k];
            if (lane == 0) {
                w.o[k][T] = tk;
                w.lo[k] = 0;
            }
        }
    }
    int A = 0, P = 0;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        if (k < nk) {
            P += lo[k];
            if (lane < T) w.dtab[k][lane] = A + (S - P);
            A += hi[k];
        }
    }
    if (lane < T) w.S[lane] = S;
    if (lane == 0) {
        w.S[T] = total;
        w.nk = nk;
        w.total = total;
    }
    wave_sync();
}

// List reader over the window (see k_stream_window): w0 holds merged entries
// base + lane, w1 the next 64.  Windows are built in order, 64 positions at
// a time, when the stream passes one; entries past the list are zero (row 0,
// alpha 0), like the padding of the HBM lists.  Loading a window's events one
// window ahead (so they arrive while w0 streams) was measured slower: it
// costs registers (the dwordx4 stream 92 -> 97 VGPRs, 5 -> 4 waves per SIMD)
// and the building, not the wait, is what costs here.
template <int KMAX>
struct WinList {
    WinCtx<KMAX>* w;
    const vd_event* ev;
    int C_in, rowbytes, T;
    int base;
    int2 w0, w1;
    __device__ __forceinline__ int2 fill(int P0) {
        const int lane = lane_id();
        const int total = uniform(w->total);
        int2 e = make_int2(0, 0);
        if (P0 >= total) return e;  // uniform
        const int P1 = P0 + 64;
        const int nk = uniform(w->nk);
        int t1 = -1;
        if (P1 < total) {  // the bin holding position P1: the last bin starting at or before it
            const int sl = lane < T ? w->S[lane] : 0x7fffffff;
            t1 = __popcll(__ballot(sl <= P1)) - 1;
        }
        int kk = 0, cbase = 0, lo_sel = 0, C = 0;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            if (k < nk) {
                const int lo = uniform(w->lo[k]);
                int hi;
                if (t1 < 0) {
                    hi = uniform(w->o[k][T]);
                } else {
                    const int ot = uniform(w->o[k][t1]), on = uniform(w->o[k][t1 + 1]);
                    const int d = P1 - uniform(w->dtab[k][t1]) - ot;
                    hi = ot + (d < 0 ? 0 : (d > on - ot ? on - ot : d));
                }
                if (lane >= C && lane < C + (hi - lo)) {  // lane takes column k's (lane - C)-th event
                    kk = k;
                    cbase = C;
                    lo_sel = lo;
                }
                C += hi - lo;
                // every lane read lo[k] above; a wave's LDS operations
                // execute in program order
                if (lane == 0) w->lo[k] = hi;
            }
        }
        int pos = lane;  // lanes past the window's events carry the zero padding
        if (lane < C) {
            const int i = lo_sel + (lane - cbase);
            const vd_event x = ev[(int64_t)w->col[kk] * C_in + i];
            const int b = (int)(x.key >> 24);
            pos = w->dtab[kk][b] + i - P0;
            e = make_int2(w->krow[kk] + (int)(x.key & 0xFFFFFFu) * rowbytes, __float_as_int(x.alpha));
        }
        e.x = __builtin_amdgcn_ds_permute(pos << 2, e.x);
        e.y = __builtin_amdgcn_ds_permute(pos << 2, e.y);
        return e;
    }
    __device__ __forceinline__ void start(const void* L_, int j, const StreamArgs& a) {
        w = static_cast<WinCtx<KMAX>*>(const_cast<void*>(L_));
        ev = a.bev;
        C_in = a.b_cin;
        rowbytes = a.b_rowbytes;
        T = a.T;
        base = j;  // 0: T <= 64 is one bin block
        w0 = fill(j);
        w1 = fill(j + 64);
    }
    __device__ __forceinline__ Group8 take(int j) {
        if (j - base >= 64) {  // uniform
            base += 64;
            w0 = w1;
            w1 = fill(base + 64);
        }
        const int k = j - base;
        Group8 g;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            g.v[i].x = __builtin_amdgcn_readlane(w0.x, k + i);
            g.v[i].y = __builtin_amdgcn_readlane(w0.y, k + i);
        }
        return g;
    }
};

template <bool COUNT, int VEC, bool CULIF, int EPI, int KMAX>
__global__ __launch_bounds__(256) void k_stream_window(MergeArgs m, StreamArgs a, float* __restrict__ out,
                                                       const float* __restrict__ theta) {
    __shared__ WinCtx<KMAX> ctx_all[4];
    const int wave = uniform(threadIdx.x >> 6);
    int cb;
    int64_t pg;
    map_block(a.n_cblk, cb, pg);
    WinCtx<KMAX>& w = ctx_all[wave];
    const int64_t pix0 = (pg * 4 + wave) * a.ppw;
    for (int q = 0; q < a.ppw; ++q) {
        const int64_t pix = pix0 + q;
        if (pix >= a.n_pix) return;  // uniform per wave
        win_setup<KMAX>(m, pix, w);
        stream_one<COUNT, VEC, CULIF, EPI, WinList<KMAX>>(a, out, &w, w.S, theta, pix, cb);
        wave_sync();  // this pixel's table reads precede the next pixel's setup
    }
}

// ---------------------------------------------------------------------------
// k_conv_small: conv layers whose receptive field has at most 32 elements
// (K_h * K_w * C_in <= 32: VGG-16's first layer, 27; LeNet's first, 25) and
// T <= 64.  No list is built: a wave packs P = 64 / C_out pixels, lane =
// (pixel p, c_out c), and each lane loads its pixel's receptive elements
// straight from the spike map into registers -- arrival bin, weight and
// decay value per element.  A bin's sum is the lane's elements of that bin
// in element order -- (kh, kw, cin), the reference's order -- as fma(w,
// alpha, acc), and closing it is carry += acc and the threshold test, as in
// k_stream.  One pixel per wave (UNI) walks the bins in lockstep; several
// pixels per wave walk each lane's own occupied bins (below).
constexpr int kSmallMaxEl = 32;
struct SmallArgs {
    const float* in;      // [n_cols][C_in] spike times (NHWC map)
    const float* alpha;   // decay LUT, T + 1 entries
    const float* W;       // [(kh*K_w + kw)*C_in + cin][C_out]
    const float* bias;
    const float* theta;   // T entries
    float* out;           // [n_pix][C_out]
    int64_t n_pix;
    int T, t_min, alpha_by_time;
    float tfs;
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad_h, pad_w;
    int nel;              // K_h * K_w * C_in
    int P;                // pixels per wave: 64 / C_out
    int in_bytes;         // bytes of `in`, below 2^31
    int w_bytes;          // bytes of W
    FastDiv div_cout, div_w, div_h;  // C_out, W_out, H_out
    // element e's offset from its field's first element, (kh * W_in + kw) *
    // C_in + ci (0 past nel): the k_conv_small<.., .., true> form
    int dk[kSmallMaxEl];
};
constexpr int kSmallMaxBins = 64;

__device__ __forceinline__ uint64_t wave_or64(uint64_t m) {
    uint32_t lo = (uint32_t)m, hi = (uint32_t)(m >> 32);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        lo |= (uint32_t)__shfl_xor((int)lo, off, 64);
        hi |= (uint32_t)__shfl_xor((int)hi, off, 64);
    }
    return ((uint64_t)__builtin_amdgcn_readfirstlane((int)hi) << 32) |
           (uint32_t)__builtin_amdgcn_readfirstlane((int)lo);
}

// Threshold tests for a lane that walks its own occupied bins (bins hold
// no event of the lane between two it visits).  Across such a run carry is
// constant, as an empty bin adds nothing.  With theta non-increasing over
// the window (checked once per wave; NaN fails) "carry >= theta[t]" holds
// on a suffix of the run and "theta[t] >= 1e-5" on a prefix of the window
// (bins below th_end), so the run fires iff carry clears theta at its last
// bin that may fire, and then at the first bin where it does -- a binary
// search per lane; otherwise the run is scanned bin by bin.  th points at
// the thresholds in LDS.  Built with every lane of the wave active.
struct RunFire {
    const float* th;
    int t_min, th_end;
    bool mono;
    __device__ RunFire(const float* th_, float v_th, int T, int t_min_) : th(th_), t_min(t_min_) {
        const int lane = lane_id();
        const float nxt = __shfl_down(v_th, 1, 64);
        mono = __ballot(lane + 1 < T && !(v_th >= nxt)) == 0;
        const uint64_t low = __ballot(lane < T && !(v_th >= 1e-5f));
        th_end = low ? (int)__builtin_ctzll(low) : T;
    }
    // theta at the last bin of [0, r1) that may fire, read ahead by the caller
    __device__ float last(int r1) const {
        const int tb = r1 < th_end ? r1 : th_end;
        return th[tb > 0 ? tb - 1 : 0];
    }
    // fire in the bins [r0, r1) (no event of the lane there) if carry
    // reaches a threshold; th_b = last(r1)
    __device__ void run(int r0, int r1, float th_b, float carry, float& res, bool& alive) const {
        const int ta = r0 > t_min ? r0 : t_min;
        if (mono) {
            const int tb = r1 < th_end ? r1 : th_end;
            if (ta < tb && carry >= th_b) {
                int lo = ta, hi = tb - 1;
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    const bool le = th[mid] <= carry;
                    hi = le ? mid : hi;
                    lo = le ? lo : mid + 1;
                }
                res = (float)lo;
                alive = false;
            }
        } else {
            for (int t = ta; t < r1; ++t) {
                const float v = th[t];
                if (v >= 1e-5f && carry >= v) {
                    res = (float)t;
                    alive = false;
                    break;
                }
            }
        }
    }
    // close an occupied bin t: carry += the bin's sum, then the test
    __device__ void bin(int t, float acc, float th_t, float& carry, float& res, bool& alive) const {
        carry = carry + acc;
        if (t >= t_min && th_t >= 1e-5f && carry >= th_t) {
            res = (float)t;
            alive = false;
        }
    }
};

// UNI: one pixel per wave (C_out > 32), so the spike times, bins and decay
// values are wave-uniform (scalar) and only the weights are per lane.  NEL:
// the elements the bin scan covers -- the layer's receptive field where an
// instantiation has it, else the 32-element limit (its extra elements hold
// bin -1).  Measured on LeNet-5's conv1 at B=1024 (25 elements, ten pixels
// per wave; A/B on one box): 0.350 -> 0.300 ms with the scan cut to 25;
// 0.300 -> 0.211 ms with each lane walking its own occupied bins (about 5
// of a pixel's 25 elements hold a spike, spread over the 64 bins, while
// the ten pixels of a wave occupy about 35 bins between them); 0.211 ->
// 0.192 ms with every spike-time and weight load issued before any is used
// (32-bit offsets from a per-lane base: 64-bit index arithmetic had made
// each load wait for the previous one); 0.192 -> 0.187 ms with the bin's
// thresholds read before its sum; 0.187 -> 0.137 ms where every tap lies
// inside the map (no padding): element offsets from a host table as the
// loads' scalar offsets, no bounds tests, and the bins and decay indices
// without branches (the preamble went from about 870 vector and 900 scalar
// instructions per wave to 440 and 200).  Tried and slower there: the fma under
// an exec mask (compare, save-exec, fmac, restore: 0.331 ms -- the scalar
// unit then issues as much as the vector unit saved); a wave-uniform branch
// skipping elements no lane holds in the bin (0.318); bin sums in LDS, each
// element added once (0.502: 25 dependent LDS round trips per wave at ten
// waves per CU).
template <bool UNI, int NEL, bool VALID>
__global__ __launch_bounds__(256) void k_conv_small(SmallArgs a) {
    // the thresholds, for per-lane bins (several pixels per wave)
    __shared__ float th_lds[UNI ? 1 : kSmallMaxBins];
    if constexpr (!UNI) {
        if ((int)threadIdx.x < a.T) th_lds[threadIdx.x] = a.theta[threadIdx.x];
        __syncthreads();
    }
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t pix0 = ((int64_t)blockIdx.x * 4 + wave) * a.P;
    if (pix0 >= a.n_pix) return;  // uniform per wave
    const int p = UNI ? 0 : fdiv(lane, a.div_cout), c = lane - p * a.C_out;
    const int64_t pix = pix0 + p;
    const bool ok = p < a.P && pix < a.n_pix && c < a.C_out;
    const bool pix_ok = UNI ? true : ok;  // the lane's pixel exists (UNI: pix0 < n_pix)
    // 32-bit pixel coordinates and offsets: the launch keeps the pixel count
    // and the map's bytes below 2^31
    const int px = (int)(UNI ? pix0 : (ok ? pix : pix0));
    const int qd = fdiv(px, a.div_w);
    const int w_out = px - qd * a.W_out;
    const int img = fdiv(qd, a.div_h);
    const int h_out = qd - img * a.H_out;
    // the lane's receptive elements: bin (-1: none), weight, decay value.
    // Every spike-time and weight load is issued before any is used (no
    // branch between them; elements outside the map load its first word and
    // are masked), so a lane waits for two rounds of loads, not one per
    // element: the spike times and weights, then the decay values.  An
    // instantiation whose NEL is not the 32-element limit runs only for
    // fields of exactly NEL elements (EXACT).
    constexpr bool EXACT = NEL != kSmallMaxEl;
    int bin[NEL];
    float wv[NEL], av[NEL];
    uint32_t inm = 0;  // bit e: element e lies inside the map
    if constexpr (VALID) {
        // every tap of every output pixel lies inside the map (no padding):
        // element e sits a.dk[e] past the field's first element, so a load's
        // per-lane offset is the field's base and its scalar offset the
        // table entry -- no per-element address or bounds arithmetic
        const __amdgpu_buffer_rsrc_t rin =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, a.in_bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rw =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.w_bytes, 0x00020000);
        const int vb = (((img * a.H_in + h_out) * a.W_in + w_out) * a.C_in) * 4;
        const int vc = (c < a.C_out ? c : 0) * 4;
#pragma unroll
        for (int e = 0; e < NEL; ++e) {
            av[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, vb, a.dk[e] * 4, 0));
            wv[e] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rw, vc, (EXACT || e < a.nel ? e : 0) * a.C_out * 4, 0));
        }
        (void)inm;
    } else {
        const __amdgpu_buffer_rsrc_t rin =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.in, (short)0, a.in_bytes, 0x00020000);
        const int cc = c < a.C_out ? c : 0;
        // the field's first element (kh = kw = ci = 0, possibly outside the
        // map); element e lies dk + ci further, dk = (kh * W_in + kw) * C_in
        const int h0 = h_out - a.pad_h, w0 = w_out - a.pad_w;
        const int base = ((img * a.H_in + h0) * a.W_in + w0) * a.C_in;
        int kh = 0, kw = 0, ci = 0, dk = 0;  // element e = (kh*K_w + kw)*C_in + ci, wave-uniform
#pragma unroll
        for (int e = 0; e < NEL; ++e) {
            const bool inb = e < a.nel && pix_ok && (unsigned)(h0 + kh) < (unsigned)a.H_in &&
                             (unsigned)(w0 + kw) < (unsigned)a.W_in;
            const int off = inb ? (base + dk + ci) * 4 : 0;
            av[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rin, off, 0, 0));
            wv[e] = a.W[(e < a.nel ? e : 0) * a.C_out + cc];
            inm |= (inb ? 1u : 0u) << e;
            ci += 1;
            const bool wrap_c = ci == a.C_in;
            ci = wrap_c ? 0 : ci;
            kw += wrap_c ? 1 : 0;
            dk += wrap_c ? a.C_in : 0;
            const bool wrap_w = kw == a.K_w;
            kw = wrap_w ? 0 : kw;
            kh += wrap_w ? 1 : 0;
            dk += wrap_w ? (a.W_in - a.K_w) * a.C_in : 0;
        }
    }
    uint64_t occ = 0;
    if constexpr (UNI) {
#pragma unroll
        for (int e = 0; e < NEL; ++e) {
            const float t = (inm >> e) & 1u ? av[e] : kInfTime;
            const int b = arrival_bin(t, a.tfs, a.T);
            const int ai = b >= 0 ? alpha_index(t, b, a.alpha_by_time, a.T) : 0;
            av[e] = a.alpha[ai];
            bin[e] = b;
            occ |= b >= 0 ? (1ull << b) : 0ull;
        }
    } else {
        // arrival_bin and alpha_index without branches, as quad_build: bin
        // floor(max(t - tfs, 0)), an event if t < kInfTime and the bin is
        // below T; LUT index the bin, or clamp(t, 0, T) by spike time (one
        // med3).  The table form loads every lane's field (lanes past the
        // last pixel load the wave's first), and only elements past nel are
        // masked: a lane without a pixel is never alive.
        const __amdgpu_buffer_rsrc_t ral =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.alpha, (short)0, (a.T + 1) * 4, 0x00020000);
#pragma unroll
        for (int e = 0; e < NEL; ++e) {
            const float t = VALID ? av[e] : ((inm >> e) & 1u ? av[e] : kInfTime);
            const int tb = (int)floorf(fmaxf(t - a.tfs, 0.0f));
            const bool ev = (!VALID || EXACT || e < a.nel) && t < kInfTime && tb < a.T;
            const int ai = a.alpha_by_time ? (int)__builtin_amdgcn_fmed3f(t, 0.0f, (float)a.T) : tb;
            av[e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ral, (ev ? ai : 0) * 4, 0, 0));
            bin[e] = ev ? tb : -1;
            occ |= ev ? (1ull << tb) : 0ull;
        }
    }
    const float v_th = lane < a.T ? a.theta[lane] : 0.0f;
    float carry = ok ? a.bias[c] : 0.0f;
    float res = kInfTime;
    bool alive = ok;
    if constexpr (!UNI) {
        // Each lane walks only its own pixel's occupied bins, in order (the
        // lowest set bit of its mask), and settles the empty bins between
        // them with RunFire.  The wave takes as many steps as its busiest
        // pixel has occupied bins, not one per bin that any of its pixels
        // occupies.
        const RunFire rf(th_lds, v_th, a.T, a.t_min);
        uint64_t rem = occ;  // the lane's occupied bins not yet integrated
        int t_done = 0;      // bins below are closed
        while (__ballot(alive && rem != 0) != 0) {
            if (alive && rem != 0) {
                const int tn = (int)__builtin_ctzll(rem);
                // both thresholds are read before the bin's sum, which hides
                // the LDS latency; the sum is dropped if the lane fires in the
                // empty bins before tn
                const float th_n = th_lds[tn], th_b = rf.last(tn);
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < NEL; ++e) acc = bin[e] == tn ? __builtin_fmaf(wv[e], av[e], acc) : acc;
                rf.run(t_done, tn, th_b, carry, res, alive);
                if (alive) rf.bin(tn, acc, th_n, carry, res, alive);
                rem &= rem - 1;
                t_done = tn + 1;
            }
        }
        if (alive) rf.run(t_done, a.T, rf.last(a.T), carry, res, alive);
        if (ok) a.out[pix * a.C_out + c] = res;
        return;
    }
    const uint64_t any = wave_or64(occ);
    for (int t = 0; t < a.T; ++t) {
        float acc = 0.0f;
        if ((any >> t) & 1) {  // uniform; elements past nel hold bin -1
#pragma unroll
            for (int e = 0; e < NEL; ++e) acc = bin[e] == t ? __builtin_fmaf(wv[e], av[e], acc) : acc;
        }
        carry = carry + acc;
        const float th = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_th), t));
        if (t >= a.t_min && th >= 1e-5f && alive && carry >= th) {
            res = (float)t;
            alive = false;
        }
        if (__ballot(alive) == 0) break;
    }
    if (ok) a.out[pix * a.C_out + c] = res;
}

// ---------------------------------------------------------------------------
// k_stream_narrow: layers with C_out < 32 (LeNet's 6-, 16- and 10-wide
// layers), where one pixel per wave would leave most lanes idle.  A wave
// packs P = 64 / C_out pixels, lane = (pixel p, c_out c); each lane walks its
// pixel's merged list (the k_merge output, (bin, tap, cin) order) through a
// window of 8 entries and their gathers W[row + c].  Bins close in lockstep,
// in order, with the neuron of the layer, as in k_stream: each adds the
// window's events that fall in it, in list order, and the window moves on
// only when some lane's open bin runs past it -- one list load and one round
// of gathers per 8 events rather than per bin.  Lanes of one pixel read the
// same list entries.  E_proc / E_bin count per lane with the
// same rules as k_stream (a neuron counts a bin's events while it was alive
// at the start of the chunk / of the bin).  The eight bins of a group are
// unrolled, each with its end in a register: with the group's bin index a
// loop variable, selecting the end had cost seven instructions per bin
// (LeNet-5 conv2 at B=1024, A/B on one box: 0.209 -> 0.176 ms with its merge).
template <bool COUNT, bool CULIF>
__global__ __launch_bounds__(256) void k_stream_narrow(StreamArgs a, float* __restrict__ out,
                                                       const int2* __restrict__ list,
                                                       const int32_t* __restrict__ bstart,
                                                       const float* __restrict__ theta) {
    const int wave = uniform(threadIdx.x >> 6);
    const int lane = lane_id();
    const int P = 64 / a.C_out;
    const int p = lane / a.C_out, c = lane - p * a.C_out;
    const int64_t pix = ((int64_t)blockIdx.x * 4 + wave) * P + p;
    if (((int64_t)blockIdx.x * 4 + wave) * P >= a.n_pix) return;  // uniform per wave
    const bool ok = p < P && pix < a.n_pix;
    const int2* __restrict__ L = list + (ok ? pix : 0) * a.cap;
    const int32_t* __restrict__ BS = bstart + (ok ? pix : 0) * (int64_t)(a.T + 1);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.w_bytes, 0x00020000);
    const int voff = c * 4;
    float carry = (ok && !CULIF) ? a.bias[c] : 0.0f;
    float cur = 0.0f, res = kInfTime;
    bool alive = ok, alive_chunk = ok;
    unsigned long long cnt_proc = 0, cnt_bin = 0;
    const int T = a.T, D = a.D;
    int j = 0;
    for (int t0 = 0; t0 < T; t0 += kBlockBins) {
        const int nb = (T - t0) < kBlockBins ? (T - t0) : kBlockBins;
        const float v_th = (!CULIF && lane < nb) ? theta[t0 + lane] : 0.0f;
        bool done = false;
        for (int b8 = 0; b8 < nb && !done; b8 += 8) {
            const int ng = (nb - b8) < 8 ? (nb - b8) : 8;  // uniform
            int ends[8];  // bin ends of the next eight bins, loaded together
#pragma unroll
            for (int g = 0; g < 8; ++g) ends[g] = (ok && g < ng) ? BS[t0 + b8 + g + 1] : j;
            // A window of 8 list entries per lane (the list is padded past its
            // end, so the loads stay in the pixel's region) serves every bin
            // it covers: bins close in lockstep, each adding the window's
            // events that fall in it, in list order; the window moves on only
            // when some lane's open bin runs past it.
            int s_ = j;   // first event of the lane's open bin
            int wj = j;   // window start
            int2 e[8];
            float w[8];
            bool need = true;  // uniform
            float acc = 0.0f;
            // the eight bins unrolled, so each reads its end from a register
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                if (g >= ng) break;  // uniform
                const int be = ends[g];
                for (;;) {  // uniform: the window moves on while some lane's bin runs past it
                    if (need) {
#pragma unroll
                        for (int q = 0; q < 8; ++q) e[q] = L[wj + q];
#pragma unroll
                        for (int q = 0; q < 8; ++q)
                            w[q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, e[q].x + voff, 0, 0));
                        need = false;
                    }
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const int idx = wj + q;
                        acc = (idx >= s_ && idx < be) ? __builtin_fmaf(w[q], __int_as_float(e[q].y), acc) : acc;
                    }
                    if (__ballot(be > wj + 8) == 0) break;
                    wj = be > wj + 8 ? wj + 8 : be;
                    need = true;
                }
                const int b = b8 + g;
                const int t = t0 + b;
                if (COUNT) {
                    const unsigned long long n = (unsigned long long)(be - s_);
                    if (alive) cnt_bin += n;
                    if (alive_chunk) cnt_proc += n;
                }
                if (CULIF) {
                    cur = __builtin_fmaf(cur, a.decay, acc);
                    carry = carry + cur;
                    if (alive && carry >= a.th) {
                        res = (float)t;
                        alive = false;
                    }
                } else {
                    const float th = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_th), b));
                    carry = carry + acc;
                    if (t >= a.t_min && th >= 1e-5f && alive && carry >= th) {
                        res = (float)t;
                        alive = false;
                    }
                }
                const bool chunk_end = ((t + 1) % D) == 0;
                if (COUNT && chunk_end) alive_chunk = alive;
                acc = 0.0f;
                s_ = be;
            }
            j = s_;
            // counting forwards keep going to the end of the chunk of the
            // last firing (their counts stop with the alive flags)
            if (__ballot(COUNT ? (alive || alive_chunk) : alive) == 0) done = true;
        }
        if (done) break;
    }
    if (ok) out[pix * a.C_out + c] = res;
    if (COUNT) {
        for (int o = 32; o > 0; o >>= 1) {
            cnt_proc += __shfl_xor(cnt_proc, o, 64);
            cnt_bin += __shfl_xor(cnt_bin, o, 64);
        }
        if (lane == 0) {
            unsigned long long* cs = counter_stripe(a.counters);
            atomicAdd(&cs[0], cnt_proc);
            atomicAdd(&cs[1], cnt_bin);
        }
    }
}

// ---------------------------------------------------------------------------
struct GenArgs {
    float* out;
    const int32_t* off;
    const int32_t* ref_cin;   // REF layout
    const float* ref_tin;     // REF layout
    const vd_event* ev;       // BIN layout
    const float* W;
    const float* bias;
    const float* alpha;       // REF layout: decay LUT
    const float* theta;
    unsigned long long* counters;
    int64_t total;
    int T, D, t_min, alpha_by_time;
    float tfs;
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad_h, pad_w, is_fc;
};

template <bool BINS, int DMAX, bool COUNT>
__global__ __launch_bounds__(256) void k_integrate_generic(GenArgs a) {
    const int64_t nid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool ok = nid < a.total;
    unsigned long long my_proc = 0, my_bin = 0;
    if (ok) {
        const int c_out = (int)(nid % a.C_out);
        int img, h_out = 0, w_out = 0;
        if (a.is_fc) {
            img = (int)(nid / a.C_out);
        } else {
            const int64_t t1 = nid / a.C_out;
            w_out = (int)(t1 % a.W_out);
            const int64_t t2 = t1 / a.W_out;
            h_out = (int)(t2 % a.H_out);
            img = (int)(t2 / a.H_out);
        }
        const int T = a.T, D = a.D, NC = (T + D - 1) / D;
        const int OS = BINS ? T + 1 : NC + 1;
        const int kh_n = a.is_fc ? 1 : a.K_h, kw_n = a.is_fc ? 1 : a.K_w;
        float carry = a.bias[c_out];
        float result = kInfTime;
        bool crossed = false;
        float delta[DMAX];
        int nbin[DMAX];
        for (int tau = 0; tau < NC; ++tau) {
#pragma unroll
            for (int i = 0; i < DMAX; ++i) {
                delta[i] = 0.0f;
                if (COUNT) nbin[i] = 0;
            }
            const int base_t = tau * D;
            for (int kh = 0; kh < kh_n; ++kh) {
                const int h_in = a.is_fc ? 0 : h_out - a.pad_h + kh;
                if (!a.is_fc && (h_in < 0 || h_in >= a.H_in)) continue;
                for (int kw = 0; kw < kw_n; ++kw) {
                    const int w_in = a.is_fc ? 0 : w_out - a.pad_w + kw;
                    if (!a.is_fc && (w_in < 0 || w_in >= a.W_in)) continue;
                    const int64_t col =
                        a.is_fc ? img : ((int64_t)img * a.H_in + h_in) * a.W_in + w_in;
                    const int64_t wbase = (int64_t)(kh * a.K_w + kw) * a.C_in;
                    int s, e;
                    if (BINS) {
                        const int t1 = (base_t + D) < T ? base_t + D : T;
                        s = a.off[col * OS + base_t];
                        e = a.off[col * OS + t1];
                    } else {
                        s = a.off[col * OS + tau];
                        e = a.off[col * OS + tau + 1];
                    }
                    // caller-made buckets (the drop-in) are not trusted to
                    // match this context's T, Delta and TFS: offsets clamp to
                    // the column, and events outside this chunk's bins, the
                    // window or the input width are skipped below.  Buckets
                    // made with the context's own constants never trigger
                    // either guard, so their results are unchanged.
                    s = s < 0 ? 0 : (s > a.C_in ? a.C_in : s);
                    e = e < s ? s : (e > a.C_in ? a.C_in : e);
                    for (int p = s; p < e; ++p) {
                        int cin, tb;
                        float al, t_in = 0.0f;
                        if (BINS) {
                            const vd_event ev = a.ev[col * a.C_in + p];
                            cin = (int)(ev.key & 0xFFFFFFu);
                            tb = (int)(ev.key >> 24);
                            al = ev.alpha;
                        } else {
                            cin = a.ref_cin[col * a.C_in + p];
                            t_in = a.ref_tin[col * a.C_in + p];
                            tb = (int)floorf(t_in - a.tfs);
                            if (tb < 0) tb = 0;
                        }
                        const int di = tb - base_t;
                        if ((unsigned)di >= (unsigned)D || tb >= T || (unsigned)cin >= (unsigned)a.C_in) continue;
                        if (!BINS) al = a.alpha[alpha_index(t_in, tb, a.alpha_by_time, T)];
                        delta[di] = __builtin_fmaf(a.W[(wbase + cin) * a.C_out + c_out], al, delta[di]);
                        if (COUNT) nbin[di]++;
                    }
                }
            }
            int crossed_i = -1;
            for (int i = 0; i < D; ++i) {
                const int t = base_t + i;
                if (t >= T) break;
                carry = carry + delta[i];
                const float th = a.theta[t];
                if (t >= a.t_min && carry >= th && th >= 1e-5f) {
                    result = (float)t;
                    crossed_i = i;
                    break;
                }
            }
            if (COUNT) {
                const int last = crossed_i >= 0 ? crossed_i : D - 1;
                for (int i = 0; i < D; ++i) {
                    my_proc += nbin[i];
                    if (!crossed && i <= last) my_bin += nbin[i];
                }
            }
            if (crossed_i >= 0) crossed = true;
            if (result < kInfTime) break;
        }
        a.out[nid] = result;
    }
    if (COUNT) {
        for (int o = 32; o > 0; o >>= 1) {
            my_proc += __shfl_xor(my_proc, o, 64);
            my_bin += __shfl_xor(my_bin, o, 64);
        }
        if (lane_id() == 0) {
            unsigned long long* c = counter_stripe(a.counters);
            atomicAdd(&c[0], my_proc);
            atomicAdd(&c[1], my_bin);
        }
    }
}

template <bool BINS, bool COUNT>
int launch_generic_d(vdttfs_ctx* ctx, const GenArgs& g) {
    const int64_t blocks = (g.total + 255) / 256;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
    const int D = ctx->c.delta;
    if (D <= 16)
        hipLaunchKernelGGL((k_integrate_generic<BINS, 16, COUNT>), dim3((unsigned)blocks), dim3(256), 0,
                           ctx->stream, g);
    else if (D <= 64)
        hipLaunchKernelGGL((k_integrate_generic<BINS, 64, COUNT>), dim3((unsigned)blocks), dim3(256), 0,
                           ctx->stream, g);
    else
        hipLaunchKernelGGL((k_integrate_generic<BINS, 256, COUNT>), dim3((unsigned)blocks), dim3(256), 0,
                           ctx->stream, g);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

}  // namespace

int check_integ_shape(const vdttfs_ctx* ctx, const IntegShape& s) {
    if (s.B <= 0 || s.C_in <= 0 || s.C_out <= 0)
        return set_error(VDTTFS_E_INVALID, "integrate: B, C_in, C_out must be positive");
    if (!s.is_fc) {
        if (s.H_in <= 0 || s.W_in <= 0 || s.H_out <= 0 || s.W_out <= 0 || s.K_h <= 0 || s.K_w <= 0)
            return set_error(VDTTFS_E_INVALID, "integrate: conv dims must be positive");
        // every receptive column of every output pixel must be addressable
        if (s.pad_h == 0 && s.pad_w == 0 && (s.H_out + s.K_h - 1 > s.H_in || s.W_out + s.K_w - 1 > s.W_in))
            return set_error(VDTTFS_E_INVALID,
                             "integrate: valid conv needs H_in >= H_out+K_h-1 (got %d < %d+%d-1)",
                             s.H_in, s.H_out, s.K_h);
    }
    const int64_t cols = s.is_fc ? s.B : (int64_t)s.B * s.H_in * s.W_in;
    const int64_t neurons =
        (int64_t)s.B * (s.is_fc ? 1 : (int64_t)s.H_out * s.W_out) * s.C_out;
    if (cols * s.C_in > INT64_C(0x7fffffff) * 8 || neurons > INT64_C(1) << 40)
        return set_error(VDTTFS_E_UNSUPPORTED, "integrate: problem too large");
    (void)ctx;
    return VDTTFS_OK;
}

int launch_integrate_ref(vdttfs_ctx* ctx, float* out, const int32_t* cin, const float* tin,
                         const int32_t* off, const float* W, const float* bias,
                         const float* alpha, const float* theta, int t_min, int B, int H_in,
                         int W_in, int C_in, int H_out, int W_out, int C_out, int K_h, int K_w,
                         int is_fc) {
    GenArgs g{};
    g.out = out;
    g.off = off;
    g.ref_cin = cin;
    g.ref_tin = tin;
    g.W = W;
    g.bias = bias;
    g.alpha = alpha;
    g.theta = theta;
    g.T = ctx->c.T;
    g.D = ctx->c.delta;
    g.t_min = t_min;
    g.alpha_by_time = ctx->c.alpha_by_time;
    g.tfs = ctx->c.tfs;
    g.H_in = is_fc ? 1 : H_in;
    g.W_in = is_fc ? 1 : W_in;
    g.C_in = C_in;
    g.H_out = is_fc ? 1 : H_out;
    g.W_out = is_fc ? 1 : W_out;
    g.C_out = C_out;
    g.K_h = is_fc ? 1 : K_h;
    g.K_w = is_fc ? 1 : K_w;
    const bool same = !is_fc && ctx->c.conv_same_pad;  // T2V:109-110
    g.pad_h = same ? K_h / 2 : 0;
    g.pad_w = same ? K_w / 2 : 0;
    g.is_fc = is_fc;
    g.total = (int64_t)B * g.H_out * g.W_out * C_out;
    return launch_generic_d<false, false>(ctx, g);
}

int launch_integrate_generic_bins(vdttfs_ctx* ctx, float* out, const vd_event* ev,
                                  const int32_t* off, const float* W, const float* bias,
                                  const float* theta, int t_min, const IntegShape& sh,
                                  unsigned long long* counters) {
    const int T = ctx->c.T, D = ctx->c.delta;
    GenArgs g{};
    g.out = out;
    g.off = off;
    g.ev = ev;
    g.W = W;
    g.bias = bias;
    g.theta = theta;
    g.counters = counters;
    g.T = T;
    g.D = D;
    g.t_min = t_min;
    g.alpha_by_time = ctx->c.alpha_by_time;
    g.tfs = ctx->c.tfs;
    g.H_in = sh.H_in;
    g.W_in = sh.W_in;
    g.C_in = sh.C_in;
    g.H_out = sh.H_out;
    g.W_out = sh.W_out;
    g.C_out = sh.C_out;
    g.K_h = sh.K_h;
    g.K_w = sh.K_w;
    g.pad_h = sh.pad_h;
    g.pad_w = sh.pad_w;
    g.is_fc = sh.is_fc;
    g.total = (int64_t)sh.B * (sh.is_fc ? 1 : (int64_t)sh.H_out * sh.W_out) * sh.C_out;
    return counters ? launch_generic_d<true, true>(ctx, g) : launch_generic_d<true, false>(ctx, g);
}

int merged_list_cap(const IntegShape& sh) {
    return (sh.is_fc ? 1 : sh.K_h * sh.K_w) * sh.C_in + kListPad;
}

namespace {

// Shape limits of the merged-list path (merge + k_stream).
bool wave_path_ok(const IntegShape& sh, int64_t* wbytes) {
    const int nk_max = sh.is_fc ? 1 : sh.K_h * sh.K_w;
    *wbytes = (int64_t)nk_max * sh.C_in * sh.C_out * 4;
    return sh.C_out >= 32 && nk_max <= 25 && *wbytes < INT64_C(0x7fffffff) && sh.C_in < (1 << 24);
}

// Layers narrower than the wave path (C_out < 32) take k_stream_narrow.
bool narrow_path_ok(const IntegShape& sh, int64_t* wbytes) {
    const int nk_max = sh.is_fc ? 1 : sh.K_h * sh.K_w;
    *wbytes = (int64_t)nk_max * sh.C_in * sh.C_out * 4;
    return sh.C_out >= 1 && sh.C_out < 32 && nk_max <= 25 && *wbytes < INT64_C(0x7fffffff) &&
           sh.C_in < (1 << 24);
}

int64_t n_pixels(const IntegShape& sh) {
    return (int64_t)sh.B * (sh.is_fc ? 1 : (int64_t)sh.H_out * sh.W_out);
}

// Kernel arguments of a layer's stream; vec c_out per lane and epi events
// per load follow the plan's gather (1: 1/1, 2: 2/2, 4: 4/1).
StreamArgs stream_args(vdttfs_ctx* ctx, float* out, const int2* list, int64_t cap, const int32_t* bstart,
                       const float* W, int64_t wbytes, const float* bias, const float* theta, int t_min,
                       const IntegShape& sh, unsigned long long* counters, const CulifNeuron* culif,
                       const LaunchPlan& p, int* vec, int* epi) {
    StreamArgs a{};
    a.out = out;
    a.list = list;
    a.bstart = bstart;
    a.W = W;
    a.bias = bias;
    a.theta = theta;
    a.counters = counters;
    a.n_pix = n_pixels(sh);
    a.cap = cap;
    a.T = ctx->c.T;
    a.D = ctx->c.delta;
    a.t_min = t_min;
    a.C_out = sh.C_out;
    a.decay = culif ? culif->decay : 0.0f;
    a.th = culif ? culif->th : 0.0f;
    *vec = p.gather == 4 ? 4 : (p.gather == 2 ? 2 : 1);
    *epi = p.gather == 2 ? 2 : 1;
    a.n_cblk = *epi > 1 ? (sh.C_out + 127) / 128 : (sh.C_out + 64 * *vec - 1) / (64 * *vec);
    a.w_bytes = (int)wbytes;
    a.ppw = p.ppw > 0 ? p.ppw : 1;
    return a;
}

int launch_stream(vdttfs_ctx* ctx, float* out, const int2* list, int64_t cap, const int32_t* bstart,
                  const float* W, int64_t wbytes, const float* bias, const float* theta, int t_min,
                  const IntegShape& sh, unsigned long long* counters, const CulifNeuron* culif,
                  const LaunchPlan& p) {
    int vec, epi;
    const StreamArgs a = stream_args(ctx, out, list, cap, bstart, W, wbytes, bias, theta, t_min, sh,
                                     counters, culif, p, &vec, &epi);
    const int64_t n_pix = a.n_pix;
    const int waves = 4;
    const int64_t n_pg = (n_pix + waves * a.ppw - 1) / (waves * a.ppw);
    const int64_t blocks = n_pg * a.n_cblk;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
#define VD_LAUNCH_STREAM(C, V, L, E)                                                               \
    hipLaunchKernelGGL((k_stream<C, V, L, E>), dim3((unsigned)blocks), dim3(64 * waves), 0, ctx->stream, \
                       a, out, list, bstart, theta)
#define VD_LAUNCH_STREAM_V(C, L)              \
    do {                                      \
        if (epi == 2)                         \
            VD_LAUNCH_STREAM(C, 2, L, 2);     \
        else if (vec == 4)                    \
            VD_LAUNCH_STREAM(C, 4, L, 1);     \
        else                                  \
            VD_LAUNCH_STREAM(C, 1, L, 1);     \
    } while (0)
#define VD_LAUNCH_LEAN(G, L)                                                                                \
    hipLaunchKernelGGL((k_stream_lean<G, L>), dim3((unsigned)blocks), dim3(64 * waves), 0, ctx->stream, a, out, \
                       list, bstart, theta)
    if (!counters && a.T <= kBlockBins && (epi == 2 || vec == 4)) {
        if (epi == 2) {
            if (culif)
                VD_LAUNCH_LEAN(2, true);
            else
                VD_LAUNCH_LEAN(2, false);
        } else {
            if (culif)
                VD_LAUNCH_LEAN(4, true);
            else
                VD_LAUNCH_LEAN(4, false);
        }
    } else if (culif) {
        if (counters)
            VD_LAUNCH_STREAM_V(true, true);
        else
            VD_LAUNCH_STREAM_V(false, true);
    } else {
        if (counters)
            VD_LAUNCH_STREAM_V(true, false);
        else
            VD_LAUNCH_STREAM_V(false, false);
    }
#undef VD_LAUNCH_LEAN
#undef VD_LAUNCH_STREAM_V
#undef VD_LAUNCH_STREAM
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

// The window path: bucketize output -> k_stream_window (merge + stream).
int launch_stream_window(vdttfs_ctx* ctx, const MergeArgs& m, float* out, const vd_event* ev, const float* W,
                         int64_t wbytes, const float* bias, const float* theta, int t_min, const IntegShape& sh,
                         unsigned long long* counters, const CulifNeuron* culif, const LaunchPlan& p) {
    int vec, epi;
    StreamArgs a = stream_args(ctx, out, nullptr, 0, nullptr, W, wbytes, bias, theta, t_min, sh, counters, culif,
                               p, &vec, &epi);
    a.bev = ev;
    a.b_cin = sh.C_in;
    a.b_rowbytes = sh.C_out * 4;
    const int waves = 4;
    const int64_t n_pg = (a.n_pix + waves * a.ppw - 1) / (waves * a.ppw);
    const int64_t blocks = n_pg * a.n_cblk;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
    if (m.T > kBlockBins || (!m.is_fc && m.K_h * m.K_w > 9))
        return set_error(VDTTFS_E_UNSUPPORTED, "window path: T <= 64 and at most 9 taps");
#define VD_LAUNCH_WIN(C, V, L, E, K)                                                                     \
    hipLaunchKernelGGL((k_stream_window<C, V, L, E, K>), dim3((unsigned)blocks), dim3(64 * waves), 0,     \
                       ctx->stream, m, a, out, theta)
#define VD_LAUNCH_WIN_K(C, V, L, E)          \
    do {                                     \
        if (m.is_fc)                         \
            VD_LAUNCH_WIN(C, V, L, E, 1);    \
        else                                 \
            VD_LAUNCH_WIN(C, V, L, E, 9);    \
    } while (0)
#define VD_LAUNCH_WIN_V(C, L)                \
    do {                                     \
        if (epi == 2)                        \
            VD_LAUNCH_WIN_K(C, 2, L, 2);     \
        else if (vec == 4)                   \
            VD_LAUNCH_WIN_K(C, 4, L, 1);     \
        else                                 \
            VD_LAUNCH_WIN_K(C, 1, L, 1);     \
    } while (0)
    // the CuLIF engine always takes the built-in plan, which never asks for
    // this path, so only the LUT neuron is instantiated
    if (culif) return set_error(VDTTFS_E_UNSUPPORTED, "window path: LUT-threshold layers only");
    if (counters)
        VD_LAUNCH_WIN_V(true, false);
    else
        VD_LAUNCH_WIN_V(false, false);
#undef VD_LAUNCH_WIN_V
#undef VD_LAUNCH_WIN_K
#undef VD_LAUNCH_WIN
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

// Most receptive elements of one output pixel: an output row meets at most
// min(K_h, H_in) input rows whatever the padding (a 3x3 kernel on a 2x2 map
// reaches 4 taps), likewise columns.
int64_t shared_nel_max(const IntegShape& sh) {
    if (sh.is_fc) return sh.C_in;
    const int kh = sh.K_h < sh.H_in ? sh.K_h : sh.H_in;
    const int kw = sh.K_w < sh.W_in ? sh.K_w : sh.W_in;
    return (int64_t)kh * kw * sh.C_in;
}

// Waves of one shared-list workgroup: one per c_out block, covering at most
// 256 c_out (four 64-wide, two 128-wide or one 256-wide block).  Wider layers take several
// workgroups per pixel (c_out groups), which the kernel pins to XCDs:
// VGG-16's 512-wide layers take two groups, so that an XCD's L2 holds half
// of a 9.4 MB weight tensor (measured on conv 8, 512 -> 512 at 4x4: L2 hit
// rate 0.69 with one group of four 128-wide waves, 0.99 with two groups).
int shared_waves(int64_t n_cblk, int gather) {
    const int64_t most = gather == 4 ? 1 : (gather == 2 ? 2 : kSharedMaxWaves);
    return (int)(n_cblk < most ? n_cblk : most);
}

// List capacity of a shared-list workgroup, in entries: the pixel's most
// receptive elements, but at most what keeps the workgroup's LDS near 5 KB
// per wave (eight waves per SIMD on the 160 KB of a CU), rounded to 16.  A
// pixel with more events streams its list in windows of this size (VGG-16
// conv 8: 4,608 receptive elements, ~2,150 events per interior pixel, a
// capacity of 2,640 at four waves: 0.633 -> 0.533 ms against lists sized to
// the field).
constexpr int kSharedLdsPerWave = 5 * 1024;
// A 256-wide wave (one event per load) keeps 16 loads in flight, so fewer of
// them hide the gathers' latency: about 16 KB of list per wave.
constexpr int kSharedLdsPerLeanWave = 16 * 1024;
int shared_cap(int64_t nel_max, int waves, bool alphas, int gather) {
    const int64_t per = alphas ? 6 : 4;  // 16-bit row and alpha, or row byte offset
    const int64_t budget = gather == 4 ? kSharedLdsPerLeanWave : kSharedLdsPerWave;
    const int64_t lim = ((budget - 4 * kSharedWaveWords) * waves / per) & ~INT64_C(15);
    const int64_t want = (nel_max + 15) & ~INT64_C(15);
    return (int)(want < lim ? want : lim);
}
// The shared-list kernel: one workgroup per (output pixel, group of up to
// four c_out blocks), the W waves building the pixel's list together and
// each streaming one c_out block (64 c_out at epi 1, 128 at epi 2).
// k_stream_multi's later-list capacity: four images' receptive elements
// (every event of the field past bin 0), at most kMultiCapMax entries
// (about 12 KB of LDS per wave with the ring and tables: 13 waves per CU).
constexpr int kMultiCapMax = 2048;
int multi_cap(int64_t nel_max) {
    const int64_t want = (kMultiImages * nel_max + 3) & ~INT64_C(3);
    return (int)(want < kMultiCapMax ? want : kMultiCapMax);
}

int launch_stream_multi(vdttfs_ctx* ctx, const DenseMergeArgs& m, const StreamArgs& a, float* out,
                        const float* theta, int64_t nel_max, const IntegShape& sh) {
    const int n_pos = sh.H_out * sh.W_out;
    const int64_t n_prob = (int64_t)((sh.B + kMultiImages - 1) / kMultiImages) * n_pos;
    const int64_t blocks = n_prob * a.n_cblk;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
    const int cap = multi_cap(nel_max);
    const size_t lds = (size_t)multi_wave_words(cap) * sizeof(int);
    hipLaunchKernelGGL(k_stream_multi, dim3((unsigned)blocks), dim3(64), lds, ctx->stream, m, a, out, theta, cap,
                       n_pos, sh.B);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_stream_shared(vdttfs_ctx* ctx, const DenseMergeArgs& m, const StreamArgs& a, float* out,
                         const float* theta, int64_t nel_max, int gather, bool culif, bool pool) {
    const int waves = shared_waves(a.n_cblk, gather);
    const int64_t n_grp = (a.n_cblk + waves - 1) / waves;
    const int64_t blocks = a.n_pix * n_grp;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
    const int cap = shared_cap(nel_max, waves, !culif, gather);
    const size_t lds = (size_t)shared_block_words(cap, m.T, !culif, waves) * sizeof(int);
    if (lds > kFusedMaxLds) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: shared list exceeds LDS");
#define VD_LAUNCH_SHARED(G, NB, L, P)                                                                      \
    hipLaunchKernelGGL((k_stream_quad<G, NB, L, P>), dim3((unsigned)blocks), dim3(64 * waves), lds, ctx->stream, \
                       m, a, out, theta, cap)
#define VD_LAUNCH_SHARED_NB(G, L, P)       \
    do {                                   \
        if (cap < nel_max)                 \
            VD_LAUNCH_SHARED(G, -1, L, P); \
        else                               \
            VD_LAUNCH_SHARED(G, 0, L, P);  \
    } while (0)
    if (culif && pool) return set_error(VDTTFS_E_INVALID, "integrate: the pool is fused into LUT-neuron builds only");
    if (gather == 4) {  // one event per load, four c_out per lane
        if (culif)
            VD_LAUNCH_SHARED_NB(1, true, false);
        else if (pool)
            VD_LAUNCH_SHARED_NB(1, false, true);
        else
            VD_LAUNCH_SHARED_NB(1, false, false);
    } else if (gather == 2) {
        if (culif)
            VD_LAUNCH_SHARED_NB(2, true, false);
        else if (pool)
            VD_LAUNCH_SHARED_NB(2, false, true);
        else
            VD_LAUNCH_SHARED_NB(2, false, false);
    } else {
        if (culif)
            VD_LAUNCH_SHARED_NB(4, true, false);
        else if (pool)
            VD_LAUNCH_SHARED_NB(4, false, true);
        else
            VD_LAUNCH_SHARED_NB(4, false, false);
    }
#undef VD_LAUNCH_SHARED_NB
#undef VD_LAUNCH_SHARED
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_stream_narrow(vdttfs_ctx* ctx, float* out, const int2* list, int64_t cap, const int32_t* bstart,
                         const float* W, int64_t wbytes, const float* bias, const float* theta, int t_min,
                         const IntegShape& sh, unsigned long long* counters, const CulifNeuron* culif) {
    int vec, epi;
    const StreamArgs a = stream_args(ctx, out, list, cap, bstart, W, wbytes, bias, theta, t_min, sh,
                                     counters, culif, LaunchPlan{}, &vec, &epi);
    const int P = 64 / sh.C_out;
    const int64_t waves = (a.n_pix + P - 1) / P;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
#define VD_LAUNCH_NARROW(C, L)                                                                      \
    hipLaunchKernelGGL((k_stream_narrow<C, L>), dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a, out, \
                       list, bstart, theta)
    if (culif) {
        if (counters)
            VD_LAUNCH_NARROW(true, true);
        else
            VD_LAUNCH_NARROW(false, true);
    } else {
        if (counters)
            VD_LAUNCH_NARROW(true, false);
        else
            VD_LAUNCH_NARROW(false, false);
    }
#undef VD_LAUNCH_NARROW
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

}  // namespace

// Measured per VGG layer against bucketize + k_merge: the dense merge is
// faster up to C_in = 64 and slower beyond, where each pixel's wave has many
// chunks and few pixels share the work; up to 9 taps (a 5x5 kernel's 25
// chunks spill registers).
bool integrate_dense_ok(const vdttfs_ctx* ctx, const IntegShape& sh) {
    int64_t wbytes;
    const int taps = sh.K_h * sh.K_w;
    // narrow layers (k_stream_narrow) take 5x5 kernels too: their pixels have
    // few receptive elements (LeNet: 25 and 150), where the closed-form merge
    // spends its time on a 25-column x T table per pixel
    const bool shape_ok = wave_path_ok(sh, &wbytes) ? taps <= 9 : (narrow_path_ok(sh, &wbytes) && taps <= 25);
    return !sh.is_fc && shape_ok && ctx->c.T <= kDenseMaxBins && sh.C_in <= kDenseMaxCin;
}

// Conv layers past the dense path's C_in limit whose lists k_stream_quad
// still builds in LDS straight from the dense map (no counters; a counting
// forward of such a layer takes bucketize + merge + stream): up to 9 taps
// and C_in <= 128 (18 chunks of 64), T <= 64, the four- or two-event gather
// (C_out <= 64, or <= 128 and a multiple of 4), 32-bit input offsets.
bool quad_wide_ok(const vdttfs_ctx* ctx, const IntegShape& sh) {
    int64_t wbytes;
    const int64_t in_bytes = (int64_t)sh.B * sh.H_in * sh.W_in * sh.C_in * 4;
    return !sh.is_fc && sh.K_h * sh.K_w <= 9 && ctx->c.T <= kBlockBins && sh.C_in > kDenseMaxCin &&
           sh.C_in <= kQuadMaxCin && !narrow_path_ok(sh, &wbytes) && wave_path_ok(sh, &wbytes) &&
           in_bytes < (INT64_C(1) << 31) && (sh.C_out <= 64 || (sh.C_out <= 128 && sh.C_out % 4 == 0));
}

namespace {
bool fused_ok(const vdttfs_ctx* ctx, const IntegShape& sh, int gather);

}  // namespace

// Layers whose lists the shared-list kernel builds (k_stream_quad<GEO, 0>,
// one output pixel per workgroup of up to four waves that share its list):
// conv with at most 9 taps or FC, T <= 64, gather 1 (64 c_out per wave), 2
// (128 per wave, C_out % 4 == 0) or 4 (one event per load, 256 c_out per
// wave, C_out > 128), weight rows below 2^16 (16-bit entries),
// 32-bit input offsets and a workgroup's list within the LDS limit.  No
// counters: a counting forward takes bucketize + merge + stream.
bool shared_ok(const vdttfs_ctx* ctx, const IntegShape& sh, int gather) {
    int64_t wbytes;
    const int taps = sh.is_fc ? 1 : sh.K_h * sh.K_w;
    const int64_t in_bytes = (int64_t)sh.B * sh.H_in * sh.W_in * sh.C_in * 4;
    const int64_t nel_max = shared_nel_max(sh);
    // weight rows tap * C_in + cin go in 16 bits (the tap of the full kernel:
    // a 3x3 conv on a 1x1 map still reads rows 4 C_in ...)
    const int64_t rows = (int64_t)taps * sh.C_in;
    // FC layers narrower than 32 outputs too (one 64-wide wave per image,
    // gather 1): LeNet-5's 84 -> 10
    const bool narrow_fc = sh.is_fc && narrow_path_ok(sh, &wbytes);
    if (ctx->c.T > kBlockBins || taps > 9 || !(wave_path_ok(sh, &wbytes) || narrow_fc) ||
        in_bytes >= (INT64_C(1) << 31) || nel_max > 0xFFFF || rows > 0x10000 || (narrow_fc && gather != 1))
        return false;
    // gather 4 (256 c_out per wave) for layers wider than 128 only
    if (gather != 1 && !(gather == 2 && sh.C_out % 4 == 0) && !(gather == 4 && sh.C_out % 4 == 0 && sh.C_out > 128))
        return false;
    const int cw = gather == 4 ? 256 : (gather == 2 ? 128 : 64);
    const int64_t n_cblk = (sh.C_out + cw - 1) / cw;
    const int waves = shared_waves(n_cblk, gather);
    const int cap = shared_cap(nel_max, waves, true, gather);
    return (size_t)shared_block_words(cap, ctx->c.T, true, waves) * sizeof(int) <= kFusedMaxLds;
}

// The shared-list kernel's built-in gather: 128 c_out per wave (two events
// per load, fewer transposes per byte) up to 256 c_out, where one group of
// waves covers the layer; 64 per wave (four events per load) past that, so
// that each c_out group of four waves holds a smaller share of the weights
// in its XCD's L2, and where C_out <= 64 or is not a multiple of 4.
// For 64 < C_out <= 128 the pair gather is one wave per pixel, which builds
// the list alone; where the launch fits one round of resident waves (at most
// 32 per CU), two 64-wide waves that build together and stream half the
// c_out each finish first (LeNet-5's FC 256 -> 120 and 120 -> 84 at B=1024,
// 1,024 pixels: 0.025 / 0.017 -> 0.020 / 0.016 ms).
namespace {
int64_t cu_count(const vdttfs_ctx* ctx);
}  // namespace
int shared_gather(const vdttfs_ctx* ctx, const IntegShape& sh) {
    if (!(sh.C_out % 4 == 0 && sh.C_out > 64 && sh.C_out <= 256)) return 1;
    if (sh.C_out <= 128) {
        const int64_t cus = cu_count(ctx);
        if (cus > 0 && n_pixels(sh) * 2 <= cus * 32) return 1;
    }
    return 2;
}

// The kernel a fused plan with this gather runs: 1 the per-wave kernels
// (k_stream_quad's own lists, k_stream_dense), 2 the shared-list kernel,
// 0 none.
int fused_kind(const vdttfs_ctx* ctx, const IntegShape& sh, int gather) {
    if ((integrate_dense_ok(ctx, sh) || quad_wide_ok(ctx, sh)) && fused_ok(ctx, sh, gather)) return 1;
    return shared_ok(ctx, sh, gather) ? 2 : 0;
}

// Layers k_stream_multi takes (the shared-list kernel's four-c_out layers:
// C_out > 128, C_out % 4 == 0; the LUT neuron only): plan FUSED, gather 4,
// four pixels per wave -- the same position of four images.
bool multi_ok(const vdttfs_ctx* ctx, const IntegShape& sh, bool culif) {
    if (culif || fused_kind(ctx, sh, 4) != 2) return false;
    return (size_t)multi_wave_words(multi_cap(shared_nel_max(sh))) * sizeof(int) <= kFusedMaxLds;
}

bool plan_from_dense(const vdttfs_ctx* ctx, const IntegShape& sh, const LaunchPlan& p, bool counters) {
    if (plan_bins(p)) return false;
    return integrate_dense_ok(ctx, sh) ||
           (!counters && p.path == VDTTFS_PATH_FUSED && fused_kind(ctx, sh, p.gather) != 0);
}

bool plan_lds_list(const vdttfs_ctx* ctx, const IntegShape& sh, const LaunchPlan& p, bool counters, bool culif) {
    if (p.path == VDTTFS_PATH_WINDOW) return true;
    if (p.path == VDTTFS_PATH_REG) return !counters && !culif;
    if (p.path != VDTTFS_PATH_FUSED) return false;
    // the shared-list kernel runs no counters: a counting forward takes
    // k_merge_dense + stream (C_in <= 64) or bucketize + merge + stream
    if (fused_kind(ctx, sh, p.gather) == 2) return !counters;
    // past the dense limits a counting forward takes bucketize + merge + stream
    if (counters && !integrate_dense_ok(ctx, sh)) return false;
    // two events per load: k_stream_quad only (no counters, 32-bit input
    // offsets); otherwise k_merge_dense + k_stream
    (void)culif;
    const int64_t in_bytes = (int64_t)sh.B * sh.H_in * sh.W_in * sh.C_in * 4;
    return p.gather != 2 || (!counters && in_bytes < (INT64_C(1) << 31));
}

namespace {

// The fused path: one c_out per lane up to 64 c_out (k_stream_quad, or
// k_stream_dense for counting and CuLIF forwards), or two events per load
// up to 128 (k_stream_quad; counting and CuLIF forwards of such a layer
// take k_merge_dense + k_stream, as the dense path).
bool fused_ok(const vdttfs_ctx* ctx, const IntegShape& sh, int gather) {
    const int nel_max = sh.K_h * sh.K_w * sh.C_in;
    const size_t lds = (size_t)kMergeWaves * fused_wave_words(nel_max, ctx->c.T) * sizeof(int);
    const size_t qlds = (size_t)kQuadWaves * quad_wave_words(nel_max, ctx->c.T) * sizeof(int);
    if (ctx->c.T > kBlockBins) return false;
    // past the dense limits only k_stream_quad runs (no counters)
    const bool wide = quad_wide_ok(ctx, sh);
    if (gather == 1) return sh.C_out <= 64 && (wide ? qlds : lds) <= kFusedMaxLds;
    return gather == 2 && sh.C_out <= 128 && sh.C_out % 4 == 0 && qlds <= kFusedMaxLds;
}

// k_stream_window's limits: one bin block, the per-pixel tables of <= 9 columns
bool window_ok(const vdttfs_ctx* ctx, const IntegShape& sh) {
    return ctx->c.T <= kBlockBins && (sh.is_fc || sh.K_h * sh.K_w <= 9);
}

// k_conv_small's limits (the receptive field and the bins fit in registers)
bool small_ok(const vdttfs_ctx* ctx, const IntegShape& sh) {
    const int64_t in_bytes = (int64_t)sh.B * sh.H_in * sh.W_in * sh.C_in * 4;
    return !sh.is_fc && sh.K_h * sh.K_w * sh.C_in <= kSmallMaxEl && sh.C_out <= 64 &&
           ctx->c.T <= kSmallMaxBins && integrate_dense_ok(ctx, sh) && in_bytes < (INT64_C(1) << 31) &&
           n_pixels(sh) < (INT64_C(1) << 31);
}

int launch_conv_small(vdttfs_ctx* ctx, float* out, const float* in, const float* alpha, const float* W,
                      const float* bias, const float* theta, int t_min, const IntegShape& sh) {
    SmallArgs a{};
    a.in = in;
    a.alpha = alpha;
    a.W = W;
    a.bias = bias;
    a.theta = theta;
    a.out = out;
    a.n_pix = n_pixels(sh);
    a.T = ctx->c.T;
    a.t_min = t_min;
    a.alpha_by_time = ctx->c.alpha_by_time;
    a.tfs = ctx->c.tfs;
    a.H_in = sh.H_in;
    a.W_in = sh.W_in;
    a.C_in = sh.C_in;
    a.H_out = sh.H_out;
    a.W_out = sh.W_out;
    a.C_out = sh.C_out;
    a.K_h = sh.K_h;
    a.K_w = sh.K_w;
    a.pad_h = sh.pad_h;
    a.pad_w = sh.pad_w;
    a.nel = sh.K_h * sh.K_w * sh.C_in;
    a.P = 64 / sh.C_out;
    const int64_t in_bytes = (int64_t)sh.B * sh.H_in * sh.W_in * sh.C_in * 4;
    if (a.nel > kSmallMaxEl || sh.C_out > 64 || a.T > kSmallMaxBins || in_bytes >= (INT64_C(1) << 31) ||
        a.n_pix >= (INT64_C(1) << 31))
        return set_error(VDTTFS_E_UNSUPPORTED, "conv_small: layer outside its limits");
    a.in_bytes = (int)in_bytes;
    a.div_cout = make_fastdiv(sh.C_out);
    a.div_w = make_fastdiv(sh.W_out);
    a.div_h = make_fastdiv(sh.H_out);
    const int64_t waves = (a.n_pix + a.P - 1) / a.P;
    const int64_t blocks = (waves + 3) / 4;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "conv_small: grid too large");
    // the bin scan covers exactly the receptive field of LeNet-5's conv1 (25)
    // and VGG-16's conv 0 (27), the 32-element limit otherwise
    // every tap of every output pixel inside the map (no padding): the
    // element offsets come from a table
    const bool valid = sh.pad_h == 0 && sh.pad_w == 0 && sh.H_out <= sh.H_in - sh.K_h + 1 &&
                       sh.W_out <= sh.W_in - sh.K_w + 1;
    a.w_bytes = (int)((int64_t)a.nel * sh.C_out * 4);
    for (int e = 0; e < kSmallMaxEl; ++e) a.dk[e] = 0;
    for (int kh = 0, e = 0; kh < sh.K_h; ++kh)
        for (int kw = 0; kw < sh.K_w; ++kw)
            for (int ci = 0; ci < sh.C_in; ++ci, ++e) a.dk[e] = (kh * sh.W_in + kw) * sh.C_in + ci;
#define VD_LAUNCH_SMALL(U, N, V) \
    hipLaunchKernelGGL((k_conv_small<U, N, V>), dim3((unsigned)blocks), dim3(256), 0, ctx->stream, a)
    if (a.P == 1) {
        if (a.nel == 27)
            VD_LAUNCH_SMALL(true, 27, false);
        else
            VD_LAUNCH_SMALL(true, kSmallMaxEl, false);
    } else if (valid) {
        if (a.nel == 25)
            VD_LAUNCH_SMALL(false, 25, true);
        else
            VD_LAUNCH_SMALL(false, kSmallMaxEl, true);
    } else {
        if (a.nel == 25)
            VD_LAUNCH_SMALL(false, 25, false);
        else
            VD_LAUNCH_SMALL(false, kSmallMaxEl, false);
    }
#undef VD_LAUNCH_SMALL
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

// Waves of the gather's k_stream instantiation the device holds at once
// (resident blocks per CU from the compiled kernel's registers, times CUs);
// 0 if the runtime cannot tell.  Cached per device and gather width.
int64_t stream_wave_capacity(const vdttfs_ctx* ctx, int gather) {
    constexpr int kMaxDev = 64;
    static std::atomic<int> blocks_per_cu[3][kMaxDev];
    static std::atomic<int> cus[kMaxDev];
    const int dev = ctx->device;
    if (dev < 0 || dev >= kMaxDev) return 0;
    const int gi = gather == 4 ? 2 : (gather == 2 ? 1 : 0);
    int nb = blocks_per_cu[gi][dev].load(std::memory_order_relaxed);
    int nc = cus[dev].load(std::memory_order_relaxed);
    if (nb <= 0 || nc <= 0) {
        hipError_t e;
        if (gi == 2)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_stream<false, 4, false, 1>, 256, 0);
        else if (gi == 1)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_stream<false, 2, false, 2>, 256, 0);
        else
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_stream<false, 1, false, 1>, 256, 0);
        if (e != hipSuccess || hipDeviceGetAttribute(&nc, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            nb <= 0 || nc <= 0) {
            (void)hipGetLastError();
            return 0;
        }
        blocks_per_cu[gi][dev].store(nb, std::memory_order_relaxed);
        cus[dev].store(nc, std::memory_order_relaxed);
    }
    return (int64_t)nb * 4 * nc;  // 4 waves per block
}

// Compute units of the context's device (0 if the runtime cannot tell),
// cached per device.
int64_t cu_count(const vdttfs_ctx* ctx) {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cus[kMaxDev];
    const int dev = ctx->device;
    if (dev < 0 || dev >= kMaxDev) return 0;
    int nc = cus[dev].load(std::memory_order_relaxed);
    if (nc <= 0) {
        if (hipDeviceGetAttribute(&nc, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || nc <= 0) {
            (void)hipGetLastError();
            return 0;
        }
        cus[dev].store(nc, std::memory_order_relaxed);
    }
    return nc;
}

// Whether the built-in plan takes the shared-list kernel where it applies:
// where a pixel's c_out fit at most two workgroups.  Each workgroup builds
// the pixel's list itself, so wider layers (config 5's 4096-wide FC: 16
// groups of 256 c_out) keep bucketize + merge, which build it once.
bool shared_builtin(const vdttfs_ctx* ctx, const IntegShape& sh) {
    (void)ctx;
    const int g = shared_gather(ctx, sh);
    const int cw = g == 4 ? 256 : (g == 2 ? 128 : 64);
    const int64_t n_cblk = (sh.C_out + cw - 1) / cw;
    const int waves = shared_waves(n_cblk, g);
    return (n_cblk + waves - 1) / waves <= 2;
}

int plan_error(const IntegShape& sh, const char* what) {
    return set_error(VDTTFS_E_UNSUPPORTED, "plan: %s (layer %dx%dx%d -> %d, %dx%d taps%s)", what, sh.H_in, sh.W_in,
                     sh.C_in, sh.C_out, sh.K_h, sh.K_w, sh.is_fc ? ", fc" : "");
}

}  // namespace

int resolve_plan(const vdttfs_ctx* ctx, const IntegShape& sh, const LaunchPlan& req, LaunchPlan* out) {
    if (req.path < 0 || req.path > VDTTFS_PATH_WINDOW || req.gather < 0 || req.ppw < 0 || req.ppw > 64)
        return set_error(VDTTFS_E_INVALID, "plan: path %d, gather %d, ppw %d out of range", req.path,
                         req.gather, req.ppw);
    int64_t wbytes;
    const bool narrow = narrow_path_ok(sh, &wbytes);
    const bool wave = !narrow && wave_path_ok(sh, &wbytes);
    const bool dense = integrate_dense_ok(ctx, sh);
    LaunchPlan p{};
    if (!narrow && !wave) {  // the generic integrator: nothing to choose
        if ((req.path && req.path != VDTTFS_PATH_BINS) || req.gather || req.ppw)
            return plan_error(sh, "the generic integrator has no launch choices");
        p.path = VDTTFS_PATH_BINS;
        *out = p;
        return VDTTFS_OK;
    }
    // no list (k_conv_small).  Built-in for layers narrower than 32 outputs
    // (LeNet conv1, B=1024: 0.37 ms against 0.58 for k_merge_dense +
    // k_stream_narrow).  A wave-wide layer keeps the fused list: k_conv_small
    // scans every element for each occupied bin, about 5,400 instructions
    // per VGG-16 L0 pixel against 2,600 for k_stream_dense (1.42 against
    // 0.70 ms), which touches each event once.
    const bool small = small_ok(ctx, sh);
    const int P_small = 64 / sh.C_out;
    if (req.path == VDTTFS_PATH_REG || (req.path == 0 && small && narrow && !req.gather && !req.ppw)) {
        if (!small) return plan_error(sh, "the register path needs K_h*K_w*C_in <= 32, C_out <= 64, T <= 64");
        if (req.gather > 1 || (req.ppw && req.ppw != P_small))
            return plan_error(sh, "the register path takes gather 1 and 64 / C_out pixels per wave");
        p.path = VDTTFS_PATH_REG;
        p.gather = 1;
        p.ppw = P_small;
        *out = p;
        return VDTTFS_OK;
    }
    // FC layers narrower than 32 outputs: the shared-list kernel (one wave
    // per image, the list built in LDS) where it takes them, in place of
    // bucketize + k_merge + k_stream_narrow (LeNet-5's 84 -> 10 at B=1024:
    // three launches of a few microseconds of work each)
    if (narrow && sh.is_fc && shared_ok(ctx, sh, 1) && (req.path == 0 || req.path == VDTTFS_PATH_FUSED) &&
        req.gather <= 1 && req.ppw <= 1) {
        p.path = VDTTFS_PATH_FUSED;
        p.gather = 1;
        p.ppw = 1;
        *out = p;
        return VDTTFS_OK;
    }
    if (narrow) {  // one pixel per C_out lanes
        const int P = 64 / sh.C_out;
        if (req.path == VDTTFS_PATH_FUSED || req.path == VDTTFS_PATH_WINDOW || (req.gather && req.gather != 1) ||
            (req.ppw && req.ppw != P))
            return plan_error(sh, "narrow layers take gather 1, 64 / C_out pixels per wave, paths bins or dense");
        p.path = req.path ? req.path : (dense ? VDTTFS_PATH_DENSE : VDTTFS_PATH_BINS);
        if (p.path == VDTTFS_PATH_DENSE && !dense) return plan_error(sh, "dense path outside its limits");
        p.gather = 1;
        p.ppw = P;
        *out = p;
        return VDTTFS_OK;
    }
    // gather: 64 < C_out <= 128 (multiple of 4): 2 events per 1 KB load;
    // wider layers: 4 c_out per lane (dwordx4), 64*4 c_out per block.
    // C_out <= 64 keeps one dword load per event: measured faster than 2 or 4
    // events per load there, as lanes whose neurons fired skip their loads.
    if (req.gather) {
        if (req.gather != 1 && req.gather != 2 && req.gather != 4) return plan_error(sh, "gather is 1, 2 or 4");
        if (req.gather != 1 && sh.C_out % 4 != 0) return plan_error(sh, "gather 2 and 4 need C_out % 4 == 0");
        p.gather = req.gather;
    } else {
        p.gather = (sh.C_out % 4 == 0 && sh.C_out > 64) ? (sh.C_out <= 128 ? 2 : 4) : 1;
        // an FC layer's pixels are its batch: where four c_out per lane would
        // leave fewer waves than the device has SIMDs, the pair gather (2x
        // the c_out blocks, two events per load) is faster (VGG-16's 512 ->
        // 512 FC at B=256: 512 waves, 0.072 ms; one c_out per lane, 0.055;
        // the pair, 0.047; the 2x2 conv L14's 2,048 keep four)
        const int64_t simds = 4 * cu_count(ctx);
        if (p.gather == 4 && sh.is_fc && simds > 0 && n_pixels(sh) * ((sh.C_out + 255) / 256) < simds) p.gather = 2;
        // where no per-wave fused kernel serves, the shared-list kernel's
        // gather (shared_gather)
        const int pw = (dense || quad_wide_ok(ctx, sh)) && fused_ok(ctx, sh, p.gather) ? 1 : 0;
        if ((req.path == 0 || req.path == VDTTFS_PATH_FUSED) && !pw) {
            const int g = shared_gather(ctx, sh);
            if (shared_ok(ctx, sh, g) && (req.path == VDTTFS_PATH_FUSED || shared_builtin(ctx, sh))) p.gather = g;
        }
    }
    // measured: 2 pixels per wave pays at >= 2^20 pixels (CuLIF conv2 at
    // 128x128 x 64 samples: 9.16 -> 8.56 ms) and loses on smaller layers
    // (VGG-16 B=256 at 2, 4, 8 pixels per wave: 30.4K -> 29.3K, 26.0K, 20.0K
    // images/s; the 2^18-pixel CuLIF conv3: 3.68 -> 3.88 ms).  It also pays
    // where one pixel per wave needs more than one but at most two rounds of
    // resident waves and two pixels per wave fit in one (VGG-16's 4x4 layers:
    // 8,192 waves against 5,120 resident, 0.42 -> 0.39 ms each): the second
    // round would run mostly empty.
    if (req.ppw > kMaxPixPerWave) return plan_error(sh, "at most 8 pixels per wave");
    const int kind = fused_kind(ctx, sh, p.gather);
    const bool fused = kind == 1 || (kind == 2 && (req.path == VDTTFS_PATH_FUSED || shared_builtin(ctx, sh)));
    if (req.path == VDTTFS_PATH_DENSE && !dense) return plan_error(sh, "dense path outside its limits");
    if (req.path == VDTTFS_PATH_FUSED && !fused)
        return plan_error(sh, "fused path needs T <= 64, at most 9 taps (or FC), gather 1, 2 or 4 (C_out % 4 == 0), "
                              "and the pixel's list within the LDS limit");
    if (req.path == VDTTFS_PATH_WINDOW && !window_ok(ctx, sh))
        return plan_error(sh, "window path needs T <= 64 and at most 9 taps (or an FC layer)");
    p.path = req.path ? req.path : (fused ? VDTTFS_PATH_FUSED : (dense ? VDTTFS_PATH_DENSE : VDTTFS_PATH_BINS));
    if (p.path == VDTTFS_PATH_FUSED && kind == 2) {
        // the shared-list kernel: one output pixel per workgroup; or, with
        // gather 4 and four pixels per wave, k_stream_multi (one position of
        // four images per wave)
        if (req.ppw == kMultiImages && p.gather == 4 && multi_ok(ctx, sh, false)) {
            p.ppw = kMultiImages;
        } else {
            if (req.ppw > 1)
                return plan_error(sh, "the shared-list fused kernel takes one pixel per workgroup, or four "
                                      "(the same position of four images) with gather 4");
            p.ppw = 1;
        }
    } else if (req.ppw) {
        p.ppw = req.ppw;
    } else {
        const int64_t n_pix = n_pixels(sh);
        p.ppw = n_pix >= (INT64_C(1) << 20) ? 2 : 1;
        // the one-chunk fused kernel (receptive field <= 64 elements) spends
        // a large share of a pixel on the wave's set-up: four pixels per wave
        // where that still leaves 16K waves (VGG-16's conv 0 at B=256:
        // 0.295 -> 0.283 ms; the nine-chunk conv 1 gains nothing at 2 or 4)
        if (p.path == VDTTFS_PATH_FUSED && !sh.is_fc && sh.K_h * sh.K_w * sh.C_in <= 64 && n_pix >= (INT64_C(1) << 16))
            p.ppw = 4;
        if (p.ppw == 1 && p.path != VDTTFS_PATH_FUSED && p.path != VDTTFS_PATH_WINDOW) {
            // k_stream's residency (the fused and window kernels' is LDS-bound).
            // The rule keeps k_stream's figures (six waves per SIMD at four
            // c_out per lane) where the timed forward runs k_stream_lean
            // (eight): with k_stream_lean's own, VGG-16's 8x8 layers would
            // take two pixels per wave and its 4x4 layers one, and both lose
            // (0.447 -> 0.478 and 0.349 -> 0.415 ms).
            const int vec = p.gather == 4 ? 4 : (p.gather == 2 ? 2 : 1);
            const int64_t n_cblk = p.gather == 2 ? (sh.C_out + 127) / 128 : (sh.C_out + 64 * vec - 1) / (64 * vec);
            // Past 8 c_out blocks an XCD streams one block at a time over all
            // the pixels (map_block), so only that block's waves are in
            // flight on it and the rule does not hold: config 5's FC 4096 x
            // 4096 at B=512 (16 blocks) 0.147 -> 0.109 ms at one pixel per wave.
            const int64_t cap = stream_wave_capacity(ctx, p.gather);
            if (cap > 0 && n_cblk < 8 && n_pix * n_cblk > cap && (n_pix + 1) / 2 * n_cblk <= cap) p.ppw = 2;
        }
    }
    *out = p;
    return VDTTFS_OK;
}

int launch_integrate_bins(vdttfs_ctx* ctx, float* out, const vd_event* ev, const int32_t* off,
                          int2* list, int64_t list_cap, int32_t* bstart, const float* W,
                          const float* bias, const float* theta, int t_min, const IntegShape& sh,
                          unsigned long long* counters, const CulifNeuron* culif, const LaunchPlan* plan) {
    LaunchPlan p;
    VD_TRY(resolve_plan(ctx, sh, plan ? *plan : LaunchPlan{}, &p));
    // a fused plan past the dense limits falls back here for counting forwards
    if (plan && plan->path && !plan_bins(*plan) &&
        !(plan->path == VDTTFS_PATH_FUSED && (quad_wide_ok(ctx, sh) || fused_kind(ctx, sh, p.gather) == 2)))
        return set_error(VDTTFS_E_INVALID, "integrate_bins: the plan asks for a dense path");
    int64_t wbytes;
    const bool narrow = narrow_path_ok(sh, &wbytes);
    if (!narrow && !wave_path_ok(sh, &wbytes)) {
        if (culif)
            return set_error(VDTTFS_E_UNSUPPORTED,
                             "CuLIF engine layers need <= 25 taps and < 2 GB of weights");
        return launch_integrate_generic_bins(ctx, out, ev, off, W, bias, theta, t_min, sh, counters);
    }
    const int nk_max = sh.is_fc ? 1 : sh.K_h * sh.K_w;
    const int64_t n_pix = n_pixels(sh);
    const int64_t cap = (int64_t)nk_max * sh.C_in + kListPad;
    if (p.path != VDTTFS_PATH_WINDOW && (!list || !bstart || list_cap < cap))
        return set_error(VDTTFS_E_INVALID, "integrate: merged-list scratch too small");
    MergeArgs m{};
    m.list = list;
    m.bstart = bstart;
    m.ev = ev;
    m.off = off;
    m.n_pix = n_pix;
    m.cap = cap;
    m.T = ctx->c.T;
    m.H_in = sh.H_in;
    m.W_in = sh.W_in;
    m.C_in = sh.C_in;
    m.H_out = sh.H_out;
    m.W_out = sh.W_out;
    m.K_h = sh.K_h;
    m.K_w = sh.K_w;
    m.pad_h = sh.pad_h;
    m.pad_w = sh.pad_w;
    m.is_fc = sh.is_fc;
    m.rowbytes = sh.C_out * 4;
    if (n_pix >= (INT64_C(1) << 31)) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: 2^31 output pixels or more");
    m.div_w = make_fastdiv(sh.W_out);
    m.div_h = make_fastdiv(sh.H_out);
    if (p.path == VDTTFS_PATH_WINDOW)
        return launch_stream_window(ctx, m, out, ev, W, wbytes, bias, theta, t_min, sh, counters, culif, p);
    const int64_t mblocks = (n_pix + kMergeWaves - 1) / kMergeWaves;
    if (mblocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
    if (nk_max == 1)
        hipLaunchKernelGGL(k_merge<1>, dim3((unsigned)mblocks), dim3(64 * kMergeWaves), 0, ctx->stream, m);
    else if (nk_max <= 9)
        hipLaunchKernelGGL(k_merge<9>, dim3((unsigned)mblocks), dim3(64 * kMergeWaves), 0, ctx->stream, m);
    else
        hipLaunchKernelGGL(k_merge<25>, dim3((unsigned)mblocks), dim3(64 * kMergeWaves), 0, ctx->stream, m);
    VD_HIP(hipGetLastError());
    if (narrow) return launch_stream_narrow(ctx, out, list, cap, bstart, W, wbytes, bias, theta, t_min, sh,
                                            counters, culif);
    return launch_stream(ctx, out, list, cap, bstart, W, wbytes, bias, theta, t_min, sh, counters, culif, p);
}

bool pool_fusable(const vdttfs_ctx* ctx, const IntegShape& sh, const LaunchPlan& p, int H_u, int W_u) {
    if (p.path != VDTTFS_PATH_FUSED) return false;
    if (H_u / 2 != sh.H_in || W_u / 2 != sh.W_in || H_u < 2 || W_u < 2) return false;
    if ((int64_t)sh.B * H_u * W_u * sh.C_in * 4 >= (INT64_C(1) << 31)) return false;
    int64_t wbytes;
    if (narrow_path_ok(sh, &wbytes) || !plan_lds_list(ctx, sh, p, false, false)) return false;
    const int kind = fused_kind(ctx, sh, p.gather);
    // the shared-list kernel, or the per-wave kernel of 9 or 18 chunks
    return (kind == 2 && p.ppw != kMultiImages) || (kind == 1 && sh.K_h * sh.K_w * sh.C_in > 64);
}

int launch_integrate_dense(vdttfs_ctx* ctx, float* out, const float* in, const float* alpha, int2* list,
                           int64_t list_cap, int32_t* bstart, const float* W, const float* bias,
                           const float* theta, int t_min, const IntegShape& sh,
                           unsigned long long* counters, const CulifNeuron* culif, const LaunchPlan* plan,
                           const PoolIn* pool) {
    int64_t wbytes;
    const bool narrow = narrow_path_ok(sh, &wbytes);
    const bool wide = !integrate_dense_ok(ctx, sh) && quad_wide_ok(ctx, sh);
    LaunchPlan p;
    VD_TRY(resolve_plan(ctx, sh, plan ? *plan : LaunchPlan{}, &p));
    // the shared-list kernel: any conv (<= 9 taps) or FC layer in its limits
    const bool shared = !counters && p.path == VDTTFS_PATH_FUSED && fused_kind(ctx, sh, p.gather) == 2;
    if (!shared && ((!integrate_dense_ok(ctx, sh) && !(wide && !counters)) || (!narrow && !wave_path_ok(sh, &wbytes))))
        return set_error(VDTTFS_E_UNSUPPORTED, "integrate_dense: conv layers of the merged-list path only");
    if (shared) (void)wave_path_ok(sh, &wbytes);
    if (wide && p.path != VDTTFS_PATH_FUSED)
        return set_error(VDTTFS_E_UNSUPPORTED, "integrate_dense: past C_in %d only the fused path builds from the map",
                         kDenseMaxCin);
    if (plan_bins(p))
        return set_error(VDTTFS_E_INVALID, "integrate_dense: the plan asks for the bins path");
    if (p.path == VDTTFS_PATH_REG) {
        if (!counters && !culif) return launch_conv_small(ctx, out, in, alpha, W, bias, theta, t_min, sh);
        // counting forwards and the CuLIF neuron take a list path: same results
        LaunchPlan req{};
        req.path = (!narrow && fused_ok(ctx, sh, 1)) ? VDTTFS_PATH_FUSED : VDTTFS_PATH_DENSE;
        VD_TRY(resolve_plan(ctx, sh, req, &p));
    }
    const int nk_max = sh.K_h * sh.K_w;
    const int64_t n_pix = n_pixels(sh);
    const int64_t cap = (int64_t)nk_max * sh.C_in + kListPad;
    // the fused kernels keep their lists in LDS; the others need the scratch
    const bool lds_list = plan_lds_list(ctx, sh, p, counters != nullptr, culif != nullptr);
    if (!lds_list && (!list || !bstart || list_cap < cap))
        return set_error(VDTTFS_E_INVALID, "integrate: merged-list scratch too small");
    DenseMergeArgs m{};
    m.list = list;
    m.bstart = bstart;
    m.in = in;
    m.alpha = alpha;
    m.n_pix = n_pix;
    m.cap = cap;
    m.T = ctx->c.T;
    m.tfs = ctx->c.tfs;
    m.alpha_by_time = ctx->c.alpha_by_time;
    int nbits = 0;
    while ((1 << nbits) < m.T) ++nbits;
    m.nbits = nbits;
    m.H_in = sh.H_in;
    m.W_in = sh.W_in;
    m.C_in = sh.C_in;
    m.H_out = sh.H_out;
    m.W_out = sh.W_out;
    m.K_h = sh.K_h;
    m.K_w = sh.K_w;
    m.pad_h = sh.pad_h;
    m.pad_w = sh.pad_w;
    m.rowbytes = sh.C_out * 4;
    m.inv_cin = 1.0f / (float)sh.C_in;
    m.fired = culif ? culif->fired : nullptr;
    if (n_pix >= (INT64_C(1) << 31)) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: 2^31 output pixels or more");
    m.div_w = make_fastdiv(sh.W_out);
    m.div_h = make_fastdiv(sh.H_out);
    const int64_t in_bytes = (int64_t)sh.B * sh.H_in * sh.W_in * sh.C_in * 4;
    m.in_bytes = in_bytes < (INT64_C(1) << 31) ? (int)in_bytes : 0;
    if (pool) {
        if (counters || culif || !pool_fusable(ctx, sh, p, pool->H_u, pool->W_u))
            return set_error(VDTTFS_E_INVALID, "integrate: this layer's list build cannot take the pool");
        m.H_u = pool->H_u;
        m.W_u = pool->W_u;
        m.pdx = sh.C_in * 4;
        m.pdy = pool->W_u * sh.C_in * 4;
        m.in_bytes = (int)((int64_t)sh.B * pool->H_u * pool->W_u * sh.C_in * 4);  // < 2^31 (pool_fusable)
    }
    const int64_t mblocks = (n_pix + kMergeWaves - 1) / kMergeWaves;
    if (mblocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
    if (narrow && !shared) {
        if (nk_max <= 9)
            hipLaunchKernelGGL(k_merge_dense<9>, dim3((unsigned)mblocks), dim3(64 * kMergeWaves), 0, ctx->stream,
                               m);
        else
            hipLaunchKernelGGL(k_merge_dense<25>, dim3((unsigned)mblocks), dim3(64 * kMergeWaves), 0,
                               ctx->stream, m);
        VD_HIP(hipGetLastError());
        return launch_stream_narrow(ctx, out, list, cap, bstart, W, wbytes, bias, theta, t_min, sh, counters,
                                    culif);
    }
    int vec, epi;
    const StreamArgs a = stream_args(ctx, out, list, cap, bstart, W, wbytes, bias, theta, t_min, sh,
                                     counters, culif, p, &vec, &epi);
    const int nel_max = nk_max * sh.C_in;
    const size_t lds = (size_t)kMergeWaves * fused_wave_words(nel_max, m.T) * sizeof(int);
    if (p.path == VDTTFS_PATH_FUSED && lds_list) {
        if (shared && p.ppw == kMultiImages && !culif)
            return launch_stream_multi(ctx, m, a, out, theta, shared_nel_max(sh), sh);
        if (shared)
            return launch_stream_shared(ctx, m, a, out, theta, shared_nel_max(sh), p.gather, culif != nullptr,
                                        pool != nullptr);
        // build the list in LDS and stream it there
        const int64_t fblocks = (n_pix + kMergeWaves * a.ppw - 1) / (kMergeWaves * a.ppw);
        if (!counters && m.in_bytes > 0) {
            // waves per workgroup: one, except the one-chunk four-event
            // kernel (VGG conv 0), measured A/B on one box: CuLIF conv2
            // 4.08 -> 3.31 ms with 1 (4.23 with 2), VGG conv 1 -0.8% and
            // conv 2 -1.4% with 1, conv 0 +1.4% with 1
            const int qw = (epi != 2 && nel_max <= 64) ? kQuadWaves : 1;
            const size_t qlds = (size_t)qw * quad_wave_words(nel_max, m.T, culif == nullptr) * sizeof(int);
            const int64_t qblocks = (n_pix + qw * a.ppw - 1) / (qw * a.ppw);
#define VD_LAUNCH_QUAD(G, NB, L, P)                                                                        \
    hipLaunchKernelGGL((k_stream_quad<G, NB, L, P>), dim3((unsigned)qblocks), dim3(64 * qw), qlds, \
                       ctx->stream, m, a, out, theta, nel_max)
#define VD_LAUNCH_QUAD_NB(G, L)              \
    do {                                     \
        if (nel_max <= 64)                   \
            VD_LAUNCH_QUAD(G, 1, L, false);  \
        else if (nel_max <= 9 * 64)          \
            VD_LAUNCH_QUAD(G, 9, L, false);  \
        else                                 \
            VD_LAUNCH_QUAD(G, 18, L, false); \
    } while (0)
            if (pool) {  // nel_max > 64 (pool_fusable)
                if (nel_max <= 9 * 64) {
                    if (epi == 2)
                        VD_LAUNCH_QUAD(2, 9, false, true);
                    else
                        VD_LAUNCH_QUAD(4, 9, false, true);
                } else {
                    if (epi == 2)
                        VD_LAUNCH_QUAD(2, 18, false, true);
                    else
                        VD_LAUNCH_QUAD(4, 18, false, true);
                }
            } else if (epi == 2) {
                if (culif)
                    VD_LAUNCH_QUAD_NB(2, true);
                else
                    VD_LAUNCH_QUAD_NB(2, false);
            } else {
                if (culif)
                    VD_LAUNCH_QUAD_NB(4, true);
                else
                    VD_LAUNCH_QUAD_NB(4, false);
            }
#undef VD_LAUNCH_QUAD_NB
#undef VD_LAUNCH_QUAD
            VD_HIP(hipGetLastError());
            return VDTTFS_OK;
        }
        // pixels of at most 64 elements (VGG-16 L0: 27) build from one chunk
        // in the fewest registers
#define VD_LAUNCH_FUSED_NB(C, L, NB)                                                                      \
    hipLaunchKernelGGL((k_stream_dense<C, 1, L, 1, NB>), dim3((unsigned)fblocks), dim3(64 * kMergeWaves), \
                       lds, ctx->stream, m, a, out, theta, nel_max)
#define VD_LAUNCH_FUSED(C, L)                \
    do {                                     \
        if (nel_max <= 64)                   \
            VD_LAUNCH_FUSED_NB(C, L, 1);     \
        else                                 \
            VD_LAUNCH_FUSED_NB(C, L, 9);     \
    } while (0)
        if (culif) {
            if (counters)
                VD_LAUNCH_FUSED(true, true);
            else
                VD_LAUNCH_FUSED(false, true);
        } else {
            if (counters)
                VD_LAUNCH_FUSED(true, false);
            else
                VD_LAUNCH_FUSED(false, false);
        }
#undef VD_LAUNCH_FUSED
#undef VD_LAUNCH_FUSED_NB
        VD_HIP(hipGetLastError());
        return VDTTFS_OK;
    }
    hipLaunchKernelGGL(k_merge_dense<9>, dim3((unsigned)mblocks), dim3(64 * kMergeWaves), 0, ctx->stream, m);
    VD_HIP(hipGetLastError());
    return launch_stream(ctx, out, list, cap, bstart, W, wbytes, bias, theta, t_min, sh, counters, culif, p);
}

}  // namespace vdttfs
