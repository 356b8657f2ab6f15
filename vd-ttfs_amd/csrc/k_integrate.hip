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
// k_integrate_wave (engine path): one wave64 per (output pixel, 64-wide
// c_out block); lanes are c_out, so every event is wave-uniform and each
// weight gather is one coalesced 256-byte row segment.  Per chunk the wave
// merges the receptive columns' bin-sorted lists into (bin, column, cin)
// order in LDS using a closed-form position table, then streams the merged
// list in batches of 8 independent gathers, finalising one bin at a time;
// lanes that fired are masked off (no fetch) and the wave leaves as soon as
// its ballot of live lanes is empty.
//
// k_integrate_generic: one thread per neuron, the reference loop nest over
// either the reference bucket layout (drop-in) or the engine's bin layout
// (narrow layers), with the chunk's delta[] in private memory.
#include "common.h"
#include "wave.h"

namespace vdttfs {
namespace {

struct WaveArgs {
    float* out;
    const vd_event* ev;
    const int32_t* off;
    const float* W;
    const float* bias;
    const float* theta;
    unsigned long long* counters;
    int64_t n_units;
    int T, D, t_min;
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad, is_fc;
    int n_cblk, nk_max, pmax;
    int lds_wave_ints, lds_flat_off;
};

struct WaveLds {
    int* kcol;  // [nk_max] column index of each in-bounds receptive column
    int* krow;  // [nk_max] byte offset of its (kh,kw) weight plane
    int* kcum;  // [nk_max+1] exclusive prefix of column run lengths
    int* otab;  // [nk_max][D+1] bin offsets O_k[t0+d]
    int* dtab;  // [nk_max][D] merged-position bases
    int* bst;   // [D+1] bin starts in merged order
    int2* flat; // [pmax] merged events: (weight byte offset, alpha bits)
};

// Merge the events of bins [d0,d1) of the current chunk into lds.flat.
// multi: positions from the table (whole bins); otherwise a single bin whose
// merged order equals the column-major order, windowed to [lo,hi).
__device__ __forceinline__ void fill_flat(const WaveArgs& a, const WaveLds& s, int nk, int t0,
                                          int d0, int d1, int lo, int hi, bool multi,
                                          int rowbytes) {
    const int lane = lane_id();
    const int os = a.D + 1;
    int len = 0;
    if (lane < nk) len = s.otab[lane * os + d1] - s.otab[lane * os + d0];
    const int incl = wave_incl_scan(len);
    if (lane < nk) s.kcum[lane] = incl - len;
    wave_sync();
    const int base = multi ? uniform(s.bst[d0]) : 0;
    for (int f0 = lo; f0 < hi; f0 += 64) {
        const int f = f0 + lane;
        if (f < hi) {
            int k = 0;
            for (int kk = 1; kk < nk; ++kk) k += (s.kcum[kk] <= f) ? 1 : 0;
            const int i = s.otab[k * os + d0] + (f - s.kcum[k]);
            const vd_event e = a.ev[(int64_t)s.kcol[k] * a.C_in + i];
            int pos;
            if (multi) {
                const int br = (int)(e.key >> 24) - t0;
                pos = s.dtab[k * a.D + br] + i - base;
            } else {
                pos = f - lo;
            }
            s.flat[pos] = make_int2(s.krow[k] + (int)(e.key & 0xFFFFFFu) * rowbytes,
                                    __float_as_int(e.alpha));
        }
    }
    wave_sync();
}

// acc = fma-chain over merged events [j0, j1), in order.  Only live lanes
// fetch; the batch of 8 gathers is issued before the first fma.
__device__ __forceinline__ float stream_events(const WaveArgs& a, const int2* flat, int j0,
                                               int j1, float acc, bool live, uint32_t row_lane) {
    if (live) {
        const char* Wb = reinterpret_cast<const char*>(a.W);
        for (int j = j0; j < j1; j += 8) {
            const int n = j1 - j;
            float w[8], al[8];
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const int2 v = flat[j + (g < n ? g : n - 1)];
                al[g] = __int_as_float(v.y);
                w[g] = *reinterpret_cast<const float*>(Wb + ((uint32_t)v.x + row_lane));
            }
#pragma unroll
            for (int g = 0; g < 8; ++g)
                if (g < n) acc = __builtin_fmaf(w[g], al[g], acc);
        }
    }
    return acc;
}

template <bool COUNT>
__global__ __launch_bounds__(256) void k_integrate_wave(WaveArgs a) {
    extern __shared__ int lds_all[];
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t unit = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
    if (unit >= a.n_units) return;  // uniform per wave

    int* L = lds_all + wave * a.lds_wave_ints;
    WaveLds s;
    s.kcol = L;
    s.krow = s.kcol + a.nk_max;
    s.kcum = s.krow + a.nk_max;
    s.otab = s.kcum + a.nk_max + 1;
    s.dtab = s.otab + a.nk_max * (a.D + 1);
    s.bst = s.dtab + a.nk_max * a.D;
    s.flat = reinterpret_cast<int2*>(L + a.lds_flat_off);

    const int cb = (int)(unit % a.n_cblk);
    const int64_t pix = unit / a.n_cblk;
    const int c = cb * 64 + lane;
    const bool lane_ok = c < a.C_out;
    const uint32_t row_lane = (uint32_t)(lane_ok ? c : 0) * 4u;
    const int rowbytes = a.C_out * 4;

    int img, h_out = 0, w_out = 0;
    if (a.is_fc) {
        img = (int)pix;
    } else {
        w_out = (int)(pix % a.W_out);
        const int64_t q = pix / a.W_out;
        h_out = (int)(q % a.H_out);
        img = (int)(q / a.H_out);
    }

    // in-bounds receptive columns in (kh, kw) order
    int nk;
    if (a.is_fc) {
        nk = 1;
        if (lane == 0) {
            s.kcol[0] = img;
            s.krow[0] = 0;
        }
    } else {
        bool v = false;
        int col = 0;
        if (lane < a.K_h * a.K_w) {
            const int kh = lane / a.K_w, kw = lane - kh * a.K_w;
            const int hi = h_out - a.pad + kh, wi = w_out - a.pad + kw;
            v = hi >= 0 && hi < a.H_in && wi >= 0 && wi < a.W_in;
            col = (img * a.H_in + hi) * a.W_in + wi;
        }
        const uint64_t m = __ballot(v);
        nk = __popcll(m);
        if (v) {
            const int slot = __popcll(m & lanemask_lt());
            s.kcol[slot] = col;
            s.krow[slot] = lane * a.C_in * rowbytes;
        }
    }
    wave_sync();

    float carry = lane_ok ? a.bias[c] : 0.0f;
    float res = kInfTime;
    bool live = lane_ok;
    unsigned long long cnt_proc = 0, cnt_bin = 0;
    const int T = a.T, D = a.D;
    const int NC = (T + D - 1) / D;
    const int osb = T + 1;   // offsets per column in the bin layout
    const int os = D + 1;
    bool done = false;

    for (int tau = 0; tau < NC && !done; ++tau) {
        const int t0 = tau * D;
        const int nb = (T - t0) < D ? (T - t0) : D;
        // closed-form merge table: for event i of column k in bin t0+d,
        // merged position = dtab[k][d] + i (relative to the chunk start)
        int S = 0;
        for (int k = 0; k < nk; ++k) {
            const int col = uniform(s.kcol[k]);
            if (lane < nb) S += a.off[(int64_t)col * osb + t0 + lane];
        }
        const int C0 = uniform(S);
        int A = 0, P = 0;
        for (int k = 0; k < nk; ++k) {
            const int col = uniform(s.kcol[k]);
            int o = 0, on = 0;
            if (lane < nb) {
                const int32_t* ob = a.off + (int64_t)col * osb + t0 + lane;
                o = ob[0];
                on = ob[1];
            }
            P += o;
            if (lane < nb) {
                s.dtab[k * D + lane] = A + (S - P) - C0;
                s.otab[k * os + lane] = o;
            }
            if (lane == nb - 1) s.otab[k * os + nb] = on;
            A += on;
        }
        if (lane < nb) s.bst[lane] = S - C0;
        if (lane == nb - 1) s.bst[nb] = A - C0;
        wave_sync();
        const uint64_t live_start = __ballot(live);

        int d = 0;
        while (d < nb && !done) {
            const int sd = uniform(s.bst[d]);
            int d1 = d + 1;
            while (d1 < nb && uniform(s.bst[d1 + 1]) - sd <= a.pmax) ++d1;
            const int n_range = uniform(s.bst[d1]) - sd;
            if (n_range <= a.pmax) {
                fill_flat(a, s, nk, t0, d, d1, 0, n_range, true, rowbytes);
                for (int dd = d; dd < d1; ++dd) {
                    const int j0 = uniform(s.bst[dd]) - sd, j1 = uniform(s.bst[dd + 1]) - sd;
                    const float acc = stream_events(a, s.flat, j0, j1, 0.0f, live, row_lane);
                    if (COUNT) {
                        cnt_bin += (unsigned long long)(j1 - j0) * __popcll(__ballot(live));
                        cnt_proc += (unsigned long long)(j1 - j0) * __popcll(live_start);
                    }
                    carry = carry + acc;
                    const int t = t0 + dd;
                    const float th = a.theta[t];
                    if (t >= a.t_min && th >= 1e-5f && live && carry >= th) {
                        res = (float)t;
                        live = false;
                    }
                    if (!COUNT && __ballot(live) == 0) {
                        done = true;
                        break;
                    }
                }
            } else {
                // one bin larger than the merged list: stream it in windows
                float acc = 0.0f;
                for (int lo = 0; lo < n_range; lo += a.pmax) {
                    const int hi = (n_range - lo) < a.pmax ? n_range : lo + a.pmax;
                    fill_flat(a, s, nk, t0, d, d + 1, lo, hi, false, rowbytes);
                    acc = stream_events(a, s.flat, 0, hi - lo, acc, live, row_lane);
                }
                if (COUNT) {
                    cnt_bin += (unsigned long long)n_range * __popcll(__ballot(live));
                    cnt_proc += (unsigned long long)n_range * __popcll(live_start);
                }
                carry = carry + acc;
                const int t = t0 + d;
                const float th = a.theta[t];
                if (t >= a.t_min && th >= 1e-5f && live && carry >= th) {
                    res = (float)t;
                    live = false;
                }
                if (!COUNT && __ballot(live) == 0) done = true;
                d1 = d + 1;
            }
            d = d1;
        }
        if (COUNT && __ballot(live) == 0) done = true;
    }
    if (lane_ok) a.out[pix * a.C_out + c] = res;
    if (COUNT && lane == 0) {
        atomicAdd(&a.counters[0], cnt_proc);
        atomicAdd(&a.counters[1], cnt_bin);
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
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad, is_fc;
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
                const int h_in = a.is_fc ? 0 : h_out - a.pad + kh;
                if (!a.is_fc && (h_in < 0 || h_in >= a.H_in)) continue;
                for (int kw = 0; kw < kw_n; ++kw) {
                    const int w_in = a.is_fc ? 0 : w_out - a.pad + kw;
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
                    for (int p = s; p < e; ++p) {
                        int cin, tb;
                        float al;
                        if (BINS) {
                            const vd_event ev = a.ev[col * a.C_in + p];
                            cin = (int)(ev.key & 0xFFFFFFu);
                            tb = (int)(ev.key >> 24);
                            al = ev.alpha;
                        } else {
                            cin = a.ref_cin[col * a.C_in + p];
                            const float t_in = a.ref_tin[col * a.C_in + p];
                            tb = (int)floorf(t_in - a.tfs);
                            if (tb < 0) tb = 0;
                            al = a.alpha[alpha_index(t_in, tb, a.alpha_by_time, T)];
                        }
                        const int di = tb - base_t;
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
            atomicAdd(&a.counters[0], my_proc);
            atomicAdd(&a.counters[1], my_bin);
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
        if (s.pad == 0 && (s.H_out + s.K_h - 1 > s.H_in || s.W_out + s.K_w - 1 > s.W_in))
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
    g.pad = (is_fc || !ctx->c.conv_same_pad) ? 0 : K_h / 2;
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
    g.pad = sh.pad;
    g.is_fc = sh.is_fc;
    g.total = (int64_t)sh.B * (sh.is_fc ? 1 : (int64_t)sh.H_out * sh.W_out) * sh.C_out;
    return counters ? launch_generic_d<true, true>(ctx, g) : launch_generic_d<true, false>(ctx, g);
}

int launch_integrate_bins(vdttfs_ctx* ctx, float* out, const vd_event* ev, const int32_t* off,
                          const float* W, const float* bias, const float* theta, int t_min,
                          const IntegShape& sh, unsigned long long* counters) {
    const int T = ctx->c.T, D = ctx->c.delta;
    const int nk_max = sh.is_fc ? 1 : sh.K_h * sh.K_w;
    const int64_t wbytes = (int64_t)nk_max * sh.C_in * sh.C_out * 4;
    const bool wave_ok = sh.C_out >= 32 && D <= 64 && nk_max <= 64 && wbytes < INT64_C(0x7fffffff) &&
                         sh.C_in < (1 << 24);
    if (!wave_ok)
        return launch_integrate_generic_bins(ctx, out, ev, off, W, bias, theta, t_min, sh, counters);
    WaveArgs a{};
    a.out = out;
    a.ev = ev;
    a.off = off;
    a.W = W;
    a.bias = bias;
    a.theta = theta;
    a.counters = counters;
    a.T = T;
    a.D = D;
    a.t_min = t_min;
    a.H_in = sh.H_in;
    a.W_in = sh.W_in;
    a.C_in = sh.C_in;
    a.H_out = sh.H_out;
    a.W_out = sh.W_out;
    a.C_out = sh.C_out;
    a.K_h = sh.K_h;
    a.K_w = sh.K_w;
    a.pad = sh.pad;
    a.is_fc = sh.is_fc;
    a.n_cblk = (sh.C_out + 63) / 64;
    a.nk_max = nk_max;
    a.pmax = 256;
    const int64_t n_pix = (int64_t)sh.B * (sh.is_fc ? 1 : (int64_t)sh.H_out * sh.W_out);
    a.n_units = n_pix * a.n_cblk;
    int ints = nk_max * 2 + (nk_max + 1) + nk_max * (D + 1) + nk_max * D + (D + 1);
    ints = (ints + 1) & ~1;  // 8-byte align the merged list
    a.lds_flat_off = ints;
    a.lds_wave_ints = ints + 2 * a.pmax;
    const int waves = 4;
    const size_t lds = (size_t)a.lds_wave_ints * 4 * waves;
    if (lds > 64 * 1024) {
        // large Delta x receptive field: the per-neuron kernel has no LDS need
            return launch_integrate_generic_bins(ctx, out, ev, off, W, bias, theta, t_min, sh, counters);
    }
    const int64_t blocks = (a.n_units + waves - 1) / waves;
    if (blocks <= 0) return VDTTFS_OK;
    if (blocks > 0x7fffffff) return set_error(VDTTFS_E_UNSUPPORTED, "integrate: grid too large");
    if (counters)
        hipLaunchKernelGGL(k_integrate_wave<true>, dim3((unsigned)blocks), dim3(64 * waves), lds,
                           ctx->stream, a);
    else
        hipLaunchKernelGGL(k_integrate_wave<false>, dim3((unsigned)blocks), dim3(64 * waves), lds,
                           ctx->stream, a);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

}  // namespace vdttfs
