// CuLIF (T3V, config 4): the drop-in entry points over the reference layouts
// and the network engine that runs the T3V main() layer sequence
// (T3V:276-289) as one stream-ordered forward.
//
// Engine layouts (all result-neutral): conv and pool maps are NHWC so that
// a conv layer's input columns are contiguous and its integrator lanes are
// c_out; conv weights are re-laid out OIHW -> HWIO once at creation (one
// weight row per event); an FC layer's input is flattened in the
// reference's NCHW order, because the order of the per-step sums follows
// the input index.  Conv layers run (bucketize ->) merge -> stream with the
// CuLIF neuron and alpha = 1 (fma(w, 1, acc) is the reference's acc + w).
// The recurrent FC layer's feed-forward sums are computed per (sample, step)
// in parallel from its dense input (k_fc_currents) before the per-step
// recurrence.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"

using namespace vdttfs;

namespace {

int dalloc(void** p, size_t bytes) {
    if (hipMalloc(p, bytes ? bytes : 4) != hipSuccess) {
        *p = nullptr;
        return set_error(VDTTFS_E_NOMEM, "device allocation of %zu bytes failed", bytes);
    }
    return VDTTFS_OK;
}

int upload(float** dst, const std::vector<float>& h) {
    VD_TRY(dalloc((void**)dst, h.size() * 4));
    if (!h.empty()) VD_HIP(hipMemcpy(*dst, h.data(), h.size() * 4, hipMemcpyHostToDevice));
    return VDTTFS_OK;
}

struct CLayer {
    vdttfs_culif_layer d{};
    int H_out = 1, W_out = 1;
    float* W = nullptr;     // engine layout
    float* Wrec = nullptr;  // FC_REC: [j][i]
    float* out = nullptr;
    int64_t out_elems = 0;  // per batch
    int nhwc = 0;           // output layout
    int64_t list_cap = 0;   // CONV: merged-list entries per pixel
};

}  // namespace

struct vdttfs_culif_net {
    vdttfs_ctx* ctx = nullptr;
    int B = 0;
    std::vector<CLayer> L;
    float* ones = nullptr;     // alpha = 1 for T+1 bins
    vd_event* ev = nullptr;    // bin-layout events
    int32_t* off = nullptr;    // bin offsets
    int2* list = nullptr;      // merged lists
    int32_t* bstart = nullptr;
    int32_t* rcin = nullptr;   // reference-layout buckets (small FC)
    float* rtin = nullptr;
    int32_t* roff = nullptr;
    float* flat = nullptr;     // NCHW flatten of a spatial map before an FC
    float* cur = nullptr;      // FC_REC feed-forward currents [B][T][out]
    FcSortScratch fcs{};           // FC_REC inputs sorted by arrival step
    uint64_t* raw_mask = nullptr;  // conv1_raw event masks (finite weights, C_in <= 4)
    uint32_t* raw_nonbin = nullptr;
    uint8_t* raw_fired = nullptr;  // per conv1 output pixel: some neuron fired (mask kernel, C_out <= 64)
    bool timing = false;
    std::vector<hipEvent_t> pool;      // 2 per layer per timed forward
    size_t pool_used = 0;
    std::vector<int> pending_layer;    // layer of each recorded pair
    int64_t forwards = 0;
};

namespace {

void destroy_impl(vdttfs_culif_net* net) {
    if (!net) return;
    if (net->ctx) {
        (void)hipSetDevice(net->ctx->device);
        (void)hipStreamSynchronize(net->ctx->stream);
    }
    for (hipEvent_t e : net->pool) (void)hipEventDestroy(e);
    for (CLayer& l : net->L)
        for (float* q : {l.W, l.Wrec, l.out})
            if (q) (void)hipFree(q);
    for (void* q : {(void*)net->ones, (void*)net->ev, (void*)net->off, (void*)net->list,
                    (void*)net->bstart, (void*)net->rcin, (void*)net->rtin, (void*)net->roff,
                    (void*)net->flat, (void*)net->cur, (void*)net->raw_mask, (void*)net->raw_nonbin, (void*)net->raw_fired,
                    (void*)net->fcs.counts, (void*)net->fcs.offs, (void*)net->fcs.binstart, (void*)net->fcs.list})
        if (q) (void)hipFree(q);
    delete net;
}

int validate(const vdttfs_ctx* ctx, const vdttfs_culif_layer* layers, int n) {
    if (!layers || n <= 0) return set_error(VDTTFS_E_INVALID, "culif net: no layers");
    if (ctx->c.tfs != 0.0f)
        return set_error(VDTTFS_E_INVALID, "culif net: the context's tfs must be 0 (T3V has no fire start)");
    if (layers[0].kind != VDTTFS_CULIF_RAW_CONV)
        return set_error(VDTTFS_E_INVALID, "culif net: layer 0 must be RAW_CONV (the dense event input)");
    int C = 0, H = 0, W = 0;
    for (int i = 0; i < n; ++i) {
        const vdttfs_culif_layer& d = layers[i];
        const bool fc = d.kind == VDTTFS_CULIF_FC || d.kind == VDTTFS_CULIF_FC_REC;
        if (d.kind < VDTTFS_CULIF_RAW_CONV || d.kind > VDTTFS_CULIF_FC)
            return set_error(VDTTFS_E_INVALID, "culif net: layer %d kind %d", i, d.kind);
        if (i > 0 && d.kind == VDTTFS_CULIF_RAW_CONV)
            return set_error(VDTTFS_E_INVALID, "culif net: RAW_CONV only as layer 0");
        if (d.C_in <= 0 || d.C_out <= 0 || (!fc && (d.H_in <= 0 || d.W_in <= 0)))
            return set_error(VDTTFS_E_INVALID, "culif net: layer %d has a non-positive shape", i);
        if (i > 0) {
            if (fc) {
                if ((int64_t)d.C_in != (int64_t)C * H * W)
                    return set_error(VDTTFS_E_INVALID, "culif net: layer %d takes %d features, previous gives %lld",
                                     i, d.C_in, (long long)C * H * W);
            } else if (d.C_in != C || d.H_in != H || d.W_in != W) {
                return set_error(VDTTFS_E_INVALID, "culif net: layer %d input shape does not match layer %d", i, i - 1);
            }
        }
        if (d.kind == VDTTFS_CULIF_POOL) {
            if (d.C_out != d.C_in || d.H_in < 2 || d.W_in < 2)
                return set_error(VDTTFS_E_INVALID, "culif net: pool layer %d", i);
        } else if (!d.weight) {
            return set_error(VDTTFS_E_INVALID, "culif net: layer %d has no weights", i);
        }
        if (d.kind == VDTTFS_CULIF_FC_REC && (!d.weight_rec || d.C_out > 1024))
            return set_error(VDTTFS_E_INVALID, "culif net: FC_REC layer %d needs weight_rec and <= 1024 outputs", i);
        if (d.kind == VDTTFS_CULIF_CONV && d.C_in >= (1 << 24))
            return set_error(VDTTFS_E_UNSUPPORTED, "culif net: conv layer %d needs C_in < 2^24", i);
        if (fc) {
            C = d.C_out;
            H = W = 1;
        } else if (d.kind == VDTTFS_CULIF_POOL) {
            C = d.C_out;
            H = d.H_in / 2;
            W = d.W_in / 2;
        } else {
            C = d.C_out;
            H = d.H_in;
            W = d.W_in;
        }
    }
    return VDTTFS_OK;
}

int create_impl(vdttfs_culif_net* net, const vdttfs_culif_layer* layers, int n) {
    vdttfs_ctx* ctx = net->ctx;
    const int T = ctx->c.T, B = net->B;
    std::vector<float> ones(T + 1, 1.0f);
    VD_TRY(upload(&net->ones, ones));
    int64_t max_ev = 1, max_cols = 1, max_list = 1, max_bstart = 1, max_flat = 1, max_cur = 1;
    int64_t max_fc_counts = 1, max_fc_binstart = 1, max_fc_list = 1;
    int64_t max_rsites = 1, max_relems = 1;
    net->L.resize(n);
    for (int i = 0; i < n; ++i) {
        CLayer& l = net->L[i];
        l.d = layers[i];
        const vdttfs_culif_layer& d = layers[i];
        l.d.weight = nullptr;
        l.d.weight_rec = nullptr;
        const bool spatial_in = i > 0 && (net->L[i - 1].H_out > 1 || net->L[i - 1].W_out > 1);
        switch (d.kind) {
            case VDTTFS_CULIF_RAW_CONV: {
                l.H_out = d.H_in;
                l.W_out = d.W_in;
                l.nhwc = 1;
                std::vector<float> w(d.weight, d.weight + (size_t)d.C_out * d.C_in * 9);
                VD_TRY(upload(&l.W, w));
                // integrating from event masks skips zero inputs, exact only
                // when w * 0 == 0 for every weight
                bool finite = true;
                for (float v : w) finite = finite && std::isfinite(v);
                if (finite && culif_conv1_mask_ok(d.C_in)) {
                    const size_t units = (size_t)B * d.C_in * d.H_in * d.W_in * ((T + 63) / 64);
                    VD_TRY(dalloc((void**)&net->raw_mask, units * sizeof(uint64_t)));
                    VD_TRY(dalloc((void**)&net->raw_nonbin, units * sizeof(uint32_t)));
                    if (d.C_out <= 64)
                        VD_TRY(dalloc((void**)&net->raw_fired, (size_t)B * d.H_in * d.W_in));
                }
                break;
            }
            case VDTTFS_CULIF_CONV: {
                l.H_out = d.H_in;
                l.W_out = d.W_in;
                l.nhwc = 1;
                // OIHW -> HWIO: row (k, cin) holds the C_out weights of one event
                std::vector<float> w((size_t)9 * d.C_in * d.C_out);
                for (int o = 0; o < d.C_out; ++o)
                    for (int ci = 0; ci < d.C_in; ++ci)
                        for (int k = 0; k < 9; ++k)
                            w[((size_t)k * d.C_in + ci) * d.C_out + o] =
                                d.weight[((size_t)o * d.C_in + ci) * 9 + k];
                VD_TRY(upload(&l.W, w));
                const int64_t cols = (int64_t)B * d.H_in * d.W_in;
                const int64_t n_pix = cols;
                IntegShape sh{B, d.H_in, d.W_in, d.C_in, d.H_in, d.W_in, d.C_out, 3, 3,
                              /*pad_h=*/1, /*pad_w=*/1, /*is_fc=*/0};
                l.list_cap = merged_list_cap(sh);
                if (cols * d.C_in > max_ev) max_ev = cols * d.C_in;
                if (cols > max_cols) max_cols = cols;
                if (n_pix * l.list_cap > max_list) max_list = n_pix * l.list_cap;
                if (n_pix * (T + 1) > max_bstart) max_bstart = n_pix * (T + 1);
                break;
            }
            case VDTTFS_CULIF_POOL:
                l.H_out = d.H_in / 2;
                l.W_out = d.W_in / 2;
                l.nhwc = 1;
                break;
            case VDTTFS_CULIF_FC_REC: {
                // [out][in] -> [in][out] and W_rec [i][j] -> [j][i]
                std::vector<float> w((size_t)d.C_in * d.C_out), r((size_t)d.C_out * d.C_out);
                for (int o = 0; o < d.C_out; ++o)
                    for (int j = 0; j < d.C_in; ++j) w[(size_t)j * d.C_out + o] = d.weight[(size_t)o * d.C_in + j];
                for (int a = 0; a < d.C_out; ++a)
                    for (int b = 0; b < d.C_out; ++b)
                        r[(size_t)b * d.C_out + a] = d.weight_rec[(size_t)a * d.C_out + b];
                VD_TRY(upload(&l.W, w));
                VD_TRY(upload(&l.Wrec, r));
                if ((int64_t)B * T * d.C_out > max_cur) max_cur = (int64_t)B * T * d.C_out;
                if (spatial_in && (int64_t)B * d.C_in > max_flat) max_flat = (int64_t)B * d.C_in;
                const FcSortSizes z = fc_sort_sizes(B, d.C_in, T);
                max_fc_counts = std::max(max_fc_counts, z.counts);
                max_fc_binstart = std::max(max_fc_binstart, z.binstart);
                max_fc_list = std::max(max_fc_list, z.list);
                break;
            }
            case VDTTFS_CULIF_FC: {
                std::vector<float> w(d.weight, d.weight + (size_t)d.C_out * d.C_in);
                VD_TRY(upload(&l.W, w));
                if (B > max_rsites) max_rsites = B;
                if ((int64_t)B * d.C_in > max_relems) max_relems = (int64_t)B * d.C_in;
                if (spatial_in && (int64_t)B * d.C_in > max_flat) max_flat = (int64_t)B * d.C_in;
                break;
            }
        }
        l.out_elems = (int64_t)B * l.H_out * l.W_out * d.C_out;
        VD_TRY(dalloc((void**)&l.out, (size_t)l.out_elems * 4));
    }
    const int OS = T / ctx->c.delta + 1;
    VD_TRY(dalloc((void**)&net->ev, (size_t)max_ev * sizeof(vd_event)));
    VD_TRY(dalloc((void**)&net->off, (size_t)max_cols * (T + 1) * 4));
    VD_TRY(dalloc((void**)&net->list, (size_t)max_list * sizeof(int2)));
    VD_TRY(dalloc((void**)&net->bstart, (size_t)max_bstart * 4));
    VD_TRY(dalloc((void**)&net->rcin, (size_t)max_relems * 4));
    VD_TRY(dalloc((void**)&net->rtin, (size_t)max_relems * 4));
    VD_TRY(dalloc((void**)&net->roff, (size_t)max_rsites * OS * 4));
    VD_TRY(dalloc((void**)&net->flat, (size_t)max_flat * 4));
    VD_TRY(dalloc((void**)&net->cur, (size_t)max_cur * 4));
    VD_TRY(dalloc((void**)&net->fcs.counts, (size_t)max_fc_counts * 4));
    VD_TRY(dalloc((void**)&net->fcs.offs, (size_t)max_fc_counts * 4));
    VD_TRY(dalloc((void**)&net->fcs.binstart, (size_t)max_fc_binstart * 4));
    VD_TRY(dalloc((void**)&net->fcs.list, (size_t)max_fc_list * 4));
    return VDTTFS_OK;
}

int mark(vdttfs_culif_net* net, hipEvent_t* e) {
    if (net->pool_used == net->pool.size()) {
        hipEvent_t ev;
        VD_HIP(hipEventCreate(&ev));
        net->pool.push_back(ev);
    }
    *e = net->pool[net->pool_used++];
    VD_HIP(hipEventRecord(*e, net->ctx->stream));
    return VDTTFS_OK;
}

// counts: nullable [4][n_layers] (eproc, ebin, n_ev, n_cols) for an
// instrumented forward; counting and timing are exclusive.
int forward_impl(vdttfs_culif_net* net, const float* d_data, int32_t* d_pred, uint64_t* const* counts) {
    vdttfs_ctx* ctx = net->ctx;
    const int B = net->B;
    const float* cur = nullptr;
    const uint8_t* cur_fired = nullptr;  // per-site flags of `cur` (conv1's mask kernel), or null
    int cur_nhwc = 0, cH = 1, cW = 1, cC = 0;
    const bool timed = net->timing && !counts;
    for (size_t i = 0; i < net->L.size(); ++i) {
        CLayer& l = net->L[i];
        const vdttfs_culif_layer& d = l.d;
        CulifNeuron nrn{d.decay, d.th, d.kind == VDTTFS_CULIF_CONV ? cur_fired : nullptr};
        hipEvent_t e0 = nullptr, e1 = nullptr;  // consecutive pool slots 2k, 2k+1
        if (timed) VD_TRY(mark(net, &e0));
        const bool count_here = counts && d.kind == VDTTFS_CULIF_CONV;
        if (counts)
            for (int k = 0; k < 4; ++k) counts[k][i] = 0;
        if (count_here)
            VD_TRY(zero_counters(ctx));
        // an FC layer reads the previous map flattened in NCHW order
        const float* fc_in = cur;
        if ((d.kind == VDTTFS_CULIF_FC || d.kind == VDTTFS_CULIF_FC_REC) && cur_nhwc && (cH > 1 || cW > 1)) {
            VD_TRY(launch_nhwc_to_nchw(ctx, cur, net->flat, B, cC, cH, cW));
            fc_in = net->flat;
        }
        switch (d.kind) {
            case VDTTFS_CULIF_RAW_CONV:
                if (net->raw_mask)
                    VD_TRY(launch_culif_conv1_mask(ctx, d_data, l.out, l.W, B, d.C_in, d.C_out, d.H_in,
                                                   d.W_in, 1, d.decay, d.th, net->raw_mask, net->raw_nonbin,
                                                   net->raw_fired));
                else
                    VD_TRY(launch_culif_conv1_raw(ctx, d_data, l.out, l.W, B, d.C_in, d.C_out, d.H_in,
                                                  d.W_in, 1, d.decay, d.th));
                break;
            case VDTTFS_CULIF_CONV: {
                const int64_t cols = (int64_t)B * d.H_in * d.W_in;
                IntegShape sh{B, d.H_in, d.W_in, d.C_in, d.H_in, d.W_in, d.C_out, 3, 3,
                              /*pad_h=*/1, /*pad_w=*/1, /*is_fc=*/0};
                // inputs up to C_in 64, and outside counting forwards up to 128
                // (the fused list build), build the merged lists from the dense
                // map (the bin-layout bucketize then only counts retained events)
                LaunchPlan plan;
                VD_TRY(resolve_plan(ctx, sh, LaunchPlan{}, &plan));
                const bool dense = plan_from_dense(ctx, sh, plan, count_here);
                if (!dense || count_here)
                    VD_TRY(launch_bucketize_bins(ctx, cur, cols, d.C_in, net->ones, net->ev, net->off,
                                                 count_here ? ctx->d_counters + 2 : nullptr));
                if (dense)
                    VD_TRY(launch_integrate_dense(ctx, l.out, cur, net->ones, net->list, l.list_cap,
                                                  net->bstart, l.W, nullptr, nullptr, 0, sh,
                                                  count_here ? ctx->d_counters : nullptr, &nrn));
                else
                    VD_TRY(launch_integrate_bins(ctx, l.out, net->ev, net->off, net->list, l.list_cap,
                                                 net->bstart, l.W, nullptr, nullptr, 0, sh,
                                                 count_here ? ctx->d_counters : nullptr, &nrn));
                if (count_here) {
                    unsigned long long h[4];
                    VD_TRY(read_counters(ctx, h));
                    counts[0][i] = h[0];
                    counts[1][i] = h[1];
                    counts[2][i] = h[2];
                    counts[3][i] = (uint64_t)cols;
                }
                break;
            }
            case VDTTFS_CULIF_POOL:
                VD_TRY(launch_culif_pool(ctx, cur, l.out, B, d.C_in, d.H_in, d.W_in, cur_nhwc, 1, d.decay,
                                         d.th));
                break;
            case VDTTFS_CULIF_FC_REC:
                VD_TRY(launch_fc_currents(ctx, fc_in, l.W, net->cur, B, d.C_in, d.C_out, net->fcs));
                VD_TRY(launch_culif_fc_rec(ctx, nullptr, nullptr, nullptr, net->cur, l.out, nullptr, l.Wrec, B,
                                           d.C_in, d.C_out, d.decay, d.th));
                break;
            case VDTTFS_CULIF_FC:
                VD_TRY(launch_culif_bucketize(ctx, fc_in, B, d.C_in, 1, net->rcin, net->rtin, net->roff));
                VD_TRY(launch_culif_generic(ctx, net->rcin, net->rtin, net->roff, l.out, l.W, B, d.C_in,
                                            d.C_out, 1, 1, 1, d.decay, d.th));
                break;
        }
        if (timed) {
            VD_TRY(mark(net, &e1));
            net->pending_layer.push_back((int)i);
        }
        cur = l.out;
        cur_fired = (d.kind == VDTTFS_CULIF_RAW_CONV && net->raw_mask) ? net->raw_fired : nullptr;
        cur_nhwc = l.nhwc;
        cH = l.H_out;
        cW = l.W_out;
        cC = d.C_out;
    }
    if (d_pred) {
        const CLayer& last = net->L.back();
        VD_TRY(launch_readout(ctx, last.out, B, (int)(last.out_elems / B), d_pred, 2));
    }
    return VDTTFS_OK;
}

}  // namespace

namespace vdttfs {
int validate_culif_table(const vdttfs_ctx* ctx, const vdttfs_culif_layer* layers, int n) {
    return validate(ctx, layers, n);
}
}  // namespace vdttfs

extern "C" {

// ---- drop-in entry points (reference layouts) ----------------------------

int vdttfs_culif_conv1_raw(vdttfs_ctx* ctx, const float* d_data, float* d_out, const float* d_weight,
                           int N, int C_in, int C_out, int H, int W, float decay, float th) {
    VD_TRY(check_ctx(ctx));
    if (!d_data || !d_out || !d_weight) return set_error(VDTTFS_E_INVALID, "culif_conv1_raw: null buffer");
    return launch_culif_conv1_raw(ctx, d_data, d_out, d_weight, N, C_in, C_out, H, W, 0, decay, th);
}

int vdttfs_culif_bucketize_conv(vdttfs_ctx* ctx, const float* d_in, int N, int C, int H, int W,
                                int32_t* d_out_cin, float* d_out_tin, int32_t* d_out_off) {
    VD_TRY(check_ctx(ctx));
    if (!d_in || !d_out_cin || !d_out_tin || !d_out_off)
        return set_error(VDTTFS_E_INVALID, "culif_bucketize_conv: null buffer");
    if (N <= 0 || H <= 0 || W <= 0) return set_error(VDTTFS_E_INVALID, "culif_bucketize_conv: bad shape");
    return launch_culif_bucketize(ctx, d_in, (int64_t)N * H * W, C, H * W, d_out_cin, d_out_tin, d_out_off);
}

int vdttfs_culif_bucketize_fc(vdttfs_ctx* ctx, const float* d_in, int N, int F, int32_t* d_out_cin,
                              float* d_out_tin, int32_t* d_out_off) {
    VD_TRY(check_ctx(ctx));
    if (!d_in || !d_out_cin || !d_out_tin || !d_out_off)
        return set_error(VDTTFS_E_INVALID, "culif_bucketize_fc: null buffer");
    return launch_culif_bucketize(ctx, d_in, N, F, 1, d_out_cin, d_out_tin, d_out_off);
}

int vdttfs_culif_conv(vdttfs_ctx* ctx, const int32_t* d_bcin, const float* d_btin, const int32_t* d_boff,
                      float* d_out, const float* d_weight, int N, int C_in, int C_out, int H, int W,
                      float decay, float th) {
    VD_TRY(check_ctx(ctx));
    if (!d_bcin || !d_btin || !d_boff || !d_out || !d_weight)
        return set_error(VDTTFS_E_INVALID, "culif_conv: null buffer");
    if (N <= 0 || C_in <= 0 || C_out <= 0 || H <= 0 || W <= 0)
        return set_error(VDTTFS_E_INVALID, "culif_conv: bad shape");
    return launch_culif_generic(ctx, d_bcin, d_btin, d_boff, d_out, d_weight, N, C_in, C_out, H, W, 0,
                                decay, th);
}

int vdttfs_culif_pool(vdttfs_ctx* ctx, const float* d_in, float* d_out, int N, int C, int H_in,
                      int W_in, float decay, float th) {
    VD_TRY(check_ctx(ctx));
    if (!d_in || !d_out) return set_error(VDTTFS_E_INVALID, "culif_pool: null buffer");
    return launch_culif_pool(ctx, d_in, d_out, N, C, H_in, W_in, 0, 0, decay, th);
}

int vdttfs_culif_fc_recurrent(vdttfs_ctx* ctx, const int32_t* d_bcin, const float* d_btin,
                              const int32_t* d_boff, float* d_out, const float* d_w,
                              const float* d_w_rec, int N, int in_f, int out_f, float decay, float th) {
    VD_TRY(check_ctx(ctx));
    if (!d_bcin || !d_btin || !d_boff || !d_out || !d_w || !d_w_rec)
        return set_error(VDTTFS_E_INVALID, "culif_fc_recurrent: null buffer");
    return launch_culif_fc_rec(ctx, d_bcin, d_btin, d_boff, nullptr, d_out, d_w, d_w_rec, N, in_f, out_f,
                               decay, th);
}

int vdttfs_culif_fc(vdttfs_ctx* ctx, const int32_t* d_bcin, const float* d_btin, const int32_t* d_boff,
                    float* d_out, const float* d_w, int N, int in_f, int out_f, float decay, float th) {
    VD_TRY(check_ctx(ctx));
    if (!d_bcin || !d_btin || !d_boff || !d_out || !d_w)
        return set_error(VDTTFS_E_INVALID, "culif_fc: null buffer");
    if (N <= 0 || in_f <= 0 || out_f <= 0) return set_error(VDTTFS_E_INVALID, "culif_fc: bad shape");
    return launch_culif_generic(ctx, d_bcin, d_btin, d_boff, d_out, d_w, N, in_f, out_f, 1, 1, 1, decay, th);
}

int vdttfs_readout_argmin_first(vdttfs_ctx* ctx, const float* d_out, int B, int C, int32_t* d_pred) {
    VD_TRY(check_ctx(ctx));
    if (B < 0 || C <= 0) return set_error(VDTTFS_E_INVALID, "readout: bad sizes");
    return launch_readout(ctx, d_out, B, C, d_pred, 2);
}

// ---- engine ---------------------------------------------------------------

int vdttfs_culif_net_create(vdttfs_ctx* ctx, const vdttfs_culif_layer* layers, int n_layers, int B,
                            vdttfs_culif_net** out) {
    VD_TRY(check_ctx(ctx));
    if (!out) return set_error(VDTTFS_E_INVALID, "culif_net_create: null out");
    *out = nullptr;
    if (B <= 0) return set_error(VDTTFS_E_INVALID, "culif_net_create: B = %d", B);
    VD_TRY(check_culif_consts(ctx));
    VD_TRY(validate(ctx, layers, n_layers));
    vdttfs_culif_net* net = new (std::nothrow) vdttfs_culif_net();
    if (!net) return set_error(VDTTFS_E_NOMEM, "culif_net_create: host allocation");
    net->ctx = ctx;
    net->B = B;
    const int rc = create_impl(net, layers, n_layers);
    if (rc != VDTTFS_OK) {
        destroy_impl(net);
        return rc;
    }
    *out = net;
    return VDTTFS_OK;
}

int vdttfs_culif_net_destroy(vdttfs_culif_net* net) {
    destroy_impl(net);
    return VDTTFS_OK;
}

int vdttfs_culif_net_forward(vdttfs_culif_net* net, const float* d_data, int32_t* d_pred) {
    if (!net || !d_data) return set_error(VDTTFS_E_INVALID, "culif_net_forward: null argument");
    VD_TRY(check_ctx(net->ctx));
    VD_TRY(forward_impl(net, d_data, d_pred, nullptr));
    if (net->timing) net->forwards += 1;
    return VDTTFS_OK;
}

int vdttfs_culif_net_set_timing(vdttfs_culif_net* net, int enable) {
    if (!net) return set_error(VDTTFS_E_INVALID, "null net");
    net->timing = enable != 0;
    return VDTTFS_OK;
}

int vdttfs_culif_net_read_timing(vdttfs_culif_net* net, double* ms, int64_t* forwards) {
    if (!net) return set_error(VDTTFS_E_INVALID, "null net");
    VD_TRY(check_ctx(net->ctx));
    VD_HIP(hipStreamSynchronize(net->ctx->stream));
    std::vector<double> acc(net->L.size(), 0.0);
    for (size_t k = 0; k < net->pending_layer.size(); ++k) {
        float f = 0.0f;
        VD_HIP(hipEventElapsedTime(&f, net->pool[2 * k], net->pool[2 * k + 1]));
        acc[net->pending_layer[k]] += f;
    }
    if (ms)
        for (size_t i = 0; i < acc.size(); ++i) ms[i] = acc[i];
    if (forwards) *forwards = net->forwards;
    net->pending_layer.clear();
    net->pool_used = 0;
    net->forwards = 0;
    return VDTTFS_OK;
}

int vdttfs_culif_net_count(vdttfs_culif_net* net, const float* d_data, uint64_t* eproc, uint64_t* ebin,
                           uint64_t* n_ev, uint64_t* n_cols) {
    if (!net || !d_data) return set_error(VDTTFS_E_INVALID, "culif_net_count: null argument");
    VD_TRY(check_ctx(net->ctx));
    const size_t n = net->L.size();
    std::vector<uint64_t> a(n), b(n), c(n), d(n);
    uint64_t* counts[4] = {a.data(), b.data(), c.data(), d.data()};
    VD_TRY(forward_impl(net, d_data, nullptr, counts));
    VD_HIP(hipStreamSynchronize(net->ctx->stream));
    for (size_t i = 0; i < n; ++i) {
        if (eproc) eproc[i] = a[i];
        if (ebin) ebin[i] = b[i];
        if (n_ev) n_ev[i] = c[i];
        if (n_cols) n_cols[i] = d[i];
    }
    return VDTTFS_OK;
}

int vdttfs_culif_net_layer_output(vdttfs_culif_net* net, int layer, const float** d_out, int64_t* elems,
                                  int32_t* nhwc) {
    if (!net || layer < 0 || layer >= (int)net->L.size())
        return set_error(VDTTFS_E_INVALID, "culif_net_layer_output: bad layer");
    if (d_out) *d_out = net->L[layer].out;
    if (elems) *elems = net->L[layer].out_elems;
    if (nhwc) *nhwc = net->L[layer].nhwc;
    return VDTTFS_OK;
}

}  // extern "C"
