// Network engine: the sequencing of the reference driver main()s
// (T1V:286-319, T2V:337-396) as one stream-ordered forward with no host
// synchronisation.  Differences from the reference drivers, all
// result-neutral: weights, biases and every layer's LUTs are uploaded once at
// creation and stay resident (update_LUTs per layer per batch becomes a
// pointer switch); each layer has its own output map; bucket scratch is
// pre-sized here, so forward() allocates nothing.
#include <cmath>
#include <cstdlib>
#include <new>
#include <vector>

#include "common.h"

using namespace vdttfs;

namespace {

struct NetLayer {
    vdttfs_layer_desc d{};
    float* W = nullptr;
    float* bias = nullptr;
    float* alpha = nullptr;
    float* theta = nullptr;
    float* out = nullptr;
    int64_t out_elems = 0;
    int64_t cols = 0;  // bucket columns (CONV/FC)
    int cin_col = 0;   // elements per column
    int64_t list_cap = 0;  // merged-list entries per output pixel
    int t_min = 0;
    int window = 0;  // integration window T'_l; 0 = the context's T
    LaunchPlan plan;  // requested launch plan; zero fields = built-in choice
    // POOL: the last forward ran this pool inside the next layer's list
    // build, so `out` is written only when asked for (from pool_src)
    bool fused = false;
    const float* pool_src = nullptr;
};

struct TimedPair {
    hipEvent_t a, b;
    int kind;  // 0 integrate, 1 bucketize
    int layer;
};

// A forward captured into a HIP graph for one (input, prediction) pair of
// pointers under one configuration of the network (`gen`), with the host-side
// state the capture left: which pools it fused, and from which maps.
struct GraphEntry {
    const float* img = nullptr;
    int32_t* pred = nullptr;
    unsigned gen = 0;
    hipGraphExec_t exec = nullptr;
    std::vector<unsigned char> fused;
    std::vector<const float*> pool_src;
};
constexpr size_t kMaxGraphs = 4;  // (input, prediction) pairs kept per network

}  // namespace

struct vdttfs_net {
    vdttfs_ctx* ctx = nullptr;
    std::vector<NetLayer> L;
    int B = 0;
    int64_t img_elems = 0;
    int encode_mode = 0;
    float tc_in = 0, td_in = 0;
    int readout = 0;
    float* enc = nullptr;
    vd_event* ev = nullptr;
    int32_t* off = nullptr;
    int2* list = nullptr;
    int32_t* bstart = nullptr;
    bool timing = false;
    int pool_fusion = VDTTFS_POOL_FUSE_OFF;  // which 2x2 pools run inside the next layer's list build
    bool graphs_on = false;  // forwards replay captured HIP graphs
    unsigned gen = 0;        // configuration generation: plans, windows, pool fusion
    std::vector<GraphEntry> graphs;
    std::vector<hipEvent_t> pool;
    size_t pool_used = 0;
    std::vector<TimedPair> pending;
    double ms[2] = {0, 0};
    int64_t launches[2] = {0, 0};
    std::vector<double> layer_ms;
};

namespace {

int fail_layer(int i, const char* what) {
    return set_error(VDTTFS_E_INVALID, "net layer %d: %s", i, what);
}

int validate(const vdttfs_consts& c, const vdttfs_layer_desc* ls, int n, int64_t img_elems) {
    int64_t prev_elems = img_elems;
    int ph = -1, pw = -1, pc = -1;  // previous spatial shape, -1 if flattened
    for (int i = 0; i < n; ++i) {
        const vdttfs_layer_desc& d = ls[i];
        const int64_t in_e = (int64_t)d.H_in * d.W_in * d.C_in;
        if (d.H_in <= 0 || d.W_in <= 0 || d.C_in <= 0 || d.H_out <= 0 || d.W_out <= 0 || d.C_out <= 0)
            return fail_layer(i, "non-positive dimension");
        if (in_e != prev_elems) return fail_layer(i, "input size does not match the previous output");
        if (d.kind == VDTTFS_LAYER_CONV) {
            if (ph >= 0 && (d.H_in != ph || d.W_in != pw || d.C_in != pc))
                return fail_layer(i, "conv input shape does not match the previous map");
            if (d.K_h <= 0 || d.K_w <= 0) return fail_layer(i, "kernel size");
            if (c.conv_same_pad) {
                if (d.H_out != d.H_in || d.W_out != d.W_in || d.K_h % 2 == 0 || d.K_w % 2 == 0)
                    return fail_layer(i, "same-pad conv needs odd K and H_out == H_in");
            } else if (d.H_out != d.H_in - d.K_h + 1 || d.W_out != d.W_in - d.K_w + 1) {
                return fail_layer(i, "valid conv needs H_out = H_in - K_h + 1");
            }
            if (!d.kernel || !d.bias) return fail_layer(i, "null weights");
        } else if (d.kind == VDTTFS_LAYER_FC || d.kind == VDTTFS_LAYER_VMEM) {
            if (d.H_out != 1 || d.W_out != 1) return fail_layer(i, "fc output must be 1x1xC");
            if (!d.kernel || !d.bias) return fail_layer(i, "null weights");
        } else if (d.kind == VDTTFS_LAYER_POOL) {
            if (d.H_out != d.H_in / 2 || d.W_out != d.W_in / 2 || d.C_out != d.C_in)
                return fail_layer(i, "pool needs H_out = H_in/2, C_out = C_in");
        } else {
            return fail_layer(i, "unknown layer kind");
        }
        prev_elems = (int64_t)d.H_out * d.W_out * d.C_out;
        if (d.kind == VDTTFS_LAYER_FC || d.kind == VDTTFS_LAYER_VMEM) {
            ph = pw = pc = -1;
        } else {
            ph = d.H_out;
            pw = d.W_out;
            pc = d.C_out;
        }
    }
    return VDTTFS_OK;
}

hipEvent_t take_event(vdttfs_net* net) {
    if (net->pool_used == net->pool.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        net->pool.push_back(e);
    }
    return net->pool[net->pool_used++];
}

int mark(vdttfs_net* net, hipEvent_t* e) {
    *e = take_event(net);
    if (!*e) return set_error(VDTTFS_E_HIP, "hipEventCreate failed");
    VD_HIP(hipEventRecord(*e, net->ctx->stream));
    return VDTTFS_OK;
}

// Integrator shape of a CONV or FC layer (FC: one column of H*W*C inputs).
IntegShape integ_shape(const vdttfs_net* net, const NetLayer& l) {
    const vdttfs_layer_desc& d = l.d;
    const bool fc = d.kind == VDTTFS_LAYER_FC;
    IntegShape s{};
    s.B = net->B;
    s.is_fc = fc;
    s.H_in = fc ? 1 : d.H_in;
    s.W_in = fc ? 1 : d.W_in;
    s.C_in = l.cin_col;
    s.H_out = fc ? 1 : d.H_out;
    s.W_out = fc ? 1 : d.W_out;
    s.C_out = d.C_out;
    s.K_h = fc ? 1 : d.K_h;
    s.K_w = fc ? 1 : d.K_w;
    const bool same = !fc && net->ctx->c.conv_same_pad;  // T2V:109-110
    s.pad_h = same ? d.K_h / 2 : 0;
    s.pad_w = same ? d.K_w / 2 : 0;
    return s;
}

// Narrows the context's integration window to T' for one layer's launches
// and restores it on exit.  The launchers read the window from the context,
// and the LUT entries they index under T' (alpha[0..T'], theta[0..T'-1]) are
// functions of t alone, so the layer's full-window LUTs serve unchanged.
class WindowScope {
  public:
    WindowScope(vdttfs_ctx* ctx, int window) : ctx_(ctx), T_(ctx->c.T), NC_(ctx->NC), OS_(ctx->OS) {
        if (window > 0 && window < T_) {
            ctx->c.T = window;
            ctx->NC = (window + ctx->c.delta - 1) / ctx->c.delta;
            ctx->OS = ctx->NC + 1;
        }
    }
    ~WindowScope() {
        ctx_->c.T = T_;
        ctx_->NC = NC_;
        ctx_->OS = OS_;
    }
    WindowScope(const WindowScope&) = delete;
    WindowScope& operator=(const WindowScope&) = delete;

  private:
    vdttfs_ctx* ctx_;
    int T_, NC_, OS_;
};

// counters: nullable; when set, per-layer instrumented run
int forward_impl(vdttfs_net* net, const float* d_img, int32_t* d_pred, uint64_t* eproc,
                 uint64_t* ebin, uint64_t* n_ev, uint64_t* n_cols) {
    vdttfs_ctx* ctx = net->ctx;
    const bool count = eproc || ebin || n_ev;
    const int64_t n_img = (int64_t)net->B * net->img_elems;
    const float* cur = net->enc;
    if (net->encode_mode == VDTTFS_ENCODE_LOG)
        VD_TRY(launch_encode_log(ctx, d_img, net->enc, n_img, net->tc_in, net->td_in));
    else if (net->encode_mode == VDTTFS_ENCODE_LINEAR)
        VD_TRY(launch_encode_linear(ctx, d_img, net->enc, n_img));
    else
        cur = d_img;  // VDTTFS_ENCODE_TIMES: the input already holds spike times
    // a pool whose launch waits for the next layer: that layer's list build
    // takes it where it can (pool fusion), else it runs first
    NetLayer* pend = nullptr;
    for (size_t i = 0; i < net->L.size(); ++i) {
        NetLayer& l = net->L[i];
        const vdttfs_layer_desc& d = l.d;
        WindowScope window(ctx, l.window);
        PoolIn pin{};
        const PoolIn* fuse = nullptr;  // the pending pool, taken by this layer's build
        if (pend) {
            bool take = false;
            if (d.kind == VDTTFS_LAYER_CONV || d.kind == VDTTFS_LAYER_FC) {
                LaunchPlan plan;
                const IntegShape s = integ_shape(net, l);
                take = resolve_plan(ctx, s, l.plan, &plan) == VDTTFS_OK && plan_from_dense(ctx, s, plan, false) &&
                       pool_fusable(ctx, s, plan, pend->d.H_in, pend->d.W_in);
            }
            if (take) {
                pin = PoolIn{pend->d.H_in, pend->d.W_in};
                fuse = &pin;
                pend->fused = true;
                cur = pend->pool_src;
            } else {
                VD_TRY(launch_pool_min(ctx, pend->pool_src, pend->out, net->B, pend->d.H_in, pend->d.W_in,
                                       pend->d.C_in));
            }
            pend = nullptr;
        }
        l.fused = false;
        if (d.kind == VDTTFS_LAYER_POOL) {
            l.pool_src = cur;
            const bool want = net->pool_fusion == VDTTFS_POOL_FUSE_ALL ||
                              (net->pool_fusion == VDTTFS_POOL_FUSE_AUTO && d.H_out == 1 && d.W_out == 1);
            if (want && !count && i > 0 && i + 1 < net->L.size())
                pend = &l;
            else
                VD_TRY(launch_pool_min(ctx, cur, l.out, net->B, d.H_in, d.W_in, d.C_in));
        } else if (d.kind == VDTTFS_LAYER_VMEM) {
            VD_TRY(launch_fc_vmem(ctx, cur, l.out, l.W, l.bias, l.alpha, net->B,
                                  d.H_in * d.W_in * d.C_in, d.C_out));
        } else {
            const IntegShape s = integ_shape(net, l);
            if (count) VD_TRY(zero_counters(ctx));
            // conv layers of the dense paths build their merged lists from
            // the dense map; the bin-layout bucketize runs for the bins path,
            // and in a counting forward for its retained-event count
            LaunchPlan plan;
            VD_TRY(resolve_plan(ctx, s, l.plan, &plan));
            const bool dense = plan_from_dense(ctx, s, plan, count);
            TimedPair tb{}, ti{};
            tb.layer = ti.layer = (int)i;
            if (!dense || count) {
                if (net->timing && !count) VD_TRY(mark(net, &tb.a));
                VD_TRY(launch_bucketize_bins(ctx, cur, l.cols, l.cin_col, l.alpha, net->ev, net->off,
                                             count ? ctx->d_counters + 2 : nullptr));
                if (net->timing && !count) {
                    VD_TRY(mark(net, &tb.b));
                    tb.kind = 1;
                    net->pending.push_back(tb);
                    ti.a = tb.b;
                }
            } else if (net->timing) {
                VD_TRY(mark(net, &ti.a));
            }
            if (dense)
                VD_TRY(launch_integrate_dense(ctx, l.out, cur, l.alpha, net->list, l.list_cap,
                                              net->bstart, l.W, l.bias, l.theta, l.t_min, s,
                                              count ? ctx->d_counters : nullptr, nullptr, &plan, fuse));
            else
                VD_TRY(launch_integrate_bins(ctx, l.out, net->ev, net->off, net->list, l.list_cap,
                                             net->bstart, l.W, l.bias, l.theta, l.t_min, s,
                                             count ? ctx->d_counters : nullptr, nullptr, &plan));
            if (net->timing && !count) {
                VD_TRY(mark(net, &ti.b));
                ti.kind = 0;
                net->pending.push_back(ti);
            }
            if (count) {
                unsigned long long h[4];
                VD_TRY(read_counters(ctx, h));
                if (eproc) eproc[i] = h[0];
                if (ebin) ebin[i] = h[1];
                if (n_ev) n_ev[i] = h[2];
                if (n_cols) n_cols[i] = (uint64_t)l.cols;
            }
        }
        if (count && (d.kind == VDTTFS_LAYER_POOL || d.kind == VDTTFS_LAYER_VMEM)) {
            if (eproc) eproc[i] = 0;
            if (ebin) ebin[i] = 0;
            if (n_ev) n_ev[i] = 0;
            if (n_cols) n_cols[i] = 0;
        }
        cur = l.out;
    }
    if (d_pred) {
        const vdttfs_layer_desc& last = net->L.back().d;
        VD_TRY(launch_readout(ctx, cur, net->B, last.H_out * last.W_out * last.C_out, d_pred,
                              net->readout));
    }
    return VDTTFS_OK;
}

void release(vdttfs_net* net) {
    if (!net) return;
    if (net->ctx) {
        (void)hipSetDevice(net->ctx->device);
        (void)hipStreamSynchronize(net->ctx->stream);
    }
    for (NetLayer& l : net->L) {
        void* p[] = {l.W, l.bias, l.alpha, l.theta, l.out};
        for (void* q : p)
            if (q) (void)hipFree(q);
    }
    for (GraphEntry& g : net->graphs) (void)hipGraphExecDestroy(g.exec);
    if (net->enc) (void)hipFree(net->enc);
    if (net->ev) (void)hipFree(net->ev);
    if (net->off) (void)hipFree(net->off);
    if (net->list) (void)hipFree(net->list);
    if (net->bstart) (void)hipFree(net->bstart);
    for (hipEvent_t e : net->pool) (void)hipEventDestroy(e);
    delete net;
}

int upload(vdttfs_ctx* ctx, float** dst, const float* src, size_t n) {
    if (hipMalloc((void**)dst, n * 4 ? n * 4 : 4) != hipSuccess) {
        *dst = nullptr;
        return set_error(VDTTFS_E_NOMEM, "device allocation of %zu bytes failed", n * 4);
    }
    if (n) VD_HIP(hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice));
    (void)ctx;
    return VDTTFS_OK;
}

int dalloc(void** p, size_t bytes) {
    if (hipMalloc(p, bytes ? bytes : 4) != hipSuccess) {
        *p = nullptr;
        return set_error(VDTTFS_E_NOMEM, "device allocation of %zu bytes failed", bytes);
    }
    return VDTTFS_OK;
}

int create_impl(vdttfs_net* net, const vdttfs_layer_desc* layers, int n) {
    vdttfs_ctx* ctx = net->ctx;
    const vdttfs_consts& c = ctx->c;
    VD_TRY(dalloc((void**)&net->enc, (size_t)net->B * net->img_elems * 4));
    int64_t max_elems = 1, max_cols = 1, max_list = 1, max_bstart = 1;
    float tc_i = net->tc_in, td_i = net->td_in;
    std::vector<float> ha(c.T + 1), ht(c.T);
    net->L.resize(n);
    for (int i = 0; i < n; ++i) {
        NetLayer& l = net->L[i];
        l.d = layers[i];
        const vdttfs_layer_desc& d = layers[i];
        l.out_elems = (int64_t)net->B * d.H_out * d.W_out * d.C_out;
        VD_TRY(dalloc((void**)&l.out, (size_t)l.out_elems * 4));
        if (d.kind == VDTTFS_LAYER_POOL) continue;
        const bool fc = d.kind != VDTTFS_LAYER_CONV;
        const int64_t kel = fc ? (int64_t)d.H_in * d.W_in * d.C_in * d.C_out
                               : (int64_t)d.K_h * d.K_w * d.C_in * d.C_out;
        VD_TRY(upload(ctx, &l.W, d.kernel, (size_t)kel));
        VD_TRY(upload(ctx, &l.bias, d.bias, (size_t)d.C_out));
        VD_TRY(vdttfs_build_luts_host(&c, tc_i, td_i, d.tc_fire, d.td, ha.data(), ht.data()));
        VD_TRY(upload(ctx, &l.alpha, ha.data(), ha.size()));
        VD_TRY(upload(ctx, &l.theta, ht.data(), ht.size()));
        int t_min = (int)ceilf(d.td);
        l.t_min = t_min < 0 ? 0 : t_min;
        tc_i = d.tc_fire;
        td_i = d.td;
        l.d.kernel = nullptr;
        l.d.bias = nullptr;
        if (d.kind == VDTTFS_LAYER_VMEM) continue;
        l.cols = fc ? net->B : (int64_t)net->B * d.H_in * d.W_in;
        l.cin_col = fc ? d.H_in * d.W_in * d.C_in : d.C_in;
        IntegShape s{};
        s.B = net->B;
        s.is_fc = fc;
        s.H_in = fc ? 1 : d.H_in;
        s.W_in = fc ? 1 : d.W_in;
        s.C_in = l.cin_col;
        s.H_out = fc ? 1 : d.H_out;
        s.W_out = fc ? 1 : d.W_out;
        s.C_out = d.C_out;
        s.K_h = fc ? 1 : d.K_h;
        s.K_w = fc ? 1 : d.K_w;
        const bool same = !fc && c.conv_same_pad;  // T2V:109-110
        s.pad_h = same ? d.K_h / 2 : 0;
        s.pad_w = same ? d.K_w / 2 : 0;
        VD_TRY(check_integ_shape(ctx, s));
        if (l.cols * l.cin_col > max_elems) max_elems = l.cols * l.cin_col;
        if (l.cols > max_cols) max_cols = l.cols;
        l.list_cap = merged_list_cap(s);
        const int64_t n_pix = (int64_t)net->B * (fc ? 1 : (int64_t)d.H_out * d.W_out);
        if (n_pix * l.list_cap > max_list) max_list = n_pix * l.list_cap;
        if (n_pix * (c.T + 1) > max_bstart) max_bstart = n_pix * (c.T + 1);
    }
    for (int i = 0; i < n; ++i) net->L[i].d.kernel = net->L[i].d.bias = nullptr;
    VD_TRY(dalloc((void**)&net->ev, (size_t)max_elems * sizeof(vd_event)));
    VD_TRY(dalloc((void**)&net->off, (size_t)max_cols * (c.T + 1) * 4));
    VD_TRY(dalloc((void**)&net->list, (size_t)max_list * sizeof(int2)));
    VD_TRY(dalloc((void**)&net->bstart, (size_t)max_bstart * 4));
    VD_HIP(hipDeviceSynchronize());
    return VDTTFS_OK;
}

}  // namespace

namespace vdttfs {
int validate_layer_table(const vdttfs_consts& c, const vdttfs_layer_desc* layers, int n, int64_t img_elems) {
    return validate(c, layers, n, img_elems);
}
}  // namespace vdttfs

namespace {

// Waits for the stream and moves the pending event pairs into the totals.
int drain_timing(vdttfs_net* net) {
    VD_TRY(check_ctx(net->ctx));
    VD_HIP(hipStreamSynchronize(net->ctx->stream));
    if (net->layer_ms.size() != net->L.size()) net->layer_ms.assign(net->L.size(), 0.0);
    for (const TimedPair& p : net->pending) {
        float ms = 0;
        VD_HIP(hipEventElapsedTime(&ms, p.a, p.b));
        net->ms[p.kind] += ms;
        net->launches[p.kind] += 1;
        net->layer_ms[p.layer] += ms;
    }
    net->pending.clear();
    net->pool_used = 0;
    return VDTTFS_OK;
}

}  // namespace

extern "C" {

int vdttfs_net_create(vdttfs_ctx* ctx, const vdttfs_layer_desc* layers, int n_layers, int B,
                      int64_t img_elems, int encode_mode, float tc_in, float td_in, int readout,
                      vdttfs_net** out) {
    VD_TRY(check_ctx(ctx));
    if (!out || !layers || n_layers <= 0 || B <= 0 || img_elems <= 0)
        return set_error(VDTTFS_E_INVALID, "net_create: bad argument");
    *out = nullptr;
    if (encode_mode != VDTTFS_ENCODE_LINEAR && encode_mode != VDTTFS_ENCODE_LOG &&
        encode_mode != VDTTFS_ENCODE_TIMES)
        return set_error(VDTTFS_E_INVALID, "net_create: encode mode %d", encode_mode);
    if (readout != VDTTFS_READOUT_ARGMIN && readout != VDTTFS_READOUT_ARGMAX &&
        readout != VDTTFS_READOUT_ARGMIN_FIRST)
        return set_error(VDTTFS_E_INVALID, "net_create: readout %d", readout);
    VD_TRY(validate(ctx->c, layers, n_layers, img_elems));
    vdttfs_net* net = new (std::nothrow) vdttfs_net();
    if (!net) return set_error(VDTTFS_E_NOMEM, "net_create: out of memory");
    net->ctx = ctx;
    net->B = B;
    net->img_elems = img_elems;
    net->encode_mode = encode_mode;
    net->tc_in = tc_in;
    net->td_in = td_in;
    net->readout = readout;
    const int rc = create_impl(net, layers, n_layers);
    if (rc != VDTTFS_OK) {
        release(net);
        return rc;
    }
    *out = net;
    return VDTTFS_OK;
}

int vdttfs_net_destroy(vdttfs_net* net) {
    release(net);
    return VDTTFS_OK;
}

namespace {

// Captures one forward on the context stream into a graph and instantiates it.
int capture_forward(vdttfs_net* net, const float* d_img, int32_t* d_pred, GraphEntry* g) {
    vdttfs_ctx* ctx = net->ctx;
    VD_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
    const int rc = forward_impl(net, d_img, d_pred, nullptr, nullptr, nullptr, nullptr);
    hipGraph_t graph = nullptr;
    const hipError_t ec = hipStreamEndCapture(ctx->stream, &graph);
    if (rc != VDTTFS_OK) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (ec != hipSuccess || !graph)
        return set_error(VDTTFS_E_HIP, "net_forward: graph capture failed: %s", hipGetErrorString(ec));
    const hipError_t ei = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) return set_error(VDTTFS_E_HIP, "net_forward: graph instantiation failed: %s", hipGetErrorString(ei));
    g->img = d_img;
    g->pred = d_pred;
    g->gen = net->gen;
    g->fused.resize(net->L.size());
    g->pool_src.resize(net->L.size());
    for (size_t i = 0; i < net->L.size(); ++i) {
        g->fused[i] = net->L[i].fused ? 1 : 0;
        g->pool_src[i] = net->L[i].pool_src;
    }
    return VDTTFS_OK;
}

}  // namespace

int vdttfs_net_forward(vdttfs_net* net, const float* d_img, int32_t* d_pred) {
    if (!net || !d_img) return set_error(VDTTFS_E_INVALID, "net_forward: null argument");
    VD_TRY(check_ctx(net->ctx));
    if (!net->graphs_on || net->timing) return forward_impl(net, d_img, d_pred, nullptr, nullptr, nullptr, nullptr);
    // graphs of an older configuration are dropped; a pair of pointers seen
    // before replays its graph, a new one is captured (the oldest evicted)
    for (size_t i = 0; i < net->graphs.size();) {
        if (net->graphs[i].gen != net->gen) {
            (void)hipGraphExecDestroy(net->graphs[i].exec);
            net->graphs.erase(net->graphs.begin() + (long)i);
        } else {
            ++i;
        }
    }
    GraphEntry* hit = nullptr;
    for (GraphEntry& g : net->graphs)
        if (g.img == d_img && g.pred == d_pred) hit = &g;
    if (!hit) {
        if (net->graphs.size() == kMaxGraphs) {
            (void)hipGraphExecDestroy(net->graphs.front().exec);
            net->graphs.erase(net->graphs.begin());
        }
        GraphEntry g;
        VD_TRY(capture_forward(net, d_img, d_pred, &g));
        net->graphs.push_back(std::move(g));
        hit = &net->graphs.back();
    }
    VD_HIP(hipGraphLaunch(hit->exec, net->ctx->stream));
    for (size_t i = 0; i < net->L.size(); ++i) {  // the forward's host-side state, as the capture left it
        net->L[i].fused = hit->fused[i] != 0;
        net->L[i].pool_src = hit->pool_src[i];
    }
    return VDTTFS_OK;
}

int vdttfs_net_set_graphs(vdttfs_net* net, int enable) {
    if (!net) return set_error(VDTTFS_E_INVALID, "null net");
    net->graphs_on = enable != 0;
    return VDTTFS_OK;
}

int vdttfs_net_layer_output(vdttfs_net* net, int layer, const float** d_out, int64_t* elems) {
    if (!net || !d_out || layer < 0 || layer >= (int)net->L.size())
        return set_error(VDTTFS_E_INVALID, "net_layer_output: bad argument");
    NetLayer& l = net->L[layer];
    if (l.fused) {  // a pool the last forward fused into the next build: write its map now
        VD_TRY(launch_pool_min(net->ctx, l.pool_src, l.out, net->B, l.d.H_in, l.d.W_in, l.d.C_in));
        l.fused = false;
    }
    *d_out = l.out;
    if (elems) *elems = net->L[layer].out_elems;
    return VDTTFS_OK;
}

int vdttfs_net_count(vdttfs_net* net, const float* d_img, uint64_t* eproc, uint64_t* ebin,
                     uint64_t* n_ev, uint64_t* n_cols) {
    if (!net || !d_img) return set_error(VDTTFS_E_INVALID, "net_count: null argument");
    VD_TRY(check_ctx(net->ctx));
    uint64_t dummy[1];
    (void)dummy;
    std::vector<uint64_t> a(net->L.size()), b(net->L.size()), c(net->L.size()), d(net->L.size());
    VD_TRY(forward_impl(net, d_img, nullptr, a.data(), b.data(), c.data(), d.data()));
    VD_HIP(hipStreamSynchronize(net->ctx->stream));
    for (size_t i = 0; i < net->L.size(); ++i) {
        if (eproc) eproc[i] = a[i];
        if (ebin) ebin[i] = b[i];
        if (n_ev) n_ev[i] = c[i];
        if (n_cols) n_cols[i] = d[i];
    }
    return VDTTFS_OK;
}

int vdttfs_net_set_pool_fusion(vdttfs_net* net, int mode) {
    if (!net) return set_error(VDTTFS_E_INVALID, "null net");
    if (mode != VDTTFS_POOL_FUSE_OFF && mode != VDTTFS_POOL_FUSE_ALL && mode != VDTTFS_POOL_FUSE_AUTO)
        return set_error(VDTTFS_E_INVALID, "net_set_pool_fusion: unknown mode %d", mode);
    net->pool_fusion = mode;
    ++net->gen;
    return VDTTFS_OK;
}

int vdttfs_net_set_timing(vdttfs_net* net, int enable) {
    if (!net) return set_error(VDTTFS_E_INVALID, "null net");
    net->timing = enable != 0;
    return VDTTFS_OK;
}

int vdttfs_net_set_windows(vdttfs_net* net, const int32_t* windows, int n_layers) {
    if (!net) return set_error(VDTTFS_E_INVALID, "null net");
    const int n = (int)net->L.size();
    if (windows && n_layers != n)
        return set_error(VDTTFS_E_INVALID, "net_set_windows: %d windows for %d layers", n_layers, n);
    const int T = net->ctx->c.T;
    if (windows)
        for (int i = 0; i < n; ++i)
            if (net->L[i].d.kind != VDTTFS_LAYER_POOL && (windows[i] < 0 || windows[i] > T))
                return set_error(VDTTFS_E_INVALID, "net_set_windows: layer %d window %d outside [0, %d]", i,
                                 windows[i], T);
    for (int i = 0; i < n; ++i) {
        const int w = windows && net->L[i].d.kind != VDTTFS_LAYER_POOL ? windows[i] : 0;
        net->L[i].window = w == T ? 0 : w;
    }
    ++net->gen;
    return VDTTFS_OK;
}

int vdttfs_net_set_plan(vdttfs_net* net, int layer, const vdttfs_layer_plan* plan) {
    if (!net || layer < 0 || layer >= (int)net->L.size())
        return set_error(VDTTFS_E_INVALID, "net_set_plan: bad argument");
    NetLayer& l = net->L[layer];
    const bool integ = l.d.kind == VDTTFS_LAYER_CONV || l.d.kind == VDTTFS_LAYER_FC;
    LaunchPlan req{};
    if (plan) {
        req.path = plan->path;
        req.gather = plan->gather;
        req.ppw = plan->ppw;
    }
    if (!integ) {
        if (req.path || req.gather || req.ppw)
            return set_error(VDTTFS_E_UNSUPPORTED, "net_set_plan: layer %d has no integrator", layer);
        return VDTTFS_OK;
    }
    LaunchPlan resolved;
    VD_TRY(resolve_plan(net->ctx, integ_shape(net, l), req, &resolved));
    l.plan = req;
    ++net->gen;
    return VDTTFS_OK;
}

int vdttfs_net_get_plan(vdttfs_net* net, int layer, vdttfs_layer_plan* out) {
    if (!net || !out || layer < 0 || layer >= (int)net->L.size())
        return set_error(VDTTFS_E_INVALID, "net_get_plan: bad argument");
    const NetLayer& l = net->L[layer];
    *out = vdttfs_layer_plan{0, 0, 0};
    if (l.d.kind != VDTTFS_LAYER_CONV && l.d.kind != VDTTFS_LAYER_FC) return VDTTFS_OK;
    vdttfs_ctx* ctx = net->ctx;
    WindowScope window(ctx, l.window);
    LaunchPlan p;
    VD_TRY(resolve_plan(ctx, integ_shape(net, l), l.plan, &p));
    *out = vdttfs_layer_plan{p.path, p.gather, p.ppw};
    return VDTTFS_OK;
}

int vdttfs_net_read_layer_timing(vdttfs_net* net, double* ms, int n_layers) {
    if (!net || !ms || n_layers != (int)net->L.size())
        return set_error(VDTTFS_E_INVALID, "net_read_layer_timing: bad argument");
    VD_TRY(drain_timing(net));
    for (int i = 0; i < n_layers; ++i) {
        ms[i] = net->layer_ms[i];
        net->layer_ms[i] = 0.0;
    }
    return VDTTFS_OK;
}

int vdttfs_net_read_timing(vdttfs_net* net, double* integ_ms, int64_t* integ_launches,
                           double* bucket_ms, int64_t* bucket_launches) {
    if (!net) return set_error(VDTTFS_E_INVALID, "null net");
    VD_TRY(drain_timing(net));
    if (integ_ms) *integ_ms = net->ms[0];
    if (integ_launches) *integ_launches = net->launches[0];
    if (bucket_ms) *bucket_ms = net->ms[1];
    if (bucket_launches) *bucket_launches = net->launches[1];
    net->ms[0] = net->ms[1] = 0;
    net->launches[0] = net->launches[1] = 0;
    return VDTTFS_OK;
}

}  // extern "C"
