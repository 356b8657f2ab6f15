// Step-by-step (time-driven) baseline network (T1S / T2S main loops,
// T1S:222-244 and T2S:329-352): encode once, then for every global step the
// input spikes of that step and every layer in order, then the readout.
// T3S mode (snn_dvs_stepbystep.cu:220-252) steps the CuLIF layer table over
// the dense event tensor.
// Weights are uploaded once; spike maps, membrane potentials and fire-once
// latches live on the device for the batch.
#include <cmath>
#include <new>
#include <vector>

#include "common.h"
#include "wave.h"

using namespace vdttfs;

struct StepNetLayer {
    StepLayer s{};
    float tc_i = 16.0f, td_i = 0.0f;  // the previous weighted layer's fire constants (decay kernel)
    float tc_f = 16.0f, td_f = 0.0f;  // this layer's fire constants (threshold)
    int depth = 0;                    // 1-based among weighted layers
    float* W = nullptr;
    float* bias = nullptr;
    uint8_t* spk = nullptr;
    uint8_t* fired = nullptr;
    float* vmem = nullptr;
};

struct vdttfs_stepnet {
    vdttfs_ctx* ctx = nullptr;
    int B = 0, mode = 1, encode = 0, steps = 0;
    int64_t img_elems = 0;
    float tc_in = 16.0f, td_in = 0.0f;
    std::vector<StepNetLayer> L;
    float* tin = nullptr;  // encoded first-spike times of the input
    uint8_t* s0 = nullptr;
    float* out = nullptr;
    int64_t out_elems = 0;
    // T3S mode: the CuLIF layers and every buffer they own
    std::vector<Step3Layer> L3;
    std::vector<void*> bufs3;
};

namespace {

void release(vdttfs_stepnet* net) {
    if (!net) return;
    if (net->ctx) {
        (void)hipSetDevice(net->ctx->device);
        (void)hipStreamSynchronize(net->ctx->stream);
    }
    for (StepNetLayer& l : net->L)
        for (void* p : {(void*)l.W, (void*)l.bias, (void*)l.spk, (void*)l.fired, (void*)l.vmem})
            if (p) (void)hipFree(p);
    for (void* p : {(void*)net->tin, (void*)net->s0})
        if (p) (void)hipFree(p);
    if (net->mode != VDTTFS_STEP_T3 && net->out) (void)hipFree(net->out);  // T3S: out is a layer's ft
    for (void* p : net->bufs3)
        if (p) (void)hipFree(p);
    delete net;
}

int dmalloc(void** p, size_t bytes) {
    if (hipMalloc(p, bytes ? bytes : 4) != hipSuccess) {
        *p = nullptr;
        return set_error(VDTTFS_E_NOMEM, "stepnet: device allocation of %zu bytes failed", bytes);
    }
    return VDTTFS_OK;
}

int upload(float** dst, const float* src, size_t n) {
    VD_TRY(dmalloc((void**)dst, n * 4));
    VD_HIP(hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice));
    return VDTTFS_OK;
}

int create_impl(vdttfs_stepnet* net, const vdttfs_layer_desc* layers, int n) {
    vdttfs_ctx* ctx = net->ctx;
    const vdttfs_consts& c = ctx->c;
    VD_TRY(dmalloc((void**)&net->tin, (size_t)net->B * net->img_elems * 4));
    VD_TRY(dmalloc((void**)&net->s0, (size_t)net->B * net->img_elems));
    net->L.resize(n);
    float tc = net->tc_in, td = net->td_in;
    int depth = 0;
    for (int i = 0; i < n; ++i) {
        const vdttfs_layer_desc& d = layers[i];
        StepNetLayer& l = net->L[i];
        StepLayer& s = l.s;
        s.kind = d.kind;
        s.n = (int64_t)net->B * d.H_out * d.W_out * d.C_out;
        s.H_in = d.H_in;
        s.W_in = d.W_in;
        s.C_in = d.C_in;
        s.H_out = d.H_out;
        s.W_out = d.W_out;
        s.C_out = d.C_out;
        s.K_h = d.K_h;
        s.K_w = d.K_w;
        s.is_fc = d.kind != VDTTFS_LAYER_CONV;
        const bool same = !s.is_fc && c.conv_same_pad;  // T2V:109-110
        s.pad_h = same ? d.K_h / 2 : 0;
        s.pad_w = same ? d.K_w / 2 : 0;
        VD_TRY(dmalloc((void**)&l.spk, (size_t)s.n));
        VD_TRY(dmalloc((void**)&l.fired, (size_t)s.n));
        if (d.kind == VDTTFS_LAYER_POOL) continue;
        const int64_t kel = s.is_fc ? (int64_t)d.H_in * d.W_in * d.C_in * d.C_out
                                    : (int64_t)d.K_h * d.K_w * d.C_in * d.C_out;
        VD_TRY(upload(&l.W, d.kernel, (size_t)kel));
        VD_TRY(upload(&l.bias, d.bias, (size_t)d.C_out));
        VD_TRY(dmalloc((void**)&l.vmem, (size_t)s.n * 4));
        s.W = l.W;
        s.bias = l.bias;
        l.tc_i = tc;
        l.td_i = td;
        l.tc_f = d.tc_fire;
        l.td_f = d.td;
        l.depth = ++depth;
        tc = d.tc_fire;
        td = d.td;
    }
    net->out_elems = net->L.back().s.n;
    VD_TRY(dmalloc((void**)&net->out, (size_t)net->out_elems * 4));
    // T1S:229 runs T steps; T2S runs until the last weighted layer's window
    // [(D-1)*tfs, (D-1)*tfs + T) has passed (TIME_STEPS, T2S:13)
    net->steps = net->mode == VDTTFS_STEP_T1 ? c.T : (int)ceilf((float)(depth - 1) * c.tfs + (float)c.T);
    return VDTTFS_OK;
}

int forward_impl(vdttfs_stepnet* net, const float* d_img, int32_t* d_pred) {
    vdttfs_ctx* ctx = net->ctx;
    const vdttfs_consts& c = ctx->c;
    const int T = c.T;
    const int64_t n_img = (int64_t)net->B * net->img_elems;
    if (net->encode == VDTTFS_ENCODE_LOG)
        VD_TRY(launch_encode_log(ctx, d_img, net->tin, n_img, net->tc_in, net->td_in));
    else
        VD_TRY(launch_encode_linear(ctx, d_img, net->tin, n_img));
    for (StepNetLayer& l : net->L) {
        VD_HIP(hipMemsetAsync(l.fired, 0, (size_t)l.s.n, ctx->stream));
        if (l.vmem) VD_TRY(launch_step_fill(ctx, l.vmem, l.s.n, 0.0f));
    }
    const bool t1 = net->mode == VDTTFS_STEP_T1;
    VD_TRY(launch_step_fill(ctx, net->out, net->out_elems, t1 ? kInfTime : -1e9f));
    const int last = (int)net->L.size() - 1;
    for (int t = 0; t < net->steps; ++t) {
        VD_TRY(launch_step_input(ctx, net->tin, net->s0, n_img, t));
        const uint8_t* s_in = net->s0;
        for (int i = 0; i <= last; ++i) {
            StepNetLayer& l = net->L[i];
            if (l.s.kind == VDTTFS_LAYER_POOL) {
                VD_TRY(launch_step_pool(ctx, s_in, l.spk, l.fired, l.s.n, l.s.H_in, l.s.W_in, l.s.C_in));
            } else {
                int int_ok, fire_ok;
                float kv, th;
                if (t1) {
                    // T1S:74-101: integrate every step, fire from t_min on
                    int t_min = (int)ceilf(l.td_f);
                    if (t_min < 0) t_min = 0;
                    kv = expf(-((float)t - l.td_i) / l.tc_i);
                    th = c.vth * expf(-((float)t - l.td_f) / l.tc_f);
                    int_ok = 1;
                    fire_ok = t >= t_min;
                } else {
                    // T2S:72-107: layer-local integration and firing windows
                    const float t_integ = (float)t - (float)(l.depth - 1) * c.tfs;
                    const float t_fire = (float)t - (float)l.depth * c.tfs;
                    const float start = l.td_f > 0.0f ? ceilf(l.td_f) : 0.0f;
                    kv = expf(-(t_integ - l.td_i) / l.tc_i);
                    th = c.vth * expf(-(t_fire - l.td_f) / l.tc_f);
                    int_ok = t_integ >= 0.0f && t_integ < (float)T;
                    fire_ok = t_fire >= start && t_fire < (float)T;
                    if (!int_ok && !fire_ok && i != last) {
                        // outside both windows the step only clears the spikes of
                        // the neurons that have not fired; nothing spikes
                        VD_HIP(hipMemsetAsync(l.spk, 0, (size_t)l.s.n, ctx->stream));
                        s_in = l.spk;
                        continue;
                    }
                }
                const int out_layer = i == last ? (t1 ? 1 : 2) : 0;
                VD_TRY(launch_step_neuron(ctx, l.s, s_in, l.spk, l.vmem, l.fired, net->out, net->mode, int_ok,
                                          fire_ok, out_layer, kv, th, t));
            }
            s_in = l.spk;
        }
    }
    if (d_pred) {
        const StepLayer& o = net->L.back().s;
        VD_TRY(launch_readout(ctx, net->out, net->B, o.H_out * o.W_out * o.C_out, d_pred, t1 ? 0 : 1));
    }
    return VDTTFS_OK;
}

// T3S (snn_dvs_stepbystep.cu:173-214): per layer, the CuIF state and the
// fire-once latch of every neuron, its 0/1 spikes and first-spike steps.
int create3_impl(vdttfs_stepnet* net, const vdttfs_culif_layer* layers, int n) {
    const int B = net->B;
    auto alloc = [&](void** p, size_t bytes) -> int {
        VD_TRY(dmalloc(p, bytes));
        net->bufs3.push_back(*p);
        return VDTTFS_OK;
    };
    auto upload3 = [&](const float** dst, const float* src, size_t elems) -> int {
        float* d = nullptr;
        VD_TRY(alloc((void**)&d, elems * 4));
        VD_HIP(hipMemcpy(d, src, elems * 4, hipMemcpyHostToDevice));
        *dst = d;
        return VDTTFS_OK;
    };
    net->L3.resize(n);
    for (int i = 0; i < n; ++i) {
        const vdttfs_culif_layer& d = layers[i];
        Step3Layer& l = net->L3[i];
        l = Step3Layer{};
        l.kind = d.kind;
        l.C_in = d.C_in;
        l.H = d.H_in;
        l.W = d.W_in;
        l.C_out = d.C_out;
        l.decay = d.decay;
        l.th = d.th;
        const bool fc = d.kind == VDTTFS_CULIF_FC || d.kind == VDTTFS_CULIF_FC_REC;
        if (fc)
            l.n = (int64_t)B * d.C_out;
        else if (d.kind == VDTTFS_CULIF_POOL)
            l.n = (int64_t)B * d.C_in * (d.H_in / 2) * (d.W_in / 2);
        else
            l.n = (int64_t)B * d.C_out * d.H_in * d.W_in;
        VD_TRY(alloc((void**)&l.I, (size_t)l.n * 4));
        VD_TRY(alloc((void**)&l.V, (size_t)l.n * 4));
        VD_TRY(alloc((void**)&l.s, (size_t)l.n * 4));
        VD_TRY(alloc((void**)&l.ft, (size_t)l.n * 4));
        VD_TRY(alloc((void**)&l.fired, (size_t)l.n));
        if (d.kind == VDTTFS_CULIF_POOL) continue;
        if (!fc) {
            VD_TRY(upload3(&l.weight, d.weight, (size_t)d.C_out * d.C_in * 9));
            if (d.kind == VDTTFS_CULIF_RAW_CONV)  // the step's raw events
                VD_TRY(alloc((void**)&l.cur, (size_t)B * d.C_in * d.H_in * d.W_in * 4));
            continue;
        }
        // FC weights transposed to [in][out]: a wave's threads are
        // consecutive outputs, so each step of their (unchanged, i-ascending)
        // sums reads one contiguous row instead of 64 rows far apart
        std::vector<float> tw((size_t)d.C_out * d.C_in);
        for (int o = 0; o < d.C_out; ++o)
            for (int i2 = 0; i2 < d.C_in; ++i2) tw[(size_t)i2 * d.C_out + o] = d.weight[(size_t)o * d.C_in + i2];
        VD_TRY(upload3(&l.weight, tw.data(), tw.size()));
        if (d.kind == VDTTFS_CULIF_FC_REC) {
            std::vector<float> tr((size_t)d.C_out * d.C_out);
            for (int o = 0; o < d.C_out; ++o)
                for (int j = 0; j < d.C_out; ++j) tr[(size_t)j * d.C_out + o] = d.weight_rec[(size_t)o * d.C_out + j];
            VD_TRY(upload3(&l.weight_rec, tr.data(), tr.size()));
            VD_TRY(alloc((void**)&l.cur, (size_t)l.n * 4));
        }
    }
    net->out = net->L3.back().ft;
    net->out_elems = net->L3.back().n;
    net->steps = net->ctx->c.T;
    return VDTTFS_OK;
}

// T3S main loop (T3S:220-252), then its first-spike readout (T3S:274-279,
// argmin from class 0).
int forward3_impl(vdttfs_stepnet* net, const float* d_data, int32_t* d_pred) {
    vdttfs_ctx* ctx = net->ctx;
    for (Step3Layer& l : net->L3) {
        VD_TRY(launch_step_fill(ctx, l.I, l.n, 0.0f));
        VD_TRY(launch_step_fill(ctx, l.V, l.n, 0.0f));
        VD_TRY(launch_step_fill(ctx, l.s, l.n, 0.0f));
        VD_TRY(launch_step_fill(ctx, l.ft, l.n, kInfTime));
        VD_HIP(hipMemsetAsync(l.fired, 0, (size_t)l.n, ctx->stream));
    }
    const int T = net->steps;
    for (int t = 0; t < T; ++t) {
        const float* in = d_data;
        for (const Step3Layer& l : net->L3) {
            VD_TRY(launch_step3_layer(ctx, l, in, net->B, T, t));
            in = l.s;
        }
    }
    if (d_pred) VD_TRY(launch_readout(ctx, net->out, net->B, (int)(net->out_elems / net->B), d_pred, 2));
    return VDTTFS_OK;
}

}  // namespace

extern "C" {

int vdttfs_stepnet_create_culif(vdttfs_ctx* ctx, const vdttfs_culif_layer* layers, int n_layers, int B,
                                vdttfs_stepnet** out) {
    VD_TRY(check_ctx(ctx));
    if (!out || !layers || n_layers <= 0 || B <= 0)
        return set_error(VDTTFS_E_INVALID, "stepnet_create_culif: bad argument");
    *out = nullptr;
    VD_TRY(validate_culif_table(ctx, layers, n_layers));
    vdttfs_stepnet* net = new (std::nothrow) vdttfs_stepnet();
    if (!net) return set_error(VDTTFS_E_NOMEM, "stepnet_create_culif: out of memory");
    net->ctx = ctx;
    net->B = B;
    net->mode = VDTTFS_STEP_T3;
    net->img_elems = (int64_t)layers[0].C_in * layers[0].H_in * layers[0].W_in * ctx->c.T;
    const int rc = create3_impl(net, layers, n_layers);
    if (rc != VDTTFS_OK) {
        release(net);
        return rc;
    }
    *out = net;
    return VDTTFS_OK;
}

int vdttfs_stepnet_create(vdttfs_ctx* ctx, const vdttfs_layer_desc* layers, int n_layers, int B,
                          int64_t img_elems, int encode_mode, float tc_in, float td_in, int mode,
                          vdttfs_stepnet** out) {
    VD_TRY(check_ctx(ctx));
    if (!out || !layers || n_layers <= 0 || B <= 0 || img_elems <= 0)
        return set_error(VDTTFS_E_INVALID, "stepnet_create: bad argument");
    *out = nullptr;
    if (mode != VDTTFS_STEP_T1 && mode != VDTTFS_STEP_T2)
        return set_error(VDTTFS_E_INVALID, "stepnet_create: mode %d", mode);
    if (encode_mode != VDTTFS_ENCODE_LINEAR && encode_mode != VDTTFS_ENCODE_LOG)
        return set_error(VDTTFS_E_INVALID, "stepnet_create: encode mode %d", encode_mode);
    VD_TRY(validate_layer_table(ctx->c, layers, n_layers, img_elems));
    if (layers[n_layers - 1].kind == VDTTFS_LAYER_POOL)
        return set_error(VDTTFS_E_INVALID, "stepnet_create: the last layer must be a weighted layer");
    vdttfs_stepnet* net = new (std::nothrow) vdttfs_stepnet();
    if (!net) return set_error(VDTTFS_E_NOMEM, "stepnet_create: out of memory");
    net->ctx = ctx;
    net->B = B;
    net->img_elems = img_elems;
    net->encode = encode_mode;
    net->tc_in = tc_in;
    net->td_in = td_in;
    net->mode = mode;
    const int rc = create_impl(net, layers, n_layers);
    if (rc != VDTTFS_OK) {
        release(net);
        return rc;
    }
    *out = net;
    return VDTTFS_OK;
}

int vdttfs_stepnet_destroy(vdttfs_stepnet* net) {
    release(net);
    return VDTTFS_OK;
}

int vdttfs_stepnet_forward(vdttfs_stepnet* net, const float* d_img, int32_t* d_pred) {
    if (!net || !d_img) return set_error(VDTTFS_E_INVALID, "stepnet_forward: null argument");
    VD_TRY(check_ctx(net->ctx));
    if (net->mode == VDTTFS_STEP_T3) return forward3_impl(net, d_img, d_pred);
    return forward_impl(net, d_img, d_pred);
}

int vdttfs_stepnet_output(vdttfs_stepnet* net, const float** d_out, int64_t* elems, int* steps) {
    if (!net || !d_out) return set_error(VDTTFS_E_INVALID, "stepnet_output: bad argument");
    *d_out = net->out;
    if (elems) *elems = net->out_elems;
    if (steps) *steps = net->steps;
    return VDTTFS_OK;
}

}  // extern "C"
