// Step-by-step (time-driven) baseline kernels: the reference's own GPU
// denominator (T1S = task1_lenet_mnist/stepbystep_cuda/snn_mnist_stepbystep.cu,
// T2S = task2_vgg16_cifar10/stepbystep_cuda/bench_vgg_timedriven_baseline.cu),
// rebuilt for gfx950 with the reference's work structure: every global step
// launches every layer, one thread per neuron scans its whole receptive field
// for inputs that spike at that step, and neurons fire once on the decaying
// threshold.  No event lists and no early exit: this is the baseline the
// event-driven engine is measured against.
//   k_step_input  input spikes of step t from the encoded first-spike times;
//   k_step_neuron conv / FC step (T1S:47-103, T2S:53-108 and 141-200);
//   k_step_pool   spiking 2x2 pool (T1S:107-127, T2S:110-139);
//   k_s3_*        the CuLIF network of T3S (below).
// The step's decay kv(t) and threshold th(t) are the same for every neuron of
// a layer; the host evaluates them once per (layer, step) with the same expf
// expressions and passes them in.  Threads are numbered c_out fastest, so a
// wave's threads read the same input spikes and consecutive weights.
#include "common.h"
#include "wave.h"

namespace vdttfs {
namespace {

__global__ __launch_bounds__(256) void k_step_input(const float* __restrict__ tin, uint8_t* __restrict__ s,
                                                    int64_t n, float t) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        s[i] = tin[i] == t ? 1 : 0;
}

struct StepArgs {
    const uint8_t* s_in;
    uint8_t* s_out;
    float* vmem;
    uint8_t* fired;
    const float* W;
    const float* bias;
    float* out;  // output layer: first-spike steps (T1S) or max(V + b) (T2S)
    int64_t n;
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad_h, pad_w, is_fc;
    int mode;          // 1: T1S (psp = sum w; V = fma(psp, kv, V)); 2: T2S (psp = fma chain of w*kv; V += psp)
    int int_ok, fire_ok;
    int out_layer;     // 1: T1S output (records its first spike); 2: T2S output (keeps max V + b)
    float kv, th, t;
};

__global__ __launch_bounds__(256) void k_step_neuron(StepArgs a) {
    for (int64_t nid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; nid < a.n;
         nid += (int64_t)gridDim.x * blockDim.x) {
        const bool keep_max = a.out_layer == 2;
        if (!keep_max && a.fired[nid]) {
            a.s_out[nid] = 0;
            continue;
        }
        const int co = (int)(nid % a.C_out);
        float V = a.vmem[nid];
        if (a.int_ok) {
            float psp = 0.0f;
            if (a.is_fc) {
                const int cin = a.H_in * a.W_in * a.C_in;
                const uint8_t* src = a.s_in + (nid / a.C_out) * cin;
                for (int ci = 0; ci < cin; ++ci)
                    if (src[ci]) {
                        const float w = a.W[(int64_t)ci * a.C_out + co];
                        psp = a.mode == 1 ? psp + w : __builtin_fmaf(w, a.kv, psp);
                    }
            } else {
                const int64_t q = nid / a.C_out;
                const int wo = (int)(q % a.W_out);
                const int ho = (int)((q / a.W_out) % a.H_out);
                const int64_t img = q / ((int64_t)a.W_out * a.H_out);
                for (int kh = 0; kh < a.K_h; ++kh) {
                    const int hi = ho - a.pad_h + kh;
                    if (hi < 0 || hi >= a.H_in) continue;
                    for (int kw = 0; kw < a.K_w; ++kw) {
                        const int wi = wo - a.pad_w + kw;
                        if (wi < 0 || wi >= a.W_in) continue;
                        const uint8_t* src = a.s_in + ((img * a.H_in + hi) * a.W_in + wi) * a.C_in;
                        const int64_t wb = (int64_t)(kh * a.K_w + kw) * a.C_in;
                        for (int ci = 0; ci < a.C_in; ++ci)
                            if (src[ci]) {
                                const float w = a.W[(wb + ci) * a.C_out + co];
                                psp = a.mode == 1 ? psp + w : __builtin_fmaf(w, a.kv, psp);
                            }
                    }
                }
            }
            V = a.mode == 1 ? __builtin_fmaf(psp, a.kv, V) : V + psp;
            a.vmem[nid] = V;
        }
        uint8_t spike = 0;
        if (keep_max) {
            if (a.int_ok) {
                const float v = V + a.bias[co];
                if (v > a.out[nid]) a.out[nid] = v;
            }
        } else if (a.fire_ok && V + a.bias[co] >= a.th && a.th >= 1e-5f) {
            spike = 1;
            a.fired[nid] = 1;
            if (a.out_layer == 1 && a.out[nid] >= kInfTime) a.out[nid] = a.t;
        }
        a.s_out[nid] = spike;
    }
}

__global__ __launch_bounds__(256) void k_step_pool(const uint8_t* __restrict__ s_in, uint8_t* __restrict__ s_out,
                                                   uint8_t* __restrict__ fired, int64_t n, int H_in, int W_in,
                                                   int C) {
    const int Ho = H_in / 2, Wo = W_in / 2;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        if (fired[idx]) {
            s_out[idx] = 0;
            continue;
        }
        const int c = (int)(idx % C), w = (int)((idx / C) % Wo), h = (int)((idx / C / Wo) % Ho);
        const int64_t b = idx / ((int64_t)C * Wo * Ho);
        uint8_t spike = 0;
        for (int i = 0; i < 2 && !spike; ++i)
            for (int j = 0; j < 2; ++j) {
                const int hi = h * 2 + i, wi = w * 2 + j;
                if (hi < H_in && wi < W_in && s_in[((b * H_in + hi) * W_in + wi) * C + c]) {
                    spike = 1;
                    break;
                }
            }
        if (spike) fired[idx] = 1;
        s_out[idx] = spike;
    }
}

__global__ __launch_bounds__(256) void k_step_fill(float* __restrict__ p, int64_t n, float v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

unsigned step_grid(int64_t n) {
    int64_t b = (n + 255) / 256;
    if (b > (1 << 20)) b = 1 << 20;
    return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

int launch_step_input(vdttfs_ctx* ctx, const float* tin, uint8_t* s, int64_t n, int t) {
    hipLaunchKernelGGL(k_step_input, dim3(step_grid(n)), dim3(256), 0, ctx->stream, tin, s, n, (float)t);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_step_neuron(vdttfs_ctx* ctx, const StepLayer& L, const uint8_t* s_in, uint8_t* s_out, float* vmem,
                       uint8_t* fired, float* out, int mode, int int_ok, int fire_ok, int out_layer, float kv,
                       float th, int t) {
    StepArgs a{};
    a.s_in = s_in;
    a.s_out = s_out;
    a.vmem = vmem;
    a.fired = fired;
    a.W = L.W;
    a.bias = L.bias;
    a.out = out;
    a.n = L.n;
    a.H_in = L.H_in;
    a.W_in = L.W_in;
    a.C_in = L.C_in;
    a.H_out = L.H_out;
    a.W_out = L.W_out;
    a.C_out = L.C_out;
    a.K_h = L.K_h;
    a.K_w = L.K_w;
    a.pad_h = L.pad_h;
    a.pad_w = L.pad_w;
    a.is_fc = L.is_fc;
    a.mode = mode;
    a.int_ok = int_ok;
    a.fire_ok = fire_ok;
    a.out_layer = out_layer;
    a.kv = kv;
    a.th = th;
    a.t = (float)t;
    hipLaunchKernelGGL(k_step_neuron, dim3(step_grid(L.n)), dim3(256), 0, ctx->stream, a);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_step_pool(vdttfs_ctx* ctx, const uint8_t* s_in, uint8_t* s_out, uint8_t* fired, int64_t n, int H_in,
                     int W_in, int C) {
    hipLaunchKernelGGL(k_step_pool, dim3(step_grid(n)), dim3(256), 0, ctx->stream, s_in, s_out, fired, n, H_in,
                       W_in, C);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

int launch_step_fill(vdttfs_ctx* ctx, float* p, int64_t n, float v) {
    hipLaunchKernelGGL(k_step_fill, dim3(step_grid(n)), dim3(256), 0, ctx->stream, p, n, v);
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

// ---------------------------------------------------------------------------
// T3S = task3_dvsgesture/stepbystep_cuda/snn_dvs_stepbystep.cu: the CuLIF
// network stepped densely.  Every step, every layer computes every neuron's
// input current from that step's 0/1 spike map (the raw event values for the
// first layer) in the reference's order -- conv over c_in, ky, kx
// (T3S:53-64), FC over i ascending (T3S:104-106), all as fma(in, w, sum) --
// and runs the CuIF neuron I = fma(I, decay, cur); V = V + I; spike once at
// V >= th (T3S:119-140).  Maps are NCHW, threads numbered like the
// reference's (x fastest, FC: output fastest).  The current and the neuron
// share one kernel (the reference's separate current buffer changes
// nothing), except for the recurrent FC, whose current reads the layer's own
// spikes of step t-1 and so must complete before any of them is replaced.
namespace {

struct Step3Args {
    const float* in;
    const float* weight;
    const float* weight_rec;
    float* I;
    float* V;
    float* s;
    uint8_t* fired;
    float* ft;
    float* cur;
    int64_t n;
    int C_in, H, Wd, C_out, T, t;
    float decay, th;
};

__device__ __forceinline__ void s3_neuron(const Step3Args& a, int64_t i, float cur) {
    const float ci = __builtin_fmaf(a.I[i], a.decay, cur);
    const float cv = a.V[i] + ci;
    a.I[i] = ci;
    a.V[i] = cv;
    if (!a.fired[i] && cv >= a.th) {
        a.s[i] = 1.0f;
        a.fired[i] = 1;
        a.ft[i] = (float)a.t;
    } else {
        a.s[i] = 0.0f;
    }
}

// extract_input_step (T3S:33-39): the raw events of step t, NCHW
__global__ __launch_bounds__(256) void k_s3_extract(const float* __restrict__ data, float* __restrict__ out,
                                                    int64_t n, int T, int t) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = data[i * T + t];
}

// conv2d_kernel (T3S:41-68) + neuron.  Taps outside the map are skipped as
// in the reference (a select keeps sum unchanged, whatever the weight).
// A thread computes COB consecutive c_out of one pixel (threads numbered
// x fastest, then y, c_out block, n), so each input load feeds COB
// independent fma chains, each in the reference's c_in, ky, kx order.
// UNI: H*W is a multiple of 64, so a wave's threads share (n, c_out block)
// and read each weight as one scalar load.
template <bool UNI, int COB>
__global__ __launch_bounds__(256) void k_s3_conv(Step3Args a) {
    const int H = a.H, W = a.Wd, C_in = a.C_in, n_cb = a.C_out / COB;
    const int64_t HW = (int64_t)H * W;
    const int64_t n_thr = a.n / COB;
    for (int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; tid < n_thr;
         tid += (int64_t)gridDim.x * blockDim.x) {
        const int x = (int)(tid % W), y = (int)((tid / W) % H);
        int cb = (int)((tid / HW) % n_cb);
        int64_t nb = tid / (HW * n_cb);
        if (UNI) {
            cb = __builtin_amdgcn_readfirstlane(cb);
            nb = ((int64_t)__builtin_amdgcn_readfirstlane((int)(nb >> 32)) << 32) |
                 (uint32_t)__builtin_amdgcn_readfirstlane((int)nb);
        }
        bool ok[9];
        int off[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const int iy = y + k / 3 - 1, ix = x + k % 3 - 1;
            ok[k] = iy >= 0 && iy < H && ix >= 0 && ix < W;
            off[k] = ok[k] ? iy * W + ix : 0;
        }
        const int co0 = cb * COB;
        const float* ip = a.in + nb * C_in * HW;
        float sum[COB];
#pragma unroll
        for (int o = 0; o < COB; ++o) sum[o] = 0.0f;
        for (int c = 0; c < C_in; ++c) {
            float v[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) v[k] = ip[off[k]];
#pragma unroll
            for (int o = 0; o < COB; ++o) {
                const float* wk = a.weight + ((int64_t)(co0 + o) * C_in + c) * 9;
#pragma unroll
                for (int k = 0; k < 9; ++k) sum[o] = ok[k] ? __builtin_fmaf(v[k], wk[k], sum[o]) : sum[o];
            }
            ip += HW;
        }
#pragma unroll
        for (int o = 0; o < COB; ++o) s3_neuron(a, ((nb * a.C_out + co0 + o) * H + y) * (int64_t)W + x, sum[o]);
    }
}

// maxpool2d_kernel (T3S:70-94) + neuron
__global__ __launch_bounds__(256) void k_s3_pool(Step3Args a) {
    const int H_in = a.H, W_in = a.Wd, H_out = H_in / 2, W_out = W_in / 2, C = a.C_in;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int xo = (int)(idx % W_out), yo = (int)((idx / W_out) % H_out);
        const int c = (int)((idx / ((int64_t)W_out * H_out)) % C);
        const int64_t nb = idx / ((int64_t)C * H_out * W_out);
        const float* p = a.in + ((nb * C + c) * H_in + yo * 2) * (int64_t)W_in + xo * 2;
        float m = -1e9f;
        m = fmaxf(m, p[0]);
        m = fmaxf(m, p[1]);
        m = fmaxf(m, p[W_in]);
        m = fmaxf(m, p[W_in + 1]);
        s3_neuron(a, idx, m);
    }
}

// sum over i ascending of x[i] * w[i * stride] (FC weights are stored
// [in][out], stride = out)
__device__ __forceinline__ float s3_dot(const float* __restrict__ x, const float* __restrict__ w, int n,
                                        int stride) {
    float sum = 0.0f;
    int i = 0;
    // 16 loads in flight per thread; the fma chain keeps the i-ascending order
    for (; i + 16 <= n; i += 16) {
        float xv[16], wv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            xv[k] = x[i + k];
            wv[k] = w[(int64_t)(i + k) * stride];
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) sum = __builtin_fmaf(xv[k], wv[k], sum);
    }
    for (; i < n; ++i) sum = __builtin_fmaf(x[i], w[(int64_t)i * stride], sum);
    return sum;
}

// fc_kernel (T3S:96-109) + neuron
__global__ __launch_bounds__(256) void k_s3_fc(Step3Args a) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = idx / a.C_out;
        const int col = (int)(idx % a.C_out);
        s3_neuron(a, idx, s3_dot(a.in + row * a.C_in, a.weight + col, a.C_in, a.C_out));
    }
}

// recurrent FC current (T3S:244-246): the FC of the input plus, added after,
// the FC of the layer's own spikes of step t-1
__global__ __launch_bounds__(256) void k_s3_fcrec_current(Step3Args a) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = idx / a.C_out;
        const int col = (int)(idx % a.C_out);
        const float f = s3_dot(a.in + row * a.C_in, a.weight + col, a.C_in, a.C_out);
        const float r = s3_dot(a.s + row * a.C_out, a.weight_rec + col, a.C_out, a.C_out);
        a.cur[idx] = f + r;
    }
}

__global__ __launch_bounds__(256) void k_s3_neuron(Step3Args a) {
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < a.n;
         idx += (int64_t)gridDim.x * blockDim.x)
        s3_neuron(a, idx, a.cur[idx]);
}

}  // namespace

int launch_step3_layer(vdttfs_ctx* ctx, const Step3Layer& L, const float* in, int N, int T, int t) {
    Step3Args a{};
    a.in = in;
    a.weight = L.weight;
    a.weight_rec = L.weight_rec;
    a.I = L.I;
    a.V = L.V;
    a.s = L.s;
    a.fired = L.fired;
    a.ft = L.ft;
    a.cur = L.cur;
    a.n = L.n;
    a.C_in = L.C_in;
    a.H = L.H;
    a.Wd = L.W;
    a.C_out = L.C_out;
    a.T = T;
    a.t = t;
    a.decay = L.decay;
    a.th = L.th;
    const dim3 grid(step_grid(L.n)), block(256);
    const bool uni = ((int64_t)L.H * L.W) % 64 == 0;
    switch (L.kind) {
        case VDTTFS_CULIF_RAW_CONV: {
            // the step's events first, as the reference does
            if (!L.cur) return set_error(VDTTFS_E_INVALID, "step3: raw conv without a step-input buffer");
            const int64_t n_in = (int64_t)N * L.C_in * L.H * L.W;
            hipLaunchKernelGGL(k_s3_extract, dim3(step_grid(n_in)), block, 0, ctx->stream, in, L.cur, n_in, T, t);
            VD_HIP(hipGetLastError());
            a.in = L.cur;
        }
            [[fallthrough]];
        case VDTTFS_CULIF_CONV: {
            const bool cob4 = L.C_out % 4 == 0;
            const dim3 cgrid(step_grid(cob4 ? L.n / 4 : L.n));
            if (uni && cob4)
                hipLaunchKernelGGL((k_s3_conv<true, 4>), cgrid, block, 0, ctx->stream, a);
            else if (cob4)
                hipLaunchKernelGGL((k_s3_conv<false, 4>), cgrid, block, 0, ctx->stream, a);
            else if (uni)
                hipLaunchKernelGGL((k_s3_conv<true, 1>), cgrid, block, 0, ctx->stream, a);
            else
                hipLaunchKernelGGL((k_s3_conv<false, 1>), cgrid, block, 0, ctx->stream, a);
            break;
        }
        case VDTTFS_CULIF_POOL: hipLaunchKernelGGL(k_s3_pool, grid, block, 0, ctx->stream, a); break;
        case VDTTFS_CULIF_FC: hipLaunchKernelGGL(k_s3_fc, grid, block, 0, ctx->stream, a); break;
        case VDTTFS_CULIF_FC_REC:
            if (!L.cur) return set_error(VDTTFS_E_INVALID, "step3: recurrent layer without a current buffer");
            hipLaunchKernelGGL(k_s3_fcrec_current, grid, block, 0, ctx->stream, a);
            VD_HIP(hipGetLastError());
            hipLaunchKernelGGL(k_s3_neuron, grid, block, 0, ctx->stream, a);
            break;
        default: return set_error(VDTTFS_E_INVALID, "step3: layer kind %d", L.kind);
    }
    VD_HIP(hipGetLastError());
    return VDTTFS_OK;
}

}  // namespace vdttfs
