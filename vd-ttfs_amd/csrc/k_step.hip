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
//   k_step_pool   spiking 2x2 pool (T1S:107-127, T2S:110-139).
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
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad, is_fc;
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
                    const int hi = ho - a.pad + kh;
                    if (hi < 0 || hi >= a.H_in) continue;
                    for (int kw = 0; kw < a.K_w; ++kw) {
                        const int wi = wo - a.pad + kw;
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
    a.pad = L.pad;
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

}  // namespace vdttfs
