/*
 * vdttfs_oracle.h -- CPU restatement of the reference VD-TTFS algorithm.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * MI355X engine and the CPU baseline timed beside it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product (vd-ttfs_amd/) never links, loads or calls it.
 *
 * Every function follows the reference CUDA program loop-for-loop (file:line
 * cited per function, paths relative to the reference repository root):
 *   T1V = task1_lenet_mnist/vdttfs_cuda/snn_timesorted_earlyexit.cu
 *   T2V = task2_vgg16_cifar10/vdttfs_cuda/bench_vgg_eventdriven_timesorted_earlyexit.cu
 *   T3V = task3_dvsgesture/vdttfs_cuda/snn_inference_timesorted.cu
 *   T2M = task2_vgg16_cifar10/macs/stat_timesorted_macs.cu
 *   T1S = task1_lenet_mnist/stepbystep_cuda/snn_mnist_stepbystep.cu
 *
 * Floating point: built with -ffp-contract=off; the accumulation sites that
 * the reference writes as `x += a*b` / `I = I*d + x` are written as explicit
 * fmaf() (nvcc's default --fmad=true contracts them).  LUTs use the host
 * libm expf, exactly as the reference's update_LUTs does.
 *
 * Pins (what checks each function; parity is never asserted by re-typing
 * a formula):
 *   orc_build_luts        closed form alpha(td)=1, monotone theta, libm expf
 *   orc_encode_*          exact rule on hand-picked pixels (tests)
 *   orc_bucketize*        brute-force stable sort + invariants (tests)
 *   orc_integrate         brute-force time-driven simulator (below), Delta
 *                         invariance, E_proc closed forms (no-early-exit
 *                         count = retained receptive-field events), single-
 *                         input closed form, hand-computed golden fixtures
 *   orc_pool_min          exact min (tests)
 *   orc_fc_vmem           fp64 dot product (tests)
 *   orc_readout_*         tie rules on hand-built rows (tests)
 *   CuLIF set             brute-force step-by-step simulator (below)
 */
#ifndef VDTTFS_ORACLE_H
#define VDTTFS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_INF 9999.0f

/* Per-task constants (T1V:12-19, T2V:12-18). */
typedef struct orc_consts {
    int   T;              /* TIME_WINDOW */
    float tfs;            /* TIME_FIRE_START */
    int   delta;          /* CHUNK */
    int   alpha_by_time;  /* 0: alpha[tb] (T1V:128,144); 1: alpha[clamp((int)t,0,T)] (T2V:132,150) */
    float vth;            /* VTH_INIT */
} orc_consts;

int orc_num_chunks(const orc_consts* c);

/* update_LUTs (T1V:208-216, T2V:236-243): alpha has T+1 entries, theta T. */
void orc_build_luts(int T, float vth, float tc_i, float td_i, float tc_f, float td_f,
                    float* alpha, float* theta);

/* k_encode_image (T1V:32-42) and the configs' linear rule t=floor(T(1-x)). */
void orc_encode_log(const float* img, float* out, int64_t n, float tc, float td, int T);
void orc_encode_linear(const float* img, float* out, int64_t n, int T);

/* k_bucketize (T1V:45-80, T2V:45-81): reference layout, OS = NC+1. */
void orc_bucketize(const orc_consts* c, const float* in, int64_t n_cols, int c_in,
                   int32_t* out_cin, float* out_tin, int32_t* out_off, int nthreads);

/* k_conv_bucketed (T1V:83-162, T2V:84-170; E_proc as T2M:99-176).
 * pad_h = pad_w = 0 gives T1V's valid conv; pad_h = K_h/2, pad_w = K_w/2 with
 * out-of-bounds taps skipped gives T2V's same conv (T2V:109-110, 136-141).
 * eproc: events integrated under the reference's chunk-granular exit.
 * ebin : events integrated under a per-bin exit (events with bin <= fire bin).
 * Either may be NULL. */
void orc_integrate(const orc_consts* c, float* out,
                   const int32_t* bcin, const float* btin, const int32_t* boff,
                   const float* W, const float* bias, const float* alpha, const float* theta,
                   int t_min, int B, int H_in, int W_in, int C_in,
                   int H_out, int W_out, int C_out, int K_h, int K_w, int pad_h, int pad_w, int is_fc,
                   int no_early_exit, uint64_t* eproc, uint64_t* ebin, int nthreads);

/* Brute-force time-driven restatement of the same neuron: for every time bin
 * t in [0,T) it scans the whole dense receptive field for inputs arriving at
 * t (no buckets, no chunks).  Same per-bin summation order as the reference
 * ((kh,kw) outer, cin ascending). */
void orc_integrate_timedriven(const orc_consts* c, float* out, const float* spikes,
                              const float* W, const float* bias, const float* alpha,
                              const float* theta, int t_min, int B, int H_in, int W_in,
                              int C_in, int H_out, int W_out, int C_out, int K_h, int K_w,
                              int pad_h, int pad_w, int is_fc, int nthreads);

/* Decision margin in fp64 along the reference path: per neuron, the smallest
 * |carry - theta| / (|bias| + sum|w*alpha|) over every checked bin up to the
 * firing bin.  Neurons with a tiny margin are the documented threshold ties. */
void orc_integrate_margin(const orc_consts* c, double* margin, const float* spikes,
                          const float* W, const float* bias, const float* alpha,
                          const float* theta, int t_min, int B, int H_in, int W_in,
                          int C_in, int H_out, int W_out, int C_out, int K_h, int K_w,
                          int pad_h, int pad_w, int is_fc, int nthreads);

/* k_pooling (T1V:164-181, T2V:192-209). */
void orc_pool_min(const float* in, float* out, int B, int H_in, int W_in, int C, int nthreads);

/* k_layer_vmem (T2V:172-190). */
void orc_fc_vmem(const orc_consts* c, const float* in, float* out, const float* W,
                 const float* bias, const float* alpha, int B, int C_in, int C_out);

/* Readouts: T1V:312-319 (argmin, -1 if none), T2V:389-396 (argmax),
 * T3V:291-298 (argmin starting from class 0). */
void orc_readout_argmin(const float* out, int B, int C, int32_t* pred);
void orc_readout_argmax(const float* out, int B, int C, int32_t* pred);
void orc_readout_t3(const float* out, int B, int C, int32_t* pred);

/* ---- network runner (the driver main()s: T1V:286-319, T2V:337-396) ---- */
enum { ORC_CONV = 0, ORC_FC = 1, ORC_POOL = 2, ORC_VMEM = 3 };
/* ORC_ENC_TIMES: the input already holds spike times (copied unchanged) */
enum { ORC_ENC_LINEAR = 0, ORC_ENC_LOG = 1, ORC_ENC_TIMES = 2 };
enum { ORC_READ_ARGMIN = 0, ORC_READ_ARGMAX = 1, ORC_READ_T3 = 2 };

typedef struct orc_layer {
    int kind;
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad_h, pad_w;
    const float* W;
    const float* bias;
    float tc_fire, td;
} orc_layer;

/* Runs encode -> every layer -> readout for a batch.  layer_outs[i] (may be
 * NULL, or entries NULL) receives layer i's output map.  eproc/ebin are per
 * layer (may be NULL).  final_out receives the last layer's output, pred the
 * predicted classes.  Returns 0, or a negative code for an inconsistent
 * layer table. */
int orc_net_forward(const orc_consts* c, const orc_layer* layers, int n_layers, int B,
                    const float* img, int64_t img_elems_per_image, int encode_mode,
                    float tc_in, float td_in, int readout,
                    float** layer_outs, float* final_out, int32_t* pred,
                    uint64_t* eproc, uint64_t* ebin, int nthreads);

/* ---- step-by-step (time-driven) baselines ----
 * T1S = task1_lenet_mnist/stepbystep_cuda/snn_mnist_stepbystep.cu
 * T2S = task2_vgg16_cifar10/stepbystep_cuda/bench_vgg_timedriven_baseline.cu
 * Every weighted layer integrates, at each global step, the binary spikes
 * its inputs emit at that step, and fires (once) on the decaying threshold.
 *   mode 1 (T1S:47-103, 222-244): all layers share the step; psp = sum of the
 *          spiking inputs' weights, V = fma(psp, kv(t), V); fire when
 *          t >= t_min and V + b >= th(t) >= 1e-5; the output layer records its
 *          first spike (argmin readout).
 *   mode 2 (T2S:53-200, 329-352): weighted layer d (1-based) integrates at
 *          t - (d-1)*tfs in [0, T) with psp = fma chain of w*kv, V += psp, and
 *          fires at t - d*tfs in [ceil(td)+, T); the last weighted layer keeps
 *          max(V + b) over its window (argmax readout).
 * kv(t) = expf(-(t - td_prev)/tc_prev), th(t) = vth * expf(-(t - td)/tc),
 * evaluated once per (layer, step).  Pools fire at the first step any of
 * their 2x2 inputs spikes.  final_out (B x C of the last layer) gets the
 * first-spike steps (mode 1) or max(V + b) (mode 2); steps_out the number
 * of global steps run.  A VMEM layer is treated as the output FC. */
int orc_stepnet_forward(const orc_consts* c, const orc_layer* layers, int n_layers, int B,
                        const float* img, int64_t img_elems_per_image, int encode_mode,
                        float tc_in, float td_in, int mode, float* final_out, int32_t* pred,
                        int* steps_out, int nthreads);

/* ---- CuLIF (T3V), config 4 ---- */
/* conv1_raw_early (T3V:30-65): dense events [N][C_in][H][W][T], OIHW 3x3 pad 1. */
void orc_culif_conv1_raw(const float* data, float* out, const float* weight, int N, int C_in,
                         int C_out, int H, int W, int T, int delta, float decay, float th,
                         int nthreads);
/* k_bucketize_conv (T3V:70-90): NCHW sites; k_bucketize_fc (T3V:93-106). */
void orc_culif_bucketize_nchw(const float* in, int N, int C, int H, int W, int T, int delta,
                              int32_t* out_cin, float* out_tin, int32_t* out_off, int nthreads);
void orc_culif_bucketize_fc(const float* in, int N, int F, int T, int delta,
                            int32_t* out_cin, float* out_tin, int32_t* out_off, int nthreads);
/* conv_bucketed_early (T3V:109-143): OIHW 3x3 pad 1, NCHW out. */
void orc_culif_conv(const int32_t* bcin, const float* btin, const int32_t* boff, float* out,
                    const float* weight, int N, int C_in, int C_out, int H, int W, int T,
                    int delta, float decay, float th, int nthreads);
/* pool_chunk_early (T3V:146-168). */
void orc_culif_pool(const float* in, float* out, int N, int C, int H_in, int W_in, int T,
                    int delta, float decay, float th, int nthreads);
/* fc1_bucketed_recurrent (T3V:171-200): out_f neurons per sample, W [out][in],
 * W_rec [out][out]. */
void orc_culif_fc_recurrent(const int32_t* bcin, const float* btin, const int32_t* boff,
                            float* out, const float* w, const float* w_rec, int N, int in_f,
                            int out_f, int T, int delta, float decay, float th, int nthreads);
/* fc2_bucketed_early (T3V:203-225): W [out][in]. */
void orc_culif_fc(const int32_t* bcin, const float* btin, const int32_t* boff, float* out,
                  const float* w, int N, int in_f, int out_f, int T, int delta, float decay,
                  float th, int nthreads);
/* Step-by-step CuLIF neuron on a dense per-step input current, for pinning:
 * in[t] for t in [0,T); returns first t with V>=th or INF. */
float orc_culif_neuron_steps(const float* in, int T, float decay, float th);

/* ---- step-by-step CuLIF baseline (T3S =
 *      task3_dvsgesture/stepbystep_cuda/snn_dvs_stepbystep.cu) ----
 * For t = 0..T-1 (T3S:220-252), every layer in order: the layer's input
 * current from that step's input (raw events data[...][t] for the first
 * layer, else the previous layer's 0/1 spike map), then the CuIF neuron
 * I = fma(I, decay, cur); V = V + I; spike once at V >= th (T3S:119-140).
 *   RAW_CONV / CONV (T3S:41-68): 3x3 pad 1, OIHW, sum = fma(in, w, sum) over
 *     c_in, ky, kx in that order (in-bounds taps only);
 *   POOL (T3S:70-94): max of the 2x2 window, from -1e9;
 *   FC (T3S:96-109): sum = fma(in[i], W[o][i], sum) over i ascending;
 *   FC_REC (T3S:243-247): FC over the input plus, added after, the FC of
 *     the layer's own spikes of step t-1 through W_rec[o][j].
 * Kinds as ORC_CULIF_*.  layer_outs[i] (may be NULL, or entries NULL)
 * receive each layer's first-spike steps (NCHW, 9999 = none), final_out the
 * last layer's, pred the T3V/T3S readout (argmin from class 0).  Returns 0,
 * or -1 for an inconsistent table, -2 when out of memory. */
enum { ORC_CULIF_RAW_CONV = 0, ORC_CULIF_CONV = 1, ORC_CULIF_POOL = 2, ORC_CULIF_FC_REC = 3, ORC_CULIF_FC = 4 };
typedef struct orc_culif_layer {
    int kind;
    int C_in, H_in, W_in, C_out; /* FC: C_in = input features, H_in = W_in = 1 */
    const float* w;
    const float* w_rec;
    float decay, th;
} orc_culif_layer;
int orc_culif_stepnet_forward(const orc_culif_layer* layers, int n_layers, int N, const float* data,
                              int T, float** layer_outs, float* final_out, int32_t* pred, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
