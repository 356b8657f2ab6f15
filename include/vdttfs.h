/*
 * vdttfs.h -- C ABI of the MI355X-native VD-TTFS engine (libvdttfs.so).
 *
 * Plain C types only: device pointers are `float*` / `int32_t*` returned by
 * vdttfs_dev_alloc() (or any hipMalloc'ed memory), sizes are int / int64_t.
 * Every entry point returns an int status (VDTTFS_OK = 0, negative = error
 * class) and never calls exit(); vdttfs_last_error() describes the last
 * failure on the calling thread.  Work is stream-ordered on the context's
 * stream; the `_sync` launch wrappers also synchronise, as the reference's
 * launch_* helpers do.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   T1V = task1_lenet_mnist/vdttfs_cuda/snn_timesorted_earlyexit.cu
 *   T2V = task2_vgg16_cifar10/vdttfs_cuda/bench_vgg_eventdriven_timesorted_earlyexit.cu
 *   T2M = task2_vgg16_cifar10/macs/stat_timesorted_macs.cu
 *   WIO = task1_lenet_mnist/torch_ann/weights_io.py (blob format)
 */
#ifndef VDTTFS_H
#define VDTTFS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define VDTTFS_OK             0
#define VDTTFS_E_INVALID     -1  /* bad argument / inconsistent shapes     */
#define VDTTFS_E_HIP         -2  /* HIP runtime error                      */
#define VDTTFS_E_IO          -3  /* file missing / unreadable              */
#define VDTTFS_E_FORMAT      -4  /* malformed weights blob                 */
#define VDTTFS_E_NOMEM       -5  /* host or device allocation failed       */
#define VDTTFS_E_UNSUPPORTED -6  /* shape outside what the kernels handle  */
#define VDTTFS_E_NODEVICE    -7  /* no HIP device visible                  */

#define VDTTFS_INF_TIME 9999.0f  /* "no spike" (T1V:14, T2V:15) */

/* Last error message of the calling thread ("" if none). */
const char* vdttfs_last_error(void);
/* Library version string. */
const char* vdttfs_version(void);

/* ---- per-task constants: the reference's compile-time macros ---------- */
/* T1V:12-19 (TIME_WINDOW, VTH_INIT, TIME_FIRE_START, CHUNK) and T2V:12-18.
 * alpha_by_time = 0 reproduces T1V's alpha[tb] indexing (T1V:128,144);
 * 1 reproduces T2V's alpha[clamp((int)t,0,T)] (T2V:132,150).
 * conv_same_pad = 0 is T1V's valid convolution (T1V:131-133); 1 is T2V's
 * zero-padded "same" convolution with out-of-bounds columns skipped
 * (T2V:112-113,136-141). */
typedef struct vdttfs_consts {
    int32_t T;             /* TIME_WINDOW, 1..256                       */
    float   tfs;           /* TIME_FIRE_START                           */
    int32_t delta;         /* CHUNK, 1..T                               */
    float   vth;           /* VTH_INIT                                  */
    int32_t alpha_by_time;
    int32_t conv_same_pad;
} vdttfs_consts;

typedef struct vdttfs_ctx vdttfs_ctx;

/* Replaces the reference's file-static state (T2V:246-248, 321-329): the
 * context owns the constants, a HIP stream and the bucket scratch. */
int vdttfs_create(const vdttfs_consts* consts, int device, vdttfs_ctx** out);
int vdttfs_destroy(vdttfs_ctx* ctx);
int vdttfs_get_consts(const vdttfs_ctx* ctx, vdttfs_consts* out);
/* NC = ceil(T/delta) and OFF_STRIDE = NC+1 (T1V:18-19, T2V:17-18). */
int vdttfs_num_chunks(const vdttfs_ctx* ctx);
int vdttfs_synchronize(vdttfs_ctx* ctx);
/* HIP-event timer on the context's stream (no reference counterpart; the
 * reference times its batch with cudaEventRecord around main()'s layer
 * loop, T2V:339-388).  begin records a start event; end records a stop
 * event, waits for it and returns the milliseconds in between. */
int vdttfs_timer_begin(vdttfs_ctx* ctx);
int vdttfs_timer_end(vdttfs_ctx* ctx, double* ms);
int vdttfs_device_count(int* out);

/* ---- device memory plumbing (cudaMalloc/cudaMemcpy in the reference) -- */
int vdttfs_dev_alloc(vdttfs_ctx* ctx, size_t bytes, void** dptr);
int vdttfs_dev_free(vdttfs_ctx* ctx, void* dptr);
int vdttfs_h2d(vdttfs_ctx* ctx, void* dst, const void* src, size_t bytes);  /* synchronous */
int vdttfs_d2h(vdttfs_ctx* ctx, void* dst, const void* src, size_t bytes);  /* synchronous */
int vdttfs_memset(vdttfs_ctx* ctx, void* dptr, int value, size_t bytes);

/* ---- LUT builder: update_LUTs (T1V:208-216, T2V:236-243) -------------- */
/* alpha[t] = expf(-((float)t - td_integ)/tc_integ), t in [0,T] (T+1 entries);
 * theta[t] = vth*expf(-((float)t - td_fire)/tc_fire), t in [0,T).
 * Host libm expf, then a blocking upload to d_lut_decay / d_lut_th. */
int vdttfs_update_luts(vdttfs_ctx* ctx, float* d_lut_decay, float* d_lut_th,
                       float tc_integ, float td_integ, float tc_fire, float td_fire);
/* The same tables on the host (what update_LUTs uploads). */
int vdttfs_build_luts_host(const vdttfs_consts* c, float tc_integ, float td_integ,
                           float tc_fire, float td_fire, float* alpha, float* theta);

/* ---- encoders: k_encode_image (T1V:32-42, T2V:32-42) ------------------ */
int vdttfs_encode_image(vdttfs_ctx* ctx, const float* d_img, float* d_out, int64_t size,
                        float tc, float td);
/* Synthetic configs' rule: x<1e-5 -> INF, else floorf(T*(1-x)). */
int vdttfs_encode_linear(vdttfs_ctx* ctx, const float* d_img, float* d_out, int64_t size);

/* ---- k_bucketize (T1V:45-80, T2V:45-81) -------------------------------- */
/* Reference layout, bit-exact: out_off[col*OS + c] (OS = NC+1) holds the
 * chunk offsets, out_cin/out_tin[col*C_in + pos] the events of each chunk in
 * ascending cin order (the raw float spike time is copied). */
int vdttfs_bucketize(vdttfs_ctx* ctx, const float* d_in, int64_t n_cols, int c_in,
                     int32_t* d_out_cin, float* d_out_tin, int32_t* d_out_off);

/* ---- k_conv_bucketed (T1V:83-162, T2V:84-170) -------------------------- */
/* Consumes the reference bucket layout; writes first-spike times (INF if a
 * neuron never fires), NHWC with c_out fastest.  This is the reference-layout
 * export path, kept for bit-exact checks of caller-made buckets: one thread
 * per neuron, several times slower than vdttfs_layer_forward, which takes the
 * dense map.  Buckets are expected from this context's constants; events
 * outside their chunk's bins or the window, at cin >= C_in, and offsets past
 * the column are skipped / clamped rather than read out of range. */
int vdttfs_integrate(vdttfs_ctx* ctx, float* d_out, const int32_t* d_bkt_cin,
                     const float* d_bkt_tin, const int32_t* d_bkt_off, const float* d_kernel,
                     const float* d_bias, const float* d_lut_decay, const float* d_lut_th,
                     int t_min, int B, int H_in, int W_in, int C_in, int H_out, int W_out,
                     int C_out, int K_h, int K_w, int is_fc);

/* ---- fused path: bucketize + integrate from a spike-time map ----------- */
/* The engine's own path (same results as vdttfs_bucketize followed by
 * vdttfs_integrate): events are sorted per arrival bin into context scratch
 * and integrated by the wave-per-pixel kernel.  eproc / ebin (nullable,
 * host pointers) receive the integrated-synapse counts: eproc under the
 * reference's chunk-granular early exit (T2M:136,155,176), ebin under the
 * per-bin exit this kernel executes.  Counting adds a device counter and a
 * synchronisation; pass NULL for both on the hot path. */
int vdttfs_layer_forward(vdttfs_ctx* ctx, float* d_out, const float* d_in,
                         const float* d_kernel, const float* d_bias, const float* d_lut_decay,
                         const float* d_lut_th, int t_min, int B, int H_in, int W_in, int C_in,
                         int H_out, int W_out, int C_out, int K_h, int K_w, int is_fc,
                         uint64_t* eproc, uint64_t* ebin);

/* ---- the layer path without device allocation ------------------------- */
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same kernels and results as vdttfs_layer_forward
 * (without the work counters), with the layer's merged lists and bucket
 * scratch in a 64 MiB device buffer that the library holds per GPU until the
 * process ends, instead of context scratch grown with hipMalloc.  The call
 * allocates and frees nothing.  A layer whose scratch exceeds 64 MiB fails
 * with VDTTFS_E_UNSUPPORTED (the LDS-list and register paths need none: every
 * layer of the VGG-16 and LeNet-5 configurations runs; a layer on the
 * bucketize + merge path, e.g. a 5x5 conv with C_in > 64, needs about
 * (25*C_in + 32)*8 + 4*(T+1) bytes per output pixel).  Every call on one GPU
 * shares that GPU's buffer, so calls that use it are ordered on the device in
 * the order they are made, across contexts, streams and host threads (each
 * waits on a per-device event the previous one recorded).  A call on a
 * stream under graph capture records no such event: replays of captured
 * graphs that use the buffer must be ordered by the caller. */
int vdttfs_layer_forward_noalloc(vdttfs_ctx* ctx, float* d_out, const float* d_in, const float* d_kernel,
                                 const float* d_bias, const float* d_lut_decay, const float* d_lut_th, int t_min,
                                 int B, int H_in, int W_in, int C_in, int H_out, int W_out, int C_out, int K_h,
                                 int K_w, int is_fc);

/* ---- k_pooling (T1V:164-181, T2V:192-209) ------------------------------ */
int vdttfs_pool_min(vdttfs_ctx* ctx, const float* d_in, float* d_out, int B, int H_in,
                    int W_in, int C);

/* ---- k_layer_vmem (T2V:172-190) ---------------------------------------- */
int vdttfs_fc_vmem(vdttfs_ctx* ctx, const float* d_in, float* d_out, const float* d_kernel,
                   const float* d_bias, const float* d_lut_decay, int B, int C_in, int C_out);

/* ---- readout (T1V:312-319 argmin, T2V:389-396 argmax) on the device ---- */
int vdttfs_readout_argmin(vdttfs_ctx* ctx, const float* d_out, int B, int C, int32_t* d_pred);
int vdttfs_readout_argmax(vdttfs_ctx* ctx, const float* d_out, int B, int C, int32_t* d_pred);

/* ---- per-layer launch wrappers (T1V:222-240, T2V:250-287) -------------- */
/* Synchronous like the reference: one layer's bucketize + integrate, then a
 * stream synchronisation.  Runs the engine's kernels (the same as
 * vdttfs_layer_forward, with the built-in launch plan and context-owned
 * scratch); the reference's wrapper fills file-static buckets its caller
 * never reads, so only d_out is observable, and it is bit-identical.
 * t_min = max(0, ceilf(td)) as T1V:225. */
int vdttfs_launch_layer_sync(vdttfs_ctx* ctx, const float* d_in, float* d_out, int H_in,
                             int W_in, int C_in, int H_out, int W_out, int C_out, int K_h,
                             int K_w, float td, const float* d_kernel, const float* d_bias,
                             const float* d_lut_decay, const float* d_lut_th, int B, int is_fc);
int vdttfs_launch_pool_sync(vdttfs_ctx* ctx, const float* d_in, float* d_out, int H_in,
                            int W_in, int C, int B);
int vdttfs_launch_fc_vmem_sync(vdttfs_ctx* ctx, const float* d_in, float* d_out, int C_in,
                               int C_out, const float* d_kernel, const float* d_bias,
                               const float* d_lut_decay, int B);

/* ---- weights blob (T1V:185-206, T2V:213-234; format WIO:1-13) ---------- */
typedef struct vdttfs_blob_layer {
    int32_t ndim;          /* 4: [k_h,k_w,c_in,c_out] (HWIO); 2: [c_in,c_out] */
    int32_t shape[4];
    int32_t k_h, k_w, c_in, c_out;
    int64_t kernel_elems;
    float*  kernel;        /* host, C order of `shape`                       */
    int32_t bias_ndim;
    int32_t bias_size;
    float*  bias;          /* host                                           */
    int32_t tc_ndim, td_ndim;
    float   tc_fire, td;
} vdttfs_blob_layer;

typedef struct vdttfs_blob {
    int32_t num_layers;
    vdttfs_blob_layer* layers;
} vdttfs_blob;

/* Parses and validates the whole file (ndim in {2,4}, positive shapes,
 * bias size = c_out, one tc and one td float, no short read, no trailing
 * bytes -- the consumption check of WIO:69). */
int vdttfs_blob_read(const char* path, vdttfs_blob** out);
int vdttfs_blob_write(const char* path, const vdttfs_blob* blob);
int vdttfs_blob_free(vdttfs_blob* blob);

/* load_weights: the reference's LayerWeights (T1V:26-30) on the device. */
typedef struct vdttfs_dev_layer {
    float*  d_kernel;
    float*  d_bias;
    float   tc_fire, td;
    int32_t k_h, k_w, c_in, c_out;
} vdttfs_dev_layer;
int vdttfs_load_weights(vdttfs_ctx* ctx, const char* path, vdttfs_dev_layer** layers,
                        int* num_layers);
int vdttfs_free_weights(vdttfs_ctx* ctx, vdttfs_dev_layer* layers, int num_layers);

/* ---- network engine: the driver main()s (T1V:286-319, T2V:337-396) ----- */
#define VDTTFS_LAYER_CONV 0
#define VDTTFS_LAYER_FC   1
#define VDTTFS_LAYER_POOL 2   /* 2x2 min pool  */
#define VDTTFS_LAYER_VMEM 3   /* readout vmem  */
#define VDTTFS_ENCODE_LINEAR 0
#define VDTTFS_ENCODE_LOG    1
#define VDTTFS_ENCODE_TIMES  2   /* the input already holds spike times (e.g. encoded under a
                                    wider window, for temporal truncation); net engine only */
#define VDTTFS_READOUT_ARGMIN 0
#define VDTTFS_READOUT_ARGMAX 1
#define VDTTFS_READOUT_ARGMIN_FIRST 2  /* T3V:291-298: argmin seeded with class 0 */

typedef struct vdttfs_layer_desc {
    int32_t kind;
    int32_t H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w;
    const float* kernel;   /* host, reference layout (HWIO / [C_in][C_out]) */
    const float* bias;     /* host, C_out floats                            */
    float tc_fire, td;
} vdttfs_layer_desc;

typedef struct vdttfs_net vdttfs_net;

/* Uploads weights, builds every layer's LUTs once (kept resident on the
 * device) and allocates activations and scratch for batch B.
 * img_elems = H*W*C of one input image (NHWC). */
int vdttfs_net_create(vdttfs_ctx* ctx, const vdttfs_layer_desc* layers, int n_layers, int B,
                      int64_t img_elems, int encode_mode, float tc_in, float td_in,
                      int readout, vdttfs_net** out);
int vdttfs_net_destroy(vdttfs_net* net);
/* encode -> every layer -> readout, stream-ordered, no host sync.  d_img is
 * [B][img_elems]; d_pred (nullable) receives B int32 classes. */
int vdttfs_net_forward(vdttfs_net* net, const float* d_img, int32_t* d_pred);
/* Device pointer to layer i's output map (valid after a forward). */
int vdttfs_net_layer_output(vdttfs_net* net, int layer, const float** d_out, int64_t* elems);
/* One instrumented forward: per-layer integrated-synapse counts (see
 * vdttfs_layer_forward), retained events N_ev and bucket columns N_cols. */
int vdttfs_net_count(vdttfs_net* net, const float* d_img, uint64_t* eproc, uint64_t* ebin,
                     uint64_t* n_ev, uint64_t* n_cols);
/* Pool fusion.  No counterpart in the reference, whose 2x2 min pools are
 * kernels of their own between the layers (T2V:192-209, launched per pool
 * layer).  A fused pool layer (not the first or last layer) whose next
 * layer runs the fused list build -- the shared-list kernel, or the
 * per-wave kernel past 64 receptive elements, under a LUT neuron -- is
 * computed inside that build from the pool's input (each receptive element
 * the min over its 2x2 window, compared as the pool kernel does), so the
 * pooled map is not written; other pools run as their own pass.  Outputs
 * are the same either way.  vdttfs_net_layer_output of a fused pool layer
 * writes its map then (stream-ordered).  Counting forwards never fuse.
 * mode: OFF (the default) none; ALL every pool the next build can take;
 * AUTO those whose pooled map is 1x1 (an FC layer's one window per
 * channel), where the build's extra loads are fewest.  On VGG-16 B=256 the
 * builds of the wider layers lose more to the four loads per element than
 * the pool's own pass takes (ALL: forward +0.6%), and AUTO measured even. */
#define VDTTFS_POOL_FUSE_OFF  0
#define VDTTFS_POOL_FUSE_ALL  1
#define VDTTFS_POOL_FUSE_AUTO 2
int vdttfs_net_set_pool_fusion(vdttfs_net* net, int mode);
/* HIP graphs.  No counterpart in the reference, which launches every kernel
 * of every batch from the host.  enable != 0: vdttfs_net_forward captures
 * the forward (encode, layers, readout) on the context stream into a HIP
 * graph the first time it sees a (d_img, d_pred) pair under the network's
 * current plans, windows and pool fusion, and replays that graph afterwards;
 * up to four pairs are kept, and changing a plan, the windows or the pool
 * fusion drops them.  The graph holds kernel launches only (no memset or
 * copy nodes).  Outputs are the same as without.  Forwards with event timing
 * on, and counting forwards, run without graphs.  Default 0. */
int vdttfs_net_set_graphs(vdttfs_net* net, int enable);
/* Event timing of integrator launches: when enabled, forward() brackets
 * each integrator launch with HIP events on the context stream; read_timing
 * synchronises and returns the summed milliseconds and launch count since
 * the last reset. */
int vdttfs_net_set_timing(vdttfs_net* net, int enable);
/* Per-layer integration windows T'_l (input-aware temporal truncation).  No
 * counterpart in the reference, which compiles one TIME_WINDOW per program
 * (T1V:12, T2V:12) and describes per-layer windows, chosen offline from
 * spike-time percentiles, without code (README.md:46-54).  windows[i] in
 * [1, T] runs layer i as if TIME_WINDOW were windows[i]: its bucketize keeps
 * arrival bins tb < T'_l only, its neurons fire at steps t < T'_l, and T2's
 * alpha index clamps at T'_l.  0 (or T) keeps the context window; pool
 * layers ignore their entry.  windows == NULL resets every layer.  Setting
 * every layer to T' gives the same outputs as a context created with T = T'
 * (with the inputs encoded under the wider window, VDTTFS_ENCODE_TIMES). */
int vdttfs_net_set_windows(vdttfs_net* net, const int32_t* windows, int n_layers);

/* Per-layer launch plans of the integrator.  No counterpart in the
 * reference: its one granularity knob is the compile-time chunk width Delta,
 * chosen per task by a sweep (CHUNK_SELECTION.md:44-62).  This engine's
 * results do not depend on Delta (one-step bins), and its launch choices per
 * layer are these; every plan gives bit-identical results.  Fields: 0 = the
 * built-in choice.
 *   path:   VDTTFS_PATH_BINS (bucketize + per-pixel merge), VDTTFS_PATH_DENSE
 *           (merge straight from the spike map; conv layers with <= 9 taps,
 *           C_in <= 64, or narrow layers with <= 25 taps), VDTTFS_PATH_FUSED
 *           (merge and integrate in one kernel, the list kept in LDS, T <=
 *           64: per wave for dense layers and conv layers with <= 9 taps and
 *           C_in <= 128, gather 1 with C_out <= 64, four events per 16-byte
 *           load, or gather 2 with C_out <= 128; past those limits one
 *           pixel's list shared by a workgroup's waves, conv layers with <= 9
 *           taps and FC layers, gather 1, 2 or 4 (C_out > 128), ppw 1; with
 *           gather 4 and ppw 4, one position of four images per wave, each
 *           weight row applied to every image holding the event (selectable,
 *           slower); counting forwards of a gather-2 layer run it as DENSE,
 *           of a layer past C_in 64 as BINS), VDTTFS_PATH_REG (no
 *           list: each lane keeps its receptive field in registers; conv
 *           layers with K_h*K_w*C_in <= 32, C_out <= 64, T <= 64; gather 1,
 *           ppw 64 / C_out; counting forwards run it as DENSE or FUSED),
 *           VDTTFS_PATH_WINDOW (bucketize, then one kernel merges each
 *           pixel's column lists through a 64-entry register window and
 *           streams them, no merged list in memory; conv layers with <= 9
 *           taps and FC layers, C_out >= 32, T <= 64)
 *   gather: 1 one c_out per lane; 2 two events per 16-byte load, 128 c_out
 *           per wave (C_out a multiple of 4); 4 four c_out per lane, 256
 *           c_out per wave (C_out a multiple of 4)
 *   ppw:    output pixels per wave, 1..8
 * Conv layers with C_out < 32 run one pixel per C_out lanes (gather 1, ppw =
 * 64 / C_out, paths BINS or DENSE); FC layers with C_out < 32 run that way
 * (BINS) or, built in where it takes them (T <= 64), on the shared-list
 * kernel (FUSED, gather 1, ppw 1); layers outside the merged-list limits
 * (> 25 taps) take the generic integrator (path BINS, gather and ppw 0).
 * Pool and vmem layers have no plan.  set_plan(NULL) restores the built-in
 * choice; an unsupported request fails with VDTTFS_E_UNSUPPORTED and leaves
 * the layer's plan unchanged.  get_plan returns the resolved plan the next
 * forward uses. */
#define VDTTFS_PATH_AUTO   0
#define VDTTFS_PATH_BINS   1
#define VDTTFS_PATH_DENSE  2
#define VDTTFS_PATH_FUSED  3
#define VDTTFS_PATH_REG    4
#define VDTTFS_PATH_WINDOW 5
typedef struct vdttfs_layer_plan {
    int32_t path, gather, ppw;
} vdttfs_layer_plan;
int vdttfs_net_set_plan(vdttfs_net* net, int layer, const vdttfs_layer_plan* plan);
int vdttfs_net_get_plan(vdttfs_net* net, int layer, vdttfs_layer_plan* out);
/* Per-layer event time (bucketize + integrator launches, ms) summed over the
 * timed forwards since the last read (timing enabled with
 * vdttfs_net_set_timing); ms has n_layers entries, pools and vmem read 0.
 * Resets the per-layer sums; vdttfs_net_read_timing keeps its own totals. */
int vdttfs_net_read_layer_timing(vdttfs_net* net, double* ms, int n_layers);
int vdttfs_net_read_timing(vdttfs_net* net, double* integ_ms, int64_t* integ_launches,
                           double* bucket_ms, int64_t* bucket_launches);

/* ---- step-by-step (time-driven) baseline: the reference's GPU
 *      denominator, T1S = task1_lenet_mnist/stepbystep_cuda/
 *      snn_mnist_stepbystep.cu, T2S = task2_vgg16_cifar10/stepbystep_cuda/
 *      bench_vgg_timedriven_baseline.cu ------------------------------------ */
/* Every global step launches every layer: each neuron sums the weights of
 * the inputs that spike at that step and fires once on the decaying
 * threshold.  mode VDTTFS_STEP_T1 (T1S:47-103, 222-244): all layers share
 * the step, V = fma(sum w, kv(t), V), the last layer's first spike is the
 * output (argmin readout), T steps.  mode VDTTFS_STEP_T2 (T2S:53-200,
 * 329-352): weighted layer d integrates at t - (d-1)*tfs in [0, T) with
 * psp = fma chain of w*kv and fires at t - d*tfs, the last weighted layer
 * keeps max(V + b) (argmax readout), (D-1)*tfs + T steps.  Decay and
 * threshold use the context's T, tfs, vth and each layer's tc_fire/td as in
 * vdttfs_net_create; convs use the context's padding rule. */
#define VDTTFS_STEP_T1 1
#define VDTTFS_STEP_T2 2
#define VDTTFS_STEP_T3 3  /* CuLIF network: vdttfs_stepnet_create_culif */
typedef struct vdttfs_stepnet vdttfs_stepnet;
int vdttfs_stepnet_create(vdttfs_ctx* ctx, const vdttfs_layer_desc* layers, int n_layers, int B,
                          int64_t img_elems, int encode_mode, float tc_in, float td_in, int mode,
                          vdttfs_stepnet** out);
int vdttfs_stepnet_destroy(vdttfs_stepnet* net);
/* encode -> all steps -> readout, stream-ordered; d_pred (nullable) gets B classes. */
int vdttfs_stepnet_forward(vdttfs_stepnet* net, const float* d_img, int32_t* d_pred);
/* The last layer's output [B][C] (first-spike steps or max V + b) and the step count. */
int vdttfs_stepnet_output(vdttfs_stepnet* net, const float** d_out, int64_t* elems, int* steps);

/* ---- CuLIF set: task 3 (T3V = task3_dvsgesture/vdttfs_cuda/
 *      snn_inference_timesorted.cu) ------------------------------------ */
/* The current-based LIF neuron of T3V:58-62: per step I = I*decay + in
 * (one fma), V += I, fire at the first step with V >= th.  The context's
 * T is T_TOTAL and delta is CHUNK_SIZE; delta must divide T (the reference
 * chunk loop has no t < T guard).  Maps are NCHW and weights OIHW / [out][in]
 * as in the reference; bucket lists are the reference layout with
 * OS = T/delta + 1 offsets per site. */

/* conv1_raw_early (T3V:30-65): 3x3, pad 1, over a dense event tensor
 * d_data [N][C_in][H][W][T]; d_out [N][C_out][H][W] first-spike steps. */
int vdttfs_culif_conv1_raw(vdttfs_ctx* ctx, const float* d_data, float* d_out,
                           const float* d_weight, int N, int C_in, int C_out, int H, int W,
                           float decay, float th);
/* k_bucketize_conv (T3V:70-90): site = (n, y, x) of an NCHW map. */
int vdttfs_culif_bucketize_conv(vdttfs_ctx* ctx, const float* d_in, int N, int C, int H, int W,
                                int32_t* d_out_cin, float* d_out_tin, int32_t* d_out_off);
/* k_bucketize_fc (T3V:93-106): one site per sample over F features. */
int vdttfs_culif_bucketize_fc(vdttfs_ctx* ctx, const float* d_in, int N, int F,
                              int32_t* d_out_cin, float* d_out_tin, int32_t* d_out_off);
/* conv_bucketed_early (T3V:109-143): 3x3, pad 1, H x W kept. */
int vdttfs_culif_conv(vdttfs_ctx* ctx, const int32_t* d_bcin, const float* d_btin,
                      const int32_t* d_boff, float* d_out, const float* d_weight, int N, int C_in,
                      int C_out, int H, int W, float decay, float th);
/* pool_chunk_early (T3V:146-168): 2x2 spiking pool. */
int vdttfs_culif_pool(vdttfs_ctx* ctx, const float* d_in, float* d_out, int N, int C, int H_in,
                      int W_in, float decay, float th);
/* fc1_bucketed_recurrent (T3V:171-200): d_w [out_f][in_f], d_w_rec
 * [out_f][out_f]; out_f <= 1024. */
int vdttfs_culif_fc_recurrent(vdttfs_ctx* ctx, const int32_t* d_bcin, const float* d_btin,
                              const int32_t* d_boff, float* d_out, const float* d_w,
                              const float* d_w_rec, int N, int in_f, int out_f, float decay,
                              float th);
/* fc2_bucketed_early (T3V:203-225): d_w [out_f][in_f]. */
int vdttfs_culif_fc(vdttfs_ctx* ctx, const int32_t* d_bcin, const float* d_btin,
                    const int32_t* d_boff, float* d_out, const float* d_w, int N, int in_f,
                    int out_f, float decay, float th);
/* Readout T3V:291-298 (argmin seeded with class 0). */
int vdttfs_readout_argmin_first(vdttfs_ctx* ctx, const float* d_out, int B, int C,
                                int32_t* d_pred);

/* CuLIF network engine: the T3V main() layer sequence (T3V:276-289).  The
 * first layer is RAW_CONV over the dense event tensor; conv maps stay NHWC
 * inside the engine (weights are re-laid out at creation), FC inputs are
 * flattened in the reference's NCHW order. */
#define VDTTFS_CULIF_RAW_CONV 0
#define VDTTFS_CULIF_CONV     1
#define VDTTFS_CULIF_POOL     2
#define VDTTFS_CULIF_FC_REC   3
#define VDTTFS_CULIF_FC       4

typedef struct vdttfs_culif_layer {
    int32_t kind;
    int32_t C_in, H_in, W_in, C_out;  /* FC: C_in = input features, H_in = W_in = 1 */
    const float* weight;              /* host: conv OIHW [C_out][C_in][3][3], FC [out][in]; pool NULL */
    const float* weight_rec;          /* host: FC_REC [out][out], else NULL */
    float decay, th;
} vdttfs_culif_layer;

typedef struct vdttfs_culif_net vdttfs_culif_net;

int vdttfs_culif_net_create(vdttfs_ctx* ctx, const vdttfs_culif_layer* layers, int n_layers,
                            int B, vdttfs_culif_net** out);
int vdttfs_culif_net_destroy(vdttfs_culif_net* net);
/* d_data [B][C_in][H][W][T] -> per-layer maps -> d_pred (nullable, B int32,
 * T3V:291-298), stream-ordered. */
int vdttfs_culif_net_forward(vdttfs_culif_net* net, const float* d_data, int32_t* d_pred);
/* Layer i's output after a forward; *nhwc = 1 when the map is NHWC
 * (engine conv / pool layers), 0 when NCHW or FC [B][C]. */
int vdttfs_culif_net_layer_output(vdttfs_culif_net* net, int layer, const float** d_out,
                                  int64_t* elems, int32_t* nhwc);
/* Per-layer event timing: when enabled, forward() brackets every layer with
 * HIP events on the context stream; read_timing synchronises and writes the
 * summed milliseconds per layer (ms[n_layers]) and the number of timed
 * forwards since the last read. */
int vdttfs_culif_net_set_timing(vdttfs_culif_net* net, int enable);
int vdttfs_culif_net_read_timing(vdttfs_culif_net* net, double* ms, int64_t* forwards);
/* One instrumented forward (T3M-style counts): for every CONV layer the
 * integrated-synapse count under the reference's chunk-granular early exit
 * (eproc) and under the per-bin exit executed (ebin), the retained input
 * events (n_ev) and bucket columns (n_cols); 0 for other layers. */
int vdttfs_culif_net_count(vdttfs_culif_net* net, const float* d_data, uint64_t* eproc,
                           uint64_t* ebin, uint64_t* n_ev, uint64_t* n_cols);

/* Step-by-step CuLIF baseline, T3S = task3_dvsgesture/stepbystep_cuda/
 * snn_dvs_stepbystep.cu: for each of the context's T steps (T3S:220-252),
 * every layer of the same table as vdttfs_culif_net_create computes every
 * neuron's input current densely from that step's 0/1 spike map (the raw
 * events for layer 0) -- conv over c_in, ky, kx, FC over inputs ascending,
 * as fma(in, w, sum); the recurrent FC adds W_rec times its own spikes of
 * step t-1 -- then runs the CuIF neuron I = fma(I, decay, cur); V += I,
 * spiking once at V >= th (T3S:119-140).  Runs on the vdttfs_stepnet_*
 * calls: forward(d_data [B][C_in][H][W][T], d_pred) with the first-spike
 * readout (argmin from class 0, T3S:274-279); output gives the last layer's
 * first-spike steps (9999 = none) and T. */
int vdttfs_stepnet_create_culif(vdttfs_ctx* ctx, const vdttfs_culif_layer* layers, int n_layers, int B,
                                vdttfs_stepnet** out);

/* ---- gather-roof probe (measurement; no reference counterpart) --------- */
/* The integrator's weight-gather pattern alone: `waves` waves each stream
 * n_ev wave-uniform random row offsets (scalar loads, 8 per group) and issue
 * one buffer_load of 4*vec bytes per lane per row (vec 1, 2 or 4: 256, 512 or
 * 1024 B per wave-gather) into a buffer of footprint_bytes; one fma per dword.
 * Allocates and frees its own buffers, times `reps` launches after a warm-up
 * on the context stream and returns the milliseconds per launch.  The rate
 * n_ev * waves * 256 * vec bytes / time is the roof the stream kernels are
 * held against (footprints inside one XCD's L2 model a layer's weights). */
int vdttfs_probe_gather(vdttfs_ctx* ctx, int vec, int64_t footprint_bytes, int n_ev, int64_t waves, int reps,
                        double* ms_per_launch);

/* ---- synthetic workloads (counter-mode splitmix64; host) --------------- */
/* u = (z>>40) * 2^-24 with z = mix(seed + 0x9E3779B97F4A7C15*(stream*2^40+i+1)). */
int vdttfs_synth_uniform(uint64_t seed, uint64_t stream, float* out, int64_t n);
/* Box-Muller in fp64, scaled by sigma, rounded to fp32. */
int vdttfs_synth_normal(uint64_t seed, uint64_t stream, float* out, int64_t n, double sigma);
/* Config 4 event tensor out[N][C][H][W][T] in {0,1}: per sample a Gaussian
 * blob of `sigma` px whose centre starts uniform in the middle half of the
 * field and moves linearly at a per-axis velocity uniform in [-vmax, vmax]
 * px/step; p(c,y,x,t) = min(1, scale*exp(-d^2/(2 sigma^2))) with scale set
 * per sample so the mean of p over (y,x,t) is `density`; every element is
 * Bernoulli(p) from stream 2000+n.  scales (nullable, N doubles) receives the
 * per-sample scale. */
int vdttfs_synth_dvs(uint64_t seed, int N, int C, int H, int W, int T, double density,
                     double sigma, double vmax, float* out, double* scales);

#ifdef __cplusplus
}
#endif
#endif
