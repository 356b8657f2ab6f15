// Internal declarations shared by the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

#include "vdttfs.h"

// One retained spike event of the engine's bin-sorted layout: presynaptic
// index and arrival bin packed in `key` (cin in bits 0..23, bin in 24..31),
// and the decay-LUT value alpha already gathered for this event.
struct __align__(8) vd_event {
    uint32_t key;
    float alpha;
};

struct vdttfs_ctx {
    vdttfs_consts c;
    int NC;  // ceil(T/delta)
    int OS;  // NC + 1
    int device;
    hipStream_t stream;
    // reference-layout bucket scratch (launch wrappers)
    void* ref_cin;
    void* ref_tin;
    void* ref_off;
    size_t ref_elems, ref_cols;
    // engine bin-layout scratch
    void* bin_ev;
    void* bin_off;
    size_t bin_elems, bin_cols;
    // engine merged per-pixel event lists
    void* mrg_list;
    void* mrg_bstart;
    size_t mrg_list_elems, mrg_bstart_elems;
    unsigned long long* d_counters;  // kCounterStripes x 4 u64 (summed on the host)
    hipEvent_t timer[2];             // vdttfs_timer_begin/end (created on first use)
    bool timer_ready;
};

namespace vdttfs {

// Work counters (E_proc, E_bin, retained events) are striped: a kernel adds
// to counters[4 * (blockIdx.x % kCounterStripes) + k], and the host sums the
// stripes, so a million waves do not serialise on one address.
constexpr int kCounterStripes = 64;
#ifdef __HIPCC__
__device__ __forceinline__ unsigned long long* counter_stripe(unsigned long long* c) {
    return c + 4 * (blockIdx.x % kCounterStripes);
}
#endif
int zero_counters(vdttfs_ctx* ctx);
// Waits for the stream and sums the stripes into out[0..3].
int read_counters(vdttfs_ctx* ctx, unsigned long long out[4]);

int set_error(int code, const char* fmt, ...);
int hip_error(hipError_t e, const char* what, int line);
int check_ctx(vdttfs_ctx* ctx);

#define VD_HIP(call)                                                        \
    do {                                                                    \
        hipError_t vd_e_ = (call);                                          \
        if (vd_e_ != hipSuccess) return vdttfs::hip_error(vd_e_, #call, __LINE__); \
    } while (0)

#define VD_TRY(expr)                  \
    do {                              \
        int vd_rc_ = (expr);          \
        if (vd_rc_ != VDTTFS_OK) return vd_rc_; \
    } while (0)

// scratch management (ctx-owned, grown on demand; hipMalloc outside any
// timed region of the engine, which pre-sizes at net creation)
int ensure_ref_scratch(vdttfs_ctx* ctx, size_t elems, size_t cols);
int ensure_bin_scratch(vdttfs_ctx* ctx, size_t elems, size_t cols);
int ensure_merge_scratch(vdttfs_ctx* ctx, size_t list_elems, size_t bstart_elems);

// ---- kernel launchers (stream-ordered on ctx->stream) ----
int launch_encode_log(vdttfs_ctx* ctx, const float* img, float* out, int64_t n, float tc, float td);
int launch_encode_linear(vdttfs_ctx* ctx, const float* img, float* out, int64_t n);

int launch_bucketize_ref(vdttfs_ctx* ctx, const float* in, int64_t n_cols, int c_in,
                         int32_t* out_cin, float* out_tin, int32_t* out_off);
int launch_bucketize_bins(vdttfs_ctx* ctx, const float* in, int64_t n_cols, int c_in,
                          const float* alpha, vd_event* out_ev, int32_t* out_off,
                          unsigned long long* n_ev_counter);

int launch_integrate_ref(vdttfs_ctx* ctx, float* out, const int32_t* cin, const float* tin,
                         const int32_t* off, const float* W, const float* bias,
                         const float* alpha, const float* theta, int t_min, int B, int H_in,
                         int W_in, int C_in, int H_out, int W_out, int C_out, int K_h, int K_w,
                         int is_fc);

// CuLIF neuron constants (T3V:24-27 per layer; one decay and threshold).
// Integration with a CuLIF neuron adds weights unscaled (the reference's
// acc + w): its callers pass an all-ones alpha LUT, and the fused kernel
// (k_stream_quad) does not read it.  fired: nullable, one byte per input
// site (NHWC pixel of the input map), nonzero exactly where some channel of
// the site holds a spike; the fused build then skips silent fields unread.
struct CulifNeuron {
    float decay, th;
    const uint8_t* fired = nullptr;
};

struct IntegShape {
    int B, H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad_h, pad_w, is_fc;
};
// Entries per pixel of the merged event list (receptive events + padding).
int merged_list_cap(const IntegShape& s);
// Launch choices of one layer on the merged-list integrator (0 = the
// built-in choice): the list path (bucketize + k_merge, k_merge_dense, or
// the fused k_stream_dense), the weight gather (1: one c_out per lane, 2: two
// events per dwordx4 load, 4: four c_out per lane) and output pixels per
// wave.  Values as VDTTFS_PATH_* / vdttfs_layer_plan.
struct LaunchPlan {
    int path = 0, gather = 0, ppw = 0;
};
constexpr int kMaxPixPerWave = 8;
// The plan's lists come from the bin-layout bucketize (the bins and window paths).
inline bool plan_bins(const LaunchPlan& p) { return p.path == VDTTFS_PATH_BINS || p.path == VDTTFS_PATH_WINDOW; }
// Whether a layer integrated under resolved plan p builds its merged lists in
// LDS (so it needs no merged-list scratch), with or without counters and the
// CuLIF neuron.
bool plan_lds_list(const vdttfs_ctx* ctx, const IntegShape& sh, const LaunchPlan& p, bool counters, bool culif);
// Fills every field of *out: a requested field is checked against the
// layer's shape (VDTTFS_E_UNSUPPORTED when the kernels cannot run it), a zero
// field takes the built-in choice.
int resolve_plan(const vdttfs_ctx* ctx, const IntegShape& s, const LaunchPlan& req, LaunchPlan* out);

// Engine integrator over the bin layout: merge per pixel, then stream.
// list/bstart: merged-list scratch of n_pix*list_cap entries and
// n_pix*(T+1) bin starts.  counters: nullable; [0] += eproc, [1] += ebin.
// culif: nullable; selects the CuLIF neuron (bias, theta and t_min unused).
int launch_integrate_bins(vdttfs_ctx* ctx, float* out, const vd_event* ev, const int32_t* off,
                          int2* list, int64_t list_cap, int32_t* bstart, const float* W,
                          const float* bias, const float* theta, int t_min, const IntegShape& s,
                          unsigned long long* counters, const CulifNeuron* culif = nullptr,
                          const LaunchPlan* plan = nullptr);
// Conv layers of the merged-list path: the merged lists are built straight
// from the dense spike map d_in (no bucketize pass); alpha is the layer's
// decay LUT.  Same results as bucketize + launch_integrate_bins.
bool integrate_dense_ok(const vdttfs_ctx* ctx, const IntegShape& s);
// Conv layers past those limits (C_in <= 128) that the fused plan still
// builds from the dense map when no counters are asked for.
bool quad_wide_ok(const vdttfs_ctx* ctx, const IntegShape& s);
// Layers the shared-list fused kernel takes under gather 1, 2 or 4 (conv with
// at most 9 taps or FC, T <= 64, no counters), and which fused kernel a
// fused plan with this gather runs: 1 per-wave lists, 2 shared lists, 0 none.
bool shared_ok(const vdttfs_ctx* ctx, const IntegShape& s, int gather);
int fused_kind(const vdttfs_ctx* ctx, const IntegShape& s, int gather);
// Whether a layer under resolved plan p takes launch_integrate_dense (its
// lists built from the dense map) rather than bucketize +
// launch_integrate_bins, with or without counters.
bool plan_from_dense(const vdttfs_ctx* ctx, const IntegShape& s, const LaunchPlan& p, bool counters);
// A 2x2 min pool (T2V:192-209) fused into a layer's list build: `in` of
// launch_integrate_dense is then the pool's input, H_u x W_u x C_in per
// image, and the layer reads its min windows (H_in = H_u / 2, W_in =
// W_u / 2; an FC layer's input is then one 1 x 1 window).
struct PoolIn {
    int H_u, W_u;
};
// Whether the layer under resolved plan p (no counters, LUT neuron) can take
// the pool in its build: the shared-list kernel, or the per-wave kernel past
// 64 receptive elements, with the pool's input below 2^31 bytes.
bool pool_fusable(const vdttfs_ctx* ctx, const IntegShape& s, const LaunchPlan& p, int H_u, int W_u);
int launch_integrate_dense(vdttfs_ctx* ctx, float* out, const float* in, const float* alpha, int2* list,
                           int64_t list_cap, int32_t* bstart, const float* W, const float* bias,
                           const float* theta, int t_min, const IntegShape& s,
                           unsigned long long* counters, const CulifNeuron* culif = nullptr,
                           const LaunchPlan* plan = nullptr, const PoolIn* pool = nullptr);

int launch_pool_min(vdttfs_ctx* ctx, const float* in, float* out, int B, int H_in, int W_in, int C);
int launch_fc_vmem(vdttfs_ctx* ctx, const float* in, float* out, const float* W, const float* bias,
                   const float* alpha, int B, int C_in, int C_out);
// mode: 0 argmin (T1V), 1 argmax (T2V), 2 argmin seeded with class 0 (T3V)
int launch_readout(vdttfs_ctx* ctx, const float* out, int B, int C, int32_t* pred, int mode);

// ---- CuLIF (T3V) ----
int check_culif_consts(const vdttfs_ctx* ctx);
// conv1_raw from per-site masks of nonzero steps (finite weights only; mask
// [N*C_in*H*W][ceil(T/64)] uint64, nonbin the same shape in uint32).
bool culif_conv1_mask_ok(int C_in);
// fired: nullable [N*H*W] bytes, 1 where some neuron of the pixel fired
// (C_out <= 64).
int launch_culif_conv1_mask(vdttfs_ctx* ctx, const float* data, float* out, const float* W, int N, int C_in,
                            int C_out, int H, int Wd, int nhwc_out, float decay, float th, uint64_t* mask,
                            uint32_t* nonbin, uint8_t* fired = nullptr);
int launch_culif_conv1_raw(vdttfs_ctx* ctx, const float* data, float* out, const float* W, int N,
                           int C_in, int C_out, int H, int Wd, int nhwc_out, float decay, float th);
// Reference layout; site s = (n, hw), element c at (n*C + c)*HW + hw (FC: HW = 1).
int launch_culif_bucketize(vdttfs_ctx* ctx, const float* in, int64_t n_sites, int C, int HW,
                           int32_t* cin, float* tin, int32_t* off);
int launch_culif_generic(vdttfs_ctx* ctx, const int32_t* cin, const float* tin, const int32_t* off,
                         float* out, const float* W, int N, int C_in, int C_out, int H, int Wd,
                         int is_fc, float decay, float th);
int launch_culif_pool(vdttfs_ctx* ctx, const float* in, float* out, int N, int C, int H_in, int W_in,
                      int nhwc_in, int nhwc_out, float decay, float th);
// Drop-in (cur == NULL): reference buckets, W [out][in], Wrec [i][j].
// Engine (cur != NULL): feed-forward input per step cur[N][T][out_f] from
// launch_fc_currents, Wrec transposed to [j][i]; cin/tin/off/W unused.
int launch_culif_fc_rec(vdttfs_ctx* ctx, const int32_t* cin, const float* tin, const int32_t* off,
                        const float* cur, float* out, const float* W, const float* Wrec, int N,
                        int in_f, int out_f, float decay, float th);
// cur[n][t][o] = sum over inputs j ascending arriving at step t of W_t[j][o],
// from the dense input x[N][F] (T3V arrival rule).  The inputs are first
// sorted by step into the scratch (sizes in int32 elements from
// fc_sort_sizes; offs has the size of counts).
struct FcSortSizes {
    int segments;
    int64_t counts, binstart, list;
};
struct FcSortScratch {
    int32_t* counts;
    int32_t* offs;
    int32_t* binstart;
    int32_t* list;
};
FcSortSizes fc_sort_sizes(int N, int F, int T);
int launch_fc_currents(vdttfs_ctx* ctx, const float* x, const float* W_t, float* cur, int N, int F, int out_f,
                       const FcSortScratch& sc);
int launch_nhwc_to_nchw(vdttfs_ctx* ctx, const float* in, float* out, int N, int C, int H, int W);

// Layer-table checks of vdttfs_net_create (shapes chain, kinds, weights).
int validate_layer_table(const vdttfs_consts& c, const vdttfs_layer_desc* layers, int n, int64_t img_elems);

// Step-by-step baseline (k_step.hip): one layer of a time-driven network.
struct StepLayer {
    int kind;
    const float* W;
    const float* bias;
    int64_t n;  // neurons: B * H_out * W_out * C_out
    int H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, pad_h, pad_w, is_fc;
};
int launch_step_input(vdttfs_ctx* ctx, const float* tin, uint8_t* s, int64_t n, int t);
int launch_step_neuron(vdttfs_ctx* ctx, const StepLayer& L, const uint8_t* s_in, uint8_t* s_out, float* vmem,
                       uint8_t* fired, float* out, int mode, int int_ok, int fire_ok, int out_layer, float kv,
                       float th, int t);
int launch_step_pool(vdttfs_ctx* ctx, const uint8_t* s_in, uint8_t* s_out, uint8_t* fired, int64_t n, int H_in,
                     int W_in, int C);
int launch_step_fill(vdttfs_ctx* ctx, float* p, int64_t n, float v);

// Step-by-step CuLIF baseline (T3S semantics): one layer of the time-driven
// network, NCHW maps.  kind as VDTTFS_CULIF_*; in/out counts per sample:
// conv C_out*H*W, pool C*(H/2)*(W/2), FC C_out.
struct Step3Layer {
    int kind;
    int C_in, H, W, C_out;
    const float* weight;      // conv OIHW [C_out][C_in][3][3], FC [in][out] (transposed at creation)
    const float* weight_rec;  // FC_REC [j][out] (transposed)
    float* I;
    float* V;
    float* s;            // 0/1 spikes of the step (FC_REC: of step t-1 until its neuron runs)
    uint8_t* fired;
    float* ft;           // first-spike steps
    float* cur;          // FC_REC: input current of the step; RAW_CONV: the step's raw events
    int64_t n;           // neurons
    float decay, th;
};
// Layer checks of vdttfs_culif_net_create (kinds, chained shapes, weights).
int validate_culif_table(const vdttfs_ctx* ctx, const vdttfs_culif_layer* layers, int n);
// One step t of layer L from its input in (RAW_CONV: the event tensor
// [N][C_in][H][W][T]; else the previous layer's spikes of step t).
int launch_step3_layer(vdttfs_ctx* ctx, const Step3Layer& L, const float* in, int N, int T, int t);

// shape validation shared by the entry points
int check_integ_shape(const vdttfs_ctx* ctx, const IntegShape& s);

// The static scratch of vdttfs_layer_forward_noalloc (noalloc.hip): looks up
// `device`'s copy once (hipGetSymbolAddress, `device` current); vdttfs_create
// calls it for every context's device.
int noalloc_setup(int device);
size_t noalloc_scratch_bytes();

}  // namespace vdttfs
