// vdttfs_layer_forward_noalloc: the engine layer path with a library-resident
// scratch buffer instead of context-grown allocations, for callers that must
// not allocate device memory (HIP graph capture, tight serving loops).
//
// The merged event lists, bin starts and the bin-layout bucketize output of a
// layer live in `scratch`, one file-scope device array per GPU the library
// runs on (held until the process ends).  In host code the array's name is a
// host-side stand-in, not a device address: each device's copy is looked up
// once with hipGetSymbolAddress when a context is created on it
// (noalloc_setup, called by vdttfs_create; if that fails the entry point
// retries and reports it) and only that pointer is ever passed to kernels.
// No kernel needs the scratch cleared: every entry a stream kernel reads
// (list, zero tail, bin starts, bucket offsets) is written by the list
// builders of the same call.
//
// Calls that use the scratch are ordered on the device in the order they are
// made, whatever their context or stream: under one lock, each waits on a
// per-device event recorded after the previous such call's kernels, then
// records it after its own.  A call on a stream under graph capture skips
// the event (the captured graph's replays are ordered by the caller).
#include <mutex>

#include "common.h"

namespace vdttfs {

constexpr size_t kScratchBytes = size_t(64) << 20;  // 64 MiB per device

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];         // device address of `scratch` per device, set once
hipEvent_t g_done[kMaxDevices];   // recorded after each scratch-using call's kernels
bool g_recorded[kMaxDevices];     // g_done has been recorded at least once

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// With g_mu held and `device` current.
int setup_locked(int device) {
    if (device < 0 || device >= kMaxDevices)
        return set_error(VDTTFS_E_UNSUPPORTED, "device %d beyond the scratch table (%d)", device, kMaxDevices);
    if (g_ptr[device]) return VDTTFS_OK;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
        (void)hipGetLastError();
        return set_error(VDTTFS_E_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", device,
                         hipGetErrorString(e));
    }
    e = hipEventCreateWithFlags(&g_done[device], hipEventDisableTiming);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_error(VDTTFS_E_HIP, "event for the scratch order on device %d: %s", device, hipGetErrorString(e));
    }
    g_ptr[device] = p;
    return VDTTFS_OK;
}

}  // namespace

// Called by vdttfs_create with `device` current.  Only the scratch-free entry
// point needs what it sets up, so a failure here does not fail the context:
// the entry point retries and returns the error.
int noalloc_setup(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    return setup_locked(device);
}

size_t noalloc_scratch_bytes() { return kScratchBytes; }

}  // namespace vdttfs

using namespace vdttfs;

extern "C" int vdttfs_layer_forward_noalloc(vdttfs_ctx* ctx, float* d_out, const float* d_in,
                                            const float* d_kernel, const float* d_bias,
                                            const float* d_lut_decay, const float* d_lut_th, int t_min,
                                            int B, int H_in, int W_in, int C_in, int H_out, int W_out,
                                            int C_out, int K_h, int K_w, int is_fc) {
    VD_TRY(check_ctx(ctx));
    if (!d_out || !d_in || !d_kernel || !d_bias || !d_lut_decay || !d_lut_th)
        return set_error(VDTTFS_E_INVALID, "layer_forward_noalloc: null buffer");
    IntegShape s{};
    s.B = B;
    s.is_fc = is_fc ? 1 : 0;
    s.H_in = is_fc ? 1 : H_in;
    s.W_in = is_fc ? 1 : W_in;
    s.C_in = C_in;
    s.H_out = is_fc ? 1 : H_out;
    s.W_out = is_fc ? 1 : W_out;
    s.C_out = C_out;
    s.K_h = is_fc ? 1 : K_h;
    s.K_w = is_fc ? 1 : K_w;
    const bool same = !is_fc && ctx->c.conv_same_pad;  // T2V:109-110
    s.pad_h = same ? K_h / 2 : 0;
    s.pad_w = same ? K_w / 2 : 0;
    VD_TRY(check_integ_shape(ctx, s));
    // held until this call's kernels are enqueued and its event recorded
    std::lock_guard<std::mutex> lk(g_mu);
    VD_TRY(setup_locked(ctx->device));
    void* base = g_ptr[ctx->device];
    LaunchPlan p;
    VD_TRY(resolve_plan(ctx, s, LaunchPlan{}, &p));
    const int64_t cols = s.is_fc ? s.B : (int64_t)s.B * s.H_in * s.W_in;
    const int64_t n_pix = s.is_fc ? s.B : (int64_t)s.B * s.H_out * s.W_out;
    const int64_t cap = merged_list_cap(s);
    const bool dense = plan_from_dense(ctx, s, p, false);
    const bool lds_list = plan_lds_list(ctx, s, p, false, false);
    // scratch layout: [merged list | bin starts | bin-layout events | bin offsets]
    const size_t list_b = lds_list ? 0 : align256((size_t)n_pix * cap * sizeof(int2));
    const size_t bs_b = lds_list ? 0 : align256((size_t)n_pix * (ctx->c.T + 1) * 4);
    const size_t ev_b = dense ? 0 : align256((size_t)cols * C_in * sizeof(vd_event));
    const size_t off_b = dense ? 0 : align256((size_t)cols * (ctx->c.T + 1) * 4);
    const size_t need = list_b + bs_b + ev_b + off_b;
    if (need > kScratchBytes)
        return set_error(VDTTFS_E_UNSUPPORTED,
                         "layer_forward_noalloc: the layer needs %zu bytes of scratch, the static buffer "
                         "holds %zu (use vdttfs_layer_forward, or a smaller batch)",
                         need, kScratchBytes);
    unsigned char* sp = static_cast<unsigned char*>(base);
    int2* list = list_b ? reinterpret_cast<int2*>(sp) : nullptr;
    int32_t* bstart = bs_b ? reinterpret_cast<int32_t*>(sp + list_b) : nullptr;
    vd_event* ev = ev_b ? reinterpret_cast<vd_event*>(sp + list_b + bs_b) : nullptr;
    int32_t* off = off_b ? reinterpret_cast<int32_t*>(sp + list_b + bs_b + ev_b) : nullptr;
    if (need == 0)  // lists in LDS: the scratch is not touched, nothing to order
        return launch_integrate_dense(ctx, d_out, d_in, d_lut_decay, list, cap, bstart, d_kernel, d_bias,
                                      d_lut_th, t_min, s, nullptr, nullptr, &p);
    // after the previous scratch-using call on this GPU, in call order
    const int dev = ctx->device;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    VD_HIP(hipStreamIsCapturing(ctx->stream, &cs));
    const bool order = cs == hipStreamCaptureStatusNone;
    if (order && g_recorded[dev]) VD_HIP(hipStreamWaitEvent(ctx->stream, g_done[dev], 0));
    int rc;
    if (dense) {
        rc = launch_integrate_dense(ctx, d_out, d_in, d_lut_decay, list, cap, bstart, d_kernel, d_bias, d_lut_th,
                                    t_min, s, nullptr, nullptr, &p);
    } else {
        rc = launch_bucketize_bins(ctx, d_in, cols, C_in, d_lut_decay, ev, off, nullptr);
        if (rc == VDTTFS_OK)
            rc = launch_integrate_bins(ctx, d_out, ev, off, list, cap, bstart, d_kernel, d_bias, d_lut_th, t_min,
                                       s, nullptr, nullptr, &p);
    }
    if (order) {
        VD_HIP(hipEventRecord(g_done[dev], ctx->stream));
        g_recorded[dev] = true;
    }
    return rc;
}
