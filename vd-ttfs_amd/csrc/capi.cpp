// C ABI entry points: context, device memory plumbing, LUT builder and the
// reference's per-kernel surface (T1V / T2V host helpers and kernels).
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"

namespace vdttfs {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_error(hipError_t e, const char* what, int line) {
    return set_error(VDTTFS_E_HIP, "HIP error %d (%s) in %s at capi line %d", (int)e,
                     hipGetErrorString(e), what, line);
}

int check_ctx(vdttfs_ctx* ctx) {
    if (ctx == nullptr) return set_error(VDTTFS_E_INVALID, "null context");
    VD_HIP(hipSetDevice(ctx->device));
    return VDTTFS_OK;
}

static int grow(void** p, size_t* have, size_t need_bytes) {
    if (*have >= need_bytes && *p != nullptr) return VDTTFS_OK;
    if (*p) VD_HIP(hipFree(*p));
    *p = nullptr;
    *have = 0;
    if (hipMalloc(p, need_bytes ? need_bytes : 4) != hipSuccess) {
        *p = nullptr;
        return set_error(VDTTFS_E_NOMEM, "device allocation of %zu bytes failed", need_bytes);
    }
    *have = need_bytes;
    return VDTTFS_OK;
}

int ensure_ref_scratch(vdttfs_ctx* ctx, size_t elems, size_t cols) {
    if (elems > ctx->ref_elems || cols > ctx->ref_cols || !ctx->ref_cin) {
        VD_HIP(hipStreamSynchronize(ctx->stream));
        size_t e = elems > ctx->ref_elems ? elems : ctx->ref_elems;
        size_t c = cols > ctx->ref_cols ? cols : ctx->ref_cols;
        size_t h1 = 0, h2 = 0, h3 = 0;
        if (ctx->ref_cin) VD_HIP(hipFree(ctx->ref_cin));
        if (ctx->ref_tin) VD_HIP(hipFree(ctx->ref_tin));
        if (ctx->ref_off) VD_HIP(hipFree(ctx->ref_off));
        ctx->ref_cin = ctx->ref_tin = ctx->ref_off = nullptr;
        VD_TRY(grow(&ctx->ref_cin, &h1, e * 4));
        VD_TRY(grow(&ctx->ref_tin, &h2, e * 4));
        VD_TRY(grow(&ctx->ref_off, &h3, c * (size_t)ctx->OS * 4));
        ctx->ref_elems = e;
        ctx->ref_cols = c;
    }
    return VDTTFS_OK;
}

int ensure_bin_scratch(vdttfs_ctx* ctx, size_t elems, size_t cols) {
    if (elems > ctx->bin_elems || cols > ctx->bin_cols || !ctx->bin_ev) {
        VD_HIP(hipStreamSynchronize(ctx->stream));
        size_t e = elems > ctx->bin_elems ? elems : ctx->bin_elems;
        size_t c = cols > ctx->bin_cols ? cols : ctx->bin_cols;
        size_t h1 = 0, h2 = 0;
        if (ctx->bin_ev) VD_HIP(hipFree(ctx->bin_ev));
        if (ctx->bin_off) VD_HIP(hipFree(ctx->bin_off));
        ctx->bin_ev = ctx->bin_off = nullptr;
        VD_TRY(grow(&ctx->bin_ev, &h1, e * sizeof(vd_event)));
        VD_TRY(grow(&ctx->bin_off, &h2, c * (size_t)(ctx->c.T + 1) * 4));
        ctx->bin_elems = e;
        ctx->bin_cols = c;
    }
    return VDTTFS_OK;
}

int zero_counters(vdttfs_ctx* ctx) {
    VD_HIP(hipMemsetAsync(ctx->d_counters, 0, 4 * kCounterStripes * sizeof(unsigned long long), ctx->stream));
    return VDTTFS_OK;
}

int read_counters(vdttfs_ctx* ctx, unsigned long long out[4]) {
    unsigned long long h[4 * kCounterStripes];
    VD_HIP(hipMemcpyAsync(h, ctx->d_counters, sizeof(h), hipMemcpyDeviceToHost, ctx->stream));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    for (int k = 0; k < 4; ++k) out[k] = 0;
    for (int s = 0; s < kCounterStripes; ++s)
        for (int k = 0; k < 4; ++k) out[k] += h[4 * s + k];
    return VDTTFS_OK;
}

int ensure_merge_scratch(vdttfs_ctx* ctx, size_t list_elems, size_t bstart_elems) {
    if (list_elems > ctx->mrg_list_elems || bstart_elems > ctx->mrg_bstart_elems || !ctx->mrg_list) {
        VD_HIP(hipStreamSynchronize(ctx->stream));
        size_t e = list_elems > ctx->mrg_list_elems ? list_elems : ctx->mrg_list_elems;
        size_t b = bstart_elems > ctx->mrg_bstart_elems ? bstart_elems : ctx->mrg_bstart_elems;
        size_t h1 = 0, h2 = 0;
        if (ctx->mrg_list) VD_HIP(hipFree(ctx->mrg_list));
        if (ctx->mrg_bstart) VD_HIP(hipFree(ctx->mrg_bstart));
        ctx->mrg_list = ctx->mrg_bstart = nullptr;
        VD_TRY(grow(&ctx->mrg_list, &h1, e * sizeof(int2)));
        VD_TRY(grow(&ctx->mrg_bstart, &h2, b * 4));
        ctx->mrg_list_elems = e;
        ctx->mrg_bstart_elems = b;
    }
    return VDTTFS_OK;
}

static int check_consts(const vdttfs_consts* c) {
    if (!c) return set_error(VDTTFS_E_INVALID, "null constants");
    if (c->T < 1 || c->T > 255)
        return set_error(VDTTFS_E_INVALID, "TIME_WINDOW %d outside [1,255]", c->T);
    // CHUNK may exceed TIME_WINDOW: the chunk loop's t < T guard then ends
    // the single chunk early (T1V:151-153)
    if (c->delta < 1 || c->delta > 256)
        return set_error(VDTTFS_E_INVALID, "CHUNK %d outside [1,256]", c->delta);
    if (!std::isfinite(c->tfs) || !std::isfinite(c->vth))
        return set_error(VDTTFS_E_INVALID, "TIME_FIRE_START / VTH_INIT must be finite");
    return VDTTFS_OK;
}

}  // namespace vdttfs

using namespace vdttfs;

extern "C" {

const char* vdttfs_last_error(void) { return g_err; }
const char* vdttfs_version(void) { return "vdttfs-mi355x 0.1 (gfx950)"; }

int vdttfs_device_count(int* out) {
    if (!out) return set_error(VDTTFS_E_INVALID, "null out");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *out = n;
    return VDTTFS_OK;
}

int vdttfs_create(const vdttfs_consts* consts, int device, vdttfs_ctx** out) {
    if (!out) return set_error(VDTTFS_E_INVALID, "null out");
    *out = nullptr;
    VD_TRY(check_consts(consts));
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return set_error(VDTTFS_E_NODEVICE, "no HIP device visible");
    if (device < 0 || device >= n)
        return set_error(VDTTFS_E_INVALID, "device %d out of range (%d devices)", device, n);
    VD_HIP(hipSetDevice(device));
    // the scratch-free entry point's per-device set-up; only that entry point
    // needs it, and it retries and reports a failure itself
    if (noalloc_setup(device) != VDTTFS_OK) (void)hipGetLastError();
    vdttfs_ctx* ctx = new (std::nothrow) vdttfs_ctx();
    if (!ctx) return set_error(VDTTFS_E_NOMEM, "context allocation failed");
    ctx->c = *consts;
    ctx->NC = (consts->T + consts->delta - 1) / consts->delta;
    ctx->OS = ctx->NC + 1;
    ctx->device = device;
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess)
        e = hipMalloc((void**)&ctx->d_counters, 4 * kCounterStripes * sizeof(unsigned long long));
    if (e != hipSuccess) {
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_error(e, "context setup", __LINE__);
    }
    *out = ctx;
    return VDTTFS_OK;
}

int vdttfs_destroy(vdttfs_ctx* ctx) {
    if (!ctx) return VDTTFS_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    void* bufs[] = {ctx->ref_cin, ctx->ref_tin,    ctx->ref_off,   ctx->bin_ev,
                    ctx->bin_off, ctx->mrg_list, ctx->mrg_bstart, ctx->d_counters};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (ctx->timer_ready) {
        (void)hipEventDestroy(ctx->timer[0]);
        (void)hipEventDestroy(ctx->timer[1]);
    }
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return VDTTFS_OK;
}

int vdttfs_timer_begin(vdttfs_ctx* ctx) {
    VD_TRY(check_ctx(ctx));
    if (!ctx->timer_ready) {
        VD_HIP(hipEventCreate(&ctx->timer[0]));
        if (hipEventCreate(&ctx->timer[1]) != hipSuccess) {
            (void)hipEventDestroy(ctx->timer[0]);
            return set_error(VDTTFS_E_HIP, "timer: event creation failed");
        }
        ctx->timer_ready = true;
    }
    VD_HIP(hipEventRecord(ctx->timer[0], ctx->stream));
    return VDTTFS_OK;
}

int vdttfs_timer_end(vdttfs_ctx* ctx, double* ms) {
    VD_TRY(check_ctx(ctx));
    if (!ctx->timer_ready || !ms) return set_error(VDTTFS_E_INVALID, "timer_end without timer_begin");
    VD_HIP(hipEventRecord(ctx->timer[1], ctx->stream));
    VD_HIP(hipEventSynchronize(ctx->timer[1]));
    float f = 0.0f;
    VD_HIP(hipEventElapsedTime(&f, ctx->timer[0], ctx->timer[1]));
    *ms = f;
    return VDTTFS_OK;
}

int vdttfs_get_consts(const vdttfs_ctx* ctx, vdttfs_consts* out) {
    if (!ctx || !out) return set_error(VDTTFS_E_INVALID, "null argument");
    *out = ctx->c;
    return VDTTFS_OK;
}

int vdttfs_num_chunks(const vdttfs_ctx* ctx) { return ctx ? ctx->NC : VDTTFS_E_INVALID; }

int vdttfs_synchronize(vdttfs_ctx* ctx) {
    VD_TRY(check_ctx(ctx));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    return VDTTFS_OK;
}

int vdttfs_dev_alloc(vdttfs_ctx* ctx, size_t bytes, void** dptr) {
    VD_TRY(check_ctx(ctx));
    if (!dptr) return set_error(VDTTFS_E_INVALID, "null out");
    *dptr = nullptr;
    if (hipMalloc(dptr, bytes ? bytes : 4) != hipSuccess) {
        *dptr = nullptr;
        return set_error(VDTTFS_E_NOMEM, "device allocation of %zu bytes failed", bytes);
    }
    return VDTTFS_OK;
}

int vdttfs_dev_free(vdttfs_ctx* ctx, void* dptr) {
    VD_TRY(check_ctx(ctx));
    if (dptr) {
        VD_HIP(hipStreamSynchronize(ctx->stream));
        VD_HIP(hipFree(dptr));
    }
    return VDTTFS_OK;
}

int vdttfs_h2d(vdttfs_ctx* ctx, void* dst, const void* src, size_t bytes) {
    VD_TRY(check_ctx(ctx));
    if (bytes == 0) return VDTTFS_OK;
    if (!dst || !src) return set_error(VDTTFS_E_INVALID, "null pointer");
    VD_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    return VDTTFS_OK;
}

int vdttfs_d2h(vdttfs_ctx* ctx, void* dst, const void* src, size_t bytes) {
    VD_TRY(check_ctx(ctx));
    if (bytes == 0) return VDTTFS_OK;
    if (!dst || !src) return set_error(VDTTFS_E_INVALID, "null pointer");
    VD_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    return VDTTFS_OK;
}

int vdttfs_memset(vdttfs_ctx* ctx, void* dptr, int value, size_t bytes) {
    VD_TRY(check_ctx(ctx));
    if (bytes == 0) return VDTTFS_OK;
    if (!dptr) return set_error(VDTTFS_E_INVALID, "null pointer");
    VD_HIP(hipMemsetAsync(dptr, value, bytes, ctx->stream));
    return VDTTFS_OK;
}

// T1V:208-216 / T2V:236-243: host expf with true division.
int vdttfs_build_luts_host(const vdttfs_consts* c, float tc_integ, float td_integ,
                           float tc_fire, float td_fire, float* alpha, float* theta) {
    VD_TRY(check_consts(c));
    if (!alpha || !theta) return set_error(VDTTFS_E_INVALID, "null LUT buffer");
    for (int t = 0; t <= c->T; ++t) alpha[t] = expf(-((float)t - td_integ) / tc_integ);
    for (int t = 0; t < c->T; ++t) theta[t] = c->vth * expf(-((float)t - td_fire) / tc_fire);
    return VDTTFS_OK;
}

int vdttfs_update_luts(vdttfs_ctx* ctx, float* d_lut_decay, float* d_lut_th, float tc_integ,
                       float td_integ, float tc_fire, float td_fire) {
    VD_TRY(check_ctx(ctx));
    if (!d_lut_decay || !d_lut_th) return set_error(VDTTFS_E_INVALID, "null LUT buffer");
    std::vector<float> a(ctx->c.T + 1), th(ctx->c.T);
    VD_TRY(vdttfs_build_luts_host(&ctx->c, tc_integ, td_integ, tc_fire, td_fire, a.data(), th.data()));
    VD_HIP(hipMemcpyAsync(d_lut_decay, a.data(), a.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    VD_HIP(hipMemcpyAsync(d_lut_th, th.data(), th.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    return VDTTFS_OK;
}

int vdttfs_encode_image(vdttfs_ctx* ctx, const float* d_img, float* d_out, int64_t size, float tc,
                        float td) {
    VD_TRY(check_ctx(ctx));
    if (size < 0 || (size > 0 && (!d_img || !d_out))) return set_error(VDTTFS_E_INVALID, "encode: bad args");
    return launch_encode_log(ctx, d_img, d_out, size, tc, td);
}

int vdttfs_encode_linear(vdttfs_ctx* ctx, const float* d_img, float* d_out, int64_t size) {
    VD_TRY(check_ctx(ctx));
    if (size < 0 || (size > 0 && (!d_img || !d_out))) return set_error(VDTTFS_E_INVALID, "encode: bad args");
    return launch_encode_linear(ctx, d_img, d_out, size);
}

int vdttfs_bucketize(vdttfs_ctx* ctx, const float* d_in, int64_t n_cols, int c_in,
                     int32_t* d_out_cin, float* d_out_tin, int32_t* d_out_off) {
    VD_TRY(check_ctx(ctx));
    if (n_cols < 0 || c_in <= 0) return set_error(VDTTFS_E_INVALID, "bucketize: bad sizes");
    if (n_cols > 0 && (!d_in || !d_out_cin || !d_out_tin || !d_out_off))
        return set_error(VDTTFS_E_INVALID, "bucketize: null buffer");
    return launch_bucketize_ref(ctx, d_in, n_cols, c_in, d_out_cin, d_out_tin, d_out_off);
}

static IntegShape make_shape(const vdttfs_ctx* ctx, int B, int H_in, int W_in, int C_in, int H_out,
                             int W_out, int C_out, int K_h, int K_w, int is_fc) {
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
    // T2V:109-110: same padding is K_h/2 rows and K_w/2 columns
    const bool same = !is_fc && ctx->c.conv_same_pad;
    s.pad_h = same ? K_h / 2 : 0;
    s.pad_w = same ? K_w / 2 : 0;
    return s;
}

// One layer on the engine's kernels (list built in LDS, from the dense map
// or from the bin-layout bucketize, then the wave-per-pixel stream) with the
// built-in launch plan and context-owned scratch.  Scratch is sized for what
// the layer's plan uses: the fused, window and register paths need no merged
// list.
static int engine_layer(vdttfs_ctx* ctx, float* d_out, const float* d_in, const float* d_kernel,
                        const float* d_bias, const float* d_lut_decay, const float* d_lut_th, int t_min,
                        const IntegShape& s, unsigned long long* counters) {
    LaunchPlan p;
    VD_TRY(resolve_plan(ctx, s, LaunchPlan{}, &p));
    const int64_t cols = s.is_fc ? s.B : (int64_t)s.B * s.H_in * s.W_in;
    const int64_t n_pix = s.is_fc ? s.B : (int64_t)s.B * s.H_out * s.W_out;
    const int64_t cap = merged_list_cap(s);
    const bool dense = plan_from_dense(ctx, s, p, counters != nullptr);
    const bool lds_list = plan_lds_list(ctx, s, p, counters != nullptr, false);
    if (!lds_list)
        VD_TRY(ensure_merge_scratch(ctx, (size_t)(n_pix * cap), (size_t)n_pix * (ctx->c.T + 1)));
    if (dense)  // conv: merged lists straight from the dense map
        return launch_integrate_dense(ctx, d_out, d_in, d_lut_decay, (int2*)ctx->mrg_list, cap,
                                      (int32_t*)ctx->mrg_bstart, d_kernel, d_bias, d_lut_th, t_min, s,
                                      counters, nullptr, &p);
    VD_TRY(ensure_bin_scratch(ctx, (size_t)cols * s.C_in, (size_t)cols));
    VD_TRY(launch_bucketize_bins(ctx, d_in, cols, s.C_in, d_lut_decay, (vd_event*)ctx->bin_ev,
                                 (int32_t*)ctx->bin_off, nullptr));
    return launch_integrate_bins(ctx, d_out, (const vd_event*)ctx->bin_ev, (const int32_t*)ctx->bin_off,
                                 (int2*)ctx->mrg_list, cap, (int32_t*)ctx->mrg_bstart, d_kernel, d_bias,
                                 d_lut_th, t_min, s, counters, nullptr, &p);
}

int vdttfs_integrate(vdttfs_ctx* ctx, float* d_out, const int32_t* d_bkt_cin,
                     const float* d_bkt_tin, const int32_t* d_bkt_off, const float* d_kernel,
                     const float* d_bias, const float* d_lut_decay, const float* d_lut_th,
                     int t_min, int B, int H_in, int W_in, int C_in, int H_out, int W_out,
                     int C_out, int K_h, int K_w, int is_fc) {
    VD_TRY(check_ctx(ctx));
    IntegShape s = make_shape(ctx, B, H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, is_fc);
    VD_TRY(check_integ_shape(ctx, s));
    if (!d_out || !d_bkt_cin || !d_bkt_tin || !d_bkt_off || !d_kernel || !d_bias || !d_lut_decay ||
        !d_lut_th)
        return set_error(VDTTFS_E_INVALID, "integrate: null buffer");
    return launch_integrate_ref(ctx, d_out, d_bkt_cin, d_bkt_tin, d_bkt_off, d_kernel, d_bias,
                                d_lut_decay, d_lut_th, t_min, B, H_in, W_in, C_in, H_out, W_out,
                                C_out, K_h, K_w, is_fc);
}

int vdttfs_layer_forward(vdttfs_ctx* ctx, float* d_out, const float* d_in,
                         const float* d_kernel, const float* d_bias, const float* d_lut_decay,
                         const float* d_lut_th, int t_min, int B, int H_in, int W_in, int C_in,
                         int H_out, int W_out, int C_out, int K_h, int K_w, int is_fc,
                         uint64_t* eproc, uint64_t* ebin) {
    VD_TRY(check_ctx(ctx));
    IntegShape s = make_shape(ctx, B, H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, is_fc);
    VD_TRY(check_integ_shape(ctx, s));
    if (!d_out || !d_in || !d_kernel || !d_bias || !d_lut_decay || !d_lut_th)
        return set_error(VDTTFS_E_INVALID, "layer_forward: null buffer");
    const bool count = eproc || ebin;
    if (count) VD_TRY(zero_counters(ctx));
    VD_TRY(engine_layer(ctx, d_out, d_in, d_kernel, d_bias, d_lut_decay, d_lut_th, t_min, s,
                        count ? ctx->d_counters : nullptr));
    if (count) {
        unsigned long long h[4];
        VD_TRY(read_counters(ctx, h));
        if (eproc) *eproc = h[0];
        if (ebin) *ebin = h[1];
    }
    return VDTTFS_OK;
}

int vdttfs_pool_min(vdttfs_ctx* ctx, const float* d_in, float* d_out, int B, int H_in, int W_in,
                    int C) {
    VD_TRY(check_ctx(ctx));
    if (B < 0 || H_in < 0 || W_in < 0 || C < 0) return set_error(VDTTFS_E_INVALID, "pool: bad sizes");
    return launch_pool_min(ctx, d_in, d_out, B, H_in, W_in, C);
}

int vdttfs_fc_vmem(vdttfs_ctx* ctx, const float* d_in, float* d_out, const float* d_kernel,
                   const float* d_bias, const float* d_lut_decay, int B, int C_in, int C_out) {
    VD_TRY(check_ctx(ctx));
    if (B < 0 || C_in <= 0 || C_out <= 0) return set_error(VDTTFS_E_INVALID, "fc_vmem: bad sizes");
    return launch_fc_vmem(ctx, d_in, d_out, d_kernel, d_bias, d_lut_decay, B, C_in, C_out);
}

int vdttfs_readout_argmin(vdttfs_ctx* ctx, const float* d_out, int B, int C, int32_t* d_pred) {
    VD_TRY(check_ctx(ctx));
    if (B < 0 || C <= 0) return set_error(VDTTFS_E_INVALID, "readout: bad sizes");
    return launch_readout(ctx, d_out, B, C, d_pred, 0);
}

int vdttfs_readout_argmax(vdttfs_ctx* ctx, const float* d_out, int B, int C, int32_t* d_pred) {
    VD_TRY(check_ctx(ctx));
    if (B < 0 || C <= 0) return set_error(VDTTFS_E_INVALID, "readout: bad sizes");
    return launch_readout(ctx, d_out, B, C, d_pred, 1);
}

// T1V:222-234 / T2V:250-274.  The reference's wrapper runs k_bucketize into
// file-static scratch, then k_conv_bucketed, then synchronises; its caller
// never reads the buckets.  This one runs the engine's kernels on the same
// dense map (same first-spike times, bit for bit), then synchronises.
int vdttfs_launch_layer_sync(vdttfs_ctx* ctx, const float* d_in, float* d_out, int H_in, int W_in,
                             int C_in, int H_out, int W_out, int C_out, int K_h, int K_w, float td,
                             const float* d_kernel, const float* d_bias, const float* d_lut_decay,
                             const float* d_lut_th, int B, int is_fc) {
    VD_TRY(check_ctx(ctx));
    int t_min = (int)ceilf(td);
    if (t_min < 0) t_min = 0;
    IntegShape s = make_shape(ctx, B, H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, is_fc);
    VD_TRY(check_integ_shape(ctx, s));
    if (!d_out || !d_in || !d_kernel || !d_bias || !d_lut_decay || !d_lut_th)
        return set_error(VDTTFS_E_INVALID, "launch_layer: null buffer");
    VD_TRY(engine_layer(ctx, d_out, d_in, d_kernel, d_bias, d_lut_decay, d_lut_th, t_min, s, nullptr));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    return VDTTFS_OK;
}

int vdttfs_launch_pool_sync(vdttfs_ctx* ctx, const float* d_in, float* d_out, int H_in, int W_in,
                            int C, int B) {
    VD_TRY(vdttfs_pool_min(ctx, d_in, d_out, B, H_in, W_in, C));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    return VDTTFS_OK;
}

int vdttfs_launch_fc_vmem_sync(vdttfs_ctx* ctx, const float* d_in, float* d_out, int C_in,
                               int C_out, const float* d_kernel, const float* d_bias,
                               const float* d_lut_decay, int B) {
    VD_TRY(vdttfs_fc_vmem(ctx, d_in, d_out, d_kernel, d_bias, d_lut_decay, B, C_in, C_out));
    VD_HIP(hipStreamSynchronize(ctx->stream));
    return VDTTFS_OK;
}

}  // extern "C"
