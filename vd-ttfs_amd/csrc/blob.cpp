// Weights blob reader / writer (format of T1V:185-206, T2V:213-234 and the
// Python parser WIO:1-13), plus load_weights onto the device.
//
// Layout, little-endian: int32 num_layers; per layer: int32 ndim, ndim x
// int32 shape, float32[prod(shape)] kernel, int32 ndim_b, int32 b_size,
// float32[b_size] bias, int32 ndim_tc, int32 tc_size, float32 tc_fire,
// int32 ndim_td, int32 td_size, float32 td.
// Unlike the reference reader, every read is checked, shapes are validated
// and trailing bytes are an error (the full-consumption check of WIO:69).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"

using namespace vdttfs;

namespace {

struct Reader {
    FILE* f;
    const char* path;
    int read_i32(int32_t* v) {
        if (fread(v, 4, 1, f) != 1) return set_error(VDTTFS_E_FORMAT, "%s: short read", path);
        return VDTTFS_OK;
    }
    int read_f32(float* v, size_t n) {
        if (n && fread(v, 4, n, f) != n) return set_error(VDTTFS_E_FORMAT, "%s: short read", path);
        return VDTTFS_OK;
    }
};

void free_layers(vdttfs_blob* b) {
    if (!b) return;
    if (b->layers)
        for (int i = 0; i < b->num_layers; ++i) {
            free(b->layers[i].kernel);
            free(b->layers[i].bias);
        }
    free(b->layers);
    free(b);
}

int read_all(FILE* f, const char* path, vdttfs_blob* b) {
    Reader r{f, path};
    int32_t n = 0;
    VD_TRY(r.read_i32(&n));
    if (n <= 0 || n > 4096) return set_error(VDTTFS_E_FORMAT, "%s: num_layers %d", path, n);
    b->layers = (vdttfs_blob_layer*)calloc((size_t)n, sizeof(vdttfs_blob_layer));
    if (!b->layers) return set_error(VDTTFS_E_NOMEM, "blob: out of memory");
    b->num_layers = n;
    for (int i = 0; i < n; ++i) {
        vdttfs_blob_layer* L = &b->layers[i];
        VD_TRY(r.read_i32(&L->ndim));
        if (L->ndim != 2 && L->ndim != 4)
            return set_error(VDTTFS_E_FORMAT, "%s: layer %d ndim %d (need 2 or 4)", path, i, L->ndim);
        int64_t prod = 1;
        for (int j = 0; j < L->ndim; ++j) {
            VD_TRY(r.read_i32(&L->shape[j]));
            if (L->shape[j] <= 0)
                return set_error(VDTTFS_E_FORMAT, "%s: layer %d dim %d = %d", path, i, j, L->shape[j]);
            prod *= L->shape[j];
            if (prod > (INT64_C(1) << 32))
                return set_error(VDTTFS_E_FORMAT, "%s: layer %d kernel too large", path, i);
        }
        if (L->ndim == 4) {
            L->k_h = L->shape[0];
            L->k_w = L->shape[1];
            L->c_in = L->shape[2];
            L->c_out = L->shape[3];
        } else {
            L->k_h = 1;
            L->k_w = 1;
            L->c_in = L->shape[0];
            L->c_out = L->shape[1];
        }
        L->kernel_elems = prod;
        L->kernel = (float*)malloc((size_t)prod * 4);
        if (!L->kernel) return set_error(VDTTFS_E_NOMEM, "blob: out of memory");
        VD_TRY(r.read_f32(L->kernel, (size_t)prod));
        VD_TRY(r.read_i32(&L->bias_ndim));
        VD_TRY(r.read_i32(&L->bias_size));
        if (L->bias_size != L->c_out)
            return set_error(VDTTFS_E_FORMAT, "%s: layer %d bias size %d != c_out %d", path, i,
                             L->bias_size, L->c_out);
        L->bias = (float*)malloc((size_t)L->bias_size * 4);
        if (!L->bias) return set_error(VDTTFS_E_NOMEM, "blob: out of memory");
        VD_TRY(r.read_f32(L->bias, (size_t)L->bias_size));
        int32_t sz = 0;
        VD_TRY(r.read_i32(&L->tc_ndim));
        VD_TRY(r.read_i32(&sz));
        if (sz != 1) return set_error(VDTTFS_E_FORMAT, "%s: layer %d tc_size %d != 1", path, i, sz);
        VD_TRY(r.read_f32(&L->tc_fire, 1));
        VD_TRY(r.read_i32(&L->td_ndim));
        VD_TRY(r.read_i32(&sz));
        if (sz != 1) return set_error(VDTTFS_E_FORMAT, "%s: layer %d td_size %d != 1", path, i, sz);
        VD_TRY(r.read_f32(&L->td, 1));
    }
    char extra;
    if (fread(&extra, 1, 1, f) == 1)
        return set_error(VDTTFS_E_FORMAT, "%s: trailing bytes after %d layers", path, n);
    return VDTTFS_OK;
}

}  // namespace

extern "C" {

int vdttfs_blob_read(const char* path, vdttfs_blob** out) {
    if (!path || !out) return set_error(VDTTFS_E_INVALID, "null argument");
    *out = nullptr;
    FILE* f = fopen(path, "rb");
    if (!f) return set_error(VDTTFS_E_IO, "File not found: %s", path);
    vdttfs_blob* b = (vdttfs_blob*)calloc(1, sizeof(vdttfs_blob));
    if (!b) {
        fclose(f);
        return set_error(VDTTFS_E_NOMEM, "blob: out of memory");
    }
    int rc = read_all(f, path, b);
    fclose(f);
    if (rc != VDTTFS_OK) {
        free_layers(b);
        return rc;
    }
    *out = b;
    return VDTTFS_OK;
}

int vdttfs_blob_write(const char* path, const vdttfs_blob* b) {
    if (!path || !b || b->num_layers <= 0 || !b->layers)
        return set_error(VDTTFS_E_INVALID, "blob_write: bad argument");
    FILE* f = fopen(path, "wb");
    if (!f) return set_error(VDTTFS_E_IO, "cannot open %s for writing", path);
    bool ok = true;
    auto wi = [&](int32_t v) { ok = ok && fwrite(&v, 4, 1, f) == 1; };
    auto wf = [&](const float* v, size_t n) { ok = ok && (n == 0 || fwrite(v, 4, n, f) == n); };
    wi(b->num_layers);
    for (int i = 0; i < b->num_layers && ok; ++i) {
        const vdttfs_blob_layer* L = &b->layers[i];
        if ((L->ndim != 2 && L->ndim != 4) || !L->kernel || !L->bias) {
            fclose(f);
            return set_error(VDTTFS_E_INVALID, "blob_write: layer %d malformed", i);
        }
        int64_t prod = 1;
        wi(L->ndim);
        for (int j = 0; j < L->ndim; ++j) {
            wi(L->shape[j]);
            prod *= L->shape[j];
        }
        wf(L->kernel, (size_t)prod);
        wi(L->bias_ndim ? L->bias_ndim : 1);
        wi(L->bias_size);
        wf(L->bias, (size_t)L->bias_size);
        wi(L->tc_ndim);
        wi(1);
        wf(&L->tc_fire, 1);
        wi(L->td_ndim);
        wi(1);
        wf(&L->td, 1);
    }
    if (fclose(f) != 0) ok = false;
    if (!ok) return set_error(VDTTFS_E_IO, "write to %s failed", path);
    return VDTTFS_OK;
}

int vdttfs_blob_free(vdttfs_blob* b) {
    free_layers(b);
    return VDTTFS_OK;
}

int vdttfs_load_weights(vdttfs_ctx* ctx, const char* path, vdttfs_dev_layer** layers,
                        int* num_layers) {
    VD_TRY(check_ctx(ctx));
    if (!layers || !num_layers) return set_error(VDTTFS_E_INVALID, "null out");
    *layers = nullptr;
    *num_layers = 0;
    vdttfs_blob* b = nullptr;
    VD_TRY(vdttfs_blob_read(path, &b));
    vdttfs_dev_layer* out = (vdttfs_dev_layer*)calloc((size_t)b->num_layers, sizeof(vdttfs_dev_layer));
    if (!out) {
        vdttfs_blob_free(b);
        return set_error(VDTTFS_E_NOMEM, "load_weights: out of memory");
    }
    int rc = VDTTFS_OK;
    for (int i = 0; i < b->num_layers && rc == VDTTFS_OK; ++i) {
        const vdttfs_blob_layer* L = &b->layers[i];
        vdttfs_dev_layer* d = &out[i];
        d->k_h = L->k_h;
        d->k_w = L->k_w;
        d->c_in = L->c_in;
        d->c_out = L->c_out;
        d->tc_fire = L->tc_fire;
        d->td = L->td;
        rc = vdttfs_dev_alloc(ctx, (size_t)L->kernel_elems * 4, (void**)&d->d_kernel);
        if (rc == VDTTFS_OK) rc = vdttfs_h2d(ctx, d->d_kernel, L->kernel, (size_t)L->kernel_elems * 4);
        if (rc == VDTTFS_OK) rc = vdttfs_dev_alloc(ctx, (size_t)L->bias_size * 4, (void**)&d->d_bias);
        if (rc == VDTTFS_OK) rc = vdttfs_h2d(ctx, d->d_bias, L->bias, (size_t)L->bias_size * 4);
    }
    const int n = b->num_layers;
    vdttfs_blob_free(b);
    if (rc != VDTTFS_OK) {
        vdttfs_free_weights(ctx, out, n);
        return rc;
    }
    *layers = out;
    *num_layers = n;
    return VDTTFS_OK;
}

int vdttfs_free_weights(vdttfs_ctx* ctx, vdttfs_dev_layer* layers, int num_layers) {
    if (!layers) return VDTTFS_OK;
    for (int i = 0; i < num_layers; ++i) {
        if (layers[i].d_kernel) vdttfs_dev_free(ctx, layers[i].d_kernel);
        if (layers[i].d_bias) vdttfs_dev_free(ctx, layers[i].d_bias);
    }
    free(layers);
    return VDTTFS_OK;
}

}  // extern "C"
