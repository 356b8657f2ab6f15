// Gather-roof probe: the weight-gather pattern of k_stream in isolation, to
// measure the ceiling that the integrator's stream kernels are held against.
// No reference counterpart (measurement only).
//
// Every wave streams n_ev wave-uniform row offsets (read through the scalar
// cache, eight per group, as k_stream reads its merged list) and issues one
// buffer_load per row with the row in soffset and the lane's 4 * VEC bytes in
// voffset -- dword, dwordx2 or dwordx4 per lane, i.e. 256, 512 or 1024 bytes
// per wave-gather -- then one fma per loaded dword so the loads stay live.
// Rows are uniformly random over a weight buffer of `footprint` bytes:
// footprints that fit one CU's L1, one XCD's L2, or only the MALL/HBM give
// the three roofs.  The only difference from k_stream is the missing bin
// logic and early exit, which is the point.
#include <cstdint>
#include <vector>

#include "common.h"
#include "wave.h"

namespace vdttfs {
namespace {

template <int VEC>
__global__ __launch_bounds__(256) void k_probe_gather(const float* __restrict__ W, int wbytes,
                                                      const int* __restrict__ rows, int n_ev, int n_tables,
                                                      float* __restrict__ out) {
    const int lane = lane_id();
    const int wave = uniform(threadIdx.x >> 6);
    const int64_t gw = (int64_t)blockIdx.x * 4 + wave;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, wbytes, 0x00020000);
    const int* __restrict__ R = rows + (gw % n_tables) * n_ev;
    const int voff = lane * 4 * VEC;
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
    for (int j = 0; j < n_ev; j += 8) {
        int rr[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) rr[g] = uniform(R[j + g]);
        if constexpr (VEC == 1) {
            float w[8];
#pragma unroll
            for (int g = 0; g < 8; ++g) w[g] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, rr[g], 0));
#pragma unroll
            for (int g = 0; g < 8; ++g) acc[0] = __builtin_fmaf(w[g], 0.5f, acc[0]);
        } else if constexpr (VEC == 2) {
            typedef unsigned int u2 __attribute__((ext_vector_type(2)));
            u2 w[8];
#pragma unroll
            for (int g = 0; g < 8; ++g) w[g] = __builtin_amdgcn_raw_buffer_load_b64(r, voff, rr[g], 0);
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                acc[0] = __builtin_fmaf(__uint_as_float(w[g].x), 0.5f, acc[0]);
                acc[1] = __builtin_fmaf(__uint_as_float(w[g].y), 0.5f, acc[1]);
            }
        } else {
            typedef unsigned int u4 __attribute__((ext_vector_type(4)));
            u4 w[8];
#pragma unroll
            for (int g = 0; g < 8; ++g) w[g] = __builtin_amdgcn_raw_buffer_load_b128(r, voff, rr[g], 0);
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                acc[0] = __builtin_fmaf(__uint_as_float(w[g].x), 0.5f, acc[0]);
                acc[1] = __builtin_fmaf(__uint_as_float(w[g].y), 0.5f, acc[1]);
                acc[2] = __builtin_fmaf(__uint_as_float(w[g].z), 0.5f, acc[2]);
                acc[3] = __builtin_fmaf(__uint_as_float(w[g].w), 0.5f, acc[3]);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < VEC; ++v) s += acc[v];
    out[gw * 64 + lane] = s;
}

// splitmix64 step (the synthetic-data generator's mixer), for the row table
uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

}  // namespace
}  // namespace vdttfs

using namespace vdttfs;

extern "C" int vdttfs_probe_gather(vdttfs_ctx* ctx, int vec, int64_t footprint_bytes, int n_ev, int64_t waves,
                                   int reps, double* ms_per_launch) {
    VD_TRY(check_ctx(ctx));
    if (!ms_per_launch) return set_error(VDTTFS_E_INVALID, "probe_gather: null out");
    if (vec != 1 && vec != 2 && vec != 4) return set_error(VDTTFS_E_INVALID, "probe_gather: vec is 1, 2 or 4");
    const int64_t row_bytes = 256 * vec;
    const int64_t n_rows = footprint_bytes / row_bytes;
    if (n_rows < 1 || footprint_bytes > INT64_C(0x7fffffff) || n_ev < 8 || n_ev % 8 != 0 || n_ev > (1 << 20) ||
        waves < 4 || waves % 4 != 0 || waves > (INT64_C(1) << 24) || reps < 1)
        return set_error(VDTTFS_E_INVALID,
                         "probe_gather: footprint >= one row and < 2 GiB, n_ev a multiple of 8, waves a "
                         "multiple of 4, reps >= 1");
    constexpr int kTables = 1024;
    std::vector<int> h((size_t)kTables * n_ev);
    for (size_t i = 0; i < h.size(); ++i)
        h[i] = (int)((mix64(0x9E3779B97F4A7C15ull * (i + 1)) % (uint64_t)n_rows) * row_bytes);
    float* dW = nullptr;
    int* dR = nullptr;
    float* dO = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = VDTTFS_OK;
    auto fail = [&](hipError_t e, int line) {
        if (rc == VDTTFS_OK) rc = hip_error(e, "probe_gather", line);
    };
    hipError_t e;
    if ((e = hipMalloc((void**)&dW, (size_t)n_rows * row_bytes)) != hipSuccess) fail(e, __LINE__);
    if (rc == VDTTFS_OK && (e = hipMalloc((void**)&dR, h.size() * 4)) != hipSuccess) fail(e, __LINE__);
    if (rc == VDTTFS_OK && (e = hipMalloc((void**)&dO, (size_t)waves * 64 * 4)) != hipSuccess) fail(e, __LINE__);
    if (rc == VDTTFS_OK && (e = hipMemsetAsync(dW, 0, (size_t)n_rows * row_bytes, ctx->stream)) != hipSuccess)
        fail(e, __LINE__);
    if (rc == VDTTFS_OK &&
        (e = hipMemcpyAsync(dR, h.data(), h.size() * 4, hipMemcpyHostToDevice, ctx->stream)) != hipSuccess)
        fail(e, __LINE__);
    if (rc == VDTTFS_OK && (e = hipEventCreate(&e0)) != hipSuccess) fail(e, __LINE__);
    if (rc == VDTTFS_OK && (e = hipEventCreate(&e1)) != hipSuccess) fail(e, __LINE__);
    const int wbytes = (int)(n_rows * row_bytes);
    const dim3 grid((unsigned)(waves / 4)), block(256);
    auto launch = [&]() {
        if (vec == 1)
            hipLaunchKernelGGL(k_probe_gather<1>, grid, block, 0, ctx->stream, dW, wbytes, dR, n_ev, kTables, dO);
        else if (vec == 2)
            hipLaunchKernelGGL(k_probe_gather<2>, grid, block, 0, ctx->stream, dW, wbytes, dR, n_ev, kTables, dO);
        else
            hipLaunchKernelGGL(k_probe_gather<4>, grid, block, 0, ctx->stream, dW, wbytes, dR, n_ev, kTables, dO);
    };
    if (rc == VDTTFS_OK) {
        launch();  // warm-up: page-in and cache fill
        if ((e = hipGetLastError()) != hipSuccess) fail(e, __LINE__);
    }
    if (rc == VDTTFS_OK && (e = hipEventRecord(e0, ctx->stream)) != hipSuccess) fail(e, __LINE__);
    for (int i = 0; rc == VDTTFS_OK && i < reps; ++i) launch();
    if (rc == VDTTFS_OK && (e = hipEventRecord(e1, ctx->stream)) != hipSuccess) fail(e, __LINE__);
    if (rc == VDTTFS_OK && (e = hipEventSynchronize(e1)) != hipSuccess) fail(e, __LINE__);
    float ms = 0.0f;
    if (rc == VDTTFS_OK && (e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess) fail(e, __LINE__);
    (void)hipStreamSynchronize(ctx->stream);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (dW) (void)hipFree(dW);
    if (dR) (void)hipFree(dR);
    if (dO) (void)hipFree(dO);
    if (rc == VDTTFS_OK) *ms_per_launch = ms / reps;
    return rc;
}
