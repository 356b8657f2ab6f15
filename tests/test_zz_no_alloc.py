"""vdttfs_layer_forward_noalloc through the C ABI: the layer path on the
library's static per-GPU scratch must give exactly what vdttfs_layer_forward
(context scratch grown with hipMalloc) gives, on two calls in a row -- the
second with a smaller input, so stale scratch from the first call cannot
leak into it -- on every list path (fused with one or two events per load,
the shared-list fused kernel, dense, bins, narrow, register, FC) and on
VGG-16's conv 4-9 shapes at B=256; reject a layer whose scratch exceeds the
buffer; leave the device's free memory unchanged on a fresh context; and
order calls from two contexts that share the buffer."""
import sys
import zlib

import numpy as np
import pytest

import vdttfs
from vdttfs import _lib

pytestmark = pytest.mark.gpu
INF = np.float32(9999.0)

# name, task2, is_fc, (B, B2), H, W, C_in, C_out, K
CASES = [
    ("fused 32->64 3x3", True, False, (5, 2), 12, 12, 32, 64, 3),
    ("fused pair 16->128 3x3", True, False, (4, 3), 16, 16, 16, 128, 3),
    ("fused shared 24->256 3x3", True, False, (3, 2), 8, 8, 24, 256, 3),
    ("fused shared 130->256 3x3", True, False, (3, 1), 8, 8, 130, 256, 3),
    ("bins 80->64 5x5", True, False, (3, 1), 8, 8, 80, 64, 5),
    ("fused wide 96->128 3x3", True, False, (3, 2), 10, 10, 96, 128, 3),
    ("narrow 6->16 5x5 valid", False, False, (40, 7), 12, 12, 6, 16, 5),
    ("register 1->6 5x5 valid", False, False, (50, 9), 28, 28, 1, 6, 5),
    ("fc 600->300", True, True, (40, 13), 1, 1, 600, 300, 1),
    # VGG-16's conv 4-9 shapes at the benchmark batch: lists in LDS, no scratch
    ("vgg conv4 128->256 8x8 B=256", True, False, (256, 64), 8, 8, 128, 256, 3),
    ("vgg conv5 256->256 8x8 B=256", True, False, (256, 64), 8, 8, 256, 256, 3),
    ("vgg conv7 256->512 4x4 B=256", True, False, (256, 64), 4, 4, 256, 512, 3),
    ("vgg conv8 512->512 4x4 B=256", True, False, (256, 64), 4, 4, 512, 512, 3),
]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def layer(rng, tc, is_fc, B, H, W, C_in, C_out, K):
    if is_fc:
        ho = wo = 1
        n_cols = B
    else:
        ho, wo = (H, W) if tc.conv_same_pad else (H - K + 1, W - K + 1)
        n_cols = B * H * W
    n_in = n_cols * C_in
    t = np.floor(rng.random(n_in) * (tc.T + tc.tfs + 2)).astype(np.float32)
    sp = np.where(rng.random(n_in) < 0.4, t, INF).astype(np.float32)
    return sp, dict(B=B, H_in=H, W_in=W, C_in=C_in, H_out=ho, W_out=wo, C_out=C_out,
                    K_h=1 if is_fc else K, K_w=1 if is_fc else K)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_layer_forward(gpu_ctx_factory, case):
    name, task2, is_fc, Bs, H, W, C_in, C_out, K = case
    say(f"noalloc {name}")
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    tc = vdttfs.TaskConsts(T=64, tfs=32.0 if task2 else 0.0, delta=8, vth=1.0, alpha_by_time=task2,
                           conv_same_pad=task2)
    ctx = gpu_ctx_factory(tc)
    fan = (1 if is_fc else K * K) * C_in
    Wt = (rng.standard_normal(fan * C_out) * np.sqrt(2.0 / fan)).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.05).astype(np.float32)
    alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    d_W, d_b, d_a, d_t = ctx.to_device(Wt), ctx.to_device(bias), ctx.to_device(alpha), ctx.to_device(theta)
    L = vdttfs.lib()
    for B in Bs:  # the second call has a smaller input
        sp, sh = layer(rng, tc, is_fc, B, H, W, C_in, C_out, K)
        n_out = B * sh["H_out"] * sh["W_out"] * C_out
        d_in = ctx.to_device(sp)
        d_ref = ctx.empty(n_out)
        d_new = ctx.empty(n_out).fill(0xFF)
        ctx.layer_forward(d_ref, d_in, d_W, d_b, d_a, d_t, 1, is_fc=is_fc, **sh)
        args = [sh[k] for k in ("B", "H_in", "W_in", "C_in", "H_out", "W_out", "C_out", "K_h", "K_w")]
        rc = L.vdttfs_layer_forward_noalloc(ctx.handle, d_new.ptr, d_in.ptr, d_W.ptr, d_b.ptr, d_a.ptr, d_t.ptr,
                                             1, *args, int(is_fc))
        assert rc == 0, _lib.last_error()
        ctx.synchronize()
        ref, new = d_ref.download(), d_new.download()
        assert 0.02 < float(np.mean(ref < INF)) < 0.98, "degenerate case"
        np.testing.assert_array_equal(new, ref, err_msg=f"{name} B={B}")
        for a in (d_in, d_ref, d_new):
            a.free()


def test_noalloc_rejects_oversized_layer(gpu_ctx_factory):
    """A 5x5 128->256 conv at 64x32x32 (bins path: 25 taps) needs ~2 GB of
    bucketize output and merged lists: refused with VDTTFS_E_UNSUPPORTED
    before any launch, the output left untouched."""
    say("noalloc oversized layer")
    tc = vdttfs.task2_consts(T=64, delta=8, tfs=32.0)
    ctx = gpu_ctx_factory(tc)
    B, H, W, C_in, C_out = 64, 32, 32, 128, 256
    d_in = ctx.empty(B * H * W * C_in).fill(0)
    d_out = ctx.empty(B * H * W * C_out).fill(0x7F)
    d_W, d_b = ctx.empty(25 * C_in * C_out).fill(0), ctx.empty(C_out).fill(0)
    d_a, d_t = ctx.empty(65).fill(0), ctx.empty(64).fill(0)
    rc = vdttfs.lib().vdttfs_layer_forward_noalloc(ctx.handle, d_out.ptr, d_in.ptr, d_W.ptr, d_b.ptr, d_a.ptr,
                                                    d_t.ptr, 0, B, H, W, C_in, H, W, C_out, 5, 5, 0)
    assert rc == _lib.E_UNSUPPORTED
    assert "scratch" in _lib.last_error()
    out = d_out.download()
    assert np.all(out.view(np.uint32) == 0x7F7F7F7F)


def hip_free_bytes():
    """Free device memory of the current device, from the HIP runtime."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def bins_layer(rng, tc, B, C_in=80, C_out=64, H=8, K=5):
    """A 5x5 conv past the dense path's C_in limit: bucketize + merge lists in
    the scratch buffer (about 1 MB per image)."""
    fan = K * K * C_in
    Wt = (rng.standard_normal(fan * C_out) * np.sqrt(2.0 / fan)).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.05).astype(np.float32)
    sp, sh = layer(rng, tc, False, B, H, H, C_in, C_out, K)
    return Wt, bias, sp, sh


def test_noalloc_fresh_context_allocates_nothing(gpu_ctx_factory):
    """On a fresh context the scratch-free call on a bins-path layer (about
    50 MB of lists in the static buffer) leaves the device's free memory
    unchanged, while vdttfs_layer_forward on the same layer grows the
    context's scratch by about as much."""
    say("noalloc fresh context, device memory")
    tc = vdttfs.task2_consts(T=64, delta=8, tfs=32.0)
    ctx = gpu_ctx_factory(tc)
    rng = np.random.default_rng(zlib.crc32(b"noalloc-fresh"))
    Wt, bias, sp, sh = bins_layer(rng, tc, 48)
    alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    d_W, d_b, d_a, d_t = ctx.to_device(Wt), ctx.to_device(bias), ctx.to_device(alpha), ctx.to_device(theta)
    d_in = ctx.to_device(sp)
    n_out = 48 * sh["H_out"] * sh["W_out"] * sh["C_out"]
    d_new, d_ref = ctx.empty(n_out), ctx.empty(n_out)
    args = [sh[k] for k in ("B", "H_in", "W_in", "C_in", "H_out", "W_out", "C_out", "K_h", "K_w")]
    L = vdttfs.lib()

    def noalloc():
        assert L.vdttfs_layer_forward_noalloc(ctx.handle, d_new.ptr, d_in.ptr, d_W.ptr, d_b.ptr, d_a.ptr, d_t.ptr,
                                              1, *args, 0) == 0, _lib.last_error()
        ctx.synchronize()

    noalloc()  # the first launches load the kernels' code
    before = hip_free_bytes()
    for _ in range(3):
        noalloc()
    assert hip_free_bytes() == before
    ctx.layer_forward(d_ref, d_in, d_W, d_b, d_a, d_t, 1, is_fc=False, **sh)
    ctx.synchronize()
    assert before - hip_free_bytes() >= 32 << 20, "layer_forward grows context scratch (the check is sensitive)"
    np.testing.assert_array_equal(d_new.download(), d_ref.download())


def test_noalloc_two_contexts_in_call_order(gpu_ctx_factory):
    """Two contexts (two streams) enqueue scratch-using calls back to back
    with no synchronisation between them; every result equals
    vdttfs_layer_forward's."""
    say("noalloc two contexts")
    tc = vdttfs.task2_consts(T=64, delta=8, tfs=32.0)
    ca, cb = gpu_ctx_factory(tc), gpu_ctx_factory(tc)
    rng = np.random.default_rng(zlib.crc32(b"noalloc-two"))
    alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    L = vdttfs.lib()
    jobs = []
    for ctx, B, C_in in ((ca, 40, 80), (cb, 24, 96), (ca, 16, 72), (cb, 32, 88)):
        Wt, bias, sp, sh = bins_layer(rng, tc, B, C_in=C_in)
        dev = [ctx.to_device(x) for x in (Wt, bias, alpha, theta, sp)]
        n_out = B * sh["H_out"] * sh["W_out"] * sh["C_out"]
        d_ref, d_new = ctx.empty(n_out), ctx.empty(n_out).fill(0xFF)
        ctx.layer_forward(d_ref, dev[4], dev[0], dev[1], dev[2], dev[3], 1, is_fc=False, **sh)
        ctx.synchronize()
        jobs.append((ctx, sh, dev, d_ref, d_new))
    for rnd in range(3):
        for ctx, sh, dev, _, d_new in (jobs if rnd % 2 == 0 else jobs[::-1]):
            args = [sh[k] for k in ("B", "H_in", "W_in", "C_in", "H_out", "W_out", "C_out", "K_h", "K_w")]
            rc = L.vdttfs_layer_forward_noalloc(ctx.handle, d_new.ptr, dev[4].ptr, dev[0].ptr, dev[1].ptr,
                                                 dev[2].ptr, dev[3].ptr, 1, *args, 0)
            assert rc == 0, _lib.last_error()
        ca.synchronize()
        cb.synchronize()
        for i, (_, _, _, d_ref, d_new) in enumerate(jobs):
            np.testing.assert_array_equal(d_new.download(), d_ref.download(), err_msg=f"round {rnd} job {i}")
            d_new.fill(0xFF)
