"""Non-square kernels on the GPU against the oracle.

The reference's same padding is K_h/2 rows and K_w/2 columns (T2V:109-110),
so a K_h != K_w conv pins both axes: a kernel that padded both by K_h/2
would read the wrong columns.  Each case checks the drop-in pair
(reference-layout bucketize + integrate), the engine layer path with and
without counters, the synchronous launch wrapper, and a one-layer network
under every launch plan the kernels accept.  The oracle itself is pinned for
non-square kernels against the exact brute force in tests/test_oracle.py.
"""
import sys

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import tune

pytestmark = pytest.mark.gpu
INF = 9999.0

# (K_h, K_w, same padding, C_in, C_out, H, W)
CASES = [
    (1, 3, True, 5, 64, 9, 7),
    (3, 1, True, 64, 128, 6, 8),
    (3, 5, True, 16, 256, 7, 9),
    (5, 3, True, 3, 40, 8, 6),
    (1, 5, True, 2, 6, 6, 10),
    (5, 1, True, 70, 96, 9, 5),
    (2, 3, False, 4, 64, 7, 8),
    (1, 4, False, 9, 12, 5, 9),
    (3, 2, False, 33, 300, 6, 7),
]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("case", range(len(CASES)))
def test_nonsquare_conv(gpu_ctx_factory, case):
    K_h, K_w, same, C_in, C_out, H, W = CASES[case]
    say(f"non-square conv {K_h}x{K_w} same={same} C_in={C_in} C_out={C_out} {H}x{W}")
    rng = np.random.default_rng(500 + case)
    T, tfs, B = 64, (32.0 if same else 0.0), 3
    tc = vdttfs.TaskConsts(T=T, tfs=tfs, delta=8, vth=1.0, alpha_by_time=same, conv_same_pad=same)
    ho, wo = (H, W) if same else (H - K_h + 1, W - K_w + 1)
    shape = dict(B=B, H_in=H, W_in=W, C_in=C_in, H_out=ho, W_out=wo, C_out=C_out, K_h=K_h, K_w=K_w)
    n_cols = B * H * W
    n_in = n_cols * C_in
    t = np.floor(rng.random(n_in) * (T + tfs + 2)).astype(np.float32)
    sp = np.where(rng.random(n_in) < 0.4, t, np.float32(INF)).astype(np.float32)
    Wt = (rng.standard_normal(K_h * K_w * C_in * C_out) * np.sqrt(2.0 / (K_h * K_w * C_in))).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.05).astype(np.float32)
    tcf, td = 16.0, 0.0
    alpha, theta = vdttfs.build_luts_host(tc, tcf, td, tcf, td)
    cc = oracle.Consts.from_task(tc)
    cin, tin, off = oracle.bucketize(cc, sp, n_cols, C_in)
    pads = (K_h // 2, K_w // 2) if same else (0, 0)
    exp, ep, eb = oracle.integrate(cc, cin, tin, off, Wt, bias, alpha, theta, 0, pad=pads, is_fc=False, **shape)
    assert np.any(exp < INF) and np.any(exp == INF)

    ctx = gpu_ctx_factory(tc)
    d_in, d_W, d_b = ctx.to_device(sp), ctx.to_device(Wt), ctx.to_device(bias)
    d_a, d_t = ctx.to_device(alpha), ctx.to_device(theta)
    OS = tc.num_chunks + 1
    d_cin = ctx.empty(n_in, np.int32)
    d_tin = ctx.empty(n_in, np.float32)
    d_off = ctx.empty(n_cols * OS, np.int32)
    d_out = ctx.empty(exp.size, np.float32)
    ctx.bucketize(d_in, n_cols, C_in, d_cin, d_tin, d_off)
    ctx.integrate(d_out, d_cin, d_tin, d_off, d_W, d_b, d_a, d_t, 0, is_fc=False, **shape)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="drop-in pair")
    gp, gb = ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, 0, is_fc=False, count=True, **shape)
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="engine, counting")
    assert (gp, gb) == (ep, eb)
    ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, 0, is_fc=False, **shape)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="engine")
    d_out.fill(0)
    ctx.launch_layer(d_in, d_out, H, W, C_in, ho, wo, C_out, K_h, K_w, td, d_W, d_b, d_a, d_t, B, False)
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="launch_layer_sync")

    layer = vdttfs.Layer(vdttfs.LAYER_CONV, H, W, C_in, ho, wo, C_out, K_h, K_w,
                         Wt.reshape(K_h, K_w, C_in, C_out), bias, tcf, td)
    net = vdttfs.Net(ctx, [layer], B, H * W * C_in, vdttfs.ENCODE_TIMES, tcf, td, vdttfs.READOUT_ARGMIN)
    try:
        x = ctx.to_device(sp)
        plans = tune.candidates(net, 0)
        assert plans, "no accepted plan"
        for plan in plans:
            net.set_plan(0, *plan)
            net.forward(x)
            ctx.synchronize()
            np.testing.assert_array_equal(net.layer_output(0), exp, err_msg=f"plan {plan}")
    finally:
        net.close()
