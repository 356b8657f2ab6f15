"""Per-layer LUT chaining with distinct fire constants (T2V:252, 343-384).

Layer l's decay LUT alpha is built from the previous weighted layer's fire
constants (tc, td) -- the input encoder's (tc_in, td_in) for the first --
and its threshold Theta and fire start t_min = max(0, ceil(td)) from its
own.  The benchmark networks give every layer the same constants, so a slip
in which constants feed alpha, or in t_min, would pass them.  Here every
weighted layer has its own (tc_fire, td), with td > 0 (so t_min > 0) and
pools between weighted layers, in a Task-2 net (same padding, alpha by spike
time, fire start, vmem readout, layers on the fused per-wave and shared-list
kernels) and a Task-1 net (valid convs, alpha by arrival bin, FC layers).

Checked against three things that do not share the engine's chaining code:
  * the whole net against oracle.net_forward;
  * each layer against a one-layer oracle network fed the engine's previous
    output, with the alpha constants chained by this test;
  * t_min as a property: no first spike before ceil(td), and some exactly
    at it (neurons whose bias alone crosses the threshold).
A one-layer chain with each layer's own constants in place of the previous
layer's must differ from the engine somewhere (the test can see the slip).
"""
import math
import sys
import zlib

import numpy as np
import pytest

import oracle
import vdttfs

pytestmark = pytest.mark.gpu
INF = np.float32(9999.0)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def conv(rng, H, W, cin, cout, K, same, tc, td, bias_mu):
    ho, wo = (H, W) if same else (H - K + 1, W - K + 1)
    k = (rng.standard_normal((K, K, cin, cout)) * math.sqrt(2.0 / (K * K * cin))).astype(np.float32)
    b = (bias_mu + 0.5 * rng.standard_normal(cout)).astype(np.float32)
    return vdttfs.Layer(vdttfs.LAYER_CONV, H, W, cin, ho, wo, cout, K, K, k, b, tc, td)


def fc(rng, cin, cout, tc, td, bias_mu, H=1, W=1, C=None, vmem=False):
    k = (rng.standard_normal((H * W * (C or cin), cout)) * math.sqrt(2.0 / (H * W * (C or cin)))).astype(np.float32)
    b = (bias_mu + 0.5 * rng.standard_normal(cout)).astype(np.float32)
    kind = vdttfs.LAYER_VMEM if vmem else vdttfs.LAYER_FC
    return vdttfs.Layer(kind, H, W, C or cin, 1, 1, cout, 1, 1, k, b, tc, td)


def pool(H, W, C):
    return vdttfs.Layer(vdttfs.LAYER_POOL, H, W, C, H // 2, W // 2, C)


def task2_net(rng):
    tc = vdttfs.TaskConsts(T=48, tfs=16.0, delta=8, vth=1.0, alpha_by_time=True, conv_same_pad=True)
    L = [
        conv(rng, 12, 12, 3, 16, 3, True, 10.0, 0.0, 0.4),
        pool(12, 12, 16),
        conv(rng, 6, 6, 16, 32, 3, True, 20.0, 1.5, 0.6),     # t_min 2
        conv(rng, 6, 6, 32, 192, 3, True, 7.0, 3.0, 0.6),     # shared-list kernel, t_min 3
        pool(6, 6, 192),
        fc(rng, 1728, 96, 25.0, 2.25, 0.6, H=3, W=3, C=192),  # shared-list FC, t_min 3
        fc(rng, 96, 10, 13.0, 0.0, 0.0, vmem=True),           # alpha from the FC's (25, 2.25)
    ]
    imgs = rng.random((8, 12, 12, 3), dtype=np.float32)
    return tc, L, imgs, 144 * 3, (12.0, 0.5), vdttfs.READOUT_ARGMAX, oracle.READ_ARGMAX


def task1_net(rng):
    tc = vdttfs.TaskConsts(T=40, tfs=0.0, delta=8, vth=1.0, alpha_by_time=False, conv_same_pad=False)
    L = [
        conv(rng, 16, 16, 1, 8, 5, False, 8.0, 0.0, 0.4),
        pool(12, 12, 8),
        conv(rng, 6, 6, 8, 40, 3, False, 15.0, 2.5, 0.6),     # t_min 3
        fc(rng, 640, 48, 11.0, 1.0, 0.6, H=4, W=4, C=40),    # t_min 1
        fc(rng, 48, 10, 6.0, 0.75, 0.6),                     # narrow, t_min 1
    ]
    x = rng.random((8, 16, 16, 1), dtype=np.float32)
    imgs = np.where(rng.random(x.shape) < 0.6, np.float32(0.0), x).astype(np.float32)
    return tc, L, imgs, 16 * 16, (6.0, 0.25), vdttfs.READOUT_ARGMIN, oracle.READ_ARGMIN


def check_map(got, ref, what, vmem):
    if vmem:
        assert np.all(np.abs(got - ref) <= 1e-5 * (np.abs(ref) + 1e-3)), what
    else:
        np.testing.assert_array_equal(got, ref, err_msg=what)


@pytest.mark.parametrize("task", ["task2", "task1"])
def test_lut_chaining_distinct_constants(gpu_ctx_factory, task):
    say(f"LUT chaining, distinct per-layer constants, {task}")
    rng = np.random.default_rng(zlib.crc32(f"lut-chain-{task}".encode()))
    tc, L, imgs, img_elems, (tc_in, td_in), readout, oread = (task2_net if task == "task2" else task1_net)(rng)
    same = tc.conv_same_pad
    B = imgs.shape[0]
    c = oracle.Consts.from_task(tc)
    ctx = gpu_ctx_factory(tc)
    net = vdttfs.Net(ctx, L, B, img_elems, vdttfs.ENCODE_LINEAR, tc_in, td_in, readout)
    try:
        d_img = ctx.to_device(imgs.reshape(-1))
        d_pred = ctx.empty(B, np.int32)
        net.forward(d_img, d_pred)
        ctx.synchronize()
        outs = [net.layer_output(i) for i in range(len(L))]
        pred = d_pred.download()
    finally:
        net.close()

    # 1. the whole net against the oracle's own chaining
    ref = oracle.net_forward(c, L, B, imgs.reshape(-1), img_elems, oracle.ENC_LINEAR, tc_in, td_in, oread,
                             same_pad=same, keep_layers=True)
    for i, (g, o) in enumerate(zip(outs, ref["outs"])):
        check_map(g, o, f"layer {i} vs oracle.net_forward", L[i].kind == vdttfs.LAYER_VMEM)
    np.testing.assert_array_equal(pred, ref["pred"])

    # 2. layer by layer, alpha's constants chained here: the previous weighted
    # layer's (tc_fire, td), the encoder's for the first; pools pass them on
    def one_layer(i, x, enc, tci, tdi):
        return oracle.net_forward(c, [L[i]], B, x, L[i].H_in * L[i].W_in * L[i].C_in if i else img_elems,
                                  enc, tci, tdi, 0, same_pad=same)["final"]

    tci, tdi = tc_in, td_in
    slipped = 0
    for i, l in enumerate(L):
        x, enc = (imgs.reshape(-1), oracle.ENC_LINEAR) if i == 0 else (outs[i - 1], oracle.ENC_TIMES)
        exp = one_layer(i, x, enc, tci, tdi)
        check_map(outs[i], exp, f"layer {i}, alpha from ({tci}, {tdi})", l.kind == vdttfs.LAYER_VMEM)
        if l.kind != vdttfs.LAYER_POOL:
            if (tci, tdi) != (l.tc_fire, l.td):  # the slip: alpha from the layer's own constants
                wrong = one_layer(i, x, enc, l.tc_fire, l.td)
                slipped += int(not np.array_equal(wrong, exp))
            tci, tdi = l.tc_fire, l.td
    assert slipped >= 1, "the distinct constants must make the chaining observable"

    # 3. the fire start t_min = max(0, ceil(td)) as a property of the maps
    at_tmin = 0
    for i, l in enumerate(L):
        if l.kind not in (vdttfs.LAYER_CONV, vdttfs.LAYER_FC) or l.td <= 0:
            continue
        tmin = math.ceil(l.td)
        fired = outs[i][outs[i] < INF]
        assert fired.size and fired.min() >= tmin, f"layer {i}: a spike before t_min {tmin}"
        at_tmin += int(np.any(fired == tmin))
    assert at_tmin >= 2, "some neurons must fire exactly at t_min"
