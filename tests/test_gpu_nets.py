"""Whole-network parity on the GPU (the driver main()s): every layer's output
map, the readout and the predicted classes against the oracle, plus
size-independent properties at the full benchmark sizes."""
import sys

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import models

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_engine(ctx, w, B, img, count=False):
    net = vdttfs.Net(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in,
                     w.readout)
    try:
        d_img = ctx.to_device(img)
        d_pred = ctx.empty(B, np.int32)
        net.forward(d_img, d_pred)
        ctx.synchronize()
        outs = [net.layer_output(i) for i in range(len(w.layers))]
        pred = d_pred.download()
        counts = net.count(d_img) if count else None
        d_img.free()
        d_pred.free()
    finally:
        net.close()
    return outs, pred, counts


def run_oracle(w, B, img):
    same = bool(w.consts.conv_same_pad)
    return oracle.net_forward(oracle.Consts.from_task(w.consts), w.layers, B, img, w.img_elems,
                              oracle.ENC_LINEAR, w.tc_in, w.td_in,
                              oracle.READ_ARGMAX if w.readout == vdttfs.READOUT_ARGMAX
                              else oracle.READ_ARGMIN, same_pad=same, keep_layers=True)


def check_layers(w, outs, ref, rel_vmem=1e-5):
    for i, (l, g, o) in enumerate(zip(w.layers, outs, ref["outs"])):
        if l.kind == vdttfs.LAYER_VMEM:
            assert np.all(np.abs(g - o) <= rel_vmem * (np.abs(o) + 1e-3)), f"layer {i}"
        else:
            assert np.array_equal(g, o), f"layer {i} ({l.kind}) differs at {np.flatnonzero(g != o)[:10]}"


def test_lenet5_config2_b1024(gpu_ctx_factory):
    say("LeNet-5 B=1024 (config 2) vs oracle")
    w = models.lenet5()
    B = 1024
    img = models.images_for(w, B)
    ctx = gpu_ctx_factory(w.consts)
    outs, pred, counts = run_engine(ctx, w, B, img, count=True)
    ref = run_oracle(w, B, img)
    check_layers(w, outs, ref)
    np.testing.assert_array_equal(pred, ref["pred"])
    eproc, ebin, n_ev, n_cols = counts
    np.testing.assert_array_equal(eproc, ref["eproc"])
    np.testing.assert_array_equal(ebin, ref["ebin"])
    # config 1 (B=1) is image 0 of the batch
    ref1 = run_oracle(w, 1, img[:1])
    assert pred[0] == ref1["pred"][0]


def test_vgg16_config3_b16(gpu_ctx_factory):
    say("VGG-16 B=16 (config 3 shapes) vs oracle")
    w = models.vgg16()
    B = 16
    img = models.images_for(w, B)
    ctx = gpu_ctx_factory(w.consts)
    outs, pred, counts = run_engine(ctx, w, B, img, count=True)
    ref = run_oracle(w, B, img)
    check_layers(w, outs, ref)
    np.testing.assert_array_equal(pred, ref["pred"])
    np.testing.assert_array_equal(counts[0], ref["eproc"])
    np.testing.assert_array_equal(counts[1], ref["ebin"])


def test_vgg16_b256_every_layer_vs_oracle(gpu_ctx_factory):
    """Config 3 at the benchmark size: every layer's map of all 256 images,
    the readout (1e-5 relative) and the classes equal the oracle's, and the
    integrated-synapse counts too; outputs are bit-identical for every chunk
    width."""
    say("VGG-16 B=256 (config 3) every layer vs oracle")
    B = 256
    w = models.vgg16()
    img = models.images_for(w, B)
    outs, pred, counts = run_engine(gpu_ctx_factory(w.consts), w, B, img, count=True)
    ref = run_oracle(w, B, img)
    check_layers(w, outs, ref)
    np.testing.assert_array_equal(pred, ref["pred"])
    np.testing.assert_array_equal(counts[0], ref["eproc"])
    np.testing.assert_array_equal(counts[1], ref["ebin"])
    for delta in (4, 16):
        say(f"VGG-16 B=256 delta={delta}")
        wd = models.vgg16(delta=delta)
        outs_d, pred_d, _ = run_engine(gpu_ctx_factory(wd.consts), wd, B, models.images_for(wd, B))
        for i, (a, b) in enumerate(zip(outs_d, outs)):
            assert np.array_equal(a, b), f"layer {i} differs at delta={delta}"
        np.testing.assert_array_equal(pred_d, pred)


@pytest.mark.parametrize("density", [0.01, 0.05, 0.2, 0.5])
def test_fc_sweep_config5(gpu_ctx_factory, density):
    """Config 5 layer at every T' of the sweep (16, 32, 64): B=512 on the
    GPU, all 512 images against the oracle, and bit-identical outputs across
    Delta in {8, 16, 32} (Delta > T' is one chunk cut at T')."""
    say(f"FC 4096x4096 sweep density={density}")
    B, cin, cout = 512, 4096, 4096
    layer = models.fc_sweep_layer()
    sp = models.fc_sweep_spikes(5, B, cin, density)
    for Tp in (16, 32, 64):
        outs = []
        for delta in (8, 16, 32):  # delta > T' is one chunk cut at T' (T1V:152-153)
            tc = vdttfs.TaskConsts(T=Tp, tfs=0.0, delta=delta, alpha_by_time=False)
            ctx = gpu_ctx_factory(tc)
            alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
            d_out = ctx.empty(B * cout)
            d_in, d_W, d_b = ctx.to_device(sp), ctx.to_device(layer.kernel), ctx.to_device(layer.bias)
            d_a, d_t = ctx.to_device(alpha), ctx.to_device(theta)
            ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, 0, B, 1, 1, cin, 1, 1, cout, 1, 1, True)
            ctx.synchronize()
            outs.append(d_out.download())
            for d in (d_out, d_in, d_W, d_b, d_a, d_t):
                d.free()
        np.testing.assert_array_equal(outs[0], outs[1])
        np.testing.assert_array_equal(outs[0], outs[2])
        c = oracle.Consts(Tp, 0.0, 8, False)
        nb = B
        cin_, tin_, off_ = oracle.bucketize(c, sp[:nb], nb, cin)
        exp, _, _ = oracle.integrate(c, cin_, tin_, off_, layer.kernel, layer.bias, alpha, theta, 0,
                                     nb, 1, 1, cin, 1, 1, cout, 1, 1, 0, True)
        np.testing.assert_array_equal(outs[0][: nb * cout], exp)
