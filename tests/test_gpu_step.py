"""The step-by-step (time-driven) baseline on the GPU against its CPU oracle
(orc_stepnet_forward), bit for bit: T1S semantics on LeNet-5 with the
configs' linear and the reference's log encoder, and T2S semantics (depth-
offset windows, same-pad convs, max(V + b) readout) on a small VGG-like net."""
import sys

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import core, models
from vdttfs.core import Layer

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_step(ctx, layers, B, img, img_elems, enc, tc_in, mode):
    net = vdttfs.StepNet(ctx, layers, B, img_elems, enc, tc_in, 0.0, mode)
    try:
        d_img = ctx.to_device(img)
        d_pred = ctx.empty(B, np.int32)
        net.forward(d_img, d_pred)
        ctx.synchronize()
        out, steps = net.output()
        pred = d_pred.download()
        d_img.free()
        d_pred.free()
    finally:
        net.close()
    return out, pred, steps


@pytest.mark.parametrize("enc", [vdttfs.ENCODE_LINEAR, vdttfs.ENCODE_LOG])
def test_lenet_t1s(gpu_ctx_factory, enc):
    say(f"step-by-step T1S LeNet-5 B=48 encode={enc}")
    w = models.lenet5()
    B = 48
    img = models.images_for(w, B)
    tc_in = w.tc_in if enc == vdttfs.ENCODE_LINEAR else 17.452274
    out, pred, steps = run_step(gpu_ctx_factory(w.consts), w.layers, B, img, w.img_elems, enc, tc_in,
                                vdttfs.STEP_T1)
    r = oracle.stepnet_forward(oracle.Consts.from_task(w.consts), w.layers, B, img, w.img_elems,
                               oracle.ENC_LINEAR if enc == vdttfs.ENCODE_LINEAR else oracle.ENC_LOG,
                               tc_in, 0.0, oracle.STEP_T1)
    assert steps == r["steps"] == w.consts.T
    np.testing.assert_array_equal(out, r["final"])
    np.testing.assert_array_equal(pred, r["pred"])
    assert np.any(out < 9999.0)


def small_vgg(seed=9, H=8):
    rng = np.random.default_rng(seed)

    def conv(Hc, cin, cout):
        k = (rng.standard_normal((3, 3, cin, cout)) * np.sqrt(2.0 / (9 * cin))).astype(np.float32)
        return Layer(core.LAYER_CONV, Hc, Hc, cin, Hc, Hc, cout, 3, 3, k,
                     (rng.standard_normal(cout) * 0.05).astype(np.float32), 8.0, 0.0)

    def fc(cin, cout, kind=core.LAYER_FC, H_in=1, C_in=None):
        k = (rng.standard_normal((cin, cout)) * np.sqrt(2.0 / cin)).astype(np.float32)
        return Layer(kind, H_in, H_in, C_in or cin, 1, 1, cout, 1, 1, k,
                     (rng.standard_normal(cout) * 0.05).astype(np.float32), 8.0, 1.5)

    return [conv(H, 3, 16), conv(H, 16, 16), Layer(core.LAYER_POOL, H, H, 16, H // 2, H // 2, 16),
            conv(H // 2, 16, 24), Layer(core.LAYER_POOL, H // 2, H // 2, 24, H // 4, H // 4, 24),
            fc((H // 4) ** 2 * 24, 32, H_in=H // 4, C_in=24), fc(32, 10, kind=core.LAYER_VMEM)]


def test_small_vgg_t2s(gpu_ctx_factory):
    say("step-by-step T2S small VGG B=16")
    T, tfs = 32, 8.0
    tc = vdttfs.task2_consts(T=T, delta=8, tfs=tfs)
    layers = small_vgg()
    B = 16
    rng = np.random.default_rng(10)
    img = rng.random((B, 8, 8, 3)).astype(np.float32)
    out, pred, steps = run_step(gpu_ctx_factory(tc), layers, B, img, 8 * 8 * 3, vdttfs.ENCODE_LINEAR, 8.0,
                                vdttfs.STEP_T2)
    r = oracle.stepnet_forward(oracle.Consts.from_task(tc), layers, B, img, 8 * 8 * 3, oracle.ENC_LINEAR,
                               8.0, 0.0, oracle.STEP_T2, same_pad=True)
    assert steps == r["steps"] == int(np.ceil(4 * tfs + T))
    np.testing.assert_array_equal(out, r["final"])
    np.testing.assert_array_equal(pred, r["pred"])
    # spikes reached the readout: max(V + b) is not the bias alone, and it
    # differs between images
    o = out.reshape(B, 10)
    assert np.any(o != layers[-1].bias[None, :])
    assert len(np.unique(o[:, 0])) > 1


# ---- T3S: the step-by-step CuLIF baseline ----------------------------------
def _t3s_run(ctx, layers, B, data):
    sn = vdttfs.CulifStepNet(ctx, layers, B)
    try:
        d = ctx.to_device(data)
        p = ctx.empty(B, np.int32)
        sn.forward(d, p)
        ctx.synchronize()
        out, steps = sn.output()
        pred = p.download()
        d.free()
        p.free()
    finally:
        sn.close()
    return out, pred, steps


def _odd_culif_net(rng, T):
    """Channel counts that are not multiples of 4 (one output per thread) and
    a 4x4 map (a wave spans several c_out planes)."""
    from vdttfs.core import CulifLayerSpec

    def kw(*shape):
        return (rng.standard_normal(shape) * np.sqrt(2.0 / np.prod(shape[1:]))).astype(np.float32)

    d, th = 0.6, 0.5
    return [CulifLayerSpec(vdttfs.CULIF_RAW_CONV, 2, 8, 8, 3, kw(3, 2, 3, 3), None, d, th),
            CulifLayerSpec(vdttfs.CULIF_CONV, 3, 8, 8, 5, kw(5, 3, 3, 3), None, d, th),
            CulifLayerSpec(vdttfs.CULIF_POOL, 5, 8, 8, 5, None, None, d, th),
            CulifLayerSpec(vdttfs.CULIF_CONV, 5, 4, 4, 6, kw(6, 5, 3, 3), None, d, th),
            CulifLayerSpec(vdttfs.CULIF_POOL, 6, 4, 4, 6, None, None, d, th),
            CulifLayerSpec(vdttfs.CULIF_FC_REC, 24, 1, 1, 7, kw(7, 24), kw(7, 7), d, th),
            CulifLayerSpec(vdttfs.CULIF_FC, 7, 1, 1, 3, kw(3, 7), None, d, th)]


@pytest.mark.parametrize("net", ["culif7-8x8", "odd-channels"])
def test_culif_t3s_every_layer_vs_oracle(gpu_ctx_factory, net):
    """Random (non-dyadic) weights: each prefix of the table ends at layer k,
    so its output is layer k's first-spike map; all equal the oracle's T3S
    restatement bit for bit, and so do the predictions."""
    from test_culif_step_oracle import events

    print(f"T3S small CuLIF net {net} vs oracle, every layer", flush=True)
    rng = np.random.default_rng(7)
    N, T = 3, 32
    w = models.culif7(H=8, W=8, T=T, delta=8, n_classes=5, th=0.6)
    layers = w.layers if net == "culif7-8x8" else _odd_culif_net(rng, T)
    data = events(rng, N, T, density=0.15)
    ctx = gpu_ctx_factory(w.consts)
    ref = oracle.culif_stepnet_forward(layers, data, N, T, keep_layers=True)
    for k in range(1, len(layers) + 1):
        out, pred, steps = _t3s_run(ctx, layers[:k], N, data)
        assert steps == T
        np.testing.assert_array_equal(out, ref["outs"][k - 1], err_msg=f"layer {k - 1}")
        assert np.any(out < 9999.0), f"layer {k - 1} never fires"
    np.testing.assert_array_equal(pred, ref["pred"])


def test_culif_t3s_equals_engine_on_exact_sums(gpu_ctx_factory):
    """Weights and event counts in quarter units make every input current
    exact, so the time-driven baseline and the event-driven engine must give
    the same last-layer first spikes and predictions."""
    from test_culif_step_oracle import events, small_net

    print("T3S vs CuLIF engine on exact sums", flush=True)
    rng = np.random.default_rng(3)
    N, T = 4, 32
    layers = small_net(rng, 0.5, 1.0)
    data = events(rng, N, T)
    ctx = gpu_ctx_factory(vdttfs.task3_consts(T=T, delta=8))
    out, pred, _ = _t3s_run(ctx, layers, N, data)
    net = vdttfs.CulifNet(ctx, layers, N)
    try:
        d = ctx.to_device(data)
        p = ctx.empty(N, np.int32)
        net.forward(d, p)
        ctx.synchronize()
        eng = net.layer_output(len(layers) - 1)
        np.testing.assert_array_equal(out, eng.ravel())
        np.testing.assert_array_equal(pred, p.download())
    finally:
        net.close()


def test_culif_t3s_config4_shapes(gpu_ctx_factory):
    """The config 4 table at a 32x32 map, B=4, T=32, against the oracle."""
    print("T3S config 4 table at 32x32 vs oracle", flush=True)
    w = models.culif7(H=32, W=32, T=32)
    B = 4
    data = models.dvs_events(w, B)
    ctx = gpu_ctx_factory(w.consts)
    out, pred, _ = _t3s_run(ctx, w.layers, B, data)
    ref = oracle.culif_stepnet_forward(w.layers, data, B, w.consts.T)
    np.testing.assert_array_equal(out, ref["final"])
    np.testing.assert_array_equal(pred, ref["pred"])
