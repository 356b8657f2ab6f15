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
