"""Degenerate event tensors through the CuLIF engine (T3V semantics) and the
step-by-step baseline (T3S), against the oracle.

* silent: no events at all -- no neuron may fire and every prediction is
  class 0, the argmin's initial best (T3V:291-298);
* burst at the first or at the last step: every site of the input spikes
  once, at step 0 or at step T-1;
* burst of value 2 at step 0: every event carries a value other than 1.0,
  the raw conv's non-binary route.

The engine must equal the oracle's T3V network at every layer, and the
time-driven network the oracle's T3S restatement; predictions too.
"""
import sys

import numpy as np
import pytest

import oracle
import vdttfs
from test_gpu_step import _t3s_run
from vdttfs import models

pytestmark = pytest.mark.gpu

INF = 9999.0
KINDS = ["silent", "burst-first", "burst-last", "burst-value2"]
N, H, W, T, D = 2, 8, 8, 32, 8


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def tensor(kind):
    x = np.zeros((N, 2, H, W, T), np.float32)
    if kind == "burst-first":
        x[..., 0] = 1.0
    elif kind == "burst-last":
        x[..., T - 1] = 1.0
    elif kind == "burst-value2":
        x[..., 0] = 2.0
    return x


def workload():
    return models.culif7(H=H, W=W, T=T, delta=D, n_classes=5, th=0.6)


@pytest.mark.parametrize("kind", KINDS)
def test_culif_engine_degenerate_events(gpu_ctx_factory, kind):
    say(f"CuLIF engine, {kind} events")
    w = workload()
    data = tensor(kind)
    ref, rpred = oracle.culif_net_forward(w.layers, data, N, T, D)
    ctx = gpu_ctx_factory(w.consts)
    net = vdttfs.CulifNet(ctx, w.layers, N)
    try:
        d = ctx.to_device(data)
        p = ctx.empty(N, np.int32)
        net.forward(d, p)
        ctx.synchronize()
        fired = 0
        for li, o in enumerate(ref):
            g = net.layer_output(li)
            assert np.array_equal(g, o.reshape(g.shape)), f"layer {li} differs"
            fired += int(np.any(g < INF))
        pred = p.download()
        np.testing.assert_array_equal(pred, rpred)
    finally:
        net.close()
    if kind == "silent":
        assert fired == 0 and np.all(pred == 0)
    else:
        assert fired > 0


@pytest.mark.parametrize("kind", KINDS)
def test_culif_t3s_degenerate_events(gpu_ctx_factory, kind):
    say(f"T3S, {kind} events")
    w = workload()
    data = tensor(kind)
    ref = oracle.culif_stepnet_forward(w.layers, data, N, T)
    ctx = gpu_ctx_factory(w.consts)
    out, pred, steps = _t3s_run(ctx, w.layers, N, data)
    assert steps == T
    np.testing.assert_array_equal(out, ref["final"])
    np.testing.assert_array_equal(pred, ref["pred"])
    if kind == "silent":
        assert np.all(out == INF) and np.all(pred == 0)
