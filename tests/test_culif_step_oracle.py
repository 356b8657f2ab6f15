"""Pins of the step-by-step CuLIF oracle (orc_culif_stepnet_forward, T3S
semantics).

* Where every input current is exact -- weights and event counts that are
  small multiples of 1/4, so any summation order gives the same fp32 sum --
  the time-driven network and the event-driven T3V network (orc_culif_*,
  pinned on their own by time-driven simulations in test_culif_oracle.py)
  run the same neuron on the same currents, so every layer's first-spike
  map must be identical.  This fixes the layer wiring, the same-step
  propagation between layers, the recurrent feedback of step t-1, the
  pool rule and the readout.
* What exact sums cannot see is the summation order.  Two hand-built
  neurons where fp32 rounding depends on the order fix it: 2^24 + 1 rounds
  back to 2^24 (ties to even), so the order of {2^24, 1, -2^24} decides
  whether the current is 0 or 1.
"""
import numpy as np
import pytest

import oracle
from vdttfs import models
from vdttfs.core import CULIF_CONV, CULIF_FC, CULIF_FC_REC, CULIF_POOL, CULIF_RAW_CONV, CulifLayerSpec


def small_net(rng, decay, th, scale=0.25):
    """2x8x8 input -> conv 4 -> conv 8 -> pool -> conv 8 -> pool -> rec FC 32 -> 6 -> FC 5."""
    def w(*shape):
        return (rng.integers(-3, 5, size=shape) * scale).astype(np.float32)

    return [
        CulifLayerSpec(CULIF_RAW_CONV, 2, 8, 8, 4, w(4, 2, 3, 3), None, decay, th),
        CulifLayerSpec(CULIF_CONV, 4, 8, 8, 8, w(8, 4, 3, 3), None, decay, th),
        CulifLayerSpec(CULIF_POOL, 8, 8, 8, 8, None, None, decay, th),
        CulifLayerSpec(CULIF_CONV, 8, 4, 4, 8, w(8, 8, 3, 3), None, decay, th),
        CulifLayerSpec(CULIF_POOL, 8, 4, 4, 8, None, None, decay, th),
        CulifLayerSpec(CULIF_FC_REC, 32, 1, 1, 6, w(6, 32), w(6, 6), decay, th),
        CulifLayerSpec(CULIF_FC, 6, 1, 1, 5, w(5, 6), None, decay, th),
    ]


def events(rng, N, T, density=0.08):
    x = rng.random((N, 2, 8, 8, T)) < density
    return (x * rng.integers(1, 3, size=x.shape)).astype(np.float32)


@pytest.mark.parametrize("decay,th,seed", [(0.5, 1.0, 0), (float(np.float32(np.exp(-1.0 / 5.0))), 2.0, 1),
                                           (0.75, 1.5, 2)])
def test_t3s_equals_event_driven_on_exact_sums(decay, th, seed):
    rng = np.random.default_rng(seed)
    N, T = 3, 32
    layers = small_net(rng, decay, th)
    data = events(rng, N, T)
    s = oracle.culif_stepnet_forward(layers, data, N, T, keep_layers=True)
    outs, pred = oracle.culif_net_forward(layers, data, N, T, 8)
    fired_layers = 0
    for i, (a, b) in enumerate(zip(s["outs"], outs)):
        np.testing.assert_array_equal(a, b.ravel(), err_msg=f"layer {i}")
        fired_layers += bool(np.any(a < 9999))
    np.testing.assert_array_equal(s["pred"], pred)
    np.testing.assert_array_equal(s["final"], outs[-1].ravel())
    assert fired_layers == len(layers)  # every layer spikes somewhere: the comparison is not vacuous


def test_t3s_conv_sums_cin_outermost():
    """One output pixel (3x3 map, centre), 2 input channels spiking at t=0.
    Channel 0 tap (0,0) = 2^24, channel 1 tap (0,0) = -2^24, channel 0 tap
    (0,1) = 1.  Channels outermost (T3S:53-55): 2^24 + 1 -> 2^24, then
    -2^24 -> 0: the neuron never fires.  Taps outermost would give 1."""
    w = np.zeros((1, 2, 3, 3), np.float32)
    w[0, 0, 0, 0] = 2.0 ** 24
    w[0, 1, 0, 0] = -(2.0 ** 24)
    w[0, 0, 0, 1] = 1.0
    T = 4
    data = np.zeros((1, 2, 3, 3, T), np.float32)
    data[0, :, :, :, 0] = 1.0
    layer = CulifLayerSpec(CULIF_RAW_CONV, 2, 3, 3, 1, w, None, 0.5, 0.5)
    out = oracle.culif_stepnet_forward([layer], data, 1, T, keep_layers=True)["outs"][0].reshape(3, 3)
    assert out[1, 1] == 9999.0
    # the mirror case: channel 0 taps (0,0) = 2^24, (0,1) = -2^24, channel 1
    # tap (0,0) = 1.  Channels outermost: 0, then + 1 = 1 >= 0.5, fires at
    # t=0; taps outermost would give (2^24 + 1) - 2^24 = 0
    w2 = np.zeros((1, 2, 3, 3), np.float32)
    w2[0, 0, 0, 0] = 2.0 ** 24
    w2[0, 0, 0, 1] = -(2.0 ** 24)
    w2[0, 1, 0, 0] = 1.0
    layer2 = CulifLayerSpec(CULIF_RAW_CONV, 2, 3, 3, 1, w2, None, 0.5, 0.5)
    out2 = oracle.culif_stepnet_forward([layer2], data, 1, T, keep_layers=True)["outs"][0].reshape(3, 3)
    assert out2[1, 1] == 0.0


def test_t3s_fc_sums_inputs_ascending():
    """FC over [2^24, 1, -2^24] with every input spiking at step 0 (through a
    1x1 raw conv whose outputs copy the input): ascending order gives 0, so
    the FC neuron never fires; reversed weights give 1 and fire at t=0."""
    T = 3
    conv_w = np.zeros((3, 3, 3, 3), np.float32)
    for c in range(3):
        conv_w[c, c, 1, 1] = 1.0  # channel c copies input channel c; fires at t=0 with th 0.5
    data = np.zeros((1, 3, 1, 1, T), np.float32)
    data[..., 0] = 1.0
    for wv, expect in [([2.0 ** 24, 1.0, -(2.0 ** 24)], 9999.0), ([-(2.0 ** 24), 1.0, 2.0 ** 24], 0.0)]:
        layers = [CulifLayerSpec(CULIF_RAW_CONV, 3, 1, 1, 3, conv_w, None, 0.5, 0.5),
                  CulifLayerSpec(CULIF_FC, 3, 1, 1, 1, np.array([wv], np.float32), None, 0.5, 0.5)]
        r = oracle.culif_stepnet_forward(layers, data, 1, T, keep_layers=True)
        np.testing.assert_array_equal(r["outs"][0], [0.0, 0.0, 0.0])
        assert r["final"][0] == expect


def test_t3s_recurrence_uses_previous_step():
    """A recurrent FC neuron pair: neuron 0 gets input at t=0 and fires; its
    spike reaches neuron 1 through W_rec only at t=1 (the previous step's
    spikes), so neuron 1 fires at t=1, not 0."""
    T = 4
    conv_w = np.zeros((1, 1, 3, 3), np.float32)
    conv_w[0, 0, 1, 1] = 1.0
    data = np.zeros((1, 1, 1, 1, T), np.float32)
    data[..., 0] = 1.0
    w = np.array([[1.0], [0.0]], np.float32)
    w_rec = np.array([[0.0, 0.0], [1.0, 0.0]], np.float32)  # neuron 1 listens to neuron 0
    layers = [CulifLayerSpec(CULIF_RAW_CONV, 1, 1, 1, 1, conv_w, None, 0.0, 0.5),
              CulifLayerSpec(CULIF_FC_REC, 1, 1, 1, 2, w, w_rec, 0.0, 0.5)]
    r = oracle.culif_stepnet_forward(layers, data, 1, T)
    np.testing.assert_array_equal(r["final"], [0.0, 1.0])


def test_config4_table_runs_on_a_small_map():
    """The config 4 builder's table (at 16x16) is accepted and spikes."""
    w = models.culif7(H=16, W=16, T=16)
    data = models.dvs_events(w, 2)
    r = oracle.culif_stepnet_forward(w.layers, data, 2, 16, keep_layers=True)
    assert r["outs"][0].min() < 9999.0 and r["pred"].shape == (2,)
