"""The configuration records under configs/ describe the synthetic workloads
the model builders produce and bench.py measures; this keeps them in step."""
import json
import os

import numpy as np

from vdttfs import models

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def cfg(name):
    with open(os.path.join(ROOT, "configs", name)) as f:
        return json.load(f)


def test_lenet_configs_match_builder():
    w = models.lenet5()
    for name, batch in (("config1_lenet5_b1_cpu.json", 1), ("config2_lenet5_b1024.json", 1024)):
        c = cfg(name)
        assert (c["T"], c["delta"], c["tfs"], c["seed"], c["batch"]) == (w.consts.T, w.consts.delta,
                                                                         w.consts.tfs, w.seed, batch)
        assert c["input"]["shape"] == [batch, 28, 28, 1]
        assert c["weights"]["tc_in"] == w.tc_in and c["weights"]["td_in"] == w.td_in
    # 80% of pixels are zero in the seeded images
    img = models.lenet5_images(1, 64)
    assert abs(float((img == 0).mean()) - cfg("config2_lenet5_b1024.json")["input"]["zero_fraction"]) < 0.02


def test_vgg_config_matches_builder():
    c = cfg("config3_vgg16_b256.json")
    w = models.vgg16()
    assert (c["T"], c["delta"], c["tfs"], c["seed"]) == (w.consts.T, w.consts.delta, w.consts.tfs, w.seed)
    n_w = sum(l.kernel.size for l in w.layers if l.kernel is not None)
    n_b = sum(l.bias.size for l in w.layers if l.bias is not None)
    assert (n_w, n_b) == (c["parameters"]["weights"], c["parameters"]["biases"])
    convs = [l for l in w.layers if l.kernel is not None and l.kernel.ndim == 4]
    assert len(convs) == 13


def test_culif_config_matches_builder():
    c = cfg("config4_culif7_b64.json")
    w = models.culif7()
    assert (c["T"], c["delta"], c["seed"]) == (w.consts.T, w.consts.delta, w.seed)
    assert (c["neuron"]["decay"], c["neuron"]["th"]) == (w.meta["decay"], w.meta["th"])
    assert (c["input"]["density"], c["input"]["sigma_px"], c["input"]["vmax_px_per_step"]) == (
        w.meta["density"], w.meta["sigma_px"], w.meta["vmax_px_per_step"])
    assert [l.C_out for l in w.layers] == [64, 128, 128, 128, 128, 128, 11]


def test_fc_sweep_config_matches_generator():
    c = cfg("config5_fc4096_sweep.json")
    x = models.fc_sweep_spikes(c["seed"], 8, 4096, 0.2)
    active = x < 9999.0
    assert abs(float(active.mean()) - 0.2) < 0.01
    assert np.all((x[active] >= 0) & (x[active] < 64)) and np.all(x[active] == np.floor(x[active]))
