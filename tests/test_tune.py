"""The granularity tuner's host side (vdttfs.tune): plan files are checked
against the workload they are applied to, and plan records round-trip."""
import json

import pytest

import vdttfs
from vdttfs import models, tune


def test_plan_records_round_trip():
    for p in [(vdttfs.PATH_BINS, 4, 2), (vdttfs.PATH_DENSE, 2, 1), (vdttfs.PATH_FUSED, 1, 8), (vdttfs.PATH_REG, 1, 10)]:
        d = tune._plan_dict(p)
        assert (tune._path_id(d["path"]), d["gather"], d["ppw"]) == p
    assert tune._plan_dict((0, 0, 0))["path"] == "none"


def test_load_plans_checks_workload(tmp_path):
    w = models.lenet5()
    plans = [None] * len(w.layers)
    plans[0] = {"path": "dense", "gather": 1, "ppw": 10}
    f = tmp_path / "p.json"
    f.write_text(json.dumps({"workload": w.name, "batch": 64, "T": w.consts.T, "plans": plans}))
    assert tune.load_plans(str(f), w, 64) == plans
    with pytest.raises(ValueError):
        tune.load_plans(str(f), w, 128)  # another batch
    with pytest.raises(ValueError):
        tune.load_plans(str(f), models.lenet5(T=32), 64)  # another window
    with pytest.raises(ValueError):
        tune.load_plans(str(f), models.vgg16(), 64)  # another network
    assert tune.load_pool_fusion(str(f), w, 64) is None  # files without a pool-fusion mode
    for name in ("off", "auto", "all"):
        f.write_text(json.dumps({"workload": w.name, "batch": 64, "T": w.consts.T, "plans": plans,
                                 "pool_fusion": name}))
        assert tune.load_pool_fusion(str(f), w, 64) == name
        assert tune.POOL_FUSION[name] in (vdttfs.POOL_FUSE_OFF, vdttfs.POOL_FUSE_AUTO, vdttfs.POOL_FUSE_ALL)
    f.write_text(json.dumps({"workload": w.name, "batch": 64, "T": w.consts.T, "plans": plans,
                             "pool_fusion": "some"}))
    with pytest.raises(ValueError):
        tune.load_pool_fusion(str(f), w, 64)


def test_committed_vgg_plans_fit_the_benchmark():
    """configs/plans_vgg16_b256.json (tuned on MI355X, bench.py --plans) names
    a plan for exactly the integrating layers of the benchmark network."""
    import os

    w = models.vgg16()
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "configs",
                        "plans_vgg16_b256.json")
    plans = tune.load_plans(path, w, 256)
    assert len(plans) == len(w.layers)
    for l, p in zip(w.layers, plans):
        integ = l.kind in (vdttfs.LAYER_CONV, vdttfs.LAYER_FC)
        assert (p is not None) == integ
        if p:
            assert p["path"] in ("bins", "dense", "fused", "reg") and p["gather"] in (1, 2, 4) and 1 <= p["ppw"] <= 64
