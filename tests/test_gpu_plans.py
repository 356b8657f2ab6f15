"""Launch plans (vdttfs_net_set_plan) and the granularity tuner: the
built-in plan of each layer, rejection of plans the kernels cannot run,
bit-exact outputs and equal work counts under every plan the kernels accept
(against the oracle), and the tuner's Delta sweep and plan sweep."""
import sys

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import models, tune

pytestmark = pytest.mark.gpu

BINS, DENSE, FUSED, REG = vdttfs.PATH_BINS, vdttfs.PATH_DENSE, vdttfs.PATH_FUSED, vdttfs.PATH_REG


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_net(ctx, w, B):
    return vdttfs.Net(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)


def test_builtin_plans_and_rejections(gpu_ctx_factory):
    say("plans: VGG-16 B=16 built-in choices and rejections")
    w = models.vgg16()
    ctx = gpu_ctx_factory(w.consts)
    net = make_net(ctx, w, 16)
    try:
        got = [net.get_plan(i) for i in range(len(w.layers))]
        # every weighted layer builds its lists in LDS: per wave up to 128 inputs
        # and 128 outputs (conv 0-3), shared by a workgroup's waves beyond, at
        # 128 c_out per wave up to 256 outputs and 64 past that
        exp = {0: (FUSED, 1, 1), 1: (FUSED, 1, 1), 3: (FUSED, 2, 1), 4: (FUSED, 2, 1), 6: (FUSED, 2, 1),
               10: (FUSED, 1, 1), 16: (FUSED, 1, 1), 18: (FUSED, 1, 1)}
        for i, p in exp.items():
            assert got[i] == p, f"layer {i}: {got[i]}"
        assert got[2] == (0, 0, 0) and got[19] == (0, 0, 0)  # pool, vmem
        bad = [(18, DENSE, 0, 0),   # FC layers have no dense path
               (10, FUSED, 0, 2),   # ... and takes one pixel per workgroup
               (0, 0, 0, 9),        # at most 8 pixels per wave
               (0, 6, 0, 0),        # unknown path
               (4, DENSE, 0, 0),    # dense merge needs C_in <= 64
               (1, FUSED, 4, 0),    # the fused kernels gather one c_out per lane or two events per load
               (3, FUSED, 4, 0),    # ... and C_out <= 128
               (4, FUSED, 4, 0),    # ... also past the dense path's C_in limit (128 -> 128)
               (0, 0, 3, 0),        # gather is 1, 2 or 4
               (2, BINS, 0, 0),     # pools have no integrator
               (1, REG, 0, 0),      # 9 * 64 receptive elements do not fit in registers
               (0, REG, 2, 0),      # the register path gathers one c_out per lane
               (18, REG, 0, 0)]     # ... and is for conv layers
        net.set_plan(0, REG)  # selectable on a wave-wide layer: the 27 elements fit
        assert net.get_plan(0) == (REG, 1, 1)
        net.set_plan(0)
        net.set_plan(3, BINS, 1, 2)
        for layer, path, gather, ppw in bad:
            with pytest.raises(vdttfs.VdttfsError):
                net.set_plan(layer, path, gather, ppw)
        assert net.get_plan(3) == (BINS, 1, 2)  # a rejected request changes nothing
        net.set_plan(3)
        assert net.get_plan(3) == (FUSED, 2, 1)
        net.set_plan(2)  # an empty plan on a pool is accepted
    finally:
        net.close()
    w = models.lenet5()
    ctx = gpu_ctx_factory(w.consts)
    net = make_net(ctx, w, 16)
    try:
        assert net.get_plan(0) == (REG, 1, 10)     # C_out 6: 10 pixels per wave
        assert net.get_plan(2) == (DENSE, 1, 4)    # 150 receptive elements: a list
        assert net.get_plan(6) == (FUSED, 1, 1)    # FC 84 -> 10: the shared-list kernel, one wave per image
        # FC 256 -> 120: the shared-list kernel; 16 images fit one round of
        # waves, so two 64-wide waves per image rather than one 128-wide
        assert net.get_plan(4) == (FUSED, 1, 1)
        with pytest.raises(vdttfs.VdttfsError):
            net.set_plan(0, 0, 0, 2)
        with pytest.raises(vdttfs.VdttfsError):
            net.set_plan(0, FUSED)
        net.set_plan(0, BINS)
        assert net.get_plan(0) == (BINS, 1, 10)
    finally:
        net.close()


def sweep_all_plans(ctx, w, B, img, ref, check_counts):
    """Round r sets layer i to its (r mod n_i)-th accepted plan, so every plan
    of every layer runs, in mixed settings; each round equals the oracle."""
    net = make_net(ctx, w, B)
    try:
        cands = {i: tune.candidates(net, i) for i, l in enumerate(w.layers)
                 if l.kind in (vdttfs.LAYER_CONV, vdttfs.LAYER_FC)}
        rounds = max(len(c) for c in cands.values())
        d_img = ctx.to_device(img)
        d_pred = ctx.empty(B, np.int32)
        for r in range(rounds):
            for i, c in cands.items():
                net.set_plan(i, *c[r % len(c)])
            net.forward(d_img, d_pred)
            ctx.synchronize()
            for i, (l, o) in enumerate(zip(w.layers, ref["outs"])):
                g = net.layer_output(i)
                if l.kind == vdttfs.LAYER_VMEM:
                    assert np.all(np.abs(g - o) <= 1e-5 * (np.abs(o) + 1e-3)), f"round {r} layer {i}"
                else:
                    assert np.array_equal(g, o), (f"round {r} layer {i} plan {net.get_plan(i)} differs at "
                                                  f"{np.flatnonzero(g != o)[:8]}")
            np.testing.assert_array_equal(d_pred.download(), ref["pred"])
            if check_counts and r % 3 == 0:
                eproc, ebin, _, _ = net.count(d_img)
                np.testing.assert_array_equal(eproc, ref["eproc"], err_msg=f"round {r}")
                np.testing.assert_array_equal(ebin, ref["ebin"], err_msg=f"round {r}")
        d_img.free()
        d_pred.free()
        return {i: len(c) for i, c in cands.items()}
    finally:
        net.close()


def oracle_ref(w, B, img):
    return oracle.net_forward(oracle.Consts.from_task(w.consts), w.layers, B, img, w.img_elems,
                              oracle.ENC_LINEAR, w.tc_in, w.td_in,
                              oracle.READ_ARGMAX if w.readout == vdttfs.READOUT_ARGMAX else oracle.READ_ARGMIN,
                              same_pad=bool(w.consts.conv_same_pad), keep_layers=True)


def test_every_plan_matches_oracle_vgg(gpu_ctx_factory):
    say("plans: VGG-16 B=16, every accepted plan of every layer vs oracle")
    w = models.vgg16()
    B = 16
    img = models.images_for(w, B)
    ref = oracle_ref(w, B, img)
    n = sweep_all_plans(gpu_ctx_factory(w.consts), w, B, img, ref, check_counts=True)
    # layer 10 (3x3, 256 -> 512) and the FC layer: bins and window paths x 3 gathers x 3 pixel
    # counts, the shared-list fused kernel at gathers 1, 2 and 4, and k_stream_multi
    assert n[0] >= 10 and n[10] == 22 and n[18] == 22
    net = make_net(gpu_ctx_factory(w.consts), w, B)
    try:
        net.set_plan(18, vdttfs.PATH_WINDOW)
        assert net.get_plan(18)[0] == vdttfs.PATH_WINDOW
    finally:
        net.close()


def test_every_plan_matches_oracle_lenet(gpu_ctx_factory):
    say("plans: LeNet-5 B=256, every accepted plan of every layer vs oracle")
    w = models.lenet5()
    B = 256
    img = models.images_for(w, B)
    ref = oracle_ref(w, B, img)
    n = sweep_all_plans(gpu_ctx_factory(w.consts), w, B, img, ref, check_counts=True)
    assert n[0] == 3 and n[6] == 2  # FC 84 -> 10: the narrow bins path and the shared-list kernel


def test_tuner_lenet(gpu_ctx_factory):
    say("tuner: LeNet-5 B=64 Delta sweep and plan sweep")
    w = models.lenet5()
    B = 64
    img = models.images_for(w, B)
    rows = tune.delta_sweep(w, img, B, (8, 16, 32), reps=1, rounds=1)
    assert rows[0]["identical_to_first"] is None
    assert all(r["identical_to_first"] for r in rows[1:])
    assert all(r["ms_per_batch"] > 0 for r in rows)
    r = tune.tune_plans(w, img, B, reps=1, rounds=1)
    assert r["tuned_identical"]
    # LeNet-5's pools feed the dense-merge conv and a flattened FC: no build takes them
    assert set(r["pool_fusion"]["modes"]) == {"off", "auto", "all"}
    assert all(v["identical"] and v["ms"] > 0 for v in r["pool_fusion"]["modes"].values())
    assert r["pool_fusion"]["best"] in ("off", "auto", "all")
    assert [L["layer"] for L in r["layers"]] == [0, 2, 4, 5, 6]
    for L in r["layers"]:
        assert L["all_identical"] and L["best"] is not None
        assert L["best"]["ms"] <= min(c["ms"] for c in L["candidates"]) + 1e-12
    assert r["plans"][1] is None and r["plans"][0]["path"] in ("bins", "dense", "reg")


def test_committed_vgg_plans_bit_identical(gpu_ctx_factory):
    """The tuned plan file that bench.py --plans applies changes no output bit
    at the benchmark size."""
    import os

    say("plans: VGG-16 B=256 committed tuned plans vs built-in")
    w = models.vgg16()
    B = 256
    ctx = gpu_ctx_factory(w.consts)
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "configs",
                        "plans_vgg16_b256.json")
    img = ctx.to_device(models.images_for(w, B))
    d_pred = ctx.empty(B, np.int32)
    net = make_net(ctx, w, B)
    try:
        net.forward(img, d_pred)
        ctx.synchronize()
        ref = [net.layer_output(i) for i in range(len(w.layers))]
        tune.apply_plans(net, tune.load_plans(path, w, B))
        net.forward(img, d_pred)
        ctx.synchronize()
        for i in range(len(w.layers)):
            assert np.array_equal(net.layer_output(i), ref[i]), f"layer {i}"
    finally:
        net.close()


REG_CASES = [
    # T, tfs, task2 (alpha by time, same pad), H, W, C_in, C_out, K
    (64, 0.0, False, 9, 9, 8, 40, 2),      # 32 elements, one pixel per wave
    (64, 32.0, True, 8, 7, 3, 64, 3),      # VGG-16 L0's shape
    (64, 32.0, True, 6, 6, 32, 32, 1),     # 1x1, two pixels per wave
    (48, 0.0, False, 10, 10, 3, 16, 3),    # T below 64
    (16, 8.0, True, 8, 8, 3, 64, 3),       # short window, fire start
    (64, 0.0, False, 12, 12, 1, 6, 5),     # LeNet conv1's shape (the built-in choice)
    (64, 0.0, False, 9, 7, 2, 7, 3),       # no padding, 18 elements, nine pixels per wave (offset table)
    (64, 16.0, True, 7, 9, 3, 12, 3),      # same padding, 27 elements, five pixels per wave (bounds tests)
]


@pytest.mark.parametrize("case", REG_CASES, ids=[f"T{c[0]}-cin{c[5]}-cout{c[6]}-k{c[7]}" for c in REG_CASES])
def test_register_path_forced_matches_oracle(gpu_ctx_factory, case):
    """A one-layer network forced onto the register path (and on its
    built-in path) equals the oracle's one-layer network bit for bit."""
    import zlib

    T, tfs, task2, H, W, C_in, C_out, K = case
    say(f"register path {case}")
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    tc = vdttfs.TaskConsts(T=T, tfs=tfs, delta=8, vth=1.0, alpha_by_time=task2, conv_same_pad=task2)
    ho, wo = (H, W) if task2 else (H - K + 1, W - K + 1)
    kern = (rng.standard_normal((K, K, C_in, C_out)) * np.sqrt(2.0 / (K * K * C_in))).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.05).astype(np.float32)
    layer = vdttfs.Layer(vdttfs.LAYER_CONV, H, W, C_in, ho, wo, C_out, K, K, kern, bias, T / 4.0, 0.0)
    B = 3
    n_in = B * H * W * C_in
    t = np.floor(rng.random(n_in) * (T + tfs)).astype(np.float32)
    t = np.where(rng.random(n_in) < 0.3, np.float32(9999.0), t).astype(np.float32)
    ref = oracle.net_forward(oracle.Consts.from_task(tc), [layer], B, t, H * W * C_in, oracle.ENC_TIMES,
                             T / 4.0, 0.0, oracle.READ_ARGMIN, same_pad=task2)["final"]
    assert 0.02 < float(np.mean(ref < 9999.0)) < 0.98
    ctx = gpu_ctx_factory(tc)
    net = vdttfs.Net(ctx, [layer], B, H * W * C_in, vdttfs.ENCODE_TIMES, T / 4.0, 0.0, vdttfs.READOUT_ARGMIN)
    try:
        x = ctx.to_device(t)
        for plan in ((0, 0, 0), (REG, 0, 0)):
            net.set_plan(0, *plan)
            net.forward(x)
            ctx.synchronize()
            got = net.layer_output(0)
            np.testing.assert_array_equal(got, ref, err_msg=f"plan {net.get_plan(0)}")
        assert net.get_plan(0)[0] == REG
    finally:
        net.close()


def test_builtin_pixels_per_wave_follow_residency(gpu_ctx_factory):
    """VGG-16 at B=256: the built-in fused plans take four pixels per wave on
    the one-chunk conv 0 and one elsewhere (the shared-list kernel runs one
    pixel per workgroup).  On the bins path, two pixels per wave exactly
    where one pixel per wave needs between one and two rounds of resident
    waves (the 4x4 layers, 8,192 waves) and two fit in one."""
    say("plans: VGG-16 B=256 pixels per wave from residency")
    w = models.vgg16()
    ctx = gpu_ctx_factory(w.consts)
    net = make_net(ctx, w, 256)
    weighted = (0, 1, 3, 4, 6, 7, 8, 10, 11, 12, 14, 15, 16, 18)
    try:
        ppw = {i: net.get_plan(i)[2] for i in weighted}
        # conv 0: the one-chunk fused kernel takes four pixels per wave at 2^18 pixels
        assert ppw == {i: (4 if i == 0 else 1) for i in weighted}, ppw
        for i in weighted[4:]:
            net.set_plan(i, BINS, 4 if i < 18 else 2)
        ppw = {i: net.get_plan(i)[2] for i in weighted[4:]}
        assert ppw == {6: 1, 7: 1, 8: 1, 10: 2, 11: 2, 12: 2, 14: 1, 15: 1, 16: 1, 18: 1}, ppw
    finally:
        net.close()
