"""Temporal-truncation calibration (vdttfs.calibrate): the percentile
window rule on the CPU, and on the GPU that the full window reproduces the
engine's own predictions while truncated windows only drop work."""
import numpy as np
import pytest

from vdttfs import calibrate, models


def test_arrival_bins_and_percentile_window():
    t = np.array([0.0, 3.0, 3.9, 40.0, 41.5, 9999.0, 63.0], np.float32)
    np.testing.assert_array_equal(calibrate.arrival_bins(t, 32.0), [0, 0, 0, 8, 9, 31])
    np.testing.assert_array_equal(calibrate.firing_steps(t), [0, 3, 3, 40, 41, 63])
    # bin rule only (T1): tb + 1; time-indexed decay (T2): also (int)t
    np.testing.assert_array_equal(calibrate.input_requirements(t, 32.0, 64, False), [1, 1, 1, 9, 10, 32])
    np.testing.assert_array_equal(calibrate.input_requirements(t, 32.0, 64, True), [1, 3, 3, 40, 41, 63])
    # spikes whose bin the full window already drops carry no requirement
    np.testing.assert_array_equal(calibrate.input_requirements(t, 0.0, 41, False), [1, 4, 4, 41])
    req = np.arange(1, 101)
    assert calibrate.percentile_window(req, 100.0, 64) == 64      # clamped to T
    assert calibrate.percentile_window(req, 50.0, 100) == 50
    assert calibrate.percentile_window(req, 1.0, 64) == 1
    assert calibrate.percentile_window(np.array([], np.int64), 99.0, 64) == 1
    # a window never exceeds T and always meets the requested share
    rng = np.random.default_rng(0)
    r = rng.integers(1, 65, 1000)
    for q in (10.0, 50.0, 90.0, 99.0, 100.0):
        Tp = calibrate.percentile_window(r, q, 64)
        assert 1 <= Tp <= 64 and np.count_nonzero(r <= Tp) / r.size >= q / 100.0 - 1e-12
        assert Tp == 1 or np.count_nonzero(r <= Tp - 1) / r.size < q / 100.0


def test_oracle_times_input_equals_encoded_input():
    """The oracle's spike-times input mode on linearly encoded images gives
    the same network as its linear encoder on the images; truncating T
    changes the output (the window is live in the oracle)."""
    import dataclasses

    import oracle

    w = models.lenet5()
    B = 4
    img = models.images_for(w, B)
    c = oracle.Consts.from_task(w.consts)
    enc = oracle.encode_linear(img.ravel(), w.consts.T)
    a = oracle.net_forward(c, w.layers, B, img, w.img_elems, oracle.ENC_LINEAR, w.tc_in, w.td_in, 0)
    b = oracle.net_forward(c, w.layers, B, enc, w.img_elems, oracle.ENC_TIMES, w.tc_in, w.td_in, 0)
    np.testing.assert_array_equal(a["final"], b["final"])
    c16 = oracle.Consts.from_task(dataclasses.replace(w.consts, T=16))
    t = oracle.net_forward(c16, w.layers, B, enc, w.img_elems, oracle.ENC_TIMES, w.tc_in, w.td_in, 0)
    assert not np.array_equal(t["final"], a["final"])
    assert np.all((t["final"] < 16) | (t["final"] == 9999.0))


@pytest.mark.gpu
def test_calibrate_lenet(gpu_ctx_factory):
    print("calibrate LeNet-5 B=128", flush=True)
    w = models.lenet5()
    B = 128
    T = w.consts.T
    r = calibrate.calibrate(w, models.images_for(w, B), B, percentiles=(50.0, 99.0, 100.0), windows=(8, T),
                            reps=2)
    uni = {s["T_window"]: s for s in r["sweep"] if s["mode"] == "uniform"}
    per = {s["percentile"]: s for s in r["sweep"] if s["mode"] == "per_layer"}
    assert uni[T]["predictions_changed"] == 0.0 and 8 in uni
    # at the 100th percentile every arrival and firing is kept: nothing changes
    assert per[100.0]["predictions_changed"] == 0.0
    assert [L["layer"] for L in r["layers"]] == [0, 2, 4, 5, 6]
    for L in r["layers"]:
        assert L["windows"]["50.0"] <= L["windows"]["99.0"] <= L["windows"]["100.0"] <= T
        assert L["windows"]["99.0"] >= L["input_windows"]["99.0"]
    v = r["suggested_windows"]["50.0"]
    assert v[1] == v[3] == 0 and v[0] == r["layers"][0]["windows"]["50.0"]


@pytest.mark.gpu
def test_calibrate_vgg_full_share_is_lossless(gpu_ctx_factory):
    """T2 semantics (TFS = T/2, time-indexed decay): per-layer windows that
    meet every requirement of the calibration inputs leave their outputs
    unchanged, while a uniform window at the bin bound T - TFS does not."""
    print("calibrate VGG-16 B=16", flush=True)
    w = models.vgg16()
    B = 16
    T = w.consts.T
    r = calibrate.calibrate(w, models.images_for(w, B), B, percentiles=(100.0,), windows=(T // 2,), reps=1)
    per = [s for s in r["sweep"] if s["mode"] == "per_layer"]
    assert len(per) == 1 and per[0]["predictions_changed"] == 0.0
    readout = r["layers"][-1]
    assert readout["kind"] == "vmem" and readout["input_windows"]["100.0"] > T // 2


@pytest.mark.gpu
@pytest.mark.parametrize("Tp", [24, 40])
def test_uniform_windows_equal_narrow_context(gpu_ctx_factory, Tp):
    """Every layer at T' through vdttfs_net_set_windows gives bit-identical
    layer outputs to a context created with T = T', and the layers of a
    per-layer setting equal the oracle run layer by layer at each T'_l."""
    import dataclasses

    import vdttfs
    import oracle

    print(f"windows LeNet-5 T'={Tp}", flush=True)
    w = models.lenet5()
    B = 64
    full = gpu_ctx_factory(w.consts)
    narrow = gpu_ctx_factory(dataclasses.replace(w.consts, T=Tp))
    img = full.to_device(models.images_for(w, B))
    x = full.empty(B * w.img_elems)
    full.encode_linear(img, x)
    enc = x.download()
    a = vdttfs.Net(full, w.layers, B, w.img_elems, vdttfs.ENCODE_TIMES, w.tc_in, w.td_in, w.readout)
    b = vdttfs.Net(narrow, w.layers, B, w.img_elems, vdttfs.ENCODE_TIMES, w.tc_in, w.td_in, w.readout)
    try:
        xb = narrow.to_device(enc)
        pa, pb = full.empty(B, np.int32), narrow.empty(B, np.int32)
        a.set_windows([Tp] * len(w.layers))
        a.forward(x, pa)
        b.forward(xb, pb)
        full.synchronize()
        narrow.synchronize()
        for i in range(len(w.layers)):
            np.testing.assert_array_equal(a.layer_output(i), b.layer_output(i), err_msg=f"layer {i}")
        np.testing.assert_array_equal(pa.download(), pb.download())
        # per-layer windows: each layer equals the oracle's one-layer network
        # at that layer's window, fed the engine's previous output
        wins = [Tp, 0, 48, 0, Tp - 8, 56, 0]
        a.set_windows(wins)
        a.forward(x, pa)
        full.synchronize()
        cur = enc
        tc_i, td_i = w.tc_in, w.td_in
        for i, l in enumerate(w.layers):
            Tl = wins[i] or w.consts.T
            c = oracle.Consts.from_task(dataclasses.replace(w.consts, T=Tl))
            ref = oracle.net_forward(c, [l], B, cur, l.H_in * l.W_in * l.C_in, oracle.ENC_TIMES, tc_i, td_i, 0)
            got = a.layer_output(i)
            np.testing.assert_array_equal(got, ref["final"], err_msg=f"layer {i} window {Tl}")
            if l.kind != vdttfs.LAYER_POOL:
                tc_i, td_i = l.tc_fire, l.td
            cur = got
        # reset: the full window again
        a.set_windows(None)
        a.forward(x, pa)
        full.synchronize()
        ref = oracle.net_forward(oracle.Consts.from_task(w.consts), w.layers, B, enc, w.img_elems,
                                 oracle.ENC_TIMES, w.tc_in, w.td_in, 0)
        np.testing.assert_array_equal(a.layer_output(len(w.layers) - 1), ref["final"])
        with pytest.raises(vdttfs.VdttfsError):
            a.set_windows([w.consts.T + 1] * len(w.layers))
        with pytest.raises(vdttfs.VdttfsError):
            a.set_windows([0] * (len(w.layers) - 1))
    finally:
        a.close()
        b.close()
