"""CuLIF (T3V, config 4) on the GPU: each drop-in kernel against the oracle on
the reference layouts, bit for bit; the engine network layer by layer; and,
at the full config-4 size, the first samples against the oracle plus
bit-identical outputs across chunk widths."""
import sys

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import models

pytestmark = pytest.mark.gpu
INF = np.float32(9999.0)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def spike_map(rng, n, T, p=0.5):
    t = rng.integers(0, T, size=n).astype(np.float32)
    s = np.where(rng.random(n) < p, t, INF).astype(np.float32)
    s[:6] = [T + 3, np.nan, 2.75, -0.5, -1.5, T - 1]  # dropped, dropped, 2, 0, dropped, last
    return s


# C_in <= 4 runs the LDS-tiled kernel (16-pixel row tiles, ragged here),
# larger C_in the lane-broadcast kernel (T > 64: several 64-step blocks)
@pytest.mark.parametrize("T,delta,C_out,C_in,W", [(64, 32, 70, 2, 37), (48, 16, 64, 2, 7),
                                                  (32, 32, 5, 1, 16), (80, 16, 40, 3, 9),
                                                  (64, 32, 64, 4, 20), (64, 32, 64, 5, 11),
                                                  (80, 16, 33, 6, 5)])
def test_conv1_raw(gpu_ctx_factory, T, delta, C_out, C_in, W):
    say(f"culif conv1_raw T={T} delta={delta} C_out={C_out} C_in={C_in} W={W}")
    ctx = gpu_ctx_factory(vdttfs.task3_consts(T=T, delta=delta))
    rng = np.random.default_rng(31)
    N, H = 2, 9
    data = (rng.random((N, C_in, H, W, T)) < 0.05).astype(np.float32)
    w = (rng.standard_normal((C_out, C_in, 3, 3)) * 0.6).astype(np.float32)
    exp = oracle.culif_conv1_raw(data, w, N, C_in, C_out, H, W, T, delta, 0.5, 1.0)
    d_out = ctx.empty(exp.size)
    ctx.culif_conv1_raw(ctx.to_device(data), d_out, ctx.to_device(w), N, C_in, C_out, H, W, 0.5, 1.0)
    got = d_out.download()
    assert np.any(exp < INF) and np.any(exp == INF)
    np.testing.assert_array_equal(got, exp)


def test_conv1_raw_nonfinite_weight(gpu_ctx_factory):
    """An infinite weight turns the reference's fma with a zero input into NaN:
    every in-bounds tap is integrated, zero inputs included."""
    say("culif conv1_raw with an infinite weight")
    T, delta = 64, 32
    ctx = gpu_ctx_factory(vdttfs.task3_consts(T=T, delta=delta))
    rng = np.random.default_rng(34)
    N, C_in, C_out, H, W = 1, 2, 64, 6, 5
    data = (rng.random((N, C_in, H, W, T)) < 0.1).astype(np.float32)
    w = (rng.standard_normal((C_out, C_in, 3, 3)) * 0.8).astype(np.float32)
    w[3, 1, 1, 1] = np.inf
    exp = oracle.culif_conv1_raw(data, w, N, C_in, C_out, H, W, T, delta, 0.5, 1.0)
    d_out = ctx.empty(exp.size)
    ctx.culif_conv1_raw(ctx.to_device(data), d_out, ctx.to_device(w), N, C_in, C_out, H, W, 0.5, 1.0)
    np.testing.assert_array_equal(d_out.download(), exp)
    # the non-finite weight changes c_out 3 (inf * 1 fires at once, inf * 0 is
    # NaN and never fires), so skipping zero inputs would have shown
    w0 = w.copy()
    w0[3, 1, 1, 1] = 0.0
    ref0 = oracle.culif_conv1_raw(data, w0, N, C_in, C_out, H, W, T, delta, 0.5, 1.0)
    assert np.any(exp.reshape(C_out, H, W)[3] != ref0.reshape(C_out, H, W)[3])


def test_bucketize_conv_and_fc(gpu_ctx_factory):
    say("culif bucketize conv/fc")
    T, delta = 64, 16
    ctx = gpu_ctx_factory(vdttfs.task3_consts(T=T, delta=delta))
    rng = np.random.default_rng(32)
    # up to 4,096 sites run one wave per site, more one thread per site
    for (N, Cc, H, W) in [(2, 64, 5, 6), (1, 3, 7, 1), (3, 130, 2, 2), (2, 5, 64, 40)]:
        x = spike_map(rng, N * Cc * H * W, T)
        cin, tin, off = oracle.culif_bucketize_nchw(x, N, Cc, H, W, T, delta)
        d_c, d_t, d_o = ctx.empty(cin.size, np.int32), ctx.empty(tin.size), ctx.empty(off.size, np.int32)
        ctx.culif_bucketize_conv(ctx.to_device(x), N, Cc, H, W, d_c, d_t, d_o)
        go = d_o.download()
        np.testing.assert_array_equal(go, off)
        gc, gt = d_c.download(), d_t.download()
        OS = T // delta + 1
        for s in range(N * H * W):  # only each site's first off[NC] entries are defined
            n = off[s * OS + OS - 1]
            np.testing.assert_array_equal(gc[s * Cc:s * Cc + n], cin[s * Cc:s * Cc + n])
            np.testing.assert_array_equal(gt[s * Cc:s * Cc + n], tin[s * Cc:s * Cc + n])
    # FC inputs (one site per sample), with 4, 64 and 1 chunks
    for d in (delta, 1, T):
        c = ctx if d == delta else gpu_ctx_factory(vdttfs.task3_consts(T=T, delta=d))
        N, F = 5, 1000
        x = spike_map(rng, N * F, T)
        cin, tin, off = oracle.culif_bucketize_fc(x, N, F, T, d)
        d_c, d_t, d_o = c.empty(cin.size, np.int32), c.empty(tin.size), c.empty(off.size, np.int32)
        c.culif_bucketize_fc(c.to_device(x), N, F, d_c, d_t, d_o)
        np.testing.assert_array_equal(d_o.download(), off)
        OS = T // d + 1
        gc, gt = d_c.download(), d_t.download()
        for n in range(N):
            k = off[n * OS + OS - 1]
            np.testing.assert_array_equal(gc[n * F:n * F + k], cin[n * F:n * F + k])
            np.testing.assert_array_equal(gt[n * F:n * F + k], tin[n * F:n * F + k])


@pytest.mark.parametrize("delta", [8, 32])
def test_conv_pool_fc_fcrec_dropin(gpu_ctx_factory, delta):
    say(f"culif conv / pool / fc / fc_recurrent drop-in delta={delta}")
    T = 64
    ctx = gpu_ctx_factory(vdttfs.task3_consts(T=T, delta=delta))
    rng = np.random.default_rng(33)
    # conv_bucketed_early
    N, C_in, C_out, H, W = 2, 24, 20, 6, 5
    x = spike_map(rng, N * C_in * H * W, T, p=0.4)
    w = (rng.standard_normal((C_out, C_in, 3, 3)) * 0.5).astype(np.float32)
    b = oracle.culif_bucketize_nchw(x, N, C_in, H, W, T, delta)
    exp = oracle.culif_conv(*b, w, N, C_in, C_out, H, W, T, delta, 0.5, 1.0)
    db = [ctx.to_device(a) for a in b]
    d_out = ctx.empty(exp.size)
    ctx.culif_conv(*db, d_out, ctx.to_device(w), N, C_in, C_out, H, W, 0.5, 1.0)
    assert np.any(exp < INF)
    np.testing.assert_array_equal(d_out.download(), exp)
    # pool_chunk_early
    xp = spike_map(rng, 3 * 7 * 8 * 6, T, p=0.3)
    exp = oracle.culif_pool(xp, 3, 7, 8, 6, T, delta, 0.5, 1.0)
    d_p = ctx.empty(exp.size)
    ctx.culif_pool(ctx.to_device(xp), d_p, 3, 7, 8, 6, 0.5, 1.0)
    assert np.any(exp < INF) and np.any(exp == INF)
    np.testing.assert_array_equal(d_p.download(), exp)
    # thresholds at or below 0: every neuron fires at step 0, input or not;
    # and a decay above 1 and below 0
    for decay, th in ((0.5, 0.0), (0.5, -1.0), (1.5, 2.5), (-0.5, 0.75)):
        exp = oracle.culif_pool(xp, 3, 7, 8, 6, T, delta, decay, th)
        ctx.culif_pool(ctx.to_device(xp), d_p, 3, 7, 8, 6, decay, th)
        np.testing.assert_array_equal(d_p.download(), exp)
    # fc2_bucketed_early and fc1_bucketed_recurrent
    for (N, F, O) in [(3, 300, 11), (2, 513, 128), (2, 70, 70)]:
        xf = spike_map(rng, N * F, T, p=0.5)
        bf = oracle.culif_bucketize_fc(xf, N, F, T, delta)
        dbf = [ctx.to_device(a) for a in bf]
        wf = (rng.standard_normal((O, F)) * (2.0 / np.sqrt(F))).astype(np.float32)
        exp = oracle.culif_fc(*bf, wf, N, F, O, T, delta, 0.5, 1.0)
        d_f = ctx.empty(exp.size)
        ctx.culif_fc(*dbf, d_f, ctx.to_device(wf), N, F, O, 0.5, 1.0)
        np.testing.assert_array_equal(d_f.download(), exp)
        wr = (rng.standard_normal((O, O)) * 0.3).astype(np.float32)
        exp = oracle.culif_fc_recurrent(*bf, wf, wr, N, F, O, T, delta, 0.5, 1.0)
        d_r = ctx.empty(exp.size)
        ctx.culif_fc_recurrent(*dbf, d_r, ctx.to_device(wf), ctx.to_device(wr), N, F, O, 0.5, 1.0)
        assert np.any(exp < INF)
        np.testing.assert_array_equal(d_r.download(), exp)
    # readout T3V:291-298 (class 0 when nothing fires)
    rows = np.array([[INF, INF, INF], [5, 3, 3], [2, 9, 1], [INF, 7, INF]], np.float32)
    d_pr = ctx.empty(4, np.int32)
    ctx.readout_argmin_first(ctx.to_device(rows), 4, 3, d_pr)
    np.testing.assert_array_equal(d_pr.download(), oracle.readout(rows, 4, 3, oracle.READ_T3))
    assert d_pr.download().tolist() == [0, 1, 2, 1]


def run_engine(ctx, w, B, ev):
    net = vdttfs.CulifNet(ctx, w.layers, B)
    try:
        d_ev = ctx.to_device(ev)
        d_pred = ctx.empty(B, np.int32)
        net.forward(d_ev, d_pred)
        ctx.synchronize()
        outs = [net.layer_output(i) for i in range(len(w.layers))]
        pred = d_pred.download()
        d_ev.free()
        d_pred.free()
    finally:
        net.close()
    return outs, pred


def test_culif_engine_small(gpu_ctx_factory):
    say("culif engine 2x32x32 B=3 vs oracle, every layer")
    w = models.culif7(H=32, W=32)
    B = 3
    ev = models.dvs_events(w, B)
    ctx = gpu_ctx_factory(w.consts)
    outs, pred = run_engine(ctx, w, B, ev)
    ref, rpred = oracle.culif_net_forward(w.layers, ev, B, w.consts.T, w.consts.delta)
    for i, (g, o) in enumerate(zip(outs, ref)):
        o = o.reshape(g.shape)
        assert np.any(o < INF), f"layer {i} silent"
        assert np.array_equal(g, o), f"layer {i} differs at {np.flatnonzero(g != o)[:8]}"
    np.testing.assert_array_equal(pred, rpred)


def test_culif_engine_narrow_convs(gpu_ctx_factory):
    """Conv layers with C_out <= 64 build their merged lists in LDS inside the
    integrating kernel (one wave per pixel), and a 20-wide conv packs three
    pixels per wave (k_stream_narrow); every layer against the oracle, and
    bit-identical across chunk widths."""
    say("culif engine with C_out <= 64 convs (lists in LDS, narrow) vs oracle")
    H, W, F = 24, 20, 20 * 12 * 10
    k = models.kaiming
    L = [vdttfs.CulifLayerSpec(vdttfs.CULIF_RAW_CONV, 2, H, W, 32, k(7, 0, (32, 2, 3, 3), 18), None, 0.5, 1.0),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_CONV, 32, H, W, 60, k(7, 1, (60, 32, 3, 3), 288), None, 0.5, 1.0),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_CONV, 60, H, W, 48, k(7, 2, (48, 60, 3, 3), 540), None, 0.5, 1.0),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_CONV, 48, H, W, 20, k(7, 4, (20, 48, 3, 3), 432), None, 0.5, 1.0),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_POOL, 20, H, W, 20, None, None, 0.5, 1.0),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_FC, F, 1, 1, 11, k(7, 3, (11, F), F), None, 0.5, 1.0)]
    w = models.CulifWorkload("narrow", vdttfs.task3_consts(T=64, delta=32), L, (2, H, W), 11, 7,
                             meta={"decay": 0.5, "th": 1.0, "density": 0.05, "sigma_px": 6.0,
                                   "vmax_px_per_step": 0.5})
    B = 3
    ev = models.dvs_events(w, B)
    outs, pred = run_engine(gpu_ctx_factory(w.consts), w, B, ev)
    ref, rpred = oracle.culif_net_forward(w.layers, ev, B, 64, 32)
    for i, (g, o) in enumerate(zip(outs, ref)):
        o = o.reshape(g.shape)
        assert np.any(o < INF), f"layer {i} silent"
        assert np.array_equal(g, o), f"layer {i} differs at {np.flatnonzero(g != o)[:8]}"
    np.testing.assert_array_equal(pred, rpred)
    outs16, _ = run_engine(gpu_ctx_factory(vdttfs.task3_consts(T=64, delta=16)), w, B, ev)
    for a, b in zip(outs16, outs):
        assert np.array_equal(a, b)


def test_culif_engine_conv1_inputs_and_weights(gpu_ctx_factory):
    """The engine's conv1 integrates from masks of nonzero steps when every
    weight is finite: inputs other than 1.0 (read back under the site's
    flag), -0.0 (skipped like 0), T > 64 (two step blocks) and T not a
    multiple of 8 (a last partial group of steps) match the oracle; an
    infinite weight keeps the dense kernel (inf * 0 = NaN)."""
    for T, delta in ((64, 32), (96, 32), (60, 20), (100, 20)):
        w = models.culif7(H=24, W=24, T=T, delta=delta)
        B = 2
        ev = models.dvs_events(w, B)
        rng = np.random.default_rng(40 + T)
        vals = np.array([0.5, 2.0, -1.0, -0.0, 1.0], np.float32)
        pick = rng.random(ev.shape) < 0.3
        ev = np.where((ev != 0) & pick, vals[rng.integers(0, vals.size, ev.shape)], ev).astype(np.float32)
        ev[1] = np.where(ev[1] != 0, 1.0, 0.0)  # sample 1 stays binary
        layers = list(w.layers)
        for inf_w in (False, True):
            say(f"culif engine conv1 T={T} non-binary inputs, inf weight={inf_w}")
            if inf_w:
                W0 = layers[0].weight.copy()
                W0[5, 1, 2, 0] = np.inf
                layers[0] = vdttfs.CulifLayerSpec(vdttfs.CULIF_RAW_CONV, 2, 24, 24, 64, W0, None, 0.5, 1.0)
            ww = models.CulifWorkload("conv1-check", w.consts, layers, w.in_shape, w.n_classes, w.seed, w.meta)
            outs, pred = run_engine(gpu_ctx_factory(w.consts), ww, B, ev)
            ref, rpred = oracle.culif_net_forward(ww.layers, ev, B, T, delta)
            g, o = outs[0], ref[0].reshape(outs[0].shape)
            assert np.any(o < INF) and np.any(o == INF)
            assert np.array_equal(g, o), f"conv1 differs at {np.flatnonzero(g != o)[:8]}"
            # the rest of the network too (recurrent FC over 4608 inputs: a
            # ragged last sort segment)
            for i in range(1, len(outs)):
                assert np.array_equal(outs[i], ref[i].reshape(outs[i].shape)), f"layer {i} differs"
            np.testing.assert_array_equal(pred, rpred)


@pytest.mark.parametrize("decay,th", [(0.9, 1.0), (0.85, 0.6), (-0.8, 0.3), (0.95, 1.0), (0.5, 0.0), (0.5, -0.5)])
def test_culif_engine_tail_steps(gpu_ctx_factory, decay, th):
    """Slow decays keep V rising long after a pixel's last input, so neurons
    fire in the input-free steps the fused conv streams close after the list
    ends (C_in 64 and 128, C_out 64 and 128, decay < 0 too): every layer
    equals the oracle, and for decay > 0 and th > 0 some spikes come after
    the pixel's last input.  Pixels with no input skip their steps: with
    th <= 0 their neurons fire at step 0, otherwise never."""
    say(f"culif engine tail steps decay={decay} th={th}")
    H = W = 16
    k = models.kaiming
    L = [vdttfs.CulifLayerSpec(vdttfs.CULIF_RAW_CONV, 2, H, W, 64, k(9, 0, (64, 2, 3, 3), 18), None, 0.5, 1.0),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_CONV, 64, H, W, 128, k(9, 1, (128, 64, 3, 3), 576), None, decay, th),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_CONV, 128, H, W, 64, k(9, 2, (64, 128, 3, 3), 1152), None, decay, th),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_CONV, 64, H, W, 128, k(9, 3, (128, 64, 3, 3), 576), None, decay, th),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_POOL, 128, H, W, 128, None, None, 0.5, 1.0),
         vdttfs.CulifLayerSpec(vdttfs.CULIF_FC, 128 * 8 * 8, 1, 1, 11, k(9, 4, (11, 128 * 64), 128 * 64), None,
                               0.5, 1.0)]
    # th <= 0: sparser events, so that some conv2 pixels see no input at all
    w = models.CulifWorkload("tail", vdttfs.task3_consts(T=64, delta=32), L, (2, H, W), 11, 9,
                             meta={"decay": 0.5, "th": 1.0, "density": 0.05 if th > 0 else 0.01, "sigma_px": 4.0,
                                   "vmax_px_per_step": 0.5})
    B = 2
    ev = models.dvs_events(w, B)
    outs, pred = run_engine(gpu_ctx_factory(w.consts), w, B, ev)
    ref, rpred = oracle.culif_net_forward(w.layers, ev, B, 64, 32)
    tail_fires = 0
    for i, (g, o) in enumerate(zip(outs, ref)):
        o = o.reshape(g.shape)
        assert np.array_equal(g, o), f"layer {i} differs at {np.flatnonzero(g != o)[:8]}"
        if i in (1, 2, 3):  # spikes after the last input step of the pixel's 3x3 field
            x = ref[i - 1].reshape(B, -1, H, W)
            step = np.where((x >= 0) & (x < 64), np.floor(x), -1).max(axis=1)
            last = np.full((B, H + 2, W + 2), -1.0)
            last[:, 1:-1, 1:-1] = step
            last = np.max([last[:, dy:dy + H, dx:dx + W] for dy in range(3) for dx in range(3)], axis=0)
            y = o.reshape(B, -1, H, W)
            tail_fires += int(np.sum((y < INF) & (y > last[:, None])))
    np.testing.assert_array_equal(pred, rpred)
    if decay > 0 and th > 0:  # an alternating I (decay < 0) rarely lifts V after its last input
        assert tail_fires > 0
    if th <= 0:  # conv2 pixels whose 3x3 field has no input at all (their neurons fire at step 0)
        x = ref[0].reshape(B, -1, H, W)
        p = np.zeros((B, H + 2, W + 2), bool)
        p[:, 1:-1, 1:-1] = ((x >= 0) & (x < 64)).any(axis=1)
        field = np.max([p[:, dy:dy + H, dx:dx + W] for dy in range(3) for dx in range(3)], axis=0)
        assert np.any(~field)
        assert np.all(ref[1].reshape(B, -1, H, W).transpose(0, 2, 3, 1)[~field] == 0)


def test_culif_config4_full(gpu_ctx_factory):
    """Config 4 at full size (2x128x128, T=64, B=64): all 64 samples equal
    the oracle at every layer; Delta in {16, 64} gives bit-identical maps."""
    w = models.culif7()
    B = 64
    ev = models.dvs_events(w, B)
    say("culif config 4 B=64 delta=32")
    outs, pred = run_engine(gpu_ctx_factory(w.consts), w, B, ev)
    k = B
    ref, rpred = oracle.culif_net_forward(w.layers, ev[:k], k, w.consts.T, w.consts.delta)
    for i, (g, o) in enumerate(zip(outs, ref)):
        o = o.reshape((k,) + g.shape[1:])
        assert np.array_equal(g[:k], o), f"layer {i} differs"
    np.testing.assert_array_equal(pred[:k], rpred)
    assert len(set(pred.tolist())) > 1
    for d in (16, 64):
        say(f"culif config 4 B=64 delta={d}")
        outs_d, pred_d = run_engine(gpu_ctx_factory(vdttfs.task3_consts(T=64, delta=d)), w, B, ev)
        for i, (a, b) in enumerate(zip(outs_d, outs)):
            assert np.array_equal(a, b), f"layer {i} differs at delta={d}"
        np.testing.assert_array_equal(pred_d, pred)
