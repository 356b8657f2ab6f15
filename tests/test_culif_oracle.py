"""Pins the CuLIF part of the CPU oracle (T3V:30-225) against time-driven
simulations: every step t gets a dense input current built directly from
the spike map (no buckets, no chunks), in exact binary32 arithmetic
(tests/pyref.py), and the neuron is stepped as the step-by-step baseline
defines it (T3S: I = I*decay + in, V += I, fire once at V >= th).  The
chunked, bucketed oracle must give the same first-spike steps for every
chunk width that divides T.
"""
import numpy as np
import pytest

import oracle
import pyref

INF = np.float32(9999.0)


def lif_steps(cur, T, decay, th):
    I = V = 0.0
    for t in range(T):
        I = pyref.fma32(I, decay, cur[t])
        V = pyref.add32(V, I)
        if V >= th:
            return float(t)
    return float(INF)


def spike_map(rng, n, T, p=0.5):
    t = rng.integers(0, T, size=n).astype(np.float32)
    s = np.where(rng.random(n) < p, t, INF).astype(np.float32)
    if n > 6:
        s[0] = np.float32(T + 3)    # beyond the window: dropped
        s[1] = np.float32(np.nan)   # dropped
        s[2] = np.float32(2.75)     # non-integer: step 2
    return s


def step_of(tf, T):
    """The arrival step of a spike under T3V:78 ((int)t, kept if 0 <= t < T)."""
    if not (tf < INF):
        return -1
    tb = int(tf)
    return tb if 0 <= tb < T else -1


@pytest.mark.parametrize("delta", [4, 8, 16])
def test_conv1_raw_matches_steps(delta):
    rng = np.random.default_rng(21)
    N, C_in, C_out, H, W, T = 1, 2, 3, 4, 5, 16
    data = (rng.random((N, C_in, H, W, T)) < 0.3).astype(np.float32)
    data[0, 0, 0, 0, 3] = 0.5  # a non-binary value: the fma is general
    w = (rng.standard_normal((C_out, C_in, 3, 3)) * 0.8).astype(np.float32)
    got = oracle.culif_conv1_raw(data, w, N, C_in, C_out, H, W, T, delta, 0.5, 1.0)
    got = got.reshape(N, C_out, H, W)
    assert np.any(got < INF) and np.any(got == INF)
    for o in range(C_out):
        for y in range(H):
            for x in range(W):
                cur = [0.0] * T
                for t in range(T):
                    for ci in range(C_in):
                        for ky in range(3):
                            for kx in range(3):
                                iy, ix = y + ky - 1, x + kx - 1
                                if 0 <= iy < H and 0 <= ix < W:
                                    cur[t] = pyref.fma32(float(w[o, ci, ky, kx]),
                                                         float(data[0, ci, iy, ix, t]), cur[t])
                assert got[0, o, y, x] == lif_steps(cur, T, 0.5, 1.0), (o, y, x)


def test_bucketize_nchw_matches_stable_sort():
    rng = np.random.default_rng(22)
    N, Cc, H, W, T, delta = 2, 9, 3, 2, 16, 4
    x = spike_map(rng, N * Cc * H * W, T)
    x[5] = np.float32(-0.5)  # (int)-0.5 == 0: kept in step 0
    x[6] = np.float32(-1.5)  # (int)-1.5 == -1: dropped
    cin, tin, off = oracle.culif_bucketize_nchw(x, N, Cc, H, W, T, delta)
    OS = T // delta + 1
    xs = x.reshape(N, Cc, H * W)
    for n in range(N):
        for hw in range(H * W):
            site = n * H * W + hw
            ev = []
            for c in range(Cc):
                tf = xs[n, c, hw]
                if tf < INF and 0 <= int(tf) < T:  # (int) truncates: -0.5 -> 0
                    ev.append((int(tf) // delta, c, tf))
            ev.sort(key=lambda e: e[0])  # stable: c ascending within a chunk
            o = off[site * OS:(site + 1) * OS]
            assert o[-1] == len(ev)
            for k in range(T // delta):
                assert o[k + 1] - o[k] == sum(1 for e in ev if e[0] == k)
            for p, (_, c, tf) in enumerate(ev):
                assert cin[site * Cc + p] == c
                assert tin[site * Cc + p] == tf


@pytest.mark.parametrize("delta", [4, 16])
def test_conv_matches_steps(delta):
    rng = np.random.default_rng(23)
    N, C_in, C_out, H, W, T = 1, 5, 3, 4, 4, 16
    x = spike_map(rng, N * C_in * H * W, T, p=0.6)
    w = (rng.standard_normal((C_out, C_in, 3, 3)) * 0.7).astype(np.float32)
    b = oracle.culif_bucketize_nchw(x, N, C_in, H, W, T, delta)
    got = oracle.culif_conv(*b, w, N, C_in, C_out, H, W, T, delta, 0.5, 1.0).reshape(N, C_out, H, W)
    xm = x.reshape(N, C_in, H, W)
    assert np.any(got < INF)
    for o in range(C_out):
        for y in range(H):
            for xx in range(W):
                cur = [0.0] * T
                # per step: taps in (ky, kx) order, then ascending cin (T3V:120-133)
                for ky in range(3):
                    for kx in range(3):
                        iy, ix = y + ky - 1, xx + kx - 1
                        if not (0 <= iy < H and 0 <= ix < W):
                            continue
                        for ci in range(C_in):
                            tb = step_of(xm[0, ci, iy, ix], T)
                            if tb >= 0:
                                cur[tb] = pyref.add32(cur[tb], float(w[o, ci, ky, kx]))
                assert got[0, o, y, xx] == lif_steps(cur, T, 0.5, 1.0), (o, y, xx)


def test_pool_matches_steps():
    rng = np.random.default_rng(24)
    N, Cc, H, W, T, delta = 1, 3, 6, 4, 16, 8
    x = spike_map(rng, N * Cc * H * W, T, p=0.4)
    got = oracle.culif_pool(x, N, Cc, H, W, T, delta, 0.5, 0.9).reshape(N, Cc, H // 2, W // 2)
    xm = x.reshape(N, Cc, H, W)
    assert np.any(got < INF) and np.any(got == INF)
    for c in range(Cc):
        for yo in range(H // 2):
            for xo in range(W // 2):
                cur = [0.0] * T
                for dy in range(2):
                    for dx in range(2):
                        tf = xm[0, c, 2 * yo + dy, 2 * xo + dx]
                        if 0 <= tf < T:
                            cur[int(tf)] = 1.0  # set, not added (T3V:159)
                assert got[0, c, yo, xo] == lif_steps(cur, T, 0.5, 0.9)


@pytest.mark.parametrize("delta", [4, 16])
def test_fc_recurrent_matches_steps(delta):
    rng = np.random.default_rng(25)
    N, F, O, T = 2, 24, 6, 16
    x = spike_map(rng, N * F, T, p=0.7)
    w = (rng.standard_normal((O, F)) * 0.6).astype(np.float32)
    wr = (rng.standard_normal((O, O)) * 0.8).astype(np.float32)
    b = oracle.culif_bucketize_fc(x, N, F, T, delta)
    got = oracle.culif_fc_recurrent(*b, w, wr, N, F, O, T, delta, 0.5, 0.8).reshape(N, O)
    assert np.any(got < INF)
    for n in range(N):
        I = [0.0] * O
        V = [0.0] * O
        fired = [False] * O
        prev = [False] * O
        res = [float(INF)] * O
        for t in range(T):
            now = [False] * O
            for i in range(O):
                ff = 0.0
                for j in range(F):
                    if step_of(x[n * F + j], T) == t:
                        ff = pyref.add32(ff, float(w[i, j]))
                rec = 0.0
                for j in range(O):
                    if prev[j]:
                        rec = pyref.add32(rec, float(wr[i, j]))
                I[i] = pyref.add32(pyref.fma32(I[i], 0.5, ff), rec)
                V[i] = pyref.add32(V[i], I[i])
                if V[i] >= 0.8 and not fired[i]:
                    now[i] = fired[i] = True
                    res[i] = float(t)
                    V[i] = -10000.0
            prev = now
        assert got[n].tolist() == res, n


def test_culif_net_is_delta_invariant():
    """The chained oracle network gives identical outputs for every chunk
    width dividing T (per-step recurrence; chunks only regroup steps)."""
    import sys
    import os
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    "vd-ttfs_amd"))
    from vdttfs import models
    w = models.culif7(H=16, W=16, T=32, delta=32)
    ev = models.dvs_events(w, 2)
    ref_outs, ref_pred = oracle.culif_net_forward(w.layers, ev, 2, 32, 32)
    assert any(np.any(o < INF) for o in ref_outs)
    for d in (4, 8, 16):
        outs, pred = oracle.culif_net_forward(w.layers, ev, 2, 32, d)
        for a, b in zip(outs, ref_outs):
            np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(pred, ref_pred)
