"""Pins of the step-by-step (time-driven) baseline oracle, orc_stepnet_forward
(T1S = task1_lenet_mnist/stepbystep_cuda/snn_mnist_stepbystep.cu,
T2S = task2_vgg16_cifar10/stepbystep_cuda/bench_vgg_timedriven_baseline.cu):

* closed forms for single-input neurons in both modes (T1S: V = w*kv(s) from
  the arrival step s on; T2S: the same in layer-local time, and the output
  layer's max(V + b) over its window);
* agreement with the event-driven oracle where the two models coincide (a
  single input per neuron: the per-step psp and the per-bin fma chain round
  the same single product);
* a brute-force re-simulation in Python of a small conv + pool + FC network
  in exact binary32 steps;
* the step counts (T for T1S; (D-1)*TFS + T for T2S, 680 at the reference's
  16 weighted layers, TFS 40, T 80)."""
import numpy as np
import pytest

import oracle
from vdttfs import core
from vdttfs.core import Layer

INF = np.float32(9999.0)
F32 = np.float32


def consts(T=64, tfs=0.0):
    return oracle.Consts(T=T, tfs=tfs, delta=8, alpha_by_time=0, vth=1.0)


def fc(C_in, C_out, w, b, tc=16.0, td=0.0, kind=core.LAYER_FC):
    return Layer(kind, 1, 1, C_in, 1, 1, C_out, 1, 1, np.asarray(w, F32).reshape(C_in, C_out),
                 np.asarray(b, F32), tc, td)


def kv_th(T, tc_i, td_i, tc_f, td_f, vth=1.0):
    a, th = oracle.build_luts(T, vth, tc_i, td_i, tc_f, td_f)
    return np.asarray(a, F32), np.asarray(th, F32)


def test_t1_single_input_closed_form():
    T = 64
    rng = np.random.default_rng(1)
    for trial in range(40):
        s = int(rng.integers(0, T))
        x = F32(1.0 - (s + 0.5) / T)           # linear encoding: floor(T(1-x)) = s
        w = F32(rng.normal() * 2.0)
        b = F32(rng.normal() * 0.3)
        td = float(rng.choice([0.0, 3.0, 7.5]))
        L = [fc(1, 1, [w], [b], tc=16.0, td=td)]
        r = oracle.stepnet_forward(consts(T), L, 1, np.array([x], F32), 1, oracle.ENC_LINEAR,
                                   16.0, 0.0, oracle.STEP_T1)
        assert r["steps"] == T
        kv, th = kv_th(T, 16.0, 0.0, 16.0, td)
        t_min = max(0, int(np.ceil(td)))
        exp = INF
        for t in range(T):
            v = F32(w * kv[s]) if t >= s else F32(0.0)   # one rounding: fma(w, kv, 0)
            if t >= t_min and F32(v + b) >= th[t] and th[t] >= F32(1e-5):
                exp = F32(t)
                break
        assert r["final"][0] == exp, (trial, s, w, b, td)


def test_t1_matches_event_driven_for_single_inputs():
    """One input per neuron: the T1S per-step psp and the T1V per-bin chain
    round the same product, so first-spike times agree."""
    T, B, Cin, Cout = 64, 8, 16, 12
    rng = np.random.default_rng(2)
    W = np.zeros((Cin, Cout), F32)
    for o in range(Cout):
        W[rng.integers(0, Cin), o] = F32(rng.normal() * 3.0)
    bias = (rng.normal(size=Cout) * 0.2).astype(F32)
    img = rng.random(B * Cin).astype(F32)
    L = [fc(Cin, Cout, W, bias)]
    r = oracle.stepnet_forward(consts(T), L, B, img, Cin, oracle.ENC_LINEAR, 16.0, 0.0, oracle.STEP_T1)
    e = oracle.net_forward(consts(T), L, B, img, Cin, oracle.ENC_LINEAR, 16.0, 0.0, oracle.READ_ARGMIN)
    np.testing.assert_array_equal(r["final"], e["final"])
    assert np.any(r["final"] < INF)


def test_t2_depth_offsets_and_max_vmem():
    """Two FC layers, one input each: layer 1 fires at local t1 (global t1 +
    TFS), layer 2 (the output) integrates it at local t1 and keeps
    max(V + b) over its window [0, T)."""
    T, tfs = 32, 8.0
    rng = np.random.default_rng(3)
    for trial in range(20):
        s = int(rng.integers(0, T))
        x = F32(1.0 - (s + 0.5) / T)
        w1, b1 = F32(abs(rng.normal()) * 3 + 0.5), F32(rng.normal() * 0.1)
        w2, b2 = F32(rng.normal() * 2.0), F32(rng.normal() * 0.3)
        L = [fc(1, 1, [w1], [b1]), fc(1, 1, [w2], [b2], kind=core.LAYER_VMEM)]
        r = oracle.stepnet_forward(consts(T, tfs), L, 1, np.array([x], F32), 1, oracle.ENC_LINEAR,
                                   16.0, 0.0, oracle.STEP_T2)
        assert r["steps"] == int(np.ceil(1 * tfs + T))
        kv1, th1 = kv_th(T, 16.0, 0.0, 16.0, 0.0)
        # layer 1 (depth 1): integrates at local t = global t, fires at local t_f = t - tfs
        v1 = F32(w1 * kv1[s])
        t1 = None
        for tf in range(T):          # local fire time; V seen at global tf + tfs
            g = tf + int(tfs)
            v = v1 if g >= s else F32(0.0)
            if F32(v + b1) >= th1[tf] and th1[tf] >= F32(1e-5):
                t1 = tf
                break
        kv2, _ = kv_th(T, 16.0, 0.0, 16.0, 0.0)
        # layer 2 (output): integrates at local ti = global - tfs in [0, T); the
        # layer-1 spike at global t1 + tfs arrives at local t1
        best = F32(-1e9)
        for ti in range(T):
            v = F32(w2 * kv2[t1]) if (t1 is not None and ti >= t1) else F32(0.0)
            best = max(best, F32(v + b2))
        assert r["final"][0] == best, (trial, s, t1)


def _brute_t1(T, img, conv_w, conv_b, fc_w, fc_b, tc_in, tcs):
    """Brute-force T1S in numpy float32: conv 3x3 valid (1 -> Co) on HxW,
    2x2 pool, FC to K outputs; returns the output first-spike steps."""
    H, W = img.shape
    Co = conv_w.shape[-1]
    Ho, Wo = H - 2, W - 2
    tin = np.where(img < 1e-5, INF, np.floor(F32(T) * (F32(1.0) - img))).astype(F32)
    Vc = np.zeros((Ho, Wo, Co), F32); fc_ = np.zeros((Ho, Wo, Co), bool)
    fp = np.zeros((Ho // 2, Wo // 2, Co), bool)
    K = fc_w.shape[1]
    Vf = np.zeros(K, F32); ff = np.zeros(K, bool); first = np.full(K, INF, F32)
    kv0, th0 = kv_th(T, tc_in, 0.0, tcs[0], 0.0)
    kv1, th1 = kv_th(T, tcs[0], 0.0, tcs[1], 0.0)
    for t in range(T):
        s0 = tin == F32(t)
        s1 = np.zeros((Ho, Wo, Co), bool)
        for y in range(Ho):
            for x in range(Wo):
                for o in range(Co):
                    if fc_[y, x, o]:
                        continue
                    psp = F32(0.0)
                    for kh in range(3):
                        for kw in range(3):
                            if s0[y + kh, x + kw]:
                                psp = F32(psp + conv_w[kh, kw, 0, o])
                    Vc[y, x, o] = F32(np.float64(psp) * np.float64(kv0[t]) + np.float64(Vc[y, x, o]))
                    if F32(Vc[y, x, o] + conv_b[o]) >= th0[t] and th0[t] >= F32(1e-5):
                        s1[y, x, o] = True
                        fc_[y, x, o] = True
        sp = np.zeros((Ho // 2, Wo // 2, Co), bool)
        for y in range(Ho // 2):
            for x in range(Wo // 2):
                for o in range(Co):
                    if fp[y, x, o]:
                        continue
                    if s1[2 * y:2 * y + 2, 2 * x:2 * x + 2, o].any():
                        sp[y, x, o] = True
                        fp[y, x, o] = True
        flat = sp.reshape(-1)
        for k in range(K):
            if ff[k]:
                continue
            psp = F32(0.0)
            for i in np.flatnonzero(flat):
                psp = F32(psp + fc_w[i, k])
            Vf[k] = F32(np.float64(psp) * np.float64(kv1[t]) + np.float64(Vf[k]))
            if F32(Vf[k] + fc_b[k]) >= th1[t] and th1[t] >= F32(1e-5):
                ff[k] = True
                if first[k] >= INF:
                    first[k] = F32(t)
    return first


def test_t1_conv_pool_fc_brute_force():
    T, H, W, Co, K = 24, 8, 8, 3, 4
    rng = np.random.default_rng(4)
    img = np.where(rng.random((H, W)) < 0.4, 0.0, rng.random((H, W))).astype(F32)
    cw = (rng.normal(size=(3, 3, 1, Co)) * 0.9).astype(F32)
    cb = (rng.normal(size=Co) * 0.1).astype(F32)
    n_flat = 3 * 3 * Co
    fw = (rng.normal(size=(n_flat, K)) * 0.8).astype(F32)
    fb = (rng.normal(size=K) * 0.1).astype(F32)
    tcs = (6.0, 6.0)
    L = [Layer(core.LAYER_CONV, H, W, 1, H - 2, W - 2, Co, 3, 3, cw, cb, tcs[0], 0.0),
         Layer(core.LAYER_POOL, H - 2, W - 2, Co, 3, 3, Co),
         Layer(core.LAYER_FC, 3, 3, Co, 1, 1, K, 1, 1, fw, fb, tcs[1], 0.0)]
    r = oracle.stepnet_forward(consts(T), L, 1, img.reshape(-1), H * W, oracle.ENC_LINEAR, 6.0, 0.0,
                               oracle.STEP_T1)
    exp = _brute_t1(T, img, cw, cb, fw, fb, 6.0, tcs)
    np.testing.assert_array_equal(r["final"], exp)
    assert np.any(exp < INF)


def test_t2_step_count_of_the_reference():
    """T2S runs TIME_STEPS = 680 for its 16 weighted layers at TFS 40, T 80."""
    L = []
    for i in range(16):
        L.append(fc(1, 1, [1.0], [0.0], kind=core.LAYER_VMEM if i == 15 else core.LAYER_FC))
    r = oracle.stepnet_forward(consts(80, 40.0), L, 1, np.array([0.5], F32), 1, oracle.ENC_LINEAR,
                               16.0, 0.0, oracle.STEP_T2)
    assert r["steps"] == 680
