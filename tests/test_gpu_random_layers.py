"""Seeded random layer configurations against the oracle.

Each case draws a valid layer -- conv (K in {1, 2, 3, 5, 7}, valid or same
padding, C_in 1..130, C_out 1..200; a share with K*K*C_in <= 32, C_out <= 64,
T <= 64) or FC (C_in 1..600, C_out 1..300) --
with random T (1..255, the window's limit), fire start, chunk width, t_min, decay and threshold
tables (monotone, or shuffled with entries below 1e-5) and spike density,
so the launch logic's branches are crossed with each other: the generic,
narrow, register, fused, dense and bins paths; one, two or four c_out per
lane and several c_out blocks; T above 64 (several bin blocks).  Every
case must equal the oracle bit for bit:

* the drop-in pair (reference-layout bucketize + integrate),
* the engine path with and without work counters (counts equal too),
* for conv layers, a one-layer network under every launch plan the kernels
  accept (vdttfs_net_set_plan).
"""
import sys
import zlib

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import tune

pytestmark = pytest.mark.gpu

N_CASES = 60
INF = 9999.0


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def draw(i):
    rng = np.random.default_rng(zlib.crc32(f"random-layer-{i}".encode()))
    T = int(rng.choice([1, 7, 16, 33, 64, 65, 80, 128, 200, 255]))
    task2 = bool(rng.random() < 0.5)
    tfs = float(rng.integers(0, T)) if rng.random() < 0.5 else 0.0
    delta = int(rng.choice([1, 4, 8, 16, 32, 64]))
    is_fc = bool(rng.random() < 0.3)
    if is_fc:
        C_in, C_out, B = int(rng.integers(1, 601)), int(rng.integers(1, 301)), int(rng.integers(1, 41))
        H = W = K = 1
    elif rng.random() < 0.3:
        # small receptive fields (K*K*C_in <= 32), C_out <= 64, T <= 64: the register path
        T = int(rng.choice([1, 7, 16, 33, 64]))
        tfs = float(rng.integers(0, T)) if rng.random() < 0.5 else 0.0
        K = int(rng.choice([1, 2, 3, 5] if not task2 else [1, 3, 5]))
        C_in = int(rng.integers(1, 32 // (K * K) + 1))
        C_out, B = int(rng.integers(1, 65)), int(rng.integers(1, 4))
        H, W = int(rng.integers(K, 13)), int(rng.integers(K, 13))
    else:
        K = int(rng.choice([1, 2, 3, 5, 7] if not task2 else [1, 3, 5, 7]))  # same padding needs odd K
        C_in = int(rng.integers(1, 9)) if rng.random() < 0.4 else int(rng.integers(1, 131))
        C_out, B = int(rng.integers(1, 201)), int(rng.integers(1, 4))
        H, W = int(rng.integers(K, 13)), int(rng.integers(K, 13))
    return dict(T=T, task2=task2, tfs=tfs, delta=delta, is_fc=is_fc, C_in=C_in, C_out=C_out, B=B, H=H,
                W=W, K=K, t_min=int(rng.integers(0, 4)), density=float(rng.uniform(0.05, 0.95)),
                shuffled=bool(rng.random() < 0.25), tc=float(rng.uniform(2.0, 2.0 * T + 2.0)),
                td=float(rng.uniform(-2.0, 4.0)), seed=int(rng.integers(1 << 30)))


def build(c):
    rng = np.random.default_rng(c["seed"])
    tc = vdttfs.TaskConsts(T=c["T"], tfs=c["tfs"], delta=c["delta"], vth=1.0, alpha_by_time=c["task2"],
                           conv_same_pad=c["task2"])
    if c["is_fc"]:
        n_cols, kshape = c["B"], (c["C_in"], c["C_out"])
        shape = dict(B=c["B"], H_in=1, W_in=1, C_in=c["C_in"], H_out=1, W_out=1, C_out=c["C_out"], K_h=1, K_w=1)
    else:
        K, H, W = c["K"], c["H"], c["W"]
        ho, wo = (H, W) if c["task2"] else (H - K + 1, W - K + 1)
        n_cols, kshape = c["B"] * H * W, (K, K, c["C_in"], c["C_out"])
        shape = dict(B=c["B"], H_in=H, W_in=W, C_in=c["C_in"], H_out=ho, W_out=wo, C_out=c["C_out"], K_h=K, K_w=K)
    n_in = n_cols * c["C_in"]
    t = np.floor(rng.random(n_in) * (c["T"] + c["tfs"] + 2)).astype(np.float32)
    sp = np.where(rng.random(n_in) < c["density"], t, np.float32(INF)).astype(np.float32)
    fan = int(np.prod(kshape[:-1]))
    Wt = (rng.standard_normal(int(np.prod(kshape))) * np.sqrt(2.0 / fan)).astype(np.float32)
    bias = (rng.standard_normal(c["C_out"]) * 0.05).astype(np.float32)
    alpha, theta = vdttfs.build_luts_host(tc, c["tc"], c["td"], c["tc"], c["td"])
    if c["shuffled"]:
        theta = rng.permutation(theta).astype(np.float32)
        theta[rng.random(theta.size) < 0.1] = np.float32(1e-6)
    return tc, sp, Wt, bias, alpha, theta, n_cols, shape


def oracle_layer(tc, sp, Wt, bias, alpha, theta, n_cols, shape, t_min, is_fc):
    cc = oracle.Consts.from_task(tc)
    cin, tin, off = oracle.bucketize(cc, sp, n_cols, shape["C_in"])
    pad = shape["K_h"] // 2 if (tc.conv_same_pad and not is_fc) else 0
    return oracle.integrate(cc, cin, tin, off, Wt, bias, alpha, theta, t_min, pad=pad, is_fc=is_fc, **shape)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_layer_matches_oracle(gpu_ctx_factory, i):
    c = draw(i)
    say(f"random layer {i}: {c}")
    tc, sp, Wt, bias, alpha, theta, n_cols, shape = build(c)
    exp, ep, eb = oracle_layer(tc, sp, Wt, bias, alpha, theta, n_cols, shape, c["t_min"], c["is_fc"])
    ctx = gpu_ctx_factory(tc)
    d_in, d_W, d_b = ctx.to_device(sp), ctx.to_device(Wt), ctx.to_device(bias)
    d_a, d_t = ctx.to_device(alpha), ctx.to_device(theta)
    # drop-in pair
    OS = tc.num_chunks + 1
    d_cin = ctx.empty(n_cols * c["C_in"], np.int32)
    d_tin = ctx.empty(n_cols * c["C_in"], np.float32)
    d_off = ctx.empty(n_cols * OS, np.int32)
    d_out = ctx.empty(exp.size, np.float32)
    ctx.bucketize(d_in, n_cols, c["C_in"], d_cin, d_tin, d_off)
    ctx.integrate(d_out, d_cin, d_tin, d_off, d_W, d_b, d_a, d_t, c["t_min"], is_fc=c["is_fc"], **shape)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="drop-in pair")
    # engine, with and without counters
    gp, gb = ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, c["t_min"], is_fc=c["is_fc"], count=True, **shape)
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="engine, counting")
    assert (gp, gb) == (ep, eb)
    ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, c["t_min"], is_fc=c["is_fc"], **shape)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="engine")


@pytest.mark.parametrize("i", [i for i in range(N_CASES) if not draw(i)["is_fc"]])
def test_random_conv_every_plan(gpu_ctx_factory, i):
    """The conv cases as one-layer networks (their own LUTs from tc/td,
    t_min = ceil(td)), under every accepted launch plan."""
    c = draw(i)
    say(f"random conv {i}, every plan")
    tc, sp, Wt, bias, _, _, n_cols, shape = build(c)
    layer = vdttfs.Layer(vdttfs.LAYER_CONV, shape["H_in"], shape["W_in"], c["C_in"], shape["H_out"],
                         shape["W_out"], c["C_out"], c["K"], c["K"], Wt.reshape(c["K"], c["K"], c["C_in"], c["C_out"]),
                         bias, c["tc"], c["td"])
    elems = shape["H_in"] * shape["W_in"] * c["C_in"]
    ref = oracle.net_forward(oracle.Consts.from_task(tc), [layer], c["B"], sp, elems, oracle.ENC_TIMES,
                             c["tc"], c["td"], oracle.READ_ARGMIN, same_pad=c["task2"])["final"]
    ctx = gpu_ctx_factory(tc)
    net = vdttfs.Net(ctx, [layer], c["B"], elems, vdttfs.ENCODE_TIMES, c["tc"], c["td"], vdttfs.READOUT_ARGMIN)
    try:
        x = ctx.to_device(sp)
        plans = tune.candidates(net, 0)
        assert plans, "no accepted plan"
        for plan in plans:
            net.set_plan(0, *plan)
            net.forward(x)
            ctx.synchronize()
            np.testing.assert_array_equal(net.layer_output(0), ref, err_msg=f"plan {plan}")
    finally:
        net.close()
