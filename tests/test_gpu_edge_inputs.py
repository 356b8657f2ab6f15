"""Degenerate inputs against the oracle, on every built-in integrator path.

* silent: no input spikes at all (every event list is empty); neurons can
  still fire from the bias alone as the threshold table decays;
* one bin: every input spikes in the first arrival bin (the largest
  possible collision: the whole receptive field in one bin's fma chain);
* last bin: every input spikes in the window's last arrival bin;
* past window: every input arrives after the window (all dropped);
* dense: every input spikes, at random times over the window (the longest
  lists, spread over all bins).

Each case must equal the oracle bit for bit through the drop-in pair
(reference-layout bucketize + integrate) and through the engine path with
and without work counters (counts equal too).  The shapes put one layer on
each path: fused list in LDS (one and two events per load, and past the
dense path's C_in limit), the shared-list kernel (64 and 128 c_out per wave,
conv and FC, with fields larger than its list capacity, so that the one-bin
and dense cases stream their lists in several windows: one split inside
bin 0, the other inside later bins), the narrow stream, the register path
and the generic integrator (> 25 taps).
"""
import sys
import zlib

import numpy as np
import pytest

import oracle
import vdttfs

pytestmark = pytest.mark.gpu

INF = 9999.0

# name, T, tfs, task2, is_fc, B, H, W, C_in, C_out, K
SHAPES = [
    ("fused-c64", 64, 32.0, True, False, 2, 6, 6, 16, 64, 3),
    ("fused-pair-c128", 64, 32.0, True, False, 2, 5, 5, 32, 128, 3),
    ("fused-wide-c128", 64, 32.0, True, False, 2, 5, 5, 128, 128, 3),
    ("shared-c256", 64, 0.0, False, False, 2, 6, 6, 96, 256, 3),
    ("shared-win-c512", 64, 32.0, True, False, 1, 4, 4, 512, 512, 3),
    ("shared-win-pair-c256", 64, 32.0, True, False, 2, 5, 5, 256, 256, 3),
    ("shared-win-fc-4096", 32, 0.0, False, True, 3, 1, 1, 4096, 256, 1),
    ("narrow-c10", 64, 0.0, False, False, 3, 8, 8, 6, 10, 5),
    ("reg-c3-o16", 64, 32.0, True, False, 2, 7, 7, 3, 16, 3),
    ("fc-512-96", 32, 0.0, False, True, 5, 1, 1, 512, 96, 1),
    ("generic-k7", 16, 0.0, False, False, 1, 9, 9, 4, 40, 7),
]
KINDS = ["silent", "one-bin", "last-bin", "past-window", "dense"]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def spike_times(kind, n, T, tfs, rng):
    if kind == "dense":
        return np.floor(rng.random(n) * (T + tfs)).astype(np.float32)
    if kind == "silent":
        v = INF
    elif kind == "one-bin":
        v = 0.0
    elif kind == "last-bin":
        v = float(T - 1) + tfs
    else:
        v = float(T) + tfs + 1.0
    return np.full(n, v, np.float32)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_degenerate_inputs_match_oracle(gpu_ctx_factory, shape, kind):
    name, T, tfs, task2, is_fc, B, H, W, C_in, C_out, K = shape
    say(f"edge input {kind} on {name}")
    tc = vdttfs.TaskConsts(T=T, tfs=tfs, delta=8 if T % 8 == 0 else 1, vth=1.0, alpha_by_time=task2,
                           conv_same_pad=task2)
    rng = np.random.default_rng(zlib.crc32(f"edge-{name}-{kind}".encode()))
    if is_fc:
        n_cols, kshape = B, (C_in, C_out)
        sh = dict(B=B, H_in=1, W_in=1, C_in=C_in, H_out=1, W_out=1, C_out=C_out, K_h=1, K_w=1)
    else:
        ho, wo = (H, W) if task2 else (H - K + 1, W - K + 1)
        n_cols, kshape = B * H * W, (K, K, C_in, C_out)
        sh = dict(B=B, H_in=H, W_in=W, C_in=C_in, H_out=ho, W_out=wo, C_out=C_out, K_h=K, K_w=K)
    sp = spike_times(kind, n_cols * C_in, T, tfs, rng)
    fan = int(np.prod(kshape[:-1]))
    Wt = (rng.standard_normal(int(np.prod(kshape))) * np.sqrt(2.0 / fan)).astype(np.float32)
    # biases large enough that some neurons fire on the bias alone
    bias = (rng.standard_normal(C_out) * 0.6).astype(np.float32)
    alpha, theta = vdttfs.build_luts_host(tc, 2.0 * T, 1.0, 2.0 * T, 1.0)
    t_min = 1
    c = oracle.Consts.from_task(tc)
    cin, tin, off = oracle.bucketize(c, sp, n_cols, C_in)
    pad = K // 2 if (task2 and not is_fc) else 0
    exp, ep, eb = oracle.integrate(c, cin, tin, off, Wt, bias, alpha, theta, t_min, pad=pad, is_fc=is_fc, **sh)
    if kind in ("one-bin", "last-bin"):
        assert (exp < INF).any() and (exp == INF).any(), "the case must fire some neurons and not others"

    ctx = gpu_ctx_factory(tc)
    d_in, d_W, d_b = ctx.to_device(sp), ctx.to_device(Wt), ctx.to_device(bias)
    d_a, d_t = ctx.to_device(alpha), ctx.to_device(theta)
    OS = tc.num_chunks + 1
    d_cin = ctx.empty(n_cols * C_in, np.int32)
    d_tin = ctx.empty(n_cols * C_in, np.float32)
    d_off = ctx.empty(n_cols * OS, np.int32)
    d_out = ctx.empty(exp.size, np.float32)
    ctx.bucketize(d_in, n_cols, C_in, d_cin, d_tin, d_off)
    ctx.integrate(d_out, d_cin, d_tin, d_off, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, **sh)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="drop-in pair")
    gp, gb = ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, count=True, **sh)
    np.testing.assert_array_equal(d_out.download(), exp, err_msg="engine, counting")
    assert (gp, gb) == (ep, eb)
    ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, **sh)
    ctx.synchronize()
    got = d_out.download()
    np.testing.assert_array_equal(got, exp, err_msg="engine")
    if kind in ("silent", "past-window"):
        assert ep == 0 and eb == 0
