"""Seeded random CuLIF networks against the oracle.

Each case draws a valid CuLIF layer table -- a raw-event conv (C_in 1..4:
the event-mask kernel up to 3 input channels, the dense kernel above), up
to two more convs and up to three pools in random order, then FC or
recurrent FC + FC -- with random map sizes, channel counts (1..140), T
(a multiple of the chunk width Delta in {8, 16, 32}), per-layer decay and
threshold, event density and binary or non-binary event values.  The
engine (vdttfs_culif_net_*) must equal the oracle's T3V network at every
layer, and its predictions must be equal too.
"""
import sys
import zlib

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import models

pytestmark = pytest.mark.gpu

N_CASES = 24
INF = 9999.0


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def draw(i):
    rng = np.random.default_rng(zlib.crc32(f"random-culif-{i}".encode()))
    D = int(rng.choice([8, 16, 32]))
    T = D * int(rng.integers(1, 255 // D + 1))
    H, W = int(rng.choice([4, 6, 8, 10, 12, 16])), int(rng.choice([4, 6, 8, 12, 16]))
    C0 = int(rng.integers(1, 5))
    B = int(rng.integers(1, 4))
    seed = int(rng.integers(1 << 30))

    def nd():
        return float(rng.uniform(0.05, 0.95)), float(rng.uniform(0.3, 3.0))

    k = models.kaiming
    L = []
    c1 = int(rng.integers(1, 81))
    L.append(vdttfs.CulifLayerSpec(vdttfs.CULIF_RAW_CONV, C0, H, W, c1, k(seed, 0, (c1, C0, 3, 3), 9 * C0), None, *nd()))
    c, h, w, idx = c1, H, W, 1
    for _ in range(int(rng.integers(0, 3))):
        if h >= 2 and w >= 2 and rng.random() < 0.5:
            L.append(vdttfs.CulifLayerSpec(vdttfs.CULIF_POOL, c, h, w, c, None, None, *nd()))
            h, w = h // 2, w // 2
        co = int(rng.integers(1, 141))
        L.append(vdttfs.CulifLayerSpec(vdttfs.CULIF_CONV, c, h, w, co, k(seed, idx, (co, c, 3, 3), 9 * c), None, *nd()))
        c, idx = co, idx + 1
    if h >= 2 and w >= 2 and rng.random() < 0.5:
        L.append(vdttfs.CulifLayerSpec(vdttfs.CULIF_POOL, c, h, w, c, None, None, *nd()))
        h, w = h // 2, w // 2
    F = c * h * w
    n_cls = int(rng.integers(2, 13))
    if rng.random() < 0.7:
        r = int(rng.integers(1, 201))
        L.append(vdttfs.CulifLayerSpec(vdttfs.CULIF_FC_REC, F, 1, 1, r, k(seed, idx, (r, F), F),
                                       k(seed, idx + 1, (r, r), r), *nd()))
        L.append(vdttfs.CulifLayerSpec(vdttfs.CULIF_FC, r, 1, 1, n_cls, k(seed, idx + 2, (n_cls, r), r), None, *nd()))
    else:
        L.append(vdttfs.CulifLayerSpec(vdttfs.CULIF_FC, F, 1, 1, n_cls, k(seed, idx, (n_cls, F), F), None, *nd()))
    density = float(rng.uniform(0.02, 0.3))
    ev = rng.random((B, C0, H, W, T)) < density
    vals = rng.integers(1, 3, size=ev.shape) if rng.random() < 0.3 else 1
    data = (ev * vals).astype(np.float32)
    return dict(T=T, D=D, B=B, layers=L, data=data)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_culif_net_matches_oracle(gpu_ctx_factory, i):
    c = draw(i)
    desc = [(l.kind, l.C_in, l.H_in, l.W_in, l.C_out) for l in c["layers"]]
    say(f"random CuLIF net {i}: T={c['T']} D={c['D']} B={c['B']} layers={desc}")
    ref, rpred = oracle.culif_net_forward(c["layers"], c["data"], c["B"], c["T"], c["D"])
    ctx = gpu_ctx_factory(vdttfs.task3_consts(T=c["T"], delta=c["D"]))
    net = vdttfs.CulifNet(ctx, c["layers"], c["B"])
    try:
        d = ctx.to_device(c["data"])
        p = ctx.empty(c["B"], np.int32)
        net.forward(d, p)
        ctx.synchronize()
        for li, o in enumerate(ref):
            g = net.layer_output(li)
            assert np.array_equal(g, o.reshape(g.shape)), (
                f"layer {li} {desc[li]} differs at {np.flatnonzero(g.ravel() != o.ravel())[:8]}")
        np.testing.assert_array_equal(p.download(), rpred)
    finally:
        net.close()
