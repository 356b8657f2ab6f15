"""Pool fusion (vdttfs_net_set_pool_fusion): a 2x2 min pool computed inside
the next layer's list build from the pool's input (the per-wave fused kernel
past 64 receptive elements, or the shared-list kernel), on request where the
pooled map is 1x1 or wherever the build can take it.  Every layer's
output -- a fused pool's map written when it is asked for -- equals the
oracle's bit for bit under every plan the kernels accept, and the forward
leaves a fused pool's map unwritten (its bytes stay as the test filled them).
"""
import ctypes
import sys
import zlib

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import models, tune
from vdttfs._lib import lib

pytestmark = pytest.mark.gpu

POOL, CONV, FC, VMEM = vdttfs.LAYER_POOL, vdttfs.LAYER_CONV, vdttfs.LAYER_FC, vdttfs.LAYER_VMEM


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def pool_buffers(net, layers):
    """Device pointer and size of every pool layer's map (asking for them
    now writes any map a previous forward left unwritten)."""
    return {i: net.layer_output_ptr(i) for i, l in enumerate(layers) if l.kind == POOL}


def poison(ctx, bufs):
    for p, n in bufs.values():
        assert lib().vdttfs_memset(ctx.handle, p, 0xFF, n * 4) == 0


def raw(ctx, p, n):
    h = np.empty(n, np.float32)
    assert lib().vdttfs_d2h(ctx.handle, h.ctypes.data_as(ctypes.c_void_p), p, h.nbytes) == 0
    return h


def forward_check(ctx, net, layers, d_img, d_pred, ref, tag):
    """One fused forward on poisoned pool maps; returns the set of pools the
    forward left unwritten, after checking every layer against the oracle."""
    bufs = pool_buffers(net, layers)
    poison(ctx, bufs)
    net.forward(d_img, d_pred)
    ctx.synchronize()
    fused = set()
    for i, (p, n) in bufs.items():
        h = raw(ctx, p, n)
        if np.all(np.isnan(h)):
            fused.add(i)
        else:  # run as its own pass: written in full
            assert not np.any(np.isnan(h)), f"{tag}: pool {i} partly written"
    for i, (l, o) in enumerate(zip(layers, ref["outs"])):
        g = net.layer_output(i)
        if l.kind == VMEM:
            assert np.all(np.abs(g - o) <= 1e-5 * (np.abs(o) + 1e-3)), f"{tag} layer {i}"
        else:
            assert np.array_equal(g, o), f"{tag} layer {i} plan {net.get_plan(i)} differs at {np.flatnonzero(g != o)[:8]}"
    if d_pred is not None:
        np.testing.assert_array_equal(d_pred.download(), ref["pred"], err_msg=tag)
    return fused


def vgg_ref(w, B, img):
    return oracle.net_forward(oracle.Consts.from_task(w.consts), w.layers, B, img, w.img_elems,
                              oracle.ENC_LINEAR, w.tc_in, w.td_in, oracle.READ_ARGMAX,
                              same_pad=bool(w.consts.conv_same_pad), keep_layers=True)


def test_pool_fusion_vgg_every_plan(gpu_ctx_factory):
    """VGG-16 at B=16: the five pools fuse into conv 2 (per-wave, 9 chunks),
    conv 4, 7, 10 and the FC (shared lists) under the built-in plans; round
    r then sets each weighted layer to its (r mod n)-th accepted plan, fused
    pools and separate ones mixed, and every round equals the oracle."""
    say("pool fusion: VGG-16 B=16 built-in plans, then every accepted plan")
    w = models.vgg16()
    B = 16
    img = models.images_for(w, B)
    ref = vgg_ref(w, B, img)
    ctx = gpu_ctx_factory(w.consts)
    net = vdttfs.Net(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)
    try:
        d_img = ctx.to_device(img)
        d_pred = ctx.empty(B, np.int32)
        pools = [i for i, l in enumerate(w.layers) if l.kind == POOL]
        # by default every pool runs as its own pass
        assert forward_check(ctx, net, w.layers, d_img, d_pred, ref, "off") == set()
        net.set_pool_fusion(vdttfs.POOL_FUSE_AUTO)  # the last pool (1x1 map) into the FC layer
        assert forward_check(ctx, net, w.layers, d_img, d_pred, ref, "auto") == {17}
        net.set_pool_fusion(vdttfs.POOL_FUSE_ALL)
        assert forward_check(ctx, net, w.layers, d_img, d_pred, ref, "built-in") == set(pools)
        with pytest.raises(vdttfs.VdttfsError):
            net.set_pool_fusion(3)
        cands = {i: tune.candidates(net, i) for i, l in enumerate(w.layers) if l.kind in (CONV, FC)}
        seen = set()
        for r in range(max(len(c) for c in cands.values())):
            for i, c in cands.items():
                net.set_plan(i, *c[r % len(c)])
            seen |= forward_check(ctx, net, w.layers, d_img, d_pred, ref, f"round {r}")
        assert seen == set(pools)
        # a counting forward runs every pool; its counts equal the oracle's
        for i in cands:
            net.set_plan(i)
        eproc, ebin, _, _ = net.count(d_img)
        np.testing.assert_array_equal(eproc, ref["eproc"])
        np.testing.assert_array_equal(ebin, ref["ebin"])
        d_img.free()
        d_pred.free()
    finally:
        net.close()


def mixed_layers(rng, T):
    """Pools over odd maps (the last row and column dropped), C_in that are
    not multiples of 64, per-layer (tc_fire, td), and a pool into an FC layer
    through its one 1x1 window."""
    def conv(H, cin, cout, tc, td):
        k = (rng.standard_normal((3, 3, cin, cout)) * np.sqrt(2.0 / (9 * cin))).astype(np.float32)
        b = (rng.standard_normal(cout) * 0.05).astype(np.float32)
        return vdttfs.Layer(CONV, H, H, cin, H, H, cout, 3, 3, k, b, tc, td)

    def fc(cin, cout, tc, td):
        k = (rng.standard_normal((cin, cout)) * np.sqrt(2.0 / cin)).astype(np.float32)
        b = (rng.standard_normal(cout) * 0.05).astype(np.float32)
        return vdttfs.Layer(FC, 1, 1, cin, 1, 1, cout, 1, 1, k, b, tc, td)

    def pool(H, c):
        return vdttfs.Layer(POOL, H, H, c, H // 2, H // 2, c)

    return [conv(11, 3, 24, T / 4, 0.0),       # 0
            pool(11, 24),                      # 1 -> 5x5, into a per-wave build of 9 chunks (216 elements)
            conv(5, 24, 96, T / 3, 1.5),       # 2
            pool(5, 96),                       # 3 -> 2x2, into a per-wave build of 18 chunks (864 elements)
            conv(2, 96, 64, T / 5, 0.5),       # 4
            conv(2, 64, 150, T / 4, 1.0),      # 5: a shared build (C_out 150)
            pool(2, 150),                      # 6 -> 1x1, into the FC layer's shared build
            fc(150, 96, T / 4, 2.0),           # 7
            fc(96, 70, T / 2, 0.0),            # 8
            ]


@pytest.mark.parametrize("task2", [True, False], ids=["alpha-by-time", "alpha-by-bin"])
def test_pool_fusion_mixed_net(gpu_ctx_factory, task2):
    """A net with odd pooled maps and distinct per-layer constants equals the
    oracle layer by layer with fusion on and off, under the built-in plans and
    every accepted plan, and under per-layer windows."""
    T = 64
    say(f"pool fusion: mixed net task2={task2}")
    rng = np.random.default_rng(zlib.crc32(f"poolfuse-mixed-{task2}".encode()))
    layers = mixed_layers(rng, T)
    tc = vdttfs.TaskConsts(T=T, tfs=16.0 if task2 else 0.0, delta=8, vth=1.0, alpha_by_time=task2,
                           conv_same_pad=True)
    B = 5
    img_elems = 11 * 11 * 3
    t = np.floor(rng.random(B * img_elems) * (T + tc.tfs)).astype(np.float32)
    t = np.where(rng.random(t.size) < 0.25, np.float32(9999.0), t).astype(np.float32)
    oc = oracle.Consts.from_task(tc)

    ref = oracle.net_forward(oc, layers, B, t, img_elems, oracle.ENC_TIMES, T / 4.0, 0.0,
                             oracle.READ_ARGMIN, same_pad=True, keep_layers=True)
    for i in (0, 2, 4, 5, 7):
        frac = float(np.mean(ref["outs"][i] < 9999.0))
        assert 0.02 < frac < 0.98, f"layer {i} fires {frac}"
    ctx = gpu_ctx_factory(tc)
    net = vdttfs.Net(ctx, layers, B, img_elems, vdttfs.ENCODE_TIMES, T / 4.0, 0.0, vdttfs.READOUT_ARGMIN)
    try:
        x = ctx.to_device(t)
        assert forward_check(ctx, net, layers, x, None, ref, "off") == set()
        net.set_pool_fusion(vdttfs.POOL_FUSE_AUTO)
        assert forward_check(ctx, net, layers, x, None, ref, "auto") == {6}
        net.set_pool_fusion(vdttfs.POOL_FUSE_ALL)
        assert net.get_plan(2)[0] == net.get_plan(4)[0] == vdttfs.PATH_FUSED
        assert forward_check(ctx, net, layers, x, None, ref, "built-in") == {1, 3, 6}
        cands = {i: tune.candidates(net, i) for i, l in enumerate(layers) if l.kind in (CONV, FC)}
        for r in range(max(len(c) for c in cands.values())):
            for i, c in cands.items():
                net.set_plan(i, *c[r % len(c)])
            forward_check(ctx, net, layers, x, None, ref, f"round {r}")
        for i in cands:
            net.set_plan(i)
        # per-layer windows (the separate-pool engine path under windows is
        # pinned against the oracle by the calibrator's tests): fused equals it
        net.set_windows([40, 0, 48, 0, 0, 56, 0, 33, 64])
        net.set_pool_fusion(vdttfs.POOL_FUSE_OFF)
        net.forward(x)
        ctx.synchronize()
        base = {"outs": [net.layer_output(i) for i in range(len(layers))]}
        net.set_pool_fusion(vdttfs.POOL_FUSE_ALL)
        assert forward_check(ctx, net, layers, x, None, base, "windows") == {1, 3, 6}
        x.free()
    finally:
        net.close()
