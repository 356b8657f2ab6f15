"""HIP-graph forwards (vdttfs_net_set_graphs): every replay of a captured
forward equals the eager forward layer by layer, with eager work and
synchronisations between the replays, for two input/prediction pairs at
once; a plan or window change recaptures; more pairs than the network keeps
evict the oldest and stay correct; pool fusion's lazily written pool maps stay
right across replays, counting forwards and eager forwards in between.  The
eager forwards these are compared with are pinned against the oracle by the
network and plan tests; the last layer and the predictions are checked
against the oracle here too."""
import sys

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import models

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def outputs(net, n):
    return [net.layer_output(i) for i in range(n)]


def check(net, ref, pred, d_pred, tag):
    for i, o in enumerate(ref):
        g = net.layer_output(i)
        assert np.array_equal(g, o), f"{tag}: layer {i} differs at {np.flatnonzero(g != o)[:8]}"
    np.testing.assert_array_equal(d_pred.download(), pred, err_msg=tag)


@pytest.mark.parametrize("name,B", [("lenet5", 64), ("vgg16", 16)])
def test_graph_replays_match_eager(gpu_ctx_factory, name, B):
    say(f"graphs: {name} B={B}")
    w = models.lenet5() if name == "lenet5" else models.vgg16()
    n = len(w.layers)
    both = np.ascontiguousarray(models.images_for(w, 2 * B), np.float32).reshape(-1)
    imgs = [both[:B * w.img_elems].copy(), both[B * w.img_elems:].copy()]
    ctx = gpu_ctx_factory(w.consts)
    net = vdttfs.Net(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)
    try:
        xs = [ctx.to_device(im) for im in imgs]
        ps = [ctx.empty(B, np.int32) for _ in imgs]
        refs, preds = [], []
        for x, p in zip(xs, ps):  # eager references
            net.forward(x, p)
            ctx.synchronize()
            refs.append(outputs(net, n))
            preds.append(p.download())
        rd = oracle.READ_ARGMAX if w.readout == vdttfs.READOUT_ARGMAX else oracle.READ_ARGMIN
        for im, ref, pred in zip(imgs, refs, preds):
            o = oracle.net_forward(oracle.Consts.from_task(w.consts), w.layers, B, im, w.img_elems,
                                   oracle.ENC_LINEAR, w.tc_in, w.td_in, rd,
                                   same_pad=bool(w.consts.conv_same_pad))
            np.testing.assert_array_equal(pred, o["pred"])
            if w.layers[-1].kind == vdttfs.LAYER_VMEM:
                assert np.all(np.abs(ref[-1] - o["final"]) <= 1e-5 * (np.abs(o["final"]) + 1e-3))
            else:
                np.testing.assert_array_equal(ref[-1], o["final"])
        net.set_graphs(True)
        for r in range(3):
            for k in (0, 1):
                for p in ps:
                    p.fill(0xFF)
                net.forward(xs[k], ps[k])  # captured on the first round, replayed after
                ctx.synchronize()
                check(net, refs[k], preds[k], ps[k], f"replay {r} input {k}")
            # eager work between replays: a forward without graphs on the other input
            net.set_graphs(False)
            net.forward(xs[1], ps[1])
            ctx.synchronize()
            check(net, refs[1], preds[1], ps[1], f"eager after replay {r}")
            net.set_graphs(True)
        # a plan change recaptures (plans give bit-identical outputs)
        last = max(i for i, l in enumerate(w.layers) if l.kind in (vdttfs.LAYER_CONV, vdttfs.LAYER_FC))
        net.set_plan(last, vdttfs.PATH_BINS)
        for r in range(2):
            net.forward(xs[0], ps[0])
            ctx.synchronize()
            check(net, refs[0], preds[0], ps[0], f"after set_plan, replay {r}")
        net.set_plan(last)
        # windows recapture too: equal to the eager forward under the same windows
        wins = [0 if l.kind == vdttfs.LAYER_POOL else 48 for l in w.layers]
        net.set_windows(wins)
        net.set_graphs(False)
        net.forward(xs[0], ps[0])
        ctx.synchronize()
        wref, wpred = outputs(net, n), ps[0].download()
        net.set_graphs(True)
        for r in range(2):
            net.forward(xs[0], ps[0])
            ctx.synchronize()
            check(net, wref, wpred, ps[0], f"windows, replay {r}")
        net.set_windows(None)
        # more (input, prediction) pairs than the network keeps graphs for
        extra = [ctx.empty(B, np.int32) for _ in range(5)]
        for r in range(2):
            for p in extra:
                net.forward(xs[0], p)
                ctx.synchronize()
                check(net, refs[0], preds[0], p, f"pair eviction, round {r}")
        for p in extra:
            p.free()
        # pool fusion: the pools' maps are written on request, also after replays
        net.set_pool_fusion(vdttfs.POOL_FUSE_ALL)
        for r in range(3):
            for k in (0, 1):
                net.forward(xs[k], ps[k])
                ctx.synchronize()
                check(net, refs[k], preds[k], ps[k], f"pool fusion replay {r} input {k}")
            net.count(xs[1])  # a counting forward runs every pool, eagerly
            ctx.synchronize()
        for x in xs:
            x.free()
        for p in ps:
            p.free()
    finally:
        net.close()
