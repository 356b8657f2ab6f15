"""k_stream_multi (plan FUSED, gather 4, four pixels per wave: one output
position of four images per wave, weight rows shared by the images) against
the oracle, bit for bit.

The kernel streams bin-0 events straight from the dense map as union entries
with per-image masks, and the later bins from a per-wave sorted list that
streams in windows past its capacity (2,048 entries).  The cases cross:
  * batches that are not a multiple of four (a partial image group),
  * C_out that is not a multiple of 256 (a partial c_out block) and several
    c_out blocks, C_in that is not a multiple of 64 (per-lane taps),
  * same and valid padding, 3x3 down to 2x2 maps, 1x1 convs and FC layers,
  * alpha by spike time (bin 0 holds many alphas) and by arrival bin, a
    fire start, t_min > 0, shuffled threshold tables, non-integer times,
  * degenerate inputs: silent, every event in bin 0 (the union ring only),
    every event in the last bin (the later list in many windows), every
    event past the window, dense random times.
"""
import sys
import zlib

import numpy as np
import pytest

import oracle
import vdttfs

pytestmark = pytest.mark.gpu
INF = np.float32(9999.0)
FUSED = vdttfs.PATH_FUSED
MULTI = (FUSED, 4, 4)

# name, task2, is_fc, B, H, W, C_in, C_out, K
SHAPES = [
    ("conv8x8-256-256-b7", True, False, 7, 8, 8, 256, 256, 3),
    ("conv4x4-512-512-b8", True, False, 8, 4, 4, 512, 512, 3),
    ("conv2x2-512-384-b5", True, False, 5, 2, 2, 512, 384, 3),
    ("conv6x6-96-132-valid-b6", False, False, 6, 6, 6, 96, 132, 3),
    ("conv5x5-72-260-b3", True, False, 3, 5, 5, 72, 260, 3),
    ("conv1x1-200-144-b9", False, False, 9, 5, 4, 200, 144, 1),
    ("fc-600-260-b9", True, True, 9, 1, 1, 600, 260, 1),
    ("fc-4096-256-b4", False, True, 4, 1, 1, 4096, 256, 1),
]
KINDS = ["random", "silent", "one-bin", "last-bin", "past-window", "dense", "fractional"]


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def spike_times(kind, n, T, tfs, rng):
    if kind == "random":
        t = np.floor(rng.random(n) * (T + tfs + 2)).astype(np.float32)
        return np.where(rng.random(n) < 0.5, t, INF).astype(np.float32)
    if kind == "dense":
        return np.floor(rng.random(n) * (T + tfs)).astype(np.float32)
    if kind == "fractional":  # times between steps: alpha by time varies inside every bin
        t = (rng.random(n) * (T + tfs + 1)).astype(np.float32)
        return np.where(rng.random(n) < 0.6, t, INF).astype(np.float32)
    v = {"silent": INF, "one-bin": 0.0, "last-bin": float(T - 1) + tfs, "past-window": float(T) + tfs + 1.0}[kind]
    return np.full(n, v, np.float32)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_multi_matches_oracle(gpu_ctx_factory, shape, kind):
    name, task2, is_fc, B, H, W, C_in, C_out, K = shape
    say(f"multi {name} {kind}")
    rng = np.random.default_rng(zlib.crc32(f"multi-{name}-{kind}".encode()))
    T = 64
    tfs = 32.0 if task2 else 0.0
    tc = vdttfs.TaskConsts(T=T, tfs=tfs, delta=8, vth=1.0, alpha_by_time=task2, conv_same_pad=task2)
    if is_fc:
        layer_in = B * C_in
        kshape = (C_in, C_out)
        ho = wo = 1
    else:
        layer_in = B * H * W * C_in
        kshape = (K, K, C_in, C_out)
        ho, wo = (H, W) if task2 else (H - K + 1, W - K + 1)
    fan = int(np.prod(kshape[:-1]))
    Wt = (rng.standard_normal(int(np.prod(kshape))) * np.sqrt(2.0 / fan)).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.6).astype(np.float32)
    tcf, td = 1.5 * T, 2.5  # t_min = 3
    if is_fc:
        layer = vdttfs.Layer(vdttfs.LAYER_FC, 1, 1, C_in, 1, 1, C_out, 1, 1, Wt.reshape(kshape), bias, tcf, td)
    else:
        layer = vdttfs.Layer(vdttfs.LAYER_CONV, H, W, C_in, ho, wo, C_out, K, K, Wt.reshape(kshape), bias, tcf, td)
    sp = spike_times(kind, layer_in, T, tfs, rng)
    elems = layer_in // B
    ref = oracle.net_forward(oracle.Consts.from_task(tc), [layer], B, sp, elems, oracle.ENC_TIMES, 0.75 * T, 0.5,
                             oracle.READ_ARGMIN, same_pad=task2)["final"]
    if kind in ("one-bin", "last-bin", "random"):
        assert (ref < INF).any() and (ref == INF).any(), "the case must fire some neurons and not others"
    ctx = gpu_ctx_factory(tc)
    net = vdttfs.Net(ctx, [layer], B, elems, vdttfs.ENCODE_TIMES, 0.75 * T, 0.5, vdttfs.READOUT_ARGMIN)
    try:
        net.set_plan(0, *MULTI)
        assert net.get_plan(0) == MULTI
        x = ctx.to_device(sp)
        net.forward(x)
        ctx.synchronize()
        np.testing.assert_array_equal(net.layer_output(0), ref, err_msg=f"{name} {kind}")
        net.set_plan(0)  # the built-in plan gives the same maps
        net.forward(x)
        ctx.synchronize()
        np.testing.assert_array_equal(net.layer_output(0), ref, err_msg=f"{name} {kind}, built-in plan")
    finally:
        net.close()

