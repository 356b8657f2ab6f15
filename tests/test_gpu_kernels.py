"""GPU parity of every kernel against the CPU oracle, through the C ABI.

Bar: bucket offsets and event order bit-exact; first-spike times bit-exact;
integrated-synapse counts exact; vmem within 1e-5 relative (fp32 dot
product in the reference's order, so in practice exact)."""
import sys
import zlib

import numpy as np
import pytest

import oracle
import vdttfs

pytestmark = pytest.mark.gpu
INF = np.float32(9999.0)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def spikes(rng, n, T, p=0.55, edge=True):
    t = rng.integers(0, T + 6, n).astype(np.float32)
    s = np.where(rng.random(n) < p, t, INF).astype(np.float32)
    if edge and n > 6:
        s[0] = np.float32(np.nan)
        s[1] = np.float32(-2.0)
        s[2] = np.float32(T)
        s[3] = np.float32(T - 1)
        s[4] = np.float32(3.5)
    return s


def consts(T, tfs, delta, task2):
    return vdttfs.TaskConsts(T=T, tfs=tfs, delta=delta, vth=1.0, alpha_by_time=task2,
                             conv_same_pad=task2)


def valid_rows(cin, tin, off, n_cols, c_in, OS):
    """Each column's valid prefix (the reference leaves the tail unwritten)."""
    out_c, out_t = [], []
    for col in range(n_cols):
        n = off[col * OS + OS - 1]
        out_c.append(cin[col * c_in: col * c_in + n])
        out_t.append(tin[col * c_in: col * c_in + n])
    return np.concatenate(out_c), np.concatenate(out_t)


BKT_CASES = [
    # T, tfs, delta, c_in, n_cols
    (64, 0.0, 16, 1, 5000),
    (64, 32.0, 8, 3, 4097),
    (64, 32.0, 8, 64, 3000),
    (80, 40.0, 8, 100, 513),
    (64, 0.0, 16, 512, 300),
    (16, 0.0, 5, 4096, 40),
    (255, 0.0, 1, 6, 777),
    (64, 0.0, 1, 130, 200),
    # few long columns (a workgroup per column): ragged chunks, waves with no chunk, 255 bins
    (64, 32.0, 8, 700, 50),
    (255, 0.0, 1, 1000, 30),
]


@pytest.mark.parametrize("T,tfs,delta,c_in,n_cols", BKT_CASES)
def test_bucketize_bitexact(gpu_ctx_factory, T, tfs, delta, c_in, n_cols):
    say(f"bucketize T={T} tfs={tfs} delta={delta} c_in={c_in} n_cols={n_cols}")
    rng = np.random.default_rng(c_in * 7 + n_cols)
    sp = spikes(rng, n_cols * c_in, T)
    tc = consts(T, tfs, delta, False)
    ctx = gpu_ctx_factory(tc)
    OS = tc.num_chunks + 1
    d_in = ctx.to_device(sp)
    d_cin = ctx.empty(n_cols * c_in, np.int32)
    d_tin = ctx.empty(n_cols * c_in, np.float32)
    d_off = ctx.empty(n_cols * OS, np.int32)
    ctx.bucketize(d_in, n_cols, c_in, d_cin, d_tin, d_off)
    ctx.synchronize()
    g_off = d_off.download()
    ocin, otin, ooff = oracle.bucketize(oracle.Consts.from_task(tc), sp, n_cols, c_in)
    np.testing.assert_array_equal(g_off, ooff)
    gc, gt = valid_rows(d_cin.download(), d_tin.download(), g_off, n_cols, c_in, OS)
    oc, ot = valid_rows(ocin, otin, ooff, n_cols, c_in, OS)
    np.testing.assert_array_equal(gc, oc)
    np.testing.assert_array_equal(gt.view(np.int32), ot.view(np.int32))


LAYER_CASES = [
    # name, T, tfs, delta, task2, is_fc, B, H, W, C_in, C_out, K
    ("t1-conv5x5-c6", 64, 0.0, 16, False, False, 3, 12, 12, 6, 16, 5),
    ("t1-conv5x5-c1", 64, 0.0, 16, False, False, 4, 28, 28, 1, 6, 5),
    ("t2-conv3x3-c64", 64, 32.0, 8, True, False, 2, 16, 16, 64, 64, 3),
    ("t2-conv3x3-c128-o192", 64, 32.0, 8, True, False, 2, 8, 8, 128, 192, 3),
    ("t2-conv3x3-2x2", 64, 32.0, 8, True, False, 3, 2, 2, 512, 128, 3),
    ("t1-fc-256-120", 64, 0.0, 16, False, True, 37, 1, 1, 256, 120, 1),
    ("t2-fc-512-512", 64, 32.0, 8, True, True, 20, 1, 1, 512, 512, 1),
    ("t1-fc-4096-96-delta32", 32, 0.0, 32, False, True, 9, 1, 1, 4096, 96, 1),
    ("t2-conv-T80", 80, 40.0, 8, True, False, 2, 6, 6, 32, 64, 3),
    # stream gather modes: 1 event per dword load (C_out <= 64), 2 per
    # dwordx4 load (64 < C_out <= 128, partly idle lanes), and the 1-event
    # fallback (C_out % 4 != 0)
    ("t2-conv-c36", 64, 32.0, 8, True, False, 2, 7, 5, 40, 36, 3),
    ("t2-conv-c100-epi2", 64, 32.0, 8, True, False, 2, 5, 6, 48, 100, 3),
    ("t2-conv-c66-vec1", 64, 32.0, 8, True, False, 2, 5, 5, 20, 66, 3),
    ("t1-fc-300-84-epi2", 64, 0.0, 16, False, True, 33, 1, 1, 300, 84, 1),
    # C_in <= 64, <= 9 taps, C_out <= 64, T <= 64: merged list built in LDS by
    # the integrating kernel (Task 1 alpha-by-bin, valid conv; Task 2 same conv)
    ("t1-conv3x3-lds-list", 64, 0.0, 16, False, False, 3, 11, 9, 48, 40, 3),
    ("t2-conv3x3-lds-list-c3", 64, 32.0, 8, True, False, 4, 12, 10, 3, 64, 3),
    # 64 < C_in <= 128: the list still built in LDS from the dense map (18
    # chunks of 64) without counters; the counting forward takes bucketize +
    # merge + stream
    ("t2-conv3x3-wide-c96-o128", 64, 32.0, 8, True, False, 2, 7, 6, 96, 128, 3),
    ("t1-conv3x3-wide-c128-o64", 64, 0.0, 16, False, False, 2, 6, 7, 128, 64, 3),
    ("t2-conv3x3-wide-c72-o100", 64, 32.0, 8, True, False, 3, 5, 5, 72, 100, 3),
    # K_h * K_w * C_in <= 32, C_out <= 64, T <= 64: receptive field in
    # registers, 64 / C_out pixels per wave (the two cases above take it too)
    ("t1-conv2x2-reg-c8-o40", 64, 0.0, 16, False, False, 3, 9, 9, 8, 40, 2),
    ("t2-conv3x3-reg-c2-o20", 64, 32.0, 8, True, False, 3, 10, 10, 2, 20, 3),
    ("t2-conv1x1-reg-c32-o32", 64, 32.0, 8, True, False, 2, 6, 6, 32, 32, 1),
    ("t1-conv3x3-reg-T48", 48, 0.0, 16, False, False, 3, 10, 10, 3, 16, 3),
    ("t2-conv3x3-reg-T16", 16, 8.0, 4, True, False, 2, 8, 8, 3, 64, 3),
]


def layer_inputs(rng, tc, is_fc, B, H, W, C_in, C_out, K, dense_early=False):
    if is_fc:
        n_cols, kshape = B, (C_in, C_out)
        H_in = W_in = H_out = W_out = 1
        K_h = K_w = 1
    else:
        n_cols, kshape = B * H * W, (K, K, C_in, C_out)
        H_in, W_in = H, W
        H_out, W_out = (H, W) if tc.conv_same_pad else (H - K + 1, W - K + 1)
        K_h = K_w = K
    sp = spikes(rng, n_cols * C_in, tc.T, edge=False)
    if dense_early:
        sp = np.where(rng.random(sp.size) < 0.9, np.float32(0.0), sp).astype(np.float32)
    fan = int(np.prod(kshape[:-1]))
    Wt = (rng.standard_normal(int(np.prod(kshape))) * np.sqrt(2.0 / fan)).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.05).astype(np.float32)
    shape = dict(B=B, H_in=H_in, W_in=W_in, C_in=C_in, H_out=H_out, W_out=W_out, C_out=C_out,
                 K_h=K_h, K_w=K_w)
    return sp, Wt, bias, n_cols, shape


def oracle_layer(tc, sp, Wt, bias, alpha, theta, n_cols, shape, t_min, is_fc):
    c = oracle.Consts.from_task(tc)
    cin, tin, off = oracle.bucketize(c, sp, n_cols, shape["C_in"])
    pad = shape["K_h"] // 2 if (tc.conv_same_pad and not is_fc) else 0
    return oracle.integrate(c, cin, tin, off, Wt, bias, alpha, theta, t_min, pad=pad,
                            is_fc=is_fc, **shape)


@pytest.mark.parametrize("case", LAYER_CASES, ids=[c[0] for c in LAYER_CASES])
def test_integrate_paths_bitexact(gpu_ctx_factory, case):
    name, T, tfs, delta, task2, is_fc, B, H, W, C_in, C_out, K = case
    say(f"integrate {name}")
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    tc = consts(T, tfs, delta, task2)
    ctx = gpu_ctx_factory(tc)
    sp, Wt, bias, n_cols, shape = layer_inputs(rng, tc, is_fc, B, H, W, C_in, C_out, K)
    alpha, theta = vdttfs.build_luts_host(tc, T / 4.0, 0.0, T / 4.0, 0.0)
    t_min = 1
    exp, ep, eb = oracle_layer(tc, sp, Wt, bias, alpha, theta, n_cols, shape, t_min, is_fc)
    assert 0.02 < float(np.mean(exp < INF)) < 0.98, "degenerate case"
    n_out = exp.size
    d_in, d_W, d_b = ctx.to_device(sp), ctx.to_device(Wt), ctx.to_device(bias)
    d_a, d_t = ctx.to_device(alpha), ctx.to_device(theta)
    # (1) the drop-in pair: reference-layout bucketize + integrate
    OS = tc.num_chunks + 1
    d_cin = ctx.empty(n_cols * C_in, np.int32)
    d_tin = ctx.empty(n_cols * C_in, np.float32)
    d_off = ctx.empty(n_cols * OS, np.int32)
    d_out = ctx.empty(n_out, np.float32)
    ctx.bucketize(d_in, n_cols, C_in, d_cin, d_tin, d_off)
    ctx.integrate(d_out, d_cin, d_tin, d_off, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, **shape)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out.download(), exp)
    # (2) the engine path, with exact synapse counts
    d_out2 = ctx.empty(n_out, np.float32)
    gp, gb = ctx.layer_forward(d_out2, d_in, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, count=True,
                               **shape)
    np.testing.assert_array_equal(d_out2.download(), exp)
    assert (gp, gb) == (ep, eb)
    # (3) engine path without counters (the hot-path kernel variant)
    d_out3 = ctx.empty(n_out, np.float32)
    ctx.layer_forward(d_out3, d_in, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, **shape)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out3.download(), exp)


@pytest.mark.parametrize("shape", ["conv", "fc", "conv-small"])
def test_integrate_theta_not_monotone(gpu_ctx_factory, shape):
    """Threshold tables the engine may not skip empty bins on: a shuffled
    theta (rises and falls), entries below 1e-5 and t_min > 0, next to the
    monotone decaying table the skip relies on, a decaying table whose tail
    falls below 1e-5 (spikes possible in bins t_min .. 49 only), a flat one
    and a decaying one with a hole below 1e-5 (allowed bins not one range)."""
    say(f"integrate non-monotone theta ({shape})")
    rng = np.random.default_rng(77)
    tc = consts(64, 0.0, 8, True)
    ctx = gpu_ctx_factory(tc)
    is_fc = shape == "fc"
    c_in = 40 if is_fc else (3 if shape == "conv-small" else 12)  # conv-small: 27 elements, in registers
    sp, Wt, bias, n_cols, shp = layer_inputs(rng, tc, is_fc, 6 if is_fc else 2, 6, 6, c_in, 64, 3)
    sp = np.where(rng.random(sp.size) < 0.7, np.float32(9999.0), sp).astype(np.float32)  # sparse: empty bins
    alpha, theta_mono = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    theta_mix = rng.permutation(theta_mono).astype(np.float32)
    theta_mix[5:9] = np.float32(1e-6)
    d_in, d_W, d_b, d_a = ctx.to_device(sp), ctx.to_device(Wt), ctx.to_device(bias), ctx.to_device(alpha)
    theta_tail = theta_mono.copy()
    theta_tail[50:] = np.float32(1e-6)
    theta_flat = np.full_like(theta_mono, theta_mono[20])
    theta_hole = theta_mono.copy()
    theta_hole[9:12] = np.float32(1e-6)
    for theta, t_min in ((theta_mix, 3), (theta_mono, 0), (theta_mono * np.float32(0.3), 7), (theta_tail, 2),
                         (theta_flat, 0), (theta_hole, 1)):
        exp, ep, eb = oracle_layer(tc, sp, Wt, bias, alpha, theta, n_cols, shp, t_min, is_fc)
        d_t = ctx.to_device(theta)
        d_out = ctx.empty(exp.size, np.float32)
        ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, **shp)
        ctx.synchronize()
        assert np.any(exp < INF) and np.any(exp == INF)
        np.testing.assert_array_equal(d_out.download(), exp)
        gp, gb = ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, t_min, is_fc=is_fc, count=True, **shp)
        assert (gp, gb) == (ep, eb)


def test_integrate_oversized_bins(gpu_ctx_factory):
    """Bins holding more events than the wave's merged list (windowed path)."""
    say("integrate oversized bins")
    rng = np.random.default_rng(99)
    tc = consts(64, 32.0, 8, True)
    ctx = gpu_ctx_factory(tc)
    for is_fc, B, H, W, C_in, C_out, K in [(True, 6, 1, 1, 4096, 64, 1), (False, 1, 4, 4, 512, 64, 3)]:
        sp, Wt, bias, n_cols, shape = layer_inputs(rng, tc, is_fc, B, H, W, C_in, C_out, K,
                                                   dense_early=True)
        Wt *= 0.05  # keep neurons from firing at the first bin
        alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
        exp, ep, eb = oracle_layer(tc, sp, Wt, bias, alpha, theta, n_cols, shape, 0, is_fc)
        d_out = ctx.empty(exp.size, np.float32)
        gp, gb = ctx.layer_forward(d_out, ctx.to_device(sp), ctx.to_device(Wt), ctx.to_device(bias),
                                   ctx.to_device(alpha), ctx.to_device(theta), 0, is_fc=is_fc,
                                   count=True, **shape)
        np.testing.assert_array_equal(d_out.download(), exp)
        assert (gp, gb) == (ep, eb)


def test_launch_layer_sync_matches_oracle(gpu_ctx_factory):
    say("launch_layer_sync")
    rng = np.random.default_rng(5)
    tc = consts(64, 0.0, 16, False)
    ctx = gpu_ctx_factory(tc)
    sp, Wt, bias, n_cols, shape = layer_inputs(rng, tc, False, 2, 12, 12, 6, 16, 5)
    alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    d_a, d_t = ctx.empty(tc.T + 1), ctx.empty(tc.T)
    ctx.update_LUTs(d_a, d_t, 16.0, 0.0, 16.0, 0.0)
    np.testing.assert_array_equal(d_a.download(), alpha)
    np.testing.assert_array_equal(d_t.download(), theta)
    exp, _, _ = oracle_layer(tc, sp, Wt, bias, alpha, theta, n_cols, shape, 0, False)
    d_out = ctx.empty(exp.size)
    ctx.launch_layer(ctx.to_device(sp), d_out, 12, 12, 6, 8, 8, 16, 5, 5, -0.5, ctx.to_device(Wt),
                     ctx.to_device(bias), d_a, d_t, 2, False)
    np.testing.assert_array_equal(d_out.download(), exp)


@pytest.mark.parametrize("B,C_in,C_out", [(3, 100, 70), (256, 512, 10), (5, 2000, 9), (2, 9000, 3), (4, 64, 1)])
def test_fc_vmem_shapes(gpu_ctx_factory, B, C_in, C_out):
    """The wave-per-image kernel (C_in <= 2048, C_out in lane blocks of 64,
    ragged tails, weights staged in LDS up to 6144 per block and read from
    global memory beyond: 2000 x 9) and the thread-per-output kernel (wider
    inputs) run the reference's fma chain in cin order: equal to the oracle
    bit for bit."""
    say(f"fc_vmem B={B} C_in={C_in} C_out={C_out}")
    rng = np.random.default_rng(C_in + C_out)
    tc = consts(64, 32.0, 8, True)
    ctx = gpu_ctx_factory(tc)
    xs = np.where(rng.random(B * C_in) < 0.6, rng.integers(0, 100, B * C_in), 9999).astype(np.float32)
    xs[:3] = [-0.5, 96.0, 97.0]  # clamped to alpha[0]; t - TFS = T is kept; T + 1 is dropped
    Wt = rng.standard_normal(C_in * C_out).astype(np.float32)
    bias = rng.standard_normal(C_out).astype(np.float32)
    alpha, _ = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    d_v = ctx.empty(B * C_out)
    ctx.fc_vmem(ctx.to_device(xs), d_v, ctx.to_device(Wt), ctx.to_device(bias), ctx.to_device(alpha),
                B, C_in, C_out)
    exp = oracle.fc_vmem(oracle.Consts.from_task(tc), xs, Wt, bias, alpha, B, C_in, C_out)
    np.testing.assert_array_equal(d_v.download(), exp)


def test_pool_vmem_readout_encode(gpu_ctx_factory):
    say("pool / vmem / readout / encoders")
    rng = np.random.default_rng(8)
    tc = consts(64, 32.0, 8, True)
    ctx = gpu_ctx_factory(tc)
    B, H, W, Cc = 5, 9, 8, 7
    x = np.where(rng.random(B * H * W * Cc) < 0.5, rng.integers(0, 64, B * H * W * Cc), 9999).astype(np.float32)
    d_o = ctx.empty(B * (H // 2) * (W // 2) * Cc)
    ctx.pool_min(ctx.to_device(x), d_o, B, H, W, Cc)
    np.testing.assert_array_equal(d_o.download(), oracle.pool_min(x, B, H, W, Cc))
    C_in, C_out = 512, 10
    xs = np.where(rng.random(B * C_in) < 0.6, rng.integers(0, 100, B * C_in), 9999).astype(np.float32)
    Wt = rng.standard_normal(C_in * C_out).astype(np.float32)
    bias = rng.standard_normal(C_out).astype(np.float32)
    alpha, _ = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    d_v = ctx.empty(B * C_out)
    ctx.fc_vmem(ctx.to_device(xs), d_v, ctx.to_device(Wt), ctx.to_device(bias), ctx.to_device(alpha),
                B, C_in, C_out)
    got = d_v.download()
    exp = oracle.fc_vmem(oracle.Consts.from_task(tc), xs, Wt, bias, alpha, B, C_in, C_out)
    scale = np.abs(exp) + 1e-3
    assert np.all(np.abs(got - exp) <= 1e-5 * scale)
    for argmax in (False, True):
        d_p = ctx.empty(B, np.int32)
        ctx.readout(ctx.to_device(got if argmax else x[:B * 4]), B, 10 if argmax else 4, argmax, d_p)
        ref = oracle.readout(got if argmax else x[:B * 4], B, 10 if argmax else 4,
                             oracle.READ_ARGMAX if argmax else oracle.READ_ARGMIN)
        np.testing.assert_array_equal(d_p.download(), ref)
    img = rng.random(4096).astype(np.float32)
    img[:5] = [0.0, 1e-6, 1e-5, 1.0, 0.5]
    d_e = ctx.empty(img.size)
    ctx.encode_linear(ctx.to_device(img), d_e)
    np.testing.assert_array_equal(d_e.download(), oracle.encode_linear(img, tc.T))
    ctx.encode_image(ctx.to_device(img), d_e, 17.452274, 0.0)
    g = d_e.download()
    o = oracle.encode_log(img, 17.452274, 0.0, tc.T)
    # device logf may differ from glibc by an ulp: only ceil-boundary ties may move
    diff = np.flatnonzero(g != o)
    assert diff.size <= 2, diff


def test_pool_min_vector_and_unaligned(gpu_ctx_factory):
    """Channel counts that are multiples of four take the 16-byte kernel (odd
    map sides drop the last row/column as the reference does); a map that
    starts 4 bytes past an aligned address takes the scalar kernel.  Both
    equal the oracle bit for bit."""
    import ctypes
    import types
    say("pool_min float4 / unaligned")
    rng = np.random.default_rng(81)
    tc = consts(64, 32.0, 8, True)
    ctx = gpu_ctx_factory(tc)
    for B, H, W, Cc in ((3, 9, 7, 8), (2, 4, 4, 12), (1, 2, 2, 4), (4, 14, 14, 64)):
        x = np.where(rng.random(B * H * W * Cc) < 0.5, rng.integers(0, 64, B * H * W * Cc), 9999)
        x = x.astype(np.float32)
        exp = oracle.pool_min(x, B, H, W, Cc)
        d_o = ctx.empty(exp.size)
        ctx.pool_min(ctx.to_device(x), d_o, B, H, W, Cc)
        np.testing.assert_array_equal(d_o.download(), exp)
        # the same map one float past an aligned address, in and out
        d_in = ctx.to_device(np.concatenate([np.zeros(1, np.float32), x]))
        d_out = ctx.empty(exp.size + 1)
        shift = lambda d: types.SimpleNamespace(ptr=ctypes.c_void_p(d.ptr.value + 4))  # noqa: E731
        ctx.pool_min(shift(d_in), shift(d_out), B, H, W, Cc)
        np.testing.assert_array_equal(d_out.download()[1:], exp)


def test_integrate_dropin_skips_foreign_events(gpu_ctx_factory):
    """The drop-in integrator over caller buckets guards what the reference
    leaves undefined (T2V:127-131 indexes delta[tb - base_t] and the weight
    row unchecked): events appended to a column's last chunk that lie in
    another chunk's bins, past the window, or at cin >= C_in are skipped, and
    a last offset past the column is clamped.  The result equals the valid
    buckets' output."""
    say("drop-in integrate with foreign events")
    rng = np.random.default_rng(4242)
    T, tfs, delta = 64, 32.0, 8
    tc = consts(T, tfs, delta, True)
    ctx = gpu_ctx_factory(tc)
    B, H, W, C_in, C_out, K = 2, 6, 6, 16, 64, 3
    n_cols = B * H * W
    t = rng.integers(0, T + 40, n_cols * C_in).astype(np.float32)
    sp = np.where(rng.random(t.size) < 0.3, t, INF).astype(np.float32)
    Wt = (rng.standard_normal(K * K * C_in * C_out) * 0.1).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.05).astype(np.float32)
    alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
    shape = dict(B=B, H_in=H, W_in=W, C_in=C_in, H_out=H, W_out=W, C_out=C_out, K_h=K, K_w=K)
    c = oracle.Consts.from_task(tc)
    cin, tin, off = oracle.bucketize(c, sp, n_cols, C_in)
    exp, _, _ = oracle.integrate(c, cin, tin, off, Wt, bias, alpha, theta, 0, pad=1, is_fc=False, **shape)
    OS = tc.num_chunks + 1
    NC = OS - 1
    bad_c, bad_t, bad_o = cin.copy(), tin.copy(), off.copy()
    foreign = [(C_in + 3, np.float32(tfs + T - 1)),   # cin past the input width
               (2, np.float32(tfs + 1.0)),            # a bin of chunk 0
               (5, np.float32(tfs + T + 7.0))]        # past the window
    n_bad = 0
    for col in range(n_cols):
        n = int(off[col * OS + NC])
        room = C_in - n
        for k in range(min(room, len(foreign))):
            bad_c[col * C_in + n + k], bad_t[col * C_in + n + k] = foreign[k]
            n_bad += 1
        bad_o[col * OS + NC] = n + min(room, len(foreign))
        if room == 0:
            bad_o[col * OS + NC] = C_in + 50  # clamped to the column
    assert n_bad > n_cols
    d_out = ctx.empty(exp.size, np.float32)
    ctx.integrate(d_out, ctx.to_device(bad_c), ctx.to_device(bad_t), ctx.to_device(bad_o), ctx.to_device(Wt),
                  ctx.to_device(bias), ctx.to_device(alpha), ctx.to_device(theta), 0, is_fc=False, **shape)
    ctx.synchronize()
    np.testing.assert_array_equal(d_out.download(), exp)
