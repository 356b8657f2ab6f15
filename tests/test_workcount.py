"""E_noEE (the no-early-exit synapse count of T2M:170-172) from the spike map
alone, against the oracle's NOEARLYEXIT counter: the closed form in
vdttfs.workcount must equal the count of a chunk loop that never breaks, and
E_proc under the early exit can only be smaller."""
import numpy as np
import pytest

import oracle
from vdttfs import workcount

INF = np.float32(9999.0)


@pytest.mark.parametrize("K_h,K_w,same,is_fc", [(3, 3, True, False), (3, 3, False, False), (1, 3, True, False),
                                                (5, 3, True, False), (2, 3, False, False), (1, 1, False, True)])
def test_no_exit_count_matches_oracle(K_h, K_w, same, is_fc):
    rng = np.random.default_rng(10 * K_h + K_w + 100 * same + 1000 * is_fc)
    T, tfs, delta = 32, (8.0 if same else 0.0), 4
    B, H, W, C_in, C_out = 2, 6, 7, 5, 6
    if is_fc:
        H = W = 1
        C_in = 40
        ho = wo = 1
    else:
        ho, wo = (H, W) if same else (H - K_h + 1, W - K_w + 1)
    n_cols = B * H * W
    t = rng.integers(0, T + 12, n_cols * C_in).astype(np.float32)
    x = np.where(rng.random(t.size) < 0.5, t, INF).astype(np.float32)
    x[:3] = [np.nan, -4.0, T + tfs]  # absent, clamped to bin 0, past the window
    Wt = (rng.standard_normal(K_h * K_w * C_in * C_out) * 0.3).astype(np.float32)
    bias = np.zeros(C_out, np.float32)
    alpha, theta = oracle.build_luts(T, 1.0, 8.0, 0.0, 8.0, 0.0)
    c = oracle.Consts(T, tfs, delta, same)
    cin, tin, off = oracle.bucketize(c, x, n_cols, C_in)
    pads = (K_h // 2, K_w // 2) if same else (0, 0)
    shape = dict(B=B, H_in=H, W_in=W, C_in=C_in, H_out=ho, W_out=wo, C_out=C_out, K_h=K_h, K_w=K_w)
    _, e_noee, _ = oracle.integrate(c, cin, tin, off, Wt, bias, alpha, theta, 0, pad=pads, is_fc=is_fc,
                                    no_early_exit=True, **shape)
    _, e_proc, _ = oracle.integrate(c, cin, tin, off, Wt, bias, alpha, theta, 0, pad=pads, is_fc=is_fc, **shape)
    got, n_ev = workcount.no_exit_synapses(x, pad_h=pads[0], pad_w=pads[1], is_fc=is_fc, tfs=tfs, T=T, **shape)
    assert got == e_noee
    assert n_ev == int(off.reshape(n_cols, -1)[:, -1].sum())
    assert e_proc <= e_noee
