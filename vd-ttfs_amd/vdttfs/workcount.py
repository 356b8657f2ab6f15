"""Work counts of the integrator that follow from the spike maps alone.

The reference's MAC profiler has a NOEARLYEXIT mode (T2M:170-172) in which
the chunk loop never breaks, so every neuron integrates every retained event
of its receptive field.  That count, E_noEE, is a closed form of the layer's
input map: C_out times the sum, over output pixels, of the retained events in
the in-bounds receptive columns.  With E_proc (the chunk-granular count under
the early exit, T2M:136-176) it gives the early-exit skip rate
1 - E_proc / E_noEE that the reference quotes as gamma
(CHUNK_SELECTION.md:93).  Retained means kept by bucketize (T2V:57-60):
t < INF and max(0, floor(t - TFS)) < T, evaluated in binary32.
"""
from __future__ import annotations

import numpy as np

INF = np.float32(9999.0)


def retained(x: np.ndarray, tfs: float, T: int) -> np.ndarray:
    """Boolean map of the inputs bucketize keeps (same shape as x)."""
    x = np.asarray(x, np.float32)
    with np.errstate(invalid="ignore"):
        live = x < INF
        tb = np.floor(np.where(live, x, np.float32(0.0)) - np.float32(tfs))
    tb = np.maximum(tb, 0)
    return live & (tb < T)


def no_exit_synapses(x: np.ndarray, B: int, H_in: int, W_in: int, C_in: int, H_out: int, W_out: int,
                     C_out: int, K_h: int, K_w: int, pad_h: int, pad_w: int, is_fc: bool, tfs: float,
                     T: int) -> tuple[int, int]:
    """(E_noEE, retained events) of one conv or FC layer whose input map x is
    NHWC [B][H_in][W_in][C_in] (FC: [B][C_in], C_in = every input)."""
    keep = retained(x, tfs, T)
    if is_fc:
        n = keep.reshape(B, -1).sum(axis=1, dtype=np.int64)
        return int(n.sum()) * C_out, int(n.sum())
    n = keep.reshape(B, H_in, W_in, C_in).sum(axis=3, dtype=np.int64)
    # zero-pad so that input row ho - pad_h + kh of every output row is addressable
    top, left = pad_h, pad_w
    bottom = max(0, H_out - 1 - pad_h + K_h - H_in)
    right = max(0, W_out - 1 - pad_w + K_w - W_in)
    p = np.pad(n, ((0, 0), (top, bottom), (left, right)))
    tot = 0
    for kh in range(K_h):
        for kw in range(K_w):
            tot += int(p[:, kh:kh + H_out, kw:kw + W_out].sum(dtype=np.int64))
    return tot * C_out, int(n.sum())
