"""Writes tests/golden/integrate_golden.json: tiny bucketize + integrate cases
whose expected outputs come from tests/pyref.py (exact-rational, dense
time-driven restatement), never from the oracle or the HIP engine.

Run from the repository root:  python tests/golden/make_golden.py
The decay/threshold tables are stored with the case, so the fixture does not
depend on the host's expf.
"""
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import pyref  # noqa: E402


def case(seed, T, tfs, delta, abt, is_fc, same, B, H, W, C_in, C_out, K, t_min):
    rng = np.random.default_rng(seed)
    if is_fc:
        sh = dict(B=B, H_in=1, W_in=1, C_in=C_in, H_out=1, W_out=1, C_out=C_out, K_h=1, K_w=1,
                  pad=0, is_fc=1)
        n_cols = B
    else:
        pad = K // 2 if same else 0
        sh = dict(B=B, H_in=H, W_in=W, C_in=C_in, H_out=H if same else H - K + 1,
                  W_out=W if same else W - K + 1, C_out=C_out, K_h=K, K_w=K, pad=pad, is_fc=0)
        n_cols = B * H * W
    n = n_cols * C_in
    t = rng.integers(0, T + 4, n).astype(np.float32)
    sp = np.where(rng.random(n) < 0.6, t, np.float32(9999.0)).astype(np.float32)
    Wt = (rng.standard_normal(sh["K_h"] * sh["K_w"] * C_in * C_out) * 0.7).astype(np.float32)
    bias = (rng.standard_normal(C_out) * 0.2).astype(np.float32)
    tc = T / 4.0
    alpha, theta = pyref.luts(T, 1.0, tc, 0.0, tc, 0.0)
    cin, tin, off = pyref.bucketize(sp, n_cols, C_in, T, tfs, delta)
    out = pyref.integrate_dense(sp, Wt, bias, alpha, theta, t_min, T=T, tfs=tfs,
                                alpha_by_time=abt, **sh)
    return {
        "consts": {"T": T, "tfs": tfs, "delta": delta, "alpha_by_time": abt},
        "shape": sh, "t_min": t_min,
        "spikes": sp.tolist(), "W": Wt.tolist(), "bias": bias.tolist(),
        "alpha": alpha.tolist(), "theta": theta.tolist(),
        "cin": cin.tolist(), "tin": tin.tolist(), "off": off.tolist(), "out": out.tolist(),
    }


def main():
    cases = [
        case(1, 16, 0.0, 4, False, False, False, 2, 5, 5, 3, 4, 3, 0),   # Task-1 valid conv
        case(2, 16, 6.0, 4, True, False, True, 1, 4, 4, 4, 3, 3, 1),     # Task-2 same conv
        case(3, 12, 0.0, 5, False, True, False, 3, 1, 1, 9, 5, 1, 0),    # FC, Delta does not divide T
        case(4, 20, 10.0, 8, True, True, False, 2, 1, 1, 12, 6, 1, 2),   # FC with TFS
        case(5, 16, 0.0, 16, False, False, False, 1, 6, 6, 2, 3, 5, 0),  # 5x5 valid conv, one chunk
    ]
    with open(os.path.join(HERE, "integrate_golden.json"), "w") as f:
        json.dump(cases, f)
    print("wrote", len(cases), "cases")


if __name__ == "__main__":
    main()
