"""Independent pure-Python restatement used to pin the C oracle on tiny inputs.

Written from the mathematics of the reference neuron, not from the oracle's
code: arithmetic is exact rational (fractions.Fraction) with one IEEE
binary32 round-to-nearest-even per operation, so a fused multiply-add is
rounded once and a plain add once.  Loops are the obvious dense ones (every
time bin scans the whole receptive field), so this shares no structure with
the bucketed, chunked oracle.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np

INF = 9999.0


def f32_round(x: Fraction) -> float:
    """Round an exact rational to the nearest binary32 (ties to even)."""
    if x == 0:
        return 0.0
    s = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)  # subnormal range keeps the fixed 2^-149 quantum
    q = Fraction(2) ** (e - 23)
    m = a / q
    n = m.numerator // m.denominator
    r = m - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = s * float(Fraction(n) * q)
    if abs(v) > 3.4028234663852886e38:
        return s * math.inf
    return float(np.float32(v))


def fq(v) -> Fraction:
    return Fraction(float(np.float32(v)))


def fma32(a, b, c) -> float:
    return f32_round(fq(a) * fq(b) + fq(c))


def add32(a, b) -> float:
    return f32_round(fq(a) + fq(b))


def mul32(a, b) -> float:
    return f32_round(fq(a) * fq(b))


def arrival_bin(t: float, tfs: float, T: int) -> int:
    """-1 when the spike is absent or outside the window."""
    t = float(np.float32(t))
    if not (t < INF):
        return -1
    tb = math.floor(float(np.float32(t - np.float32(tfs))))
    tb = max(tb, 0)
    return tb if tb < T else -1


def bucketize(spikes: np.ndarray, n_cols: int, c_in: int, T: int, tfs: float, delta: int):
    """Stable sort of each column's retained (cin, t) pairs by chunk."""
    NC = (T + delta - 1) // delta
    OS = NC + 1
    cin = np.zeros(n_cols * c_in, np.int32)
    tin = np.zeros(n_cols * c_in, np.float32)
    off = np.zeros(n_cols * OS, np.int32)
    sp = spikes.reshape(n_cols, c_in)
    for col in range(n_cols):
        ev = []
        for i in range(c_in):
            tb = arrival_bin(sp[col, i], tfs, T)
            if tb >= 0:
                ev.append((tb // delta, i, sp[col, i]))
        ev = sorted(ev, key=lambda e: e[0])  # Python's sort is stable
        for c in range(NC + 1):
            off[col * OS + c] = sum(1 for e in ev if e[0] < c)
        for p, (_, i, t) in enumerate(ev):
            cin[col * c_in + p] = i
            tin[col * c_in + p] = t
    return cin, tin, off


def _exp_arg(t, td, tc) -> float:
    """-((float)t - td) / tc evaluated in binary32, as the formula is written."""
    d = np.float32(np.float32(t) - np.float32(td))
    return float(np.float32(np.float32(-d) / np.float32(tc)))


def luts(T, vth, tc_i, td_i, tc_f, td_f):
    """alpha / theta: exp of the binary32 argument, rounded to binary32 from
    double precision (glibc expf is within 1 ulp of this)."""
    alpha = np.array([math.exp(_exp_arg(t, td_i, tc_i)) for t in range(T + 1)], np.float32)
    theta = np.array([float(np.float32(vth)) * math.exp(_exp_arg(t, td_f, tc_f)) for t in range(T)],
                     np.float32)
    return alpha, theta


def integrate_dense(spikes, W, bias, alpha, theta, t_min, B, H_in, W_in, C_in, H_out, W_out, C_out,
                    K_h, K_w, pad, is_fc, T, tfs, alpha_by_time):
    """First-spike time of every neuron, NHWC with c_out fastest.  pad: int
    (both axes) or (pad_h, pad_w)."""
    ph, pw = (pad if isinstance(pad, (tuple, list)) else (pad, pad))
    sp = np.asarray(spikes, np.float32).reshape(-1)
    Wf = np.asarray(W, np.float32).reshape(-1)
    out = []
    n_pix = B if is_fc else B * H_out * W_out
    for pix in range(n_pix):
        if is_fc:
            img, ho, wo = pix, 0, 0
        else:
            img, rem = divmod(pix, H_out * W_out)
            ho, wo = divmod(rem, W_out)
        for co in range(C_out):
            carry = float(np.float32(bias[co]))
            res = INF
            for t in range(T):
                acc = 0.0
                for kh in range(1 if is_fc else K_h):
                    for kw in range(1 if is_fc else K_w):
                        hi, wi = (0, 0) if is_fc else (ho - ph + kh, wo - pw + kw)
                        if not is_fc and not (0 <= hi < H_in and 0 <= wi < W_in):
                            continue
                        col = img if is_fc else (img * H_in + hi) * W_in + wi
                        for ci in range(C_in):
                            tin = sp[col * C_in + ci]
                            if arrival_bin(tin, tfs, T) != t:
                                continue
                            if alpha_by_time:
                                ai = min(max(int(float(tin)), 0), T)
                            else:
                                ai = t
                            widx = ((0 if is_fc else kh * K_w + kw) * C_in + ci) * C_out + co
                            acc = fma32(Wf[widx], alpha[ai], acc)
                carry = add32(carry, acc)
                th = float(theta[t])
                if t >= t_min and carry >= th and th >= float(np.float32(1e-5)):
                    res = float(t)
                    break
            out.append(res)
    return np.array(out, np.float32)
