"""ctypes wrapper of liboracle (oracle/vdttfs_oracle.c).

TEST INFRASTRUCTURE ONLY: the CPU restatement of the reference algorithm is
the parity checker and the timed CPU baseline.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module;
the product (vd-ttfs_amd/) never does.  Build with ``make -C oracle``.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvdttfs_oracle.so")
INF = np.float32(9999.0)

ORC_CONV, ORC_FC, ORC_POOL, ORC_VMEM = 0, 1, 2, 3
ENC_LINEAR, ENC_LOG, ENC_TIMES = 0, 1, 2
READ_ARGMIN, READ_ARGMAX, READ_T3 = 0, 1, 2


class OrcConsts(C.Structure):
    _fields_ = [("T", C.c_int), ("tfs", C.c_float), ("delta", C.c_int), ("alpha_by_time", C.c_int),
                ("vth", C.c_float)]


class OrcLayer(C.Structure):
    _fields_ = [("kind", C.c_int), ("H_in", C.c_int), ("W_in", C.c_int), ("C_in", C.c_int),
                ("H_out", C.c_int), ("W_out", C.c_int), ("C_out", C.c_int), ("K_h", C.c_int),
                ("K_w", C.c_int), ("pad_h", C.c_int), ("pad_w", C.c_int),
                ("W", C.POINTER(C.c_float)),
                ("bias", C.POINTER(C.c_float)), ("tc_fire", C.c_float), ("td", C.c_float)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} not built; run `make -C oracle`")
        _lib = C.CDLL(LIB_PATH)
        _lib.orc_net_forward.restype = C.c_int
        _lib.orc_culif_neuron_steps.restype = C.c_float
    return _lib


def pads(pad, K_h, K_w):
    """(pad_h, pad_w) of a conv: a pair is taken as given; an int p means the
    same p on both axes, which only a square kernel may use (T2V:109-110 pads
    rows by K_h/2 and columns by K_w/2)."""
    if isinstance(pad, (tuple, list)):
        return int(pad[0]), int(pad[1])
    if pad and K_h != K_w:
        raise ValueError(f"non-square {K_h}x{K_w} kernel: pass pad as (pad_h, pad_w)")
    return int(pad), int(pad)


def _p(a):
    return C.c_void_p(a.ctypes.data) if a is not None else None


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


@dataclass
class Consts:
    T: int
    tfs: float = 0.0
    delta: int = 16
    alpha_by_time: bool = False
    vth: float = 1.0

    def c(self):
        return OrcConsts(self.T, self.tfs, self.delta, int(self.alpha_by_time), self.vth)

    @property
    def num_chunks(self):
        return (self.T + self.delta - 1) // self.delta

    @classmethod
    def from_task(cls, tc):
        """From vdttfs.TaskConsts (duck-typed)."""
        return cls(tc.T, tc.tfs, tc.delta, bool(tc.alpha_by_time), tc.vth)


def build_luts(T, vth, tc_i, td_i, tc_f, td_f):
    a = np.empty(T + 1, np.float32)
    t = np.empty(T, np.float32)
    lib().orc_build_luts(C.c_int(T), C.c_float(vth), C.c_float(tc_i), C.c_float(td_i),
                         C.c_float(tc_f), C.c_float(td_f), _p(a), _p(t))
    return a, t


def encode_log(img, tc, td, T):
    img = f32(img)
    out = np.empty_like(img)
    lib().orc_encode_log(_p(img), _p(out), C.c_int64(img.size), C.c_float(tc), C.c_float(td), C.c_int(T))
    return out


def encode_linear(img, T):
    img = f32(img)
    out = np.empty_like(img)
    lib().orc_encode_linear(_p(img), _p(out), C.c_int64(img.size), C.c_int(T))
    return out


def bucketize(c: Consts, spikes, n_cols, c_in, nthreads=0):
    s = f32(spikes)
    OS = c.num_chunks + 1
    cin = np.zeros(n_cols * c_in, np.int32)
    tin = np.zeros(n_cols * c_in, np.float32)
    off = np.zeros(n_cols * OS, np.int32)
    cc = c.c()
    lib().orc_bucketize(C.byref(cc), _p(s), C.c_int64(n_cols), C.c_int(c_in), _p(cin), _p(tin),
                        _p(off), C.c_int(nthreads))
    return cin, tin, off


def integrate(c: Consts, cin, tin, off, W, bias, alpha, theta, t_min, B, H_in, W_in, C_in, H_out,
              W_out, C_out, K_h, K_w, pad, is_fc, no_early_exit=False, nthreads=0):
    """Returns (first-spike times, E_proc, E_bin).  pad: int (square kernels)
    or (pad_h, pad_w)."""
    ph, pw = pads(pad, K_h, K_w)
    n = B * (1 if is_fc else H_out * W_out) * C_out
    out = np.empty(n, np.float32)
    ep = C.c_uint64()
    eb = C.c_uint64()
    cc = c.c()
    W = f32(W)
    bias = f32(bias)
    alpha = f32(alpha)
    theta = f32(theta)
    cin = i32(cin)
    tin = f32(tin)
    off = i32(off)
    lib().orc_integrate(C.byref(cc), _p(out), _p(cin), _p(tin), _p(off), _p(W), _p(bias),
                        _p(alpha), _p(theta), C.c_int(t_min), C.c_int(B), C.c_int(H_in),
                        C.c_int(W_in), C.c_int(C_in), C.c_int(H_out), C.c_int(W_out),
                        C.c_int(C_out), C.c_int(K_h), C.c_int(K_w), C.c_int(ph), C.c_int(pw), C.c_int(int(is_fc)),
                        C.c_int(int(no_early_exit)), C.byref(ep), C.byref(eb), C.c_int(nthreads))
    return out, ep.value, eb.value


def integrate_timedriven(c: Consts, spikes, W, bias, alpha, theta, t_min, B, H_in, W_in, C_in,
                         H_out, W_out, C_out, K_h, K_w, pad, is_fc, nthreads=0):
    ph, pw = pads(pad, K_h, K_w)
    n = B * (1 if is_fc else H_out * W_out) * C_out
    out = np.empty(n, np.float32)
    cc = c.c()
    sp, W, bias, alpha, theta = f32(spikes), f32(W), f32(bias), f32(alpha), f32(theta)
    lib().orc_integrate_timedriven(C.byref(cc), _p(out), _p(sp), _p(W), _p(bias), _p(alpha),
                                   _p(theta), C.c_int(t_min), C.c_int(B), C.c_int(H_in),
                                   C.c_int(W_in), C.c_int(C_in), C.c_int(H_out), C.c_int(W_out),
                                   C.c_int(C_out), C.c_int(K_h), C.c_int(K_w), C.c_int(ph),
                                   C.c_int(pw), C.c_int(int(is_fc)), C.c_int(nthreads))
    return out


def integrate_margin(c: Consts, spikes, W, bias, alpha, theta, t_min, B, H_in, W_in, C_in, H_out,
                     W_out, C_out, K_h, K_w, pad, is_fc, nthreads=0):
    ph, pw = pads(pad, K_h, K_w)
    n = B * (1 if is_fc else H_out * W_out) * C_out
    out = np.empty(n, np.float64)
    cc = c.c()
    sp, W, bias, alpha, theta = f32(spikes), f32(W), f32(bias), f32(alpha), f32(theta)
    lib().orc_integrate_margin(C.byref(cc), _p(out), _p(sp), _p(W), _p(bias), _p(alpha), _p(theta),
                               C.c_int(t_min), C.c_int(B), C.c_int(H_in), C.c_int(W_in),
                               C.c_int(C_in), C.c_int(H_out), C.c_int(W_out), C.c_int(C_out),
                               C.c_int(K_h), C.c_int(K_w), C.c_int(ph), C.c_int(pw),
                               C.c_int(int(is_fc)), C.c_int(nthreads))
    return out


def pool_min(x, B, H_in, W_in, Cc, nthreads=0):
    x = f32(x)
    out = np.empty(B * (H_in // 2) * (W_in // 2) * Cc, np.float32)
    lib().orc_pool_min(_p(x), _p(out), C.c_int(B), C.c_int(H_in), C.c_int(W_in), C.c_int(Cc),
                       C.c_int(nthreads))
    return out


def fc_vmem(c: Consts, x, W, bias, alpha, B, C_in, C_out):
    x, W, bias, alpha = f32(x), f32(W), f32(bias), f32(alpha)
    out = np.empty(B * C_out, np.float32)
    cc = c.c()
    lib().orc_fc_vmem(C.byref(cc), _p(x), _p(out), _p(W), _p(bias), _p(alpha), C.c_int(B),
                      C.c_int(C_in), C.c_int(C_out))
    return out


def readout(out, B, Cc, mode):
    out = f32(out)
    pred = np.empty(B, np.int32)
    fn = {READ_ARGMIN: lib().orc_readout_argmin, READ_ARGMAX: lib().orc_readout_argmax,
          READ_T3: lib().orc_readout_t3}[mode]
    fn(_p(out), C.c_int(B), C.c_int(Cc), _p(pred))
    return pred


def net_forward(c: Consts, layers, B, img, img_elems, encode_mode, tc_in, td_in, readout_mode,
                same_pad=False, keep_layers=False, nthreads=0):
    """layers: objects with kind/H_in/.../kernel/bias/tc_fire/td (vdttfs.Layer works).
    Returns dict(final, pred, eproc, ebin, outs)."""
    n = len(layers)
    arr = (OrcLayer * n)()
    keep = []
    for i, l in enumerate(layers):
        k = f32(l.kernel) if l.kernel is not None else None
        b = f32(l.bias) if l.bias is not None else None
        keep += [k, b]
        same = l.kind == ORC_CONV and same_pad
        fp = C.POINTER(C.c_float)
        arr[i] = OrcLayer(l.kind, l.H_in, l.W_in, l.C_in, l.H_out, l.W_out, l.C_out, l.K_h, l.K_w,
                          l.K_h // 2 if same else 0, l.K_w // 2 if same else 0, k.ctypes.data_as(fp) if k is not None else fp(),
                          b.ctypes.data_as(fp) if b is not None else fp(), l.tc_fire, l.td)
    outs = [np.empty(B * l.H_out * l.W_out * l.C_out, np.float32) for l in layers] if keep_layers else None
    outs_p = (C.POINTER(C.c_float) * n)(*[o.ctypes.data_as(C.POINTER(C.c_float)) for o in outs]) if outs else None
    last = layers[-1]
    final = np.empty(B * last.H_out * last.W_out * last.C_out, np.float32)
    pred = np.empty(B, np.int32)
    ep = (C.c_uint64 * n)()
    eb = (C.c_uint64 * n)()
    img = f32(img)
    cc = c.c()
    rc = lib().orc_net_forward(C.byref(cc), arr, C.c_int(n), C.c_int(B), _p(img),
                               C.c_int64(img_elems), C.c_int(encode_mode), C.c_float(tc_in),
                               C.c_float(td_in), C.c_int(readout_mode), outs_p, _p(final), _p(pred),
                               ep, eb, C.c_int(nthreads))
    if rc != 0:
        raise RuntimeError(f"orc_net_forward failed: {rc}")
    return {"final": final, "pred": pred, "eproc": np.array(list(ep), np.uint64),
            "ebin": np.array(list(eb), np.uint64), "outs": outs}


STEP_T1, STEP_T2 = 1, 2


def stepnet_forward(c: Consts, layers, B, img, img_elems, encode_mode, tc_in, td_in, mode,
                    same_pad=False, nthreads=0):
    """Step-by-step (time-driven) baseline network: T1S (mode 1) or T2S
    (mode 2) semantics, see orc_stepnet_forward.  Returns dict(final, pred,
    steps): final is B x C of the last layer (first-spike steps or max V+b)."""
    n = len(layers)
    arr = (OrcLayer * n)()
    keep = []
    fp = C.POINTER(C.c_float)
    for i, l in enumerate(layers):
        k = f32(l.kernel) if l.kernel is not None else None
        b = f32(l.bias) if l.bias is not None else None
        keep += [k, b]
        same = l.kind == ORC_CONV and same_pad
        arr[i] = OrcLayer(l.kind, l.H_in, l.W_in, l.C_in, l.H_out, l.W_out, l.C_out, l.K_h, l.K_w,
                          l.K_h // 2 if same else 0, l.K_w // 2 if same else 0, k.ctypes.data_as(fp) if k is not None else fp(),
                          b.ctypes.data_as(fp) if b is not None else fp(), l.tc_fire, l.td)
    last = layers[-1]
    final = np.empty(B * last.H_out * last.W_out * last.C_out, np.float32)
    pred = np.empty(B, np.int32)
    steps = C.c_int(0)
    img = f32(img)
    cc = c.c()
    rc = lib().orc_stepnet_forward(C.byref(cc), arr, C.c_int(n), C.c_int(B), _p(img), C.c_int64(img_elems),
                                   C.c_int(encode_mode), C.c_float(tc_in), C.c_float(td_in), C.c_int(mode),
                                   _p(final), _p(pred), C.byref(steps), C.c_int(nthreads))
    if rc != 0:
        raise RuntimeError(f"orc_stepnet_forward failed: {rc}")
    return {"final": final, "pred": pred, "steps": steps.value}


class OrcCulifLayer(C.Structure):
    _fields_ = [("kind", C.c_int), ("C_in", C.c_int), ("H_in", C.c_int), ("W_in", C.c_int), ("C_out", C.c_int),
                ("w", C.POINTER(C.c_float)), ("w_rec", C.POINTER(C.c_float)), ("decay", C.c_float),
                ("th", C.c_float)]


def culif_stepnet_forward(layers, data, N, T, keep_layers=False, nthreads=0):
    """Step-by-step CuLIF baseline (T3S semantics, see
    orc_culif_stepnet_forward).  layers: vdttfs.CulifLayerSpec-like; data
    [N][C][H][W][T].  Returns dict(final, pred, outs): first-spike steps of
    the last layer (and of every layer, NCHW, with keep_layers)."""
    n = len(layers)
    arr = (OrcCulifLayer * n)()
    keep = []
    fp = C.POINTER(C.c_float)
    elems = []
    for i, l in enumerate(layers):
        w = f32(l.weight) if l.weight is not None else None
        r = f32(l.weight_rec) if l.weight_rec is not None else None
        keep += [w, r]
        arr[i] = OrcCulifLayer(l.kind, l.C_in, l.H_in, l.W_in, l.C_out,
                               w.ctypes.data_as(fp) if w is not None else fp(),
                               r.ctypes.data_as(fp) if r is not None else fp(), l.decay, l.th)
        if l.kind in (3, 4):
            elems.append(N * l.C_out)
        elif l.kind == 2:
            elems.append(N * l.C_in * (l.H_in // 2) * (l.W_in // 2))
        else:
            elems.append(N * l.C_out * l.H_in * l.W_in)
    outs = [np.empty(e, np.float32) for e in elems] if keep_layers else None
    outs_p = (C.POINTER(C.c_float) * n)(*[o.ctypes.data_as(fp) for o in outs]) if outs else None
    final = np.empty(elems[-1], np.float32)
    pred = np.empty(N, np.int32)
    data = f32(data)
    rc = lib().orc_culif_stepnet_forward(arr, C.c_int(n), C.c_int(N), _p(data), C.c_int(T), outs_p, _p(final),
                                         _p(pred), C.c_int(nthreads))
    if rc != 0:
        raise RuntimeError(f"orc_culif_stepnet_forward failed: {rc}")
    return {"final": final, "pred": pred, "outs": outs}


# ---- CuLIF set (T3V:30-225) -------------------------------------------------
def _ci(*xs):
    return [C.c_int(int(x)) for x in xs]


def culif_conv1_raw(data, weight, N, C_in, C_out, H, W, T, delta, decay, th, nthreads=0):
    data, weight = f32(data), f32(weight)
    out = np.empty(N * C_out * H * W, np.float32)
    lib().orc_culif_conv1_raw(_p(data), _p(out), _p(weight), *_ci(N, C_in, C_out, H, W, T, delta),
                              C.c_float(decay), C.c_float(th), C.c_int(nthreads))
    return out


def culif_bucketize_nchw(x, N, Cc, H, W, T, delta, nthreads=0):
    x = f32(x)
    OS = T // delta + 1
    cin = np.zeros(N * H * W * Cc, np.int32)
    tin = np.zeros(N * H * W * Cc, np.float32)
    off = np.zeros(N * H * W * OS, np.int32)
    lib().orc_culif_bucketize_nchw(_p(x), *_ci(N, Cc, H, W, T, delta), _p(cin), _p(tin), _p(off),
                                   C.c_int(nthreads))
    return cin, tin, off


def culif_bucketize_fc(x, N, F, T, delta, nthreads=0):
    x = f32(x)
    OS = T // delta + 1
    cin = np.zeros(N * F, np.int32)
    tin = np.zeros(N * F, np.float32)
    off = np.zeros(N * OS, np.int32)
    lib().orc_culif_bucketize_fc(_p(x), *_ci(N, F, T, delta), _p(cin), _p(tin), _p(off),
                                 C.c_int(nthreads))
    return cin, tin, off


def culif_conv(cin, tin, off, weight, N, C_in, C_out, H, W, T, delta, decay, th, nthreads=0):
    cin, tin, off, weight = i32(cin), f32(tin), i32(off), f32(weight)
    out = np.empty(N * C_out * H * W, np.float32)
    lib().orc_culif_conv(_p(cin), _p(tin), _p(off), _p(out), _p(weight),
                         *_ci(N, C_in, C_out, H, W, T, delta), C.c_float(decay), C.c_float(th),
                         C.c_int(nthreads))
    return out


def culif_pool(x, N, Cc, H_in, W_in, T, delta, decay, th, nthreads=0):
    x = f32(x)
    out = np.empty(N * Cc * (H_in // 2) * (W_in // 2), np.float32)
    lib().orc_culif_pool(_p(x), _p(out), *_ci(N, Cc, H_in, W_in, T, delta), C.c_float(decay),
                         C.c_float(th), C.c_int(nthreads))
    return out


def culif_fc_recurrent(cin, tin, off, w, w_rec, N, in_f, out_f, T, delta, decay, th, nthreads=0):
    cin, tin, off, w, w_rec = i32(cin), f32(tin), i32(off), f32(w), f32(w_rec)
    out = np.empty(N * out_f, np.float32)
    lib().orc_culif_fc_recurrent(_p(cin), _p(tin), _p(off), _p(out), _p(w), _p(w_rec),
                                 *_ci(N, in_f, out_f, T, delta), C.c_float(decay), C.c_float(th),
                                 C.c_int(nthreads))
    return out


def culif_fc(cin, tin, off, w, N, in_f, out_f, T, delta, decay, th, nthreads=0):
    cin, tin, off, w = i32(cin), f32(tin), i32(off), f32(w)
    out = np.empty(N * out_f, np.float32)
    lib().orc_culif_fc(_p(cin), _p(tin), _p(off), _p(out), _p(w), *_ci(N, in_f, out_f, T, delta),
                       C.c_float(decay), C.c_float(th), C.c_int(nthreads))
    return out


def culif_net_forward(layers, data, N, T, delta, nthreads=0):
    """The T3V main() sequence (T3V:276-298) over the oracle's kernels.
    layers: vdttfs.CulifLayerSpec-like (kind 0 raw conv, 1 conv, 2 pool,
    3 recurrent FC, 4 FC).  Returns (per-layer NCHW outputs, predictions)."""
    outs = []
    cur = None
    for l in layers:
        if l.kind == 0:
            cur = culif_conv1_raw(data, l.weight, N, l.C_in, l.C_out, l.H_in, l.W_in, T, delta,
                                  l.decay, l.th, nthreads)
        elif l.kind == 1:
            b = culif_bucketize_nchw(cur, N, l.C_in, l.H_in, l.W_in, T, delta, nthreads)
            cur = culif_conv(*b, l.weight, N, l.C_in, l.C_out, l.H_in, l.W_in, T, delta, l.decay,
                             l.th, nthreads)
        elif l.kind == 2:
            cur = culif_pool(cur, N, l.C_in, l.H_in, l.W_in, T, delta, l.decay, l.th, nthreads)
        elif l.kind == 3:
            b = culif_bucketize_fc(cur, N, l.C_in, T, delta, nthreads)
            cur = culif_fc_recurrent(*b, l.weight, l.weight_rec, N, l.C_in, l.C_out, T, delta,
                                     l.decay, l.th, nthreads)
        else:
            b = culif_bucketize_fc(cur, N, l.C_in, T, delta, nthreads)
            cur = culif_fc(*b, l.weight, N, l.C_in, l.C_out, T, delta, l.decay, l.th, nthreads)
        outs.append(cur)
    return outs, readout(cur, N, layers[-1].C_out, READ_T3)
