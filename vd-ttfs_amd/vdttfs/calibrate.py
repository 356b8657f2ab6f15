"""Offline temporal-truncation calibration.

The paper's input-aware temporal truncation is an offline configuration, not
a runtime stage: the integration window TIME_WINDOW is a compile-time
constant, set to the full window T in the reference release and reduced, for
a bounded accuracy budget, under the guidance of layer-wise spike-time
percentiles (reference README, "Input-aware temporal truncation").  This
tool does that calibration on MI355X:

1. runs the engine on calibration inputs at the full window T and reports,
   for every integrating layer, the window that keeps a given share of
   (a) its input spikes integrated as under T: the arrival bin
   tb = max(0, floor(t - TFS)) stays below T', and with T2's time-indexed
   decay alpha[clamp((int)t, 0, T')] the clamp does not bite, (int)t <= T';
   and (b) the steps at which its neurons fire (the output time is the
   integration step t, and a window T' stops the loop at T').  With
   TFS = 0 (LeNet) the two coincide layer to layer; with TFS > 0 (VGG) the
   output steps reach T while the next layer's bins stay below T - TFS, so
   (b) and the decay clamp set the window;
2. runs the engine again under truncated windows, the inputs kept as
   encoded under T (VDTTFS_ENCODE_TIMES): one window T' for every layer
   (the largest per-layer percentile window, and any given ones), and per
   layer T'_l at each percentile (vdttfs_net_set_windows).  Under T'_l a
   layer drops arrivals at tb >= T'_l and its neurons stop firing at T'_l,
   exactly as a build of the reference with TIME_WINDOW = T'_l;
3. reports, per setting, the share of predictions that change against the
   full window and the time per batch, and the per-layer windows
   (`suggested_windows`, 0 for pools) a deployment would set.

  python -m vdttfs.calibrate --workload vgg16 --batch 256 --percentiles 90 99 99.9
  python -m vdttfs.calibrate --workload lenet5 --windows 16 24 32

Prints one JSON object.  Needs a GPU (it runs the engine).
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import numpy as np

from . import core, models

INF = 9999.0


def arrival_bins(times: np.ndarray, tfs: float) -> np.ndarray:
    """Arrival bins of the finite spike times (the engine's and the
    reference's rule: tb = max(0, floor(t - TFS)))."""
    t = times[times < INF].astype(np.float64)
    return np.maximum(0, np.floor(t - tfs)).astype(np.int64)


def input_requirements(times: np.ndarray, tfs: float, T: int, alpha_by_time: bool) -> np.ndarray:
    """Per input spike kept by the full window, the smallest window under
    which the layer integrates it exactly as under T: its bin must stay in
    the window (T' > tb), and where alpha is indexed by the raw time (T2,
    alpha[clamp((int)t, 0, T')]) the clamp must not bite (T' >= (int)t)."""
    t = times[times < INF].astype(np.float64)
    tb = np.maximum(0, np.floor(t - tfs)).astype(np.int64)
    keep = tb < T
    r = tb[keep] + 1
    if alpha_by_time:
        r = np.maximum(r, np.floor(t[keep]).astype(np.int64))
    return r


def firing_steps(times: np.ndarray) -> np.ndarray:
    """Integration steps at which the spikes of an integrating layer's
    output were fired (the output time is the step index)."""
    return np.floor(times[times < INF].astype(np.float64)).astype(np.int64)


def percentile_window(req: np.ndarray, q: float, T: int) -> int:
    """Smallest window T' (1 <= T' <= T) that meets at least q percent of
    the per-spike window requirements req (each in 1..T)."""
    r = np.sort(req)
    if r.size == 0:
        return 1
    k = int(np.ceil(q / 100.0 * r.size)) - 1
    k = min(max(k, 0), r.size - 1)
    return int(min(T, max(1, r[k])))


def _timed_forward(ctx, net, x, d_pred, reps):
    net.forward(x, d_pred)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        net.forward(x, d_pred)
    ctx.synchronize()
    return d_pred.download(), (time.perf_counter() - t0) * 1000.0 / reps


def layer_windows(w, enc: np.ndarray, outs, B: int, percentiles) -> list:
    """Per integrating layer: the windows that keep each percentile of its
    input arrivals and of its firing steps, and their maximum."""
    c = w.consts
    rows = []
    cur = enc
    for i, l in enumerate(w.layers):
        if l.kind != core.LAYER_POOL:
            bins = arrival_bins(cur, c.tfs)
            req = input_requirements(cur, c.tfs, c.T, c.alpha_by_time)
            row = {
                "layer": i,
                "kind": {core.LAYER_CONV: "conv", core.LAYER_FC: "fc", core.LAYER_VMEM: "vmem"}[l.kind],
                "input_spikes_per_image": int(np.count_nonzero(cur < INF)) / B,
                "arrivals_in_window_per_image": float(np.count_nonzero(bins < c.T)) / B,
                "input_windows": {str(q): percentile_window(req, q, c.T) for q in percentiles},
            }
            if l.kind == core.LAYER_VMEM:  # the readout integrates, it does not fire
                row["firing_windows"] = None
                row["windows"] = dict(row["input_windows"])
            else:
                steps = firing_steps(outs[i])
                row["output_spikes_per_image"] = steps.size / B
                row["firing_windows"] = {str(q): percentile_window(steps + 1, q, c.T) for q in percentiles}
                row["windows"] = {k: max(v, row["firing_windows"][k]) for k, v in row["input_windows"].items()}
            rows.append(row)
        cur = outs[i]
    return rows


def calibrate(w, img: np.ndarray, B: int, percentiles=(90.0, 99.0, 99.9), windows=(), reps: int = 5) -> dict:
    c = w.consts
    n = len(w.layers)
    ctx = core.Context(c, 0)
    try:
        # the inputs encoded once under the full window (the configs' linear rule)
        d_img = ctx.to_device(img)
        x = ctx.empty(B * w.img_elems)
        ctx.encode_linear(d_img, x)
        d_img.free()
        d_pred = ctx.empty(B, np.int32)
        net = core.Net(ctx, w.layers, B, w.img_elems, core.ENCODE_TIMES, w.tc_in, w.td_in, w.readout)
        try:
            pred_full, ms_full = _timed_forward(ctx, net, x, d_pred, reps)
            outs = [net.layer_output(i) for i in range(n)]
            enc = x.download()
            layers = layer_windows(w, enc, outs, B, percentiles)

            def run(mode, wins, **tag):
                net.set_windows(wins)
                pred, ms = _timed_forward(ctx, net, x, d_pred, reps)
                return dict(mode=mode, **tag, ms_per_batch=ms, speedup=ms_full / ms,
                            predictions_changed=float(np.mean(pred != pred_full)))

            per_layer = {}
            for q in percentiles:
                v = [0] * n
                for L in layers:
                    v[L["layer"]] = L["windows"][str(q)]
                per_layer[str(q)] = v
            uniform = {max(v) for v in per_layer.values()} | {int(t) for t in windows if 1 <= int(t) <= c.T}
            sweep = [run("uniform", [t] * n, T_window=t) for t in sorted(uniform)]
            sweep += [run("per_layer", v, percentile=float(q), windows=v) for q, v in per_layer.items()]
            net.set_windows(None)
        finally:
            net.close()
        x.free()
        d_pred.free()
    finally:
        ctx.close()
    return {"workload": w.name, "batch": B, "T": c.T, "tfs": c.tfs, "delta": c.delta,
            "full_window_ms_per_batch": ms_full, "layers": layers,
            "suggested_windows": per_layer, "sweep": sweep}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--workload", default="vgg16", choices=["vgg16", "lenet5"])
    ap.add_argument("--batch", type=int, default=None, help="default: 256 (vgg16), 1024 (lenet5)")
    ap.add_argument("--percentiles", type=float, nargs="*", default=[90.0, 99.0, 99.9])
    ap.add_argument("--windows", type=int, nargs="*", default=[])
    ap.add_argument("--reps", type=int, default=5)
    a = ap.parse_args(argv)
    vgg = a.workload == "vgg16"
    B = a.batch or (256 if vgg else 1024)
    w = models.vgg16() if vgg else models.lenet5()
    img = models.images_for(w, B)
    print(json.dumps(calibrate(w, img, B, a.percentiles, a.windows, a.reps)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
