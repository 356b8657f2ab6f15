"""Launch-granularity autotuner: the reference's chunk-width sweep, on MI355X.

The reference has one granularity knob, the compile-time chunk width Delta,
and chooses it per task by a sweep: recompile for each Delta, run the
evaluation set three times, keep the minimum time, and record the outputs at
every Delta to confirm that chunking is lossless (CHUNK_SELECTION.md:44-62).

Here Delta no longer sets the integrator's granularity: the engine sorts
events into one-step bins and exits per bin, so its outputs and its time do
not depend on Delta (Delta only defines the reference's E_proc work count).
The sweep below confirms both.  The engine's own granularity knobs are per
layer: how the merged event lists are built (bins, dense or fused) or whether
the receptive field stays in registers with no list (reg), how many
c_out a lane gathers per event (1, 2 events per load, or 4), and how many
output pixels a wave integrates.  The tuner sweeps them per layer with the
reference's procedure -- minimum of three timed rounds, outputs compared bit
for bit with the built-in choice -- and reports the best plan per layer and
the whole forward under the tuned plans; then, under those plans, which 2x2
pools run inside the next layer's list build (vdttfs_net_set_pool_fusion:
off, auto or all), timed on the whole forward.

  python -m vdttfs.tune --workload vgg16 --batch 256
  python -m vdttfs.tune --workload lenet5 --deltas 4 8 16 32 64

Prints one JSON object.  Needs a GPU.
"""
from __future__ import annotations

import argparse
import dataclasses
import itertools
import json
import sys

import numpy as np

from . import core, models

PATHS = {core.PATH_BINS: "bins", core.PATH_DENSE: "dense", core.PATH_FUSED: "fused", core.PATH_REG: "reg",
         core.PATH_WINDOW: "window"}
POOL_FUSION = {"off": core.POOL_FUSE_OFF, "auto": core.POOL_FUSE_AUTO, "all": core.POOL_FUSE_ALL}


def _min_round_ms(ctx, net, x, d_pred, reps, rounds, per_layer):
    """Minimum over rounds of the mean per-forward time: the whole forward
    (HIP events around reps forwards) or, per_layer, each layer's event time."""
    best = None
    for _ in range(rounds):
        if per_layer:
            net.set_timing(True)
            net.read_layer_timing()
            for _ in range(reps):
                net.forward(x, d_pred)
            v = net.read_layer_timing() / reps
            net.set_timing(False)
            net.read_timing()
        else:
            ctx.timer_begin()
            for _ in range(reps):
                net.forward(x, d_pred)
            v = ctx.timer_end() / reps
        best = v if best is None else np.minimum(best, v)
    return best


def delta_sweep(w, img, B, deltas, reps=3, rounds=3):
    """The reference's sweep (CHUNK_SELECTION.md:44-62) run on the engine:
    per Delta, the minimum forward time of three rounds, the E_proc count,
    and whether every layer's output equals the first Delta's."""
    rows, ref = [], None
    for D in deltas:
        c = dataclasses.replace(w.consts, delta=int(D))
        with core.Context(c, 0) as ctx:
            net = core.Net(ctx, w.layers, B, w.img_elems, core.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)
            try:
                x = ctx.to_device(img)
                d_pred = ctx.empty(B, np.int32)
                ms = float(_min_round_ms(ctx, net, x, d_pred, reps, rounds, False))
                outs = [net.layer_output(i) for i in range(len(w.layers))]
                eproc = net.count(x)[0]
                x.free()
                d_pred.free()
            finally:
                net.close()
        same = None
        if ref is None:
            ref = outs
        else:
            same = all(np.array_equal(a, b) for a, b in zip(outs, ref))
        rows.append({"delta": int(D), "ms_per_batch": ms, "eproc": int(eproc.sum()),
                     "identical_to_first": same})
    return rows


def candidates(net, layer):
    """The plans the kernels can run for a layer (set_plan accepts them),
    resolved; 0 asks for the built-in gather or pixels per wave, which is
    the only choice on layers narrower than 32 outputs."""
    out = []
    for path, gather, ppw in itertools.product(PATHS, (0, 1, 2, 4), (0, 1, 2, 4)):
        try:
            net.set_plan(layer, path, gather, ppw)
        except core.VdttfsError:
            continue
        out.append(net.get_plan(layer))
    net.set_plan(layer)
    return sorted(set(out))


def tune_plans(w, img, B, reps=3, rounds=3):
    n = len(w.layers)
    with core.Context(w.consts, 0) as ctx:
        net = core.Net(ctx, w.layers, B, w.img_elems, core.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)
        try:
            x = ctx.to_device(img)
            d_pred = ctx.empty(B, np.int32)
            auto_plans = [net.get_plan(i) for i in range(n)]
            base = _min_round_ms(ctx, net, x, d_pred, reps, rounds, True)
            ref = [net.layer_output(i) for i in range(n)]
            fwd_auto = float(_min_round_ms(ctx, net, x, d_pred, reps, rounds, False))
            rows, best_plans = [], list(auto_plans)
            for i, l in enumerate(w.layers):
                if l.kind not in (core.LAYER_CONV, core.LAYER_FC):
                    continue
                cands = []
                for plan in candidates(net, i):
                    net.set_plan(i, *plan)
                    ms = float(_min_round_ms(ctx, net, x, d_pred, reps, rounds, True)[i])
                    same = bool(np.array_equal(net.layer_output(i), ref[i]))
                    cands.append({"plan": _plan_dict(plan), "ms": ms, "identical": same})
                net.set_plan(i)
                ok = [c for c in cands if c["identical"]]
                best = min(ok, key=lambda c: c["ms"]) if ok else None
                if best is not None:
                    p = best["plan"]
                    best_plans[i] = (_path_id(p["path"]), p["gather"], p["ppw"])
                rows.append({"layer": i, "kind": "conv" if l.kind == core.LAYER_CONV else "fc",
                             "shape": [l.H_in, l.W_in, l.C_in, l.C_out, l.K_h, l.K_w],
                             "auto": {"plan": _plan_dict(auto_plans[i]), "ms": float(base[i])},
                             "best": best, "candidates": cands,
                             "all_identical": all(c["identical"] for c in cands)})
            for i, p in enumerate(best_plans):
                if w.layers[i].kind in (core.LAYER_CONV, core.LAYER_FC):
                    net.set_plan(i, *p)
            fwd_tuned = float(_min_round_ms(ctx, net, x, d_pred, reps, rounds, False))
            tuned_same = all(np.array_equal(net.layer_output(i), ref[i]) for i in range(n))
            # pool fusion under the tuned plans: the whole forward per mode
            # (a fused pool's map is written when layer_output asks for it)
            fusion = {}
            for name, mode in POOL_FUSION.items():
                net.set_pool_fusion(mode)
                ms = float(_min_round_ms(ctx, net, x, d_pred, reps, rounds, False))
                same = all(np.array_equal(net.layer_output(i), ref[i]) for i in range(n))
                fusion[name] = {"ms": ms, "identical": same}
            net.set_pool_fusion(core.POOL_FUSE_OFF)
            ok = [k for k, v in fusion.items() if v["identical"]]
            best_fusion = min(ok, key=lambda k: fusion[k]["ms"]) if ok else "off"
            x.free()
            d_pred.free()
        finally:
            net.close()
    return {"layers": rows, "forward_ms": {"auto": fwd_auto, "tuned": fwd_tuned},
            "tuned_identical": tuned_same, "pool_fusion": {"modes": fusion, "best": best_fusion},
            "plans": [_plan_dict(p) if w.layers[i].kind in (core.LAYER_CONV, core.LAYER_FC) else None
                      for i, p in enumerate(best_plans)]}


def _plan_dict(p):
    return {"path": PATHS.get(p[0], "none"), "gather": int(p[1]), "ppw": int(p[2])}


def _path_id(name):
    return {v: k for k, v in PATHS.items()}[name]


def apply_plans(net, plans):
    """Sets the plans of a tune result ("plans": one dict or None per layer)."""
    if len(plans) != len(net.layers):
        raise ValueError(f"{len(plans)} plans for {len(net.layers)} layers")
    for i, p in enumerate(plans):
        if p is not None:
            net.set_plan(i, _path_id(p["path"]), p["gather"], p["ppw"])


def apply_pool_fusion(net, name):
    """Sets the pool-fusion mode of a tune result ("off", "auto" or "all";
    None leaves the network's default)."""
    if name is not None:
        net.set_pool_fusion(POOL_FUSION[name])


def _load(path, w, B):
    with open(path) as f:
        d = json.load(f)
    if d.get("workload") != w.name or d.get("batch") != B or d.get("T") != w.consts.T:
        raise ValueError(f"{path}: plans for {d.get('workload')} B={d.get('batch')} T={d.get('T')}, "
                         f"not {w.name} B={B} T={w.consts.T}")
    return d


def load_plans(path, w, B):
    """Plans written by --out, checked against the workload and batch."""
    return _load(path, w, B)["plans"]


def load_pool_fusion(path, w, B):
    """The pool-fusion mode written by --out, or None (files without one)."""
    name = _load(path, w, B).get("pool_fusion")
    if name is not None and name not in POOL_FUSION:
        raise ValueError(f"{path}: unknown pool fusion {name!r}")
    return name


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--workload", default="vgg16", choices=["vgg16", "lenet5"])
    ap.add_argument("--batch", type=int, default=None, help="default: 256 (vgg16), 1024 (lenet5)")
    ap.add_argument("--deltas", type=int, nargs="*", default=[4, 8, 16, 32, 64])
    ap.add_argument("--reps", type=int, default=3, help="forwards per timed round")
    ap.add_argument("--rounds", type=int, default=3, help="timed rounds; the minimum is kept")
    ap.add_argument("--no-plans", action="store_true", help="run the Delta sweep only")
    ap.add_argument("--out", default=None, help="also write the tuned plans as JSON (bench.py --plans)")
    a = ap.parse_args(argv)
    vgg = a.workload == "vgg16"
    B = a.batch or (256 if vgg else 1024)
    w = models.vgg16() if vgg else models.lenet5()
    img = models.images_for(w, B)
    r = {"workload": w.name, "batch": B, "T": w.consts.T,
         "delta_sweep": delta_sweep(w, img, B, a.deltas, a.reps, a.rounds) if a.deltas else []}
    if not a.no_plans:
        r.update(tune_plans(w, img, B, a.reps, a.rounds))
        if a.out:
            with open(a.out, "w") as f:
                json.dump({"workload": w.name, "batch": B, "T": w.consts.T, "plans": r["plans"],
                           "pool_fusion": r["pool_fusion"]["best"]}, f, indent=1)
    print(json.dumps(r), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
