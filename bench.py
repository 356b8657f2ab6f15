#!/usr/bin/env python3
"""Benchmark: VGG-16 TTFS-SNN inference (config 3) on one MI355X.

One step = one batch of 256 synthetic images through the whole network:
encode -> 13 conv layers (bucketize + integrate) with 5 min-pools -> FC
512->512 -> 512->10 membrane-potential readout -> argmax, inputs already
resident in HBM.  Prints ONE JSON line (stdout) with images/s, the
integrator's roofline position and a same-host CPU baseline of the
reference algorithm (oracle/, timed on a bounded sample).

  python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu]
  python bench.py --copy-calibration   # known-size copy for FETCH/WRITE_SIZE scaling

The other synthetic workloads print one line each in the same format
(parity cases of the same engine, not the headline):

  python bench.py --workload lenet5     # config 2: LeNet-5, B=1024 (config 1 = its B=1 CPU leg)
  python bench.py --workload culif7     # config 4: 7-layer CuLIF on 2x128x128 events, B=64
  python bench.py --workload fc-sweep   # config 5: FC 4096x4096, B=512, density/T'/delta sweep
  python bench.py --workload vgg16-timedriven | lenet5-timedriven
                                        # the reference's step-by-step GPU baseline (T2S / T1S)
                                        # on configs 3 / 2, with the event-driven speedup

roofline.traffic is the integrator's HBM bytes per launch measured with
rocprofv3 FETCH_SIZE / WRITE_SIZE counter runs and written to
profiles/integrator_vgg16_b256_traffic.md (by python -m
vdttfs.rocprof_summary traffic); it is reported only when that file's
workload line matches the configuration being run, else null.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "vd-ttfs_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

METRIC = "images/sec/GPU for VGG-16 TTFS bs=256; integrator % of HBM peak"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "integrator_vgg16_b256_traffic.md")
COPY_FLOATS = 1 << 28  # 1 GiB read + 1 GiB written per calibration dispatch


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def algorithmic_bytes(w, eproc, n_ev, n_cols, B):
    """Fused bytes per integrating layer, B_int + 4*N_cols*C_in: the dense
    input map read once, 4*E_proc (one fp32 weight per integrated synapse),
    8*N_ev (event lists) + 4*OS*N_cols (chunk offsets), 4*C_out (bias) and
    4*N_out (first-spike write).  Conv layers build their event lists straight
    from the dense map; FC layers bucketize first -- either way the layer's
    whole integrate (bucketize + merge + stream) is priced and timed."""
    OS = w.consts.num_chunks + 1
    total = 0
    per_layer = []
    for i, l in enumerate(w.layers):
        if l.kind not in (0, 1):
            per_layer.append(0)
            continue
        n_out = B * l.H_out * l.W_out * l.C_out
        cin_col = l.C_in if l.kind == 0 else l.H_in * l.W_in * l.C_in
        b = (4 * int(eproc[i]) + 8 * int(n_ev[i]) + 4 * OS * int(n_cols[i]) + 4 * l.C_out + 4 * n_out
             + 4 * int(n_cols[i]) * cin_col)
        per_layer.append(b)
        total += b
    return total, per_layer


def workload_key(B, consts) -> str:
    return f"vgg16 B={B} T={consts.T} delta={consts.delta} tfs={consts.tfs:g}"


def measured_traffic(key: str):
    """(bytes per step, launches per step) from the committed counter summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            text = f.read()
    except OSError:
        return None
    wl = per_step = launches = None
    for line in text.splitlines():
        line = line.strip().strip("`")
        if line.startswith("WORKLOAD="):
            wl = line[len("WORKLOAD="):].strip()
        elif line.startswith("TRAFFIC_PER_STEP_BYTES="):
            kv = dict(t.split("=", 1) for t in line.split())
            per_step = float(kv["TRAFFIC_PER_STEP_BYTES"])
            launches = int(kv["LAUNCHES_PER_STEP"])
    if wl != key or per_step is None:
        return None
    return per_step, launches


def copy_calibration() -> int:
    """One elementwise kernel over 2^28 fp32 per dispatch (1 GiB in, 1 GiB out):
    the known-size reference that FETCH_SIZE / WRITE_SIZE are scaled by."""
    import torch

    x = torch.empty(COPY_FLOATS, dtype=torch.float32, device="cuda:0").fill_(1.0)
    y = torch.empty_like(x)
    for _ in range(3):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": COPY_FLOATS * 4,
                      "copy_calibration_bytes_written": COPY_FLOATS * 4, "dispatches": 3}), flush=True)
    return 0


def cpu_baseline(w, img, gpu_pred, threads_all, n1=16, nall=None):
    import oracle
    import vdttfs

    c = oracle.Consts.from_task(w.consts)
    rmode = oracle.READ_ARGMAX if w.readout == vdttfs.READOUT_ARGMAX else oracle.READ_ARGMIN

    def run(n, thr):
        t0 = time.perf_counter()
        r = oracle.net_forward(c, w.layers, n, img[:n], w.img_elems, oracle.ENC_LINEAR, w.tc_in,
                               w.td_in, rmode, same_pad=bool(w.consts.conv_same_pad), nthreads=thr)
        return time.perf_counter() - t0, r

    # bounded sample, ~10-20 s of CPU work in all: n1 images on 1 thread and
    # the whole batch on every thread the box grants
    n1 = min(n1, len(gpu_pred))
    run(1, 1)  # warm-up (page-in, OpenMP pool)
    dt1, r1 = run(n1, 1)
    nall = len(gpu_pred) if nall is None else min(nall, len(gpu_pred))
    dta, ra = run(nall, threads_all)
    match = bool(np.array_equal(ra["pred"], gpu_pred[:nall]) and np.array_equal(r1["pred"], gpu_pred[:n1]))
    return {
        "value": nall / dta,
        "unit": "images/s",
        "cores": threads_all,
        "kind": "port",
        "sample": f"{nall} images of the batch, whole network, {threads_all} OpenMP threads "
                  f"({dta:.2f} s); 1 thread on the first {n1} images: {n1 / dt1:.3f} images/s",
        "single_thread_value": n1 / dt1,
        "pred_match_gpu": match,
    }


def threads_all() -> int:
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def bench_culif(args) -> int:
    """Config 4: 7-layer CuLIF SNN on a synthetic 2x128x128 event stream."""
    import vdttfs
    from vdttfs import models

    B = args.batch or 64
    w = models.culif7(delta=args.delta or 32)
    T, D = w.consts.T, w.consts.delta
    ev = models.dvs_events(w, B)
    ctx = vdttfs.Context(w.consts, 0)
    net = vdttfs.CulifNet(ctx, w.layers, B)
    d_ev = ctx.to_device(ev)
    d_pred = ctx.empty(B, np.int32)
    log(f"bench: {w.name} B={B} T={T} delta={D} params={w.n_params}")
    for _ in range(args.warmup):
        net.forward(d_ev, d_pred)
    ctx.synchronize()
    net.read_timing()
    net.set_timing(True)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        net.forward(d_ev, d_pred)
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    net.set_timing(False)
    ms_layers, _ = net.read_timing()
    ms_layers = ms_layers / args.steps
    gpu_pred = d_pred.download()
    eproc, ebin, n_ev, n_cols = net.count(d_ev)
    OS = T // D + 1
    conv = [i for i, l in enumerate(w.layers) if l.kind == vdttfs.CULIF_CONV]
    b_conv = 0
    for i in conv:
        l = w.layers[i]
        n_out = B * l.H_in * l.W_in * l.C_out
        # fused form: the dense input map is read by bucketize, the rest is B_int
        b_conv += (4 * int(eproc[i]) + 8 * int(n_ev[i]) + 4 * OS * int(n_cols[i]) + 4 * l.C_out
                   + 4 * n_out + 4 * int(n_cols[i]) * l.C_in)
    conv_ms = float(sum(ms_layers[i] for i in conv))
    achieved = b_conv / (conv_ms * 1e-3) / 1e9
    l0 = w.layers[0]
    raw_bytes = B * l0.C_in * l0.H_in * l0.W_in * T * 4 + B * l0.C_out * l0.H_in * l0.W_in * 4
    ms_step = elapsed * 1000.0 / args.steps
    out = {
        "metric": f"samples/sec/GPU for CuLIF-7 DVS bs={B}; conv integrator % of HBM peak",
        "value": B / (ms_step * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: moving Gaussian blob events (sigma 12 px, density 0.03), Kaiming-normal "
                "weights (random init)",
        "config": {"workload": "CuLIF-7 SNN, config 4 (2x128x128 events, conv 64/128/128, "
                               "recurrent FC 131072-128, FC 128-11)",
                   "batch": B, "T": T, "delta": D, "decay": w.meta["decay"], "th": w.meta["th"],
                   "seed": w.seed, "parallelism": "none (one GPU)"},
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": None,
            "kernel": "conv layers after conv1 (C_in <= 64: k_merge_dense + k_stream<CuLIF>; "
                      "wider: k_bucketize + k_merge + k_stream<CuLIF>); achieved = fused "
                      "algorithmic bytes of those layers / their HIP-event time",
            "algorithmic_bytes_per_step": b_conv,
            "conv_ms_per_step": conv_ms,
        },
        "layers_ms": [round(float(x), 4) for x in ms_layers],
        "conv1_raw_dense_GBps": raw_bytes / (float(ms_layers[0]) * 1e-3) / 1e9,
        "eproc_per_sample": float(eproc.sum()) / B,
        "ebin_per_sample": float(ebin.sum()) / B,
    }
    if not args.no_cpu:
        import oracle

        thr = threads_all()

        def run(n, t):
            t0 = time.perf_counter()
            _, pred = oracle.culif_net_forward(w.layers, ev[:n], n, T, D, t)
            return time.perf_counter() - t0, pred

        run(1, thr)  # warm-up
        dt1, p1 = run(1, 1)
        nall = min(8, B)
        dta, pa = run(nall, thr)
        out["cpu_baseline"] = {
            "value": nall / dta, "unit": "samples/s", "cores": thr, "kind": "port",
            "sample": f"{nall} samples, whole network, {thr} OpenMP threads ({dta:.2f} s); "
                      f"1 thread on 1 sample: {1.0 / dt1:.3f} samples/s",
            "single_thread_value": 1.0 / dt1,
            "pred_match_gpu": bool(np.array_equal(pa, gpu_pred[:nall]) and p1[0] == gpu_pred[0]),
        }
        out["x_cpu_all_cores"] = out["value"] / out["cpu_baseline"]["value"]
    d_ev.free()
    d_pred.free()
    net.close()
    ctx.close()
    print(json.dumps(out), flush=True)
    return 0


def bench_fc_sweep(args) -> int:
    """Config 5: one FC 4096->4096 layer at B=512 over spike density, the
    truncated window T' and delta.  Every point times one whole layer call
    (bucketize + merge + stream) with HIP events on the library's stream."""
    import vdttfs
    from vdttfs import models

    B = args.batch or 512
    cin = cout = 4096
    layer = models.fc_sweep_layer()
    dens = (0.01, 0.05, 0.2, 0.5)
    spikes = {d: models.fc_sweep_spikes(5, B, cin, d) for d in dens}
    reps = max(1, min(args.steps, 10))
    rows = []
    for Tp in (16, 32, 64):
        for D in (8, 16, 32):
            tc = vdttfs.TaskConsts(T=Tp, tfs=0.0, delta=D, alpha_by_time=False)
            ctx = vdttfs.Context(tc, 0)
            alpha, theta = vdttfs.build_luts_host(tc, 16.0, 0.0, 16.0, 0.0)
            d_W, d_b = ctx.to_device(layer.kernel), ctx.to_device(layer.bias)
            d_a, d_t = ctx.to_device(alpha), ctx.to_device(theta)
            d_out = ctx.empty(B * cout)
            OS = tc.num_chunks + 1
            for d in dens:
                sp = spikes[d]
                d_in = ctx.to_device(sp)
                call = lambda cnt=False: ctx.layer_forward(d_out, d_in, d_W, d_b, d_a, d_t, 0, B, 1, 1,  # noqa: E731
                                                           cin, 1, 1, cout, 1, 1, True, count=cnt)
                call()
                ctx.synchronize()
                ctx.timer_begin()
                for _ in range(reps):
                    call()
                ms = ctx.timer_end() / reps
                eproc, ebin = call(True)
                n_ev = int(np.count_nonzero(sp < Tp))
                b_int = 4 * eproc + 8 * n_ev + 4 * OS * B + 4 * cout + 4 * B * cout
                b_fused = b_int + 4 * B * cin
                gbs = b_fused / (ms * 1e-3) / 1e9
                rows.append({"density": d, "retained_density": n_ev / (B * cin), "T_window": Tp,
                             "delta": D, "ms": ms, "achieved_GBps": gbs, "frac": gbs / HBM_PEAK_GBS,
                             "eproc": int(eproc), "ebin": int(ebin),
                             "skip_rate": 1.0 - eproc / max(1, n_ev * cout),
                             "skip_rate_per_bin": 1.0 - ebin / max(1, n_ev * cout)})
                d_in.free()
            for x in (d_W, d_b, d_a, d_t, d_out):
                x.free()
            ctx.close()
    head = next(r for r in rows if r["density"] == 0.05 and r["T_window"] == 64 and r["delta"] == 16)
    out = {
        "metric": f"integrator GB/s, FC 4096x4096 bs={B} (config 5 sweep; value at density 5%, T'=64, delta=16)",
        "value": head["achieved_GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": reps,
        "warmup": 1,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: per (image, input) active with the given density, time uniform in "
                "[0,64); Gaussian N(0, 2/4096) weights",
        "config": {"workload": "FC 4096x4096 integrator sweep, config 5", "batch": B,
                   "parallelism": "none (one GPU)"},
        "roofline": {"bound": "hbm", "achieved": head["achieved_GBps"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["frac"], "traffic": None,
                     "kernel": "one layer call = bucketize + k_merge + k_stream; fused algorithmic "
                               "bytes B_int + 4*N_cols*C_in"},
        "sweep": rows,
    }
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="vgg16",
                    choices=["vgg16", "lenet5", "culif7", "fc-sweep", "vgg16-timedriven", "lenet5-timedriven",
                             "culif7-timedriven"])
    ap.add_argument("--batch", type=int, default=None,
                    help="default: 256 (vgg16), 1024 (lenet5), 64 (culif7), 512 (fc-sweep)")
    ap.add_argument("--delta", type=int, default=None,
                    help="default: 8 (vgg16), 16 (lenet5), 32 (culif7)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--plans", default=None,
                    help="vgg16/lenet5: per-layer launch plans written by python -m vdttfs.tune --out "
                         "(default: the library's built-in choice)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only the known-size copy used to scale FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (every image "
              f"is independent, so N GPUs would each run this same per-GPU batch)", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration()
    if args.plans and args.workload not in ("vgg16", "lenet5"):
        print(f"--plans applies to the vgg16 and lenet5 engine workloads, not {args.workload}", file=sys.stderr)
        return 2
    if args.workload == "culif7":
        return bench_culif(args)
    if args.workload == "fc-sweep":
        return bench_fc_sweep(args)
    if args.workload.endswith("-timedriven"):
        return bench_timedriven(args)
    return bench_ttfs(args)


def bench_timedriven(args) -> int:
    """The reference's GPU denominator on the same configs: the step-by-step
    (time-driven) network of T1S (LeNet-5, config 2) or T2S (VGG-16, config
    3; layer d integrates at t - (d-1)*TFS and fires at t - d*TFS), one
    thread per neuron per step, against the event-driven engine on the same
    images in the same process.  The two are different neuron models (the
    baseline sums a step's spiking weights, then scales by the step's decay),
    so predictions are compared, not required to match."""
    import vdttfs
    from vdttfs import models

    if args.workload.startswith("culif7"):
        return bench_timedriven_culif(args)
    vgg = args.workload.startswith("vgg16")
    B = args.batch or (256 if vgg else 1024)
    w = models.vgg16(delta=args.delta or 8) if vgg else models.lenet5(delta=args.delta or 16)
    mode = vdttfs.STEP_T2 if vgg else vdttfs.STEP_T1
    img = models.images_for(w, B)
    ctx = vdttfs.Context(w.consts, 0)
    d_img = ctx.to_device(img)
    d_pred = ctx.empty(B, np.int32)
    steps = max(1, min(args.steps, 3))
    sn = vdttfs.StepNet(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in, mode)
    log(f"bench: {w.name} time-driven ({'T2S' if vgg else 'T1S'}) B={B}, {steps} timed forwards")
    sn.forward(d_img, d_pred)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        sn.forward(d_img, d_pred)
    ctx.synchronize()
    ms_td = (time.perf_counter() - t0) * 1000.0 / steps
    _, n_steps = sn.output()
    pred_td = d_pred.download()
    sn.close()
    net = vdttfs.Net(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)
    for _ in range(3):
        net.forward(d_img, d_pred)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        net.forward(d_img, d_pred)
    ctx.synchronize()
    ms_ev = (time.perf_counter() - t0) * 1000.0 / 20
    pred_ev = d_pred.download()
    net.close()
    ctx.close()
    name = "VGG-16" if vgg else "LeNet-5"
    out = {
        "metric": f"images/sec/GPU for {name} time-driven (step-by-step) baseline bs={B}",
        "value": B / (ms_td * 1e-3),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": ms_td,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: the same seeded images and random-init weights as the event-driven workload",
        "config": {"workload": f"{name} time-driven baseline ({'T2S' if vgg else 'T1S'} semantics)",
                   "batch": B, "T": w.consts.T, "tfs": w.consts.tfs, "global_steps": n_steps,
                   "parallelism": "none (one GPU)"},
        "event_driven_images_per_s": B / (ms_ev * 1e-3),
        "event_driven_ms_per_step": ms_ev,
        "speedup_event_driven": ms_td / ms_ev,
        "prediction_agreement": float(np.mean(pred_td == pred_ev)),
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_timedriven_culif(args) -> int:
    """Config 4's denominator: the step-by-step CuLIF network of T3S (every
    layer dense at every step, fire-once CuIF neurons), against the
    event-driven CuLIF engine on the same event tensor in the same process.
    Both run the same neuron; only fp32 summation order differs (T3S sums a
    conv over c_in outermost), so predictions agree up to threshold ties."""
    import vdttfs
    from vdttfs import models

    B = args.batch or 64
    w = models.culif7(delta=args.delta or 32)
    ev = models.dvs_events(w, B)
    ctx = vdttfs.Context(w.consts, 0)
    d_ev = ctx.to_device(ev)
    d_pred = ctx.empty(B, np.int32)
    steps = max(1, min(args.steps, 3))
    sn = vdttfs.CulifStepNet(ctx, w.layers, B)
    log(f"bench: {w.name} time-driven (T3S) B={B} T={w.consts.T}, {steps} timed forwards")
    sn.forward(d_ev, d_pred)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        sn.forward(d_ev, d_pred)
    ctx.synchronize()
    ms_td = (time.perf_counter() - t0) * 1000.0 / steps
    pred_td = d_pred.download()
    sn.close()
    net = vdttfs.CulifNet(ctx, w.layers, B)
    for _ in range(3):
        net.forward(d_ev, d_pred)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        net.forward(d_ev, d_pred)
    ctx.synchronize()
    ms_ev = (time.perf_counter() - t0) * 1000.0 / 20
    pred_ev = d_pred.download()
    net.close()
    ctx.close()
    out = {
        "metric": f"samples/sec/GPU for the CuLIF-7 time-driven (step-by-step) baseline bs={B}",
        "value": B / (ms_td * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": ms_td,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: the same event tensor and random-init weights as the culif7 workload",
        "config": {"workload": "CuLIF-7 time-driven baseline (T3S semantics), config 4",
                   "batch": B, "T": w.consts.T, "global_steps": w.consts.T, "parallelism": "none (one GPU)"},
        "event_driven_samples_per_s": B / (ms_ev * 1e-3),
        "event_driven_ms_per_step": ms_ev,
        "speedup_event_driven": ms_td / ms_ev,
        "prediction_agreement": float(np.mean(pred_td == pred_ev)),
    }
    print(json.dumps(out), flush=True)
    return 0


def bench_ttfs(args) -> int:
    """Configs 3 (VGG-16, the headline) and 2 (LeNet-5)."""
    import vdttfs
    from vdttfs import models

    vgg = args.workload == "vgg16"
    B = args.batch or (256 if vgg else 1024)
    if vgg:
        w = models.vgg16(delta=args.delta or 8)
        metric = METRIC
        workload = "VGG-16 TTFS-SNN, config 3 (3x32x32, 13 conv + FC 512-512-10)"
    else:
        w = models.lenet5(delta=args.delta or 16)
        metric = f"images/sec/GPU for LeNet-5 TTFS bs={B}; integrator % of HBM peak"
        workload = "LeNet-5 TTFS-SNN, config 2 (1x28x28, conv 6/16 + FC 256-120-84-10)"
    img = models.images_for(w, B)
    ctx = vdttfs.Context(w.consts, 0)
    net = vdttfs.Net(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)
    if args.plans:
        from vdttfs import tune
        tune.apply_plans(net, tune.load_plans(args.plans, w, B))
    d_img = ctx.to_device(img)
    d_pred = ctx.empty(B, np.int32)
    log(f"bench: {w.name} B={B} T={w.consts.T} delta={w.consts.delta} tfs={w.consts.tfs} "
        f"params={w.n_params} plans={args.plans or 'built-in'}")

    for _ in range(args.warmup):
        net.forward(d_img, d_pred)
    ctx.synchronize()
    net.read_timing()  # reset

    net.set_timing(True)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        net.forward(d_img, d_pred)
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    net.set_timing(False)
    integ_ms, integ_n, bkt_ms, bkt_n = net.read_timing()
    layer_ms = net.read_layer_timing() / args.steps
    gpu_pred = d_pred.download()

    eproc, ebin, n_ev, n_cols = net.count(d_img)
    b_int, per_layer = algorithmic_bytes(w, eproc, n_ev, n_cols, B)
    ms_step = elapsed * 1000.0 / args.steps
    # a layer's whole integrate: the bucketize pass (FC layers) + merge + stream
    integ_ms_step = (integ_ms + bkt_ms) / args.steps
    launches_per_step = integ_n / args.steps
    achieved = b_int / (integ_ms_step * 1e-3) / 1e9
    key = workload_key(B, w.consts) if vgg else f"{w.name} B={B} T={w.consts.T} delta={w.consts.delta}"
    tr = measured_traffic(key)
    dense = 0
    for l in w.layers:
        if l.kind == 0:
            dense += B * l.H_out * l.W_out * l.C_out * l.K_h * l.K_w * l.C_in
        elif l.kind == 1:
            dense += B * l.C_out * l.H_in * l.W_in * l.C_in
    out = {
        "metric": metric,
        "value": B / (ms_step * 1e-3),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded splitmix64 U[0,1) images, Kaiming-normal weights (random init)",
        "config": {"workload": workload,
                   "key": key,
                   "batch": B, "T": w.consts.T, "delta": w.consts.delta, "tfs": w.consts.tfs,
                   "seed": w.seed, "parallelism": "none (one GPU)",
                   "plans": os.path.relpath(args.plans, ROOT) if args.plans else "built-in"},
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": (tr[0] / tr[1]) if tr else None,
            "kernel": "integrator = a layer's k_stream_dense (conv, C_in <= 64, 32 <= C_out <= 64: "
                      "list built in LDS), k_merge_dense + k_stream (other conv, C_in <= 64) or "
                      "k_bucketize + k_merge + k_stream (wider conv, FC); layers with C_out < 32 "
                      "stream with k_stream_narrow, or with k_conv_small (no list) when the receptive "
                      "field has <= 32 elements; a launch is one layer's integrate, achieved = "
                      "fused algorithmic bytes of a step / integrator time of a step",
            "algorithmic_bytes_per_step": b_int,
            "algorithmic_bytes_per_launch": b_int / max(launches_per_step, 1),
            "traffic_per_step": tr[0] if tr else None,
            "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if tr else None,
            "integrator_ms_per_step": integ_ms_step,
            "integrator_launches_per_step": launches_per_step,
        },
        "bucketize_ms_per_step": bkt_ms / args.steps,
        "layers_ms": {str(i): round(float(v), 4) for i, v in enumerate(layer_ms) if v > 0},
        "eproc_per_image": float(eproc.sum()) / B,
        "ebin_per_image": float(ebin.sum()) / B,
        "dense_macs_per_image": dense / B,
        "retained_events_per_image": float(n_ev.sum()) / B,
    }
    if not args.no_cpu:
        thr = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        cb = cpu_baseline(w, img, gpu_pred, thr, n1=16 if vgg else 256)
        out["cpu_baseline"] = cb
        out["x_cpu_all_cores"] = out["value"] / cb["value"]
    net.close()
    ctx.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
