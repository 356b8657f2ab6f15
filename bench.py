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
    """B_int per integrating layer: 4*E_proc (one fp32 weight per integrated
    synapse) + 8*N_ev (event lists) + 4*OS*N_cols (chunk offsets)
    + 4*C_out (bias) + 4*N_out (first-spike write)."""
    OS = w.consts.num_chunks + 1
    total = 0
    per_layer = []
    for i, l in enumerate(w.layers):
        if l.kind not in (0, 1):
            per_layer.append(0)
            continue
        n_out = B * l.H_out * l.W_out * l.C_out
        b = 4 * int(eproc[i]) + 8 * int(n_ev[i]) + 4 * OS * int(n_cols[i]) + 4 * l.C_out + 4 * n_out
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


def cpu_baseline(w, img, gpu_pred, threads_all):
    import oracle

    c = oracle.Consts.from_task(w.consts)

    def run(n, thr):
        t0 = time.perf_counter()
        r = oracle.net_forward(c, w.layers, n, img[:n], w.img_elems, oracle.ENC_LINEAR, w.tc_in,
                               w.td_in, oracle.READ_ARGMAX, same_pad=True, nthreads=thr)
        return time.perf_counter() - t0, r

    # bounded sample, ~10-20 s of CPU work in all: 16 images on 1 thread and
    # the whole batch on every thread the box grants
    n1 = min(16, len(gpu_pred))
    run(1, 1)  # warm-up (page-in, OpenMP pool)
    dt1, r1 = run(n1, 1)
    nall = len(gpu_pred)
    dta, ra = run(nall, threads_all)
    match = bool(np.array_equal(ra["pred"], gpu_pred[:nall]) and np.array_equal(r1["pred"], gpu_pred[:n1]))
    return {
        "value": nall / dta,
        "unit": "images/s",
        "cores": threads_all,
        "kind": "port",
        "sample": f"{nall} images (the whole batch), whole network, {threads_all} OpenMP threads "
                  f"({dta:.2f} s); 1 thread on the first {n1} images: {n1 / dt1:.3f} images/s",
        "single_thread_value": n1 / dt1,
        "pred_match_gpu": match,
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--delta", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only the known-size copy used to scale FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (every image "
              f"is independent, so N GPUs would each run this same per-GPU batch)", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration()

    import vdttfs
    from vdttfs import models

    B = args.batch
    w = models.vgg16(delta=args.delta)
    img = models.images_for(w, B)
    ctx = vdttfs.Context(w.consts, 0)
    net = vdttfs.Net(ctx, w.layers, B, w.img_elems, vdttfs.ENCODE_LINEAR, w.tc_in, w.td_in, w.readout)
    d_img = ctx.to_device(img)
    d_pred = ctx.empty(B, np.int32)
    log(f"bench: VGG-16 TTFS B={B} T={w.consts.T} delta={w.consts.delta} tfs={w.consts.tfs} "
        f"params={w.n_params}")

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
    gpu_pred = d_pred.download()

    eproc, ebin, n_ev, n_cols = net.count(d_img)
    b_int, per_layer = algorithmic_bytes(w, eproc, n_ev, n_cols, B)
    ms_step = elapsed * 1000.0 / args.steps
    integ_ms_step = integ_ms / args.steps
    launches_per_step = integ_n / args.steps
    achieved = b_int / (integ_ms_step * 1e-3) / 1e9
    key = workload_key(B, w.consts)
    tr = measured_traffic(key)
    dense = 0
    for l in w.layers:
        if l.kind == 0:
            dense += B * l.H_out * l.W_out * l.C_out * l.K_h * l.K_w * l.C_in
        elif l.kind == 1:
            dense += B * l.C_out * l.H_in * l.W_in * l.C_in
    out = {
        "metric": METRIC,
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
        "config": {"workload": "VGG-16 TTFS-SNN, config 3 (3x32x32, 13 conv + FC 512-512-10)",
                   "key": key,
                   "batch": B, "T": w.consts.T, "delta": w.consts.delta, "tfs": w.consts.tfs,
                   "seed": w.seed, "parallelism": "none (one GPU)"},
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": (tr[0] / tr[1]) if tr else None,
            "kernel": "integrator = k_merge + k_stream per integrating layer; a launch is one layer's "
                      "pair, achieved = algorithmic bytes of a step / integrator time of a step",
            "algorithmic_bytes_per_step": b_int,
            "algorithmic_bytes_per_launch": b_int / max(launches_per_step, 1),
            "traffic_per_step": tr[0] if tr else None,
            "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if tr else None,
            "integrator_ms_per_step": integ_ms_step,
            "integrator_launches_per_step": launches_per_step,
        },
        "bucketize_ms_per_step": bkt_ms / args.steps,
        "eproc_per_image": float(eproc.sum()) / B,
        "ebin_per_image": float(ebin.sum()) / B,
        "dense_macs_per_image": dense / B,
        "retained_events_per_image": float(n_ev.sum()) / B,
    }
    if not args.no_cpu:
        thr = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
        cb = cpu_baseline(w, img, gpu_pred, thr)
        out["cpu_baseline"] = cb
        out["x_cpu_all_cores"] = out["value"] / cb["value"]
    net.close()
    ctx.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
