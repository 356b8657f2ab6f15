"""Summaries of rocprofv3 CSV output for the VGG-16 benchmark.

Reads the files that ``rocprofv3 --output-format csv -d DIR -o NAME`` writes
(``NAME_kernel_stats.csv``, ``NAME_kernel_trace.csv``,
``NAME_counter_collection.csv``) and prints short markdown tables:

  python -m vdttfs.rocprof_summary stats   DIR NAME            # --kernel-trace --stats
  python -m vdttfs.rocprof_summary layers  DIR NAME            # one forward, per layer
  python -m vdttfs.rocprof_summary traffic FETCH_DIR WRITE_DIR CFETCH_DIR CWRITE_DIR NAME \
         [--workload KEY] [--first PREFIX] [--copy-name NAME]
  python -m vdttfs.rocprof_summary counters DIR NAME [DIR NAME ...]  # instruction mix, occupancy, LDS conflicts
  python -m vdttfs.rocprof_summary per-wave DIR NAME [PREFIX]  # every counter per wave, per dispatch

``traffic`` takes four counter runs: FETCH_SIZE and WRITE_SIZE over the
benchmark, and the same two counters over ``bench.py --copy-calibration``
(an elementwise copy of a known number of bytes).  Each counter is scaled by
known_bytes / counted_bytes of the copy, then summed over the integrator
dispatches (bucketize + merge + stream, the fused or register kernels, or the
generic integrator) of one non-counting forward, per integrating layer and in
total.  A forward starts at a dispatch whose name begins with PREFIX
(default ``k_encode``: the engine's encoder; the config-5 layer call starts
at ``k_bucketize``, the CuLIF network at ``k_culif_event_masks``).  The last
lines are machine-readable: ``WORKLOAD=KEY`` (the bench.py configuration the
counters belong to), one ``LAYER_TRAFFIC`` line per integrating layer, and
``TRAFFIC_PER_STEP_BYTES``, which bench.py reports as ``roofline.traffic``
when its own configuration key equals KEY.  --copy-name is the -o name of the
calibration runs when it differs from NAME.
"""
from __future__ import annotations

import collections
import csv
import os
import re
import sys

# every kernel of a layer's integrate: bucketize (FC layers), merge, stream
INTEGRATOR = ("k_bucketize", "k_merge", "k_stream", "k_integrate_generic", "k_conv_small")
# the dispatch that ends a layer's integrate (lists, if any, come before it)
LAYER_END = ("k_stream", "k_integrate_generic", "k_conv_small")
COPY_BYTES_DEFAULT = 1 << 30  # bench.py --copy-calibration moves 2^28 floats each way


def short_name(n: str) -> str:
    m = re.search(r"(k_\w+(<[\w, -]+>)?)", n)
    if m:
        return m.group(1)
    return n.split("(")[0][-48:]


def _csv(d: str, name: str, kind: str):
    p = os.path.join(d, f"{name}_{kind}.csv")
    with open(p, newline="") as f:
        return list(csv.DictReader(f))


def stats(d: str, name: str) -> str:
    rows = _csv(d, name, "kernel_stats")
    out = ["| kernel | calls | avg us | total ms | % |", "|---|---:|---:|---:|---:|"]
    for r in rows:
        out.append("| %s | %s | %.1f | %.3f | %s |" % (
            short_name(r["Name"]), r["Calls"], float(r["AverageNs"]) / 1e3,
            float(r["TotalDurationNs"]) / 1e6, r["Percentage"]))
    return "\n".join(out)


def _forwards(rows, key_start="Start_Timestamp", first="k_encode"):
    """Split dispatches (sorted by start) into forwards; each starts with a
    dispatch named `first...` (the engine's encoder by default)."""
    rows = sorted(rows, key=lambda r: int(r[key_start]))
    fw, cur = [], None
    for r in rows:
        n = short_name(r["Kernel_Name"])
        if n.startswith(first) and (cur is None or first != "k_bucketize" or any(
                short_name(q["Kernel_Name"]).startswith(LAYER_END) for q in cur)):
            cur = []
            fw.append(cur)
        if cur is not None:
            cur.append(r)
    return fw


_COUNTING = re.compile(r"^(k_stream(_dense|_narrow)?<true|k_integrate_generic<\w+, \d+, true>)")


def _is_counting(forward) -> bool:
    """A forward run with the E_proc counters on (net.count), not a timed one;
    or a stretch between two encoder dispatches with no integrating layer (an
    encode on its own, as bench.py runs to read the first layer's input)."""
    return (any(_COUNTING.match(short_name(r["Kernel_Name"])) for r in forward) or
            not any(short_name(r["Kernel_Name"]).startswith(LAYER_END) for r in forward))


def layers(d: str, name: str) -> str:
    fw = [f for f in _forwards(_csv(d, name, "kernel_trace")) if not _is_counting(f)]
    if not fw:
        return "no forward found"
    f = fw[-1]
    out = ["| # | kernel | grid | us |", "|---:|---|---:|---:|"]
    tot = integ = 0.0
    for i, r in enumerate(f):
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        n = short_name(r["Kernel_Name"])
        tot += us
        if n.startswith(INTEGRATOR):
            integ += us
        out.append("| %d | %s | %s | %.1f |" % (i, n, r["Grid_Size_X"], us))
    out.append("")
    out.append("kernel time of the last non-counting forward: %.1f us, of which integrator "
               "(bucketize + merge + stream) %.1f us" % (tot, integ))
    return "\n".join(out)


def _per_dispatch(d: str, name: str, counter: str):
    """{dispatch id: (kernel name, KiB)} for one counter, forward-grouped."""
    rows = [r for r in _csv(d, name, "counter_collection") if r["Counter_Name"] == counter]
    agg = collections.OrderedDict()
    for r in rows:  # one row per dispatch (and per dimension, summed here)
        k = int(r["Dispatch_Id"])
        if k not in agg:
            agg[k] = dict(r)
            agg[k]["_v"] = 0.0
        agg[k]["_v"] += float(r["Counter_Value"])
    return list(agg.values())


def _copy_factor(d: str, name: str, counter: str, known: int) -> float:
    disp = _per_dispatch(d, name, counter)
    big = max(disp, key=lambda r: r["_v"])
    return known / (big["_v"] * 1024.0)


def traffic(fdir: str, wdir: str, cfdir: str, cwdir: str, name: str, workload: str = "",
            first: str = "k_encode", copy_name: str = "", copy_bytes: int = COPY_BYTES_DEFAULT) -> str:
    ff = _copy_factor(cfdir, copy_name or name, "FETCH_SIZE", copy_bytes)
    wf = _copy_factor(cwdir, copy_name or name, "WRITE_SIZE", copy_bytes)
    lines = [f"copy calibration ({copy_bytes} B read + {copy_bytes} B written per dispatch): "
             f"FETCH_SIZE scale {ff:.4f}, WRITE_SIZE scale {wf:.4f}", ""]
    res = {}
    for counter, d, scale in (("FETCH_SIZE", fdir, ff), ("WRITE_SIZE", wdir, wf)):
        disp = _per_dispatch(d, name, counter)
        fw = [f for f in _forwards(disp, key_start="Dispatch_Id", first=first) if not _is_counting(f)]
        f = fw[-1]
        per = [(short_name(r["Kernel_Name"]), r["_v"] * 1024.0 * scale) for r in f]
        res[counter] = per
    lines.append("| # | kernel | FETCH bytes | WRITE bytes |")
    lines.append("|---:|---|---:|---:|")
    tf = tw = 0.0
    layer_f = layer_w = 0.0
    layers = []
    for i, ((n, fb), (_, wb)) in enumerate(zip(res["FETCH_SIZE"], res["WRITE_SIZE"])):
        lines.append("| %d | %s | %.4g | %.4g |" % (i, n, fb, wb))
        if n.startswith(INTEGRATOR):
            tf += fb
            tw += wb
            layer_f += fb
            layer_w += wb
            if n.startswith(LAYER_END):
                layers.append((layer_f, layer_w))
                layer_f = layer_w = 0.0
    lines.append("")
    lines.append(f"integrator (bucketize + merge + stream) per forward: FETCH {tf:.6g} B, WRITE {tw:.6g} B, "
                 f"{len(layers)} integrating layers")
    lines.append(f"WORKLOAD={workload}")
    for i, (fb, wb) in enumerate(layers):
        lines.append(f"LAYER_TRAFFIC n={i} fetch={fb:.0f} write={wb:.0f}")
    lines.append(f"TRAFFIC_PER_STEP_BYTES={tf + tw:.0f} LAUNCHES_PER_STEP={len(layers)} "
                 f"FETCH_SCALE={ff:.5f} WRITE_SCALE={wf:.5f}")
    return "\n".join(lines)


# derived percentages rocprofv3 computes per dispatch (averaged over a
# kernel's dispatches, weighted by duration)
_PERCENT = (("VALUBusy", "VALU busy %"), ("SALUBusy", "SALU busy %"),
            ("OccupancyPercent", "occupancy % of 32 waves/CU"))


def counters(runs) -> str:
    """Per kernel (non-counting dispatches, summed over each run): waves,
    instructions per wave (VALU, SALU, LDS, vector-memory reads; whichever
    the runs collected), LDS bank conflicts per LDS instruction, and
    rocprofv3's derived percentages where collected, weighted by dispatch
    duration: VALUBusy and SALUBusy (100 * SQ_ACTIVE_INST_VALU or
    SQ_INST_CYCLES_SALU / CU_NUM / GRBM_GUI_ACTIVE: the share of the
    dispatch's cycles in which a CU's vector or scalar ALUs were busy) and
    OccupancyPercent (400 *
    SQ_WAVE_CYCLES / GRBM_GUI_ACTIVE / CU_NUM / 32: resident waves as a
    share of 32 per CU).  `runs` is a list of (DIR, NAME) pairs of counter
    runs over the same program; each counter is divided by SQ_WAVES of its
    own run, and the durations shown are those of the first run."""
    agg = collections.OrderedDict()
    for ri, (d, name) in enumerate(runs):
        by = collections.OrderedDict()
        for r in _csv(d, name, "counter_collection"):
            k = int(r["Dispatch_Id"])
            e = by.setdefault(k, {"name": short_name(r["Kernel_Name"]),
                                  "dur": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        for e in by.values():
            n = e["name"]
            if _COUNTING.match(n):
                continue
            a = agg.setdefault(n, collections.defaultdict(float))
            if ri == 0:
                a["dispatches"] += 1
                a["dur"] += e["dur"]
            a["waves%d" % ri] += e.get("SQ_WAVES", 0.0)
            for c, v in e.items():
                if c.startswith("SQ_") and c != "SQ_WAVES":
                    a[c] += v
                    a["run_of_" + c] = ri
            for c, _ in _PERCENT:
                if c in e:
                    a[c] += e[c] * e["dur"]
                    a[c + "_dur"] += e["dur"]
    have = set(c for a in agg.values() for c in a)
    per_wave_cols = [(c, h) for c, h in (("SQ_INSTS_VALU", "VALU"), ("SQ_INSTS_SALU", "SALU"),
                                         ("SQ_INSTS_LDS", "LDS"), ("SQ_INSTS_VMEM_RD", "gathers"))
                     if c in have]
    pct_cols = [(c, h) for c, h in _PERCENT if c in have]
    head = ["kernel", "dispatches", "us", "waves"] + ["%s/wave" % h for _, h in per_wave_cols]
    if "SQ_LDS_BANK_CONFLICT" in have:
        head.append("bank conflicts/LDS instr")
    head += [h for _, h in pct_cols]
    out = ["| " + " | ".join(head) + " |", "|---|" + "---:|" * (len(head) - 1)]
    for n, a in sorted(agg.items(), key=lambda kv: -kv[1]["dur"]):
        row = [n, "%d" % a["dispatches"], "%.1f" % a["dur"], "%d" % a["waves0"]]
        for c, _ in per_wave_cols:
            w = a["waves%d" % int(a.get("run_of_" + c, 0))]
            row.append("%.1f" % (a[c] / w) if w else "-")
        if "SQ_LDS_BANK_CONFLICT" in have:
            row.append(("%.3f" % (a["SQ_LDS_BANK_CONFLICT"] / a["SQ_INSTS_LDS"])) if a["SQ_INSTS_LDS"] else "-")
        for c, _ in pct_cols:
            row.append(("%.1f" % (a[c] / a[c + "_dur"])) if a[c + "_dur"] else "-")
        out.append("| " + " | ".join(row) + " |")
    return "\n".join(out)


def per_wave(d: str, name: str, first: str = "k_encode") -> str:
    """One row per dispatch of the last non-counting forward: every counter
    of the run divided by the dispatch's SQ_WAVES (so, per wave), and the
    derived OccupancyPercent as is."""
    rows = _csv(d, name, "counter_collection")
    by = collections.OrderedDict()
    for r in rows:
        k = int(r["Dispatch_Id"])
        e = by.setdefault(k, {"Kernel_Name": r["Kernel_Name"], "Dispatch_Id": k,
                              "us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
        e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    fw = [f for f in _forwards(list(by.values()), key_start="Dispatch_Id", first=first) if not _is_counting(f)]
    if not fw:
        return "no forward found"
    f = fw[-1]
    names = [c for c in f[0] if c not in ("Kernel_Name", "Dispatch_Id", "us", "SQ_WAVES")]
    out = ["| # | kernel | us | waves | " + " | ".join(n + ("" if n == "OccupancyPercent" else "/wave") for n in names)
           + " |", "|---:|---|---:|---:|" + "---:|" * len(names)]
    for i, e in enumerate(f):
        w = max(e.get("SQ_WAVES", 0.0), 1.0)
        vals = [("%.1f" % e[n]) if n == "OccupancyPercent" else ("%.1f" % (e[n] / w)) for n in names]
        out.append("| %d | %s | %.1f | %d | %s |" % (i, short_name(e["Kernel_Name"]), e["us"], e.get("SQ_WAVES", 0),
                                                     " | ".join(vals)))
    return "\n".join(out)


def main(argv) -> int:
    if len(argv) < 2:
        print(__doc__)
        return 2
    cmd = argv[1]
    if cmd == "stats":
        print(stats(argv[2], argv[3]))
    elif cmd == "layers":
        print(layers(argv[2], argv[3]))
    elif cmd == "traffic":
        rest = argv[7:]
        opts = dict(zip(rest[::2], rest[1::2]))
        print(traffic(*argv[2:7], workload=opts.get("--workload", ""), first=opts.get("--first", "k_encode"),
                      copy_name=opts.get("--copy-name", "")))
    elif cmd == "counters":
        rest = argv[2:]
        print(counters(list(zip(rest[::2], rest[1::2]))))
    elif cmd == "per-wave":
        print(per_wave(argv[2], argv[3], *argv[4:5]))
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
