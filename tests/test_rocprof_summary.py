"""The counter summary that bench.py's roofline.traffic comes from: synthetic
rocprofv3 CSV files in, the machine-readable lines out, read back by
bench.measured_traffic -- which must accept only the workload key (and build)
the counters were taken for."""
import csv
import os

import pytest

import bench
from vdttfs import rocprof_summary as rs

KIB = 1024.0


def write_counters(d, name, counter, dispatches):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, f"{name}_counter_collection.csv"), "w", newline="") as f:
        wr = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
                                           "Start_Timestamp", "End_Timestamp"])
        wr.writeheader()
        for i, (kern, kib) in enumerate(dispatches):
            wr.writerow({"Dispatch_Id": i + 1, "Kernel_Name": f"void vdttfs::(anonymous namespace)::{kern}(args)",
                         "Counter_Name": counter, "Counter_Value": kib, "Start_Timestamp": 10 * i,
                         "End_Timestamp": 10 * i + 5})


FORWARD = ["k_encode_linear", "k_stream_dense<false, 1, false, 1>", "k_pool_min", "k_merge_dense<9>",
           "k_stream<false, 2, false, 2>", "k_bucketize<true>", "k_merge<1>", "k_stream<false, 1, false, 1>",
           "k_fc_vmem_wave", "k_readout"]
COUNTING = ["k_encode_linear", "k_stream_dense<true, 1, false, 1>", "k_pool_min", "k_bucketize<true>",
            "k_merge_dense<9>", "k_stream<true, 2, false, 2>"]


@pytest.fixture
def runs(tmp_path):
    name = "vgg"
    # two timed forwards, then a counting one (ignored); kernel k of forward f reads (f+1)*(k+1) KiB
    disp = []
    for f in range(2):
        disp += [(k, (f + 1) * (j + 1)) for j, k in enumerate(FORWARD)]
    disp += [(k, 1000.0) for k in COUNTING]
    write_counters(tmp_path / "f", name, "FETCH_SIZE", disp)
    write_counters(tmp_path / "w", name, "WRITE_SIZE", [(k, 2 * v) for k, v in disp])
    # the copy: FETCH_SIZE counts half the known bytes (scale 2), WRITE_SIZE all of them
    write_counters(tmp_path / "cf", name, "FETCH_SIZE", [("k_neg", (1 << 30) / 2 / KIB)])
    write_counters(tmp_path / "cw", name, "WRITE_SIZE", [("k_neg", (1 << 30) / KIB)])
    return tmp_path, name


def test_traffic_lines_and_bench_reader(runs, monkeypatch):
    d, name = runs
    key = "vgg16 B=256 T=64 delta=8 tfs=32 plans=built-in src=0123456789"
    text = rs.traffic(str(d / "f"), str(d / "w"), str(d / "cf"), str(d / "cw"), name, workload=key)
    assert f"WORKLOAD={key}" in text
    # the last timed forward (f = 1): kernel j reads 2 (j + 1) KiB, scaled x2; writes twice that, scaled x1
    integ = [j for j, k in enumerate(FORWARD) if k.startswith(rs.INTEGRATOR)]
    fetch = {j: 2 * (j + 1) * KIB * 2 for j in integ}
    write = {j: 4 * (j + 1) * KIB for j in integ}
    layers = [[1], [3, 4], [5, 6, 7]]  # stream_dense; merge_dense + stream; bucketize + merge + stream
    p = d / "integrator_x_traffic.md"
    p.write_text("# summary\n\n```\n" + text + "\n```\n")
    monkeypatch.setattr(bench, "traffic_file", lambda tag: str(p))
    tr = bench.measured_traffic("x", key)
    assert tr is not None
    assert tr["launches"] == 3
    assert tr["per_step"] == pytest.approx(sum(fetch.values()) + sum(write.values()), rel=1e-6)
    for (fb, wb), js in zip(tr["layers"], layers):
        assert fb == pytest.approx(sum(fetch[j] for j in js), rel=1e-6)
        assert wb == pytest.approx(sum(write[j] for j in js), rel=1e-6)
    # another configuration or build of the kernels: not used
    assert bench.measured_traffic("x", key.replace("src=0123456789", "src=fffffffff0")) is None
    assert bench.measured_traffic("x", key.replace("B=256", "B=128")) is None


def test_fc_layer_calls_split_at_bucketize(runs, tmp_path):
    """Config 5's layer calls have no encoder: a call starts at k_bucketize."""
    name = "fc"
    calls = [("k_bucketize<true>", 1), ("k_merge<1>", 2), ("k_stream<false, 4, false, 1>", 3)] * 3
    calls += [("k_bucketize<true>", 50), ("k_merge<1>", 50), ("k_stream<true, 4, false, 1>", 50)]
    write_counters(tmp_path / "ff", name, "FETCH_SIZE", calls)
    write_counters(tmp_path / "fw", name, "WRITE_SIZE", calls)
    d, cname = runs
    for sub in ("cf", "cw"):
        src = d / sub / f"{cname}_counter_collection.csv"
        (tmp_path / sub).mkdir(exist_ok=True)
        (tmp_path / sub / f"{name}_counter_collection.csv").write_text(src.read_text())
    text = rs.traffic(str(tmp_path / "ff"), str(tmp_path / "fw"), str(tmp_path / "cf"), str(tmp_path / "cw"),
                      name, workload="fc", first="k_bucketize")
    line = [x for x in text.splitlines() if x.startswith("TRAFFIC_PER_STEP_BYTES=")][0]
    kv = dict(t.split("=") for t in line.split())
    assert int(kv["LAUNCHES_PER_STEP"]) == 1
    assert float(kv["TRAFFIC_PER_STEP_BYTES"]) == pytest.approx((1 + 2 + 3) * KIB * 2 + (1 + 2 + 3) * KIB, rel=1e-6)


def write_multi(d, name, rows):
    """rows: (dispatch id, kernel, {counter: value}, duration)"""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, f"{name}_counter_collection.csv"), "w", newline="") as f:
        wr = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
                                           "Start_Timestamp", "End_Timestamp"])
        wr.writeheader()
        t = 0
        for i, kern, cnt, dur in rows:
            for c, v in cnt.items():
                wr.writerow({"Dispatch_Id": i, "Kernel_Name": f"void vdttfs::(anonymous namespace)::{kern}(args)",
                             "Counter_Name": c, "Counter_Value": v, "Start_Timestamp": t,
                             "End_Timestamp": t + dur})
            t += dur + 10


def test_counters_merges_runs(tmp_path):
    """Per-wave counts from two runs over the same program, each divided by
    its own run's SQ_WAVES; derived percentages weighted by duration; the
    counting kernels left out."""
    k = "k_stream_quad<4, 9, false>"
    write_multi(tmp_path / "occ", "x", [
        (1, k, {"SQ_WAVES": 100, "SQ_INSTS_LDS": 400, "SQ_LDS_BANK_CONFLICT": 100, "SQ_INSTS_VMEM_RD": 900,
                "OccupancyPercent": 50.0}, 1000),
        (2, k, {"SQ_WAVES": 100, "SQ_INSTS_LDS": 400, "SQ_LDS_BANK_CONFLICT": 100, "SQ_INSTS_VMEM_RD": 900,
                "OccupancyPercent": 80.0}, 3000),
        (3, "k_stream<true, 1, false, 1>", {"SQ_WAVES": 7, "SQ_INSTS_LDS": 1, "OccupancyPercent": 1.0}, 9000)])
    write_multi(tmp_path / "mix", "x", [
        (1, k, {"SQ_WAVES": 50, "SQ_INSTS_VALU": 1000, "SQ_INSTS_SALU": 500, "VALUBusy": 90.0, "SALUBusy": 30.0}, 2000),
        (2, k, {"SQ_WAVES": 50, "SQ_INSTS_VALU": 1000, "SQ_INSTS_SALU": 500, "VALUBusy": 100.0, "SALUBusy": 50.0},
         2000)])
    out = rs.counters([(str(tmp_path / "occ"), "x"), (str(tmp_path / "mix"), "x")])
    lines = out.splitlines()
    head = [h.strip() for h in lines[0].strip("|").split("|")]
    assert head == ["kernel", "dispatches", "us", "waves", "VALU/wave", "SALU/wave", "LDS/wave", "gathers/wave",
                    "bank conflicts/LDS instr", "VALU busy %", "SALU busy %", "occupancy % of 32 waves/CU"]
    assert len(lines) == 3  # header, rule, one kernel (the counting kernel is left out)
    row = [c.strip() for c in lines[2].strip("|").split("|")]
    assert row[0] == k and row[1] == "2"
    assert float(row[2]) == pytest.approx(4.0)  # us, from the first run's timestamps (ns)
    assert row[3] == "200"
    assert float(row[4]) == pytest.approx(20.0)   # 2000 VALU / 100 waves of the mix run
    assert float(row[5]) == pytest.approx(10.0)
    assert float(row[6]) == pytest.approx(4.0)    # 800 LDS / 200 waves of the occupancy run
    assert float(row[7]) == pytest.approx(9.0)
    assert float(row[8]) == pytest.approx(0.25)
    assert float(row[9]) == pytest.approx(95.0)   # equal durations
    assert float(row[10]) == pytest.approx(40.0)
    assert float(row[11]) == pytest.approx(72.5)  # (50 * 1 + 80 * 3) / 4
