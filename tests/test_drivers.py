"""The per-task drivers (vd-ttfs_amd/bin/vdttfs_{lenet,vgg,dvs}, the analogues
of the reference mains T1V:242, T2V:289, T3V:234) end to end on the
reference's asset formats: a synthetic weights blob and dataset are written
in those formats with labels set to the oracle's predictions, so a driver
that parses the files, builds the topology and runs the engine correctly
reports exactly 100% (and the expected fraction once labels are altered).
Missing or malformed assets must end the run as the reference does (a
message and exit status 1) before any GPU work."""
import os
import re
import subprocess

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import models

BIN = os.path.join(os.path.dirname(vdttfs.LIB_PATH), "bin")


def drv(name):
    p = os.path.join(BIN, name)
    if not os.path.exists(p):
        pytest.fail(f"{p} is not built (make -C vd-ttfs_amd)")
    return p


def run(args, timeout=600):
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout)
    return r.returncode, r.stdout + r.stderr


def onehot(pred, n_cls, dtype=np.float32):
    y = np.zeros((len(pred), n_cls), dtype)
    for i, p in enumerate(pred):
        if p >= 0:
            y[i, p] = 1
    return y


def write_images(d, imgs):
    os.makedirs(d, exist_ok=True)
    for i, im in enumerate(imgs):
        np.ascontiguousarray(im, np.float32).tofile(os.path.join(d, f"{i}.bin"))


# ------------------------------------------------------------------ CPU
def test_drivers_fail_cleanly_without_assets(tmp_path):
    for name in ("vdttfs_lenet", "vdttfs_vgg", "vdttfs_dvs"):
        rc, out = run([drv(name), "--weights", str(tmp_path / "missing.bin")])
        assert rc == 1, out
        assert "not found" in out.lower() or "cannot open" in out.lower(), out


def test_lenet_driver_rejects_bad_topology_and_missing_images(tmp_path):
    w = models.lenet5()
    wp = str(tmp_path / "w.bin")
    # an FC layer first: 784 inputs expected, the kernel says 256
    models.write_weights_blob(wp, [w.layers[4]])
    rc, out = run([drv("vdttfs_lenet"), "--weights", wp, "--data", str(tmp_path), "--n", "1"])
    assert rc == 1 and "inputs" in out, out
    models.write_weights_blob(wp, w.layers)
    rc, out = run([drv("vdttfs_lenet"), "--weights", wp, "--data", str(tmp_path), "--n", "2"])
    assert rc == 1 and "0.bin" in out, out


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_lenet_driver_end_to_end(tmp_path):
    w = models.lenet5()
    N = 100
    img = models.images_for(w, N)
    r = oracle.net_forward(oracle.Consts.from_task(w.consts), w.layers, N, img, w.img_elems,
                           oracle.ENC_LINEAR, w.tc_in, w.td_in, oracle.READ_ARGMIN)
    wp = str(tmp_path / "snn_weights.bin")
    models.write_weights_blob(wp, w.layers)
    d = str(tmp_path / "mnist")
    write_images(d, img.reshape(N, 784))
    lab = onehot(r["pred"], 10)
    lab.tofile(os.path.join(d, "label_onehot"))
    args = [drv("vdttfs_lenet"), "--weights", wp, "--data", d, "--n", str(N), "--batch", "40",
            "--T", "64", "--delta", "16", "--encode", "linear", "--tc-in", str(w.tc_in),
            "--td-in", str(w.td_in)]
    rc, out = run(args)
    assert rc == 0, out
    assert re.search(r"Images Processed:\s+100", out), out
    assert re.search(r"Final Accuracy:\s+100%", out), out
    # 25 labels moved to another class (or to "none"): 75%
    bad = lab.copy()
    for i in range(25):
        bad[i] = np.roll(bad[i], 1) if bad[i].any() else np.eye(10, dtype=np.float32)[0]
    bad.tofile(os.path.join(d, "label_onehot"))
    rc, out = run(args)
    assert rc == 0 and re.search(r"Final Accuracy:\s+75%", out), out


@pytest.mark.gpu
def test_vgg_driver_end_to_end(tmp_path):
    w = models.vgg16()
    N = 24
    img = models.images_for(w, N)
    r = oracle.net_forward(oracle.Consts.from_task(w.consts), w.layers, N, img, w.img_elems,
                           oracle.ENC_LINEAR, w.tc_in, w.td_in, oracle.READ_ARGMAX, same_pad=True)
    wp = str(tmp_path / "snn_weights_vgg.bin")
    assert models.write_weights_blob(wp, w.layers) == 15
    d = str(tmp_path / "cifar")
    write_images(d, img.reshape(N, 3072))  # HWC per image
    onehot(r["pred"], 10).tofile(os.path.join(d, "label_onehot"))
    rc, out = run([drv("vdttfs_vgg"), "--weights", wp, "--data", d, "--n", str(N), "--batch", "10",
                   "--T", "64", "--tfs", "32", "--delta", "8", "--encode", "linear",
                   "--tc-in", str(w.tc_in), "--td-in", str(w.td_in)])
    assert rc == 0, out
    assert out.count("-> Batch [") == 3, out
    assert re.search(r"Final Accuracy:\s+100%", out), out
    # T2V's loop call for call on the drop-in entry points (update_luts,
    # launch_layer_sync, launch_pool_sync, launch_fc_vmem_sync, host argmax),
    # twice: the same classes, and one LAYER_MS line per layer
    rc, out = run([drv("vdttfs_vgg"), "--weights", wp, "--data", d, "--n", str(N), "--batch", "10",
                   "--T", "64", "--tfs", "32", "--delta", "8", "--encode", "linear",
                   "--tc-in", str(w.tc_in), "--td-in", str(w.td_in), "--dropin", "--reps", "2"])
    assert rc == 0, out
    assert out.count("-> Batch [") == 6, out
    assert len(re.findall(r"Final Accuracy:\s+100%", out)) == 2, out
    assert len(re.findall(r"^LAYER_MS i=\d+ kind=\w+ lut_ms=\S+ launch_ms=\S+$", out, re.M)) == len(w.layers), out


@pytest.mark.gpu
def test_dvs_driver_end_to_end(tmp_path):
    w = models.culif7(H=32, W=32, n_classes=10)
    N = 6
    ev = models.dvs_events(w, N)
    _, pred = oracle.culif_net_forward(w.layers, ev, N, w.consts.T, w.consts.delta)
    # the reference's flat weights file: conv1, conv2, conv3, fc1_rec, fc1, fc2
    L = w.layers
    flat = np.concatenate([L[0].weight.ravel(), L[1].weight.ravel(), L[3].weight.ravel(),
                           L[5].weight_rec.ravel(), L[5].weight.ravel(), L[6].weight.ravel()])
    wp = str(tmp_path / "dvsgesture_weights.bin")
    flat.astype(np.float32).tofile(wp)
    dp, lp = str(tmp_path / "train_data.bin"), str(tmp_path / "train_labels.bin")
    ev.tofile(dp)
    onehot(pred, 10, np.int32).tofile(lp)
    rc, out = run([drv("vdttfs_dvs"), "--weights", wp, "--data", dp, "--labels", lp, "--n", str(N),
                   "--batch", "4", "--T", "64", "--delta", "32", "--decay-conv", "0.5",
                   "--th-conv", "1", "--decay-fc", "0.5", "--th-fc", "1"])
    assert rc == 0, out
    assert re.search(r"Accuracy:\s+100\.00 %", out), out
