"""Host-side tests of libvdttfs.so that need no GPU: exported symbols, the
weights-blob format (T1V:185-206, WIO:1-13) and its failure cases, the
synthetic generator and the host LUT builder."""
import ctypes as C
import os
import re
import struct
import subprocess

import numpy as np
import pytest

import oracle
import vdttfs
from vdttfs import _lib, models

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "vdttfs.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(vdttfs_[a-z0-9_]+)\s*\(", src)))


def test_python_constants_match_the_header():
    """Every integer #define VDTTFS_X of the header that the Python mirror
    names X carries the same value there (paths, layer kinds, encoders,
    readouts, step modes, pool-fusion modes, error codes)."""
    src = open(os.path.join(ROOT, "include", "vdttfs.h")).read()
    defs = dict((k, int(v)) for k, v in re.findall(r"#define\s+VDTTFS_(\w+)\s+(-?\d+)\b", src))
    shared = [k for k in defs if hasattr(_lib, k)]
    assert len(shared) >= 20, shared
    for k in shared:
        assert getattr(_lib, k) == defs[k], k
    for k in ("POOL_FUSE_OFF", "POOL_FUSE_ALL", "POOL_FUSE_AUTO", "PATH_FUSED", "PATH_WINDOW"):
        assert k in shared


def test_library_exports_every_declared_symbol():
    syms = header_symbols()
    assert len(syms) >= 40
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(vdttfs_\w+)", out))
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    L = vdttfs.lib()
    for s in syms:
        assert hasattr(L, s)
    assert set(syms) <= set(_lib.SIGNATURES), set(syms) - set(_lib.SIGNATURES)


def test_no_gpu_create_fails_cleanly():
    if vdttfs.device_count() > 0:
        pytest.skip("a device is visible here")
    with pytest.raises(vdttfs.VdttfsError) as e:
        vdttfs.Context(vdttfs.task1_consts(), 0)
    assert e.value.code == _lib.E_NODEVICE


def test_bad_consts_rejected():
    L = vdttfs.lib()
    for bad in (_lib.Consts(0, 0, 1, 1, 0, 0), _lib.Consts(64, 0, 0, 1, 0, 0),
                _lib.Consts(64, 0, 257, 1, 0, 0), _lib.Consts(300, 0, 8, 1, 0, 0)):
        a = np.empty(400, np.float32)
        rc = L.vdttfs_build_luts_host(C.byref(bad), 16, 0, 16, 0, C.c_void_p(a.ctypes.data),
                                      C.c_void_p(a.ctypes.data))
        assert rc == _lib.E_INVALID


def test_host_luts_bit_identical_to_oracle():
    for (T, tci, tdi, tcf, tdf) in [(64, 16, 0, 16, 0), (80, 34.75016403198242, 0, 17.3, 2.5),
                                    (80, 17.452274, 0.0, 9.0, 40.0)]:
        tc = vdttfs.TaskConsts(T=T, delta=8)
        a, t = vdttfs.build_luts_host(tc, tci, tdi, tcf, tdf)
        oa, ot = oracle.build_luts(T, 1.0, tci, tdi, tcf, tdf)
        np.testing.assert_array_equal(a, oa)
        np.testing.assert_array_equal(t, ot)


# ------------------------------------------------------------------ blob
def write_blob_by_spec(path, layers):
    """Hand-rolled writer from the format text (WIO:1-13), independent of the library."""
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(layers)))
        for shape, kern, bias, tc, td in layers:
            f.write(struct.pack("<i", len(shape)))
            f.write(struct.pack(f"<{len(shape)}i", *shape))
            f.write(np.asarray(kern, "<f4").tobytes())
            f.write(struct.pack("<ii", 1, len(bias)))
            f.write(np.asarray(bias, "<f4").tobytes())
            f.write(struct.pack("<iif", 1, 1, tc))
            f.write(struct.pack("<iif", 1, 1, td))


def read_blob(path):
    L = vdttfs.lib()
    p = C.POINTER(_lib.Blob)()
    rc = L.vdttfs_blob_read(path.encode(), C.byref(p))
    if rc != 0:
        return rc, None
    b = p.contents
    out = []
    for i in range(b.num_layers):
        l = b.layers[i]
        k = np.ctypeslib.as_array(l.kernel, shape=(l.kernel_elems,)).copy()
        bi = np.ctypeslib.as_array(l.bias, shape=(l.bias_size,)).copy()
        out.append(dict(ndim=l.ndim, shape=list(l.shape)[:l.ndim], k_h=l.k_h, k_w=l.k_w,
                        c_in=l.c_in, c_out=l.c_out, kernel=k, bias=bi, tc=l.tc_fire, td=l.td))
    L.vdttfs_blob_free(p)
    return 0, out


def sample_layers():
    rng = np.random.default_rng(0)
    return [
        ([3, 3, 2, 4], rng.standard_normal(72).astype(np.float32), rng.standard_normal(4).astype(np.float32), 16.5, 0.25),
        ([8, 5], rng.standard_normal(40).astype(np.float32), rng.standard_normal(5).astype(np.float32), 9.0, 40.0),
    ]


def test_blob_read_matches_spec(tmp_path):
    p = str(tmp_path / "w.bin")
    layers = sample_layers()
    write_blob_by_spec(p, layers)
    rc, got = read_blob(p)
    assert rc == 0 and len(got) == 2
    assert (got[0]["k_h"], got[0]["k_w"], got[0]["c_in"], got[0]["c_out"]) == (3, 3, 2, 4)
    assert (got[1]["k_h"], got[1]["k_w"], got[1]["c_in"], got[1]["c_out"]) == (1, 1, 8, 5)
    for g, (shape, k, b, tc, td) in zip(got, layers):
        assert g["shape"] == shape
        np.testing.assert_array_equal(g["kernel"], k)
        np.testing.assert_array_equal(g["bias"], b)
        assert g["tc"] == np.float32(tc) and g["td"] == np.float32(td)


def test_blob_write_roundtrip(tmp_path):
    p1, p2 = str(tmp_path / "a.bin"), str(tmp_path / "b.bin")
    write_blob_by_spec(p1, sample_layers())
    L = vdttfs.lib()
    blob = C.POINTER(_lib.Blob)()
    assert L.vdttfs_blob_read(p1.encode(), C.byref(blob)) == 0
    assert L.vdttfs_blob_write(p2.encode(), blob) == 0
    L.vdttfs_blob_free(blob)
    assert open(p1, "rb").read() == open(p2, "rb").read()


@pytest.mark.parametrize("mutate,code", [
    ("truncate", _lib.E_FORMAT), ("trailing", _lib.E_FORMAT), ("ndim3", _lib.E_FORMAT),
    ("tcsize2", _lib.E_FORMAT), ("biasmismatch", _lib.E_FORMAT), ("zerodim", _lib.E_FORMAT),
    ("missing", _lib.E_IO), ("nolayers", _lib.E_FORMAT)])
def test_blob_malformed(tmp_path, mutate, code):
    p = str(tmp_path / "w.bin")
    layers = sample_layers()
    write_blob_by_spec(p, layers)
    raw = bytearray(open(p, "rb").read())
    if mutate == "truncate":
        raw = raw[:-3]
    elif mutate == "trailing":
        raw += b"\0"
    elif mutate == "ndim3":
        raw[4:8] = struct.pack("<i", 3)
    elif mutate == "zerodim":
        raw[8:12] = struct.pack("<i", 0)
    elif mutate == "nolayers":
        raw[0:4] = struct.pack("<i", 0)
    elif mutate in ("tcsize2", "biasmismatch"):
        # layer 0 tail: kernel at 4+4+16+72*4, then bias header
        boff = 4 + 4 + 16 + 72 * 4
        if mutate == "biasmismatch":
            raw[boff + 4: boff + 8] = struct.pack("<i", 3)
        else:
            tcoff = boff + 8 + 4 * 4
            raw[tcoff + 4: tcoff + 8] = struct.pack("<i", 2)
    if mutate == "missing":
        p = str(tmp_path / "nope.bin")
    else:
        open(p, "wb").write(bytes(raw))
    rc, _ = read_blob(p)
    assert rc == code
    assert vdttfs.last_error()


# ------------------------------------------------------------------ synth
def test_synth_deterministic_and_prefix_stable():
    a = models.uniform(9, 1, 1000)
    b = models.uniform(9, 1, 4000)[:1000]
    np.testing.assert_array_equal(a, b)
    assert a.min() >= 0.0 and a.max() < 1.0
    assert not np.array_equal(a, models.uniform(9, 2, 1000))
    n = models.normal(9, 3, 200001, 2.0)
    assert abs(float(n.mean())) < 0.02 and abs(float(n.std()) - 2.0) < 0.02
    # config 1 is image 0 of config 2's batch
    np.testing.assert_array_equal(models.lenet5_images(1, 1)[0], models.lenet5_images(1, 1024)[0])


def test_workloads_shapes():
    v = models.vgg16()
    assert len([l for l in v.layers if l.kind == vdttfs.LAYER_CONV]) == 13
    assert len([l for l in v.layers if l.kind == vdttfs.LAYER_POOL]) == 5
    assert 14.9e6 < v.n_params < 15.1e6
    le = models.lenet5()
    assert [l.C_out for l in le.layers] == [6, 6, 16, 16, 120, 84, 10]
    x = models.lenet5_images(1, 64)
    assert 0.75 < float((x == 0).mean()) < 0.85
