"""The synthetic workloads the engine is measured on (seeded, deterministic).

Every array comes from the library's counter-mode splitmix64 generator, so
the same (seed, stream, index) always yields the same value and image b of a
batch does not depend on the batch size.

  config 1/2  LeNet-5 TTFS-SNN, T=64, Delta=16, Task-1 semantics (T1V)
  config 3    VGG-16 TTFS-SNN,  T=64, Delta=8, TFS=32, Task-2 semantics (T2V)
  config 4    7-layer CuLIF SNN on a synthetic 2x128x128 event stream (T3V)
  config 5    one FC 4096->4096 layer, spike density / window / Delta sweep

Weights are Kaiming-normal (sigma = sqrt(2/fan_in), fan_in = K_h*K_w*C_in),
biases 0, every layer's fire constants tc_fire = T/4, td = 0, and the input
encoding constants tc_in = T/4, td_in = 0, threshold theta0 = 1.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from ._lib import Blob, BlobLayer, check, lib
from .core import (CULIF_CONV, CULIF_FC, CULIF_FC_REC, CULIF_POOL, CULIF_RAW_CONV, LAYER_CONV,
                   LAYER_FC, LAYER_POOL, LAYER_VMEM, READOUT_ARGMAX, READOUT_ARGMIN, CulifLayerSpec,
                   Layer, TaskConsts, task3_consts)

STREAM_IMG = 1
STREAM_IMG_VALUE = 2
STREAM_WEIGHT0 = 1000


def uniform(seed: int, stream: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib().vdttfs_synth_uniform(seed, stream, C.c_void_p(out.ctypes.data), n))
    return out


def normal(seed: int, stream: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib().vdttfs_synth_normal(seed, stream, C.c_void_p(out.ctypes.data), n, sigma))
    return out


def kaiming(seed: int, layer_index: int, shape, fan_in: int) -> np.ndarray:
    n = int(np.prod(shape))
    return normal(seed, STREAM_WEIGHT0 + layer_index, n, math.sqrt(2.0 / fan_in)).reshape(shape)


@dataclass
class Workload:
    name: str
    consts: TaskConsts
    layers: list
    img_shape: tuple          # (H, W, C) of one image, NHWC
    readout: int
    tc_in: float
    td_in: float
    seed: int
    meta: dict = field(default_factory=dict)

    @property
    def img_elems(self) -> int:
        return int(np.prod(self.img_shape))

    @property
    def n_params(self) -> int:
        return int(sum((l.kernel.size + l.bias.size) for l in self.layers if l.kernel is not None))


def _conv(seed, idx, H, W, cin, cout, k, same, tc, td=0.0):
    ho = H if same else H - k + 1
    wo = W if same else W - k + 1
    kern = kaiming(seed, idx, (k, k, cin, cout), k * k * cin)
    return Layer(LAYER_CONV, H, W, cin, ho, wo, cout, k, k, kern, np.zeros(cout, np.float32), tc, td)


def _fc(seed, idx, cin, cout, tc, td=0.0, vmem=False, H=1, W=1, C=None):
    Cc = cin if C is None else C
    kern = kaiming(seed, idx, (cin, cout), cin)
    return Layer(LAYER_VMEM if vmem else LAYER_FC, H, W, Cc, 1, 1, cout, 1, 1, kern,
                 np.zeros(cout, np.float32), tc, td)


def _pool(H, W, Cc):
    return Layer(LAYER_POOL, H, W, Cc, H // 2, W // 2, Cc)


def write_weights_blob(path: str, layers) -> int:
    """Writes the integrating layers (conv, FC, vmem readout) of a layer list
    in the reference's weights format (the save side of WIO1:31-70, read back
    by vdttfs_blob_read / the drivers): conv kernels HWIO, FC kernels
    [C_in][C_out], one bias per output, one tc_fire and one td float.
    Returns the number of layers written."""
    integ = [l for l in layers if l.kernel is not None]
    arr = (BlobLayer * len(integ))()
    keep = []
    fp = C.POINTER(C.c_float)
    for i, l in enumerate(integ):
        k = np.ascontiguousarray(l.kernel, np.float32).ravel()
        b = np.ascontiguousarray(l.bias, np.float32).ravel()
        keep += [k, b]
        if l.kind == LAYER_CONV:
            shape = (l.K_h, l.K_w, l.C_in, l.C_out)
        else:
            shape = (l.H_in * l.W_in * l.C_in, l.C_out)
        if k.size != int(np.prod(shape)) or b.size != l.C_out:
            raise ValueError(f"layer {i}: kernel/bias sizes do not match {shape}")
        e = arr[i]
        e.ndim = len(shape)
        for j, v in enumerate(shape):
            e.shape[j] = v
        e.kernel_elems = k.size
        e.kernel = k.ctypes.data_as(fp)
        e.bias_ndim = 1
        e.bias_size = b.size
        e.bias = b.ctypes.data_as(fp)
        e.tc_ndim = 1
        e.td_ndim = 1
        e.tc_fire = l.tc_fire
        e.td = l.td
    blob = Blob(len(integ), arr)
    check(lib().vdttfs_blob_write(path.encode(), C.byref(blob)))
    return len(integ)


def lenet5(seed: int = 1, T: int = 64, delta: int = 16) -> Workload:
    """Configs 1/2: conv 6@5x5 -> pool2 -> conv 16@5x5 -> pool2 -> FC 256-120-84-10."""
    tc = T / 4.0
    consts = TaskConsts(T=T, tfs=0.0, delta=delta, vth=1.0, alpha_by_time=False,
                        conv_same_pad=False)
    L = [
        _conv(seed, 0, 28, 28, 1, 6, 5, False, tc),
        _pool(24, 24, 6),
        _conv(seed, 1, 12, 12, 6, 16, 5, False, tc),
        _pool(8, 8, 16),
        _fc(seed, 2, 256, 120, tc, H=4, W=4, C=16),
        _fc(seed, 3, 120, 84, tc),
        _fc(seed, 4, 84, 10, tc),
    ]
    return Workload("lenet5-ttfs", consts, L, (28, 28, 1), READOUT_ARGMIN, tc, 0.0, seed)


VGG16_PLAN = [64, 64, "M", 128, 128, "M", 256, 256, 256, "M", 512, 512, 512, "M", 512, 512, 512, "M"]


def vgg16(seed: int = 3, T: int = 64, delta: int = 8, tfs: float | None = None,
          fc_hidden: int = 1) -> Workload:
    """Config 3: VGG-16 on 3x32x32, FC 512->512 (x fc_hidden) -> 512->10 vmem readout.

    TIME_FIRE_START is not stated by the config; T/2 keeps the reference's
    TFS/T ratio (40/80, T2V:12-13)."""
    tc = T / 4.0
    tfs = T / 2.0 if tfs is None else tfs
    consts = TaskConsts(T=T, tfs=tfs, delta=delta, vth=1.0, alpha_by_time=True, conv_same_pad=True)
    L = []
    H = W = 32
    cin = 3
    idx = 0
    for v in VGG16_PLAN:
        if v == "M":
            L.append(_pool(H, W, cin))
            H //= 2
            W //= 2
        else:
            L.append(_conv(seed, idx, H, W, cin, v, 3, True, tc))
            idx += 1
            cin = v
    for _ in range(fc_hidden):
        L.append(_fc(seed, idx, 512, 512, tc))
        idx += 1
    L.append(_fc(seed, idx, 512, 10, tc, vmem=True))
    return Workload("vgg16-ttfs", consts, L, (32, 32, 3), READOUT_ARGMAX, tc, 0.0, seed,
                    meta={"tfs": tfs, "fc_hidden": fc_hidden})


def lenet5_images(seed: int, B: int) -> np.ndarray:
    """Per pixel: 0 with p=0.8, else x = 1-u (u in [0,1))."""
    n = B * 28 * 28
    z = uniform(seed, STREAM_IMG, n)
    v = 1.0 - uniform(seed, STREAM_IMG_VALUE, n)
    return np.where(z < np.float32(0.8), np.float32(0.0), v).astype(np.float32).reshape(B, 28, 28, 1)


def vgg_images(seed: int, B: int) -> np.ndarray:
    """Per pixel and channel x = u in [0,1)."""
    return uniform(seed, STREAM_IMG, B * 32 * 32 * 3).reshape(B, 32, 32, 3)


def images_for(w: Workload, B: int) -> np.ndarray:
    if w.name.startswith("lenet"):
        return lenet5_images(w.seed, B)
    return vgg_images(w.seed, B)


# ---- config 5: FC roofline sweep ------------------------------------------
def fc_sweep_layer(seed: int = 5, cin: int = 4096, cout: int = 4096, T: int = 64) -> Layer:
    return _fc(seed, 0, cin, cout, T / 4.0)


def fc_sweep_spikes(seed: int, B: int, cin: int, density: float, T: int = 64) -> np.ndarray:
    """Spike times: active with probability `density`, time uniform integer in [0,T)."""
    n = B * cin
    act = uniform(seed, STREAM_IMG, n) < np.float32(density)
    t = np.floor(uniform(seed, STREAM_IMG_VALUE, n) * np.float32(T)).astype(np.float32)
    return np.where(act, t, np.float32(9999.0)).astype(np.float32).reshape(B, cin)


# ---- config 4: CuLIF on a synthetic event stream (T3V) ----------------------
@dataclass
class CulifWorkload:
    name: str
    consts: TaskConsts
    layers: list              # CulifLayerSpec
    in_shape: tuple           # (C, H, W) of one sample; events are [C][H][W][T]
    n_classes: int
    seed: int
    meta: dict = field(default_factory=dict)

    @property
    def n_params(self) -> int:
        return int(sum((0 if l.weight is None else l.weight.size) +
                       (0 if l.weight_rec is None else l.weight_rec.size) for l in self.layers))


def culif7(seed: int = 4, T: int = 64, delta: int = 32, H: int = 128, W: int = 128,
           n_classes: int = 11, decay: float = 0.5, th: float = 1.0) -> CulifWorkload:
    """Config 4, T3V's topology (T3V:276-289) at 2xHxW input:
    conv 2->64 (raw events) -> conv 64->128 -> pool -> conv 128->128 -> pool
    -> recurrent FC 128*(H/4)*(W/4) -> 128 -> FC 128 -> n_classes.
    One decay and threshold for every layer; Kaiming-normal OIHW / [out][in]
    weights (recurrent weights fan_in 128)."""
    consts = task3_consts(T=T, delta=delta)
    h2, w2 = H // 4, W // 4
    F = 128 * h2 * w2
    L = [
        CulifLayerSpec(CULIF_RAW_CONV, 2, H, W, 64, kaiming(seed, 0, (64, 2, 3, 3), 2 * 9), None, decay, th),
        CulifLayerSpec(CULIF_CONV, 64, H, W, 128, kaiming(seed, 1, (128, 64, 3, 3), 64 * 9), None, decay, th),
        CulifLayerSpec(CULIF_POOL, 128, H, W, 128, None, None, decay, th),
        CulifLayerSpec(CULIF_CONV, 128, H // 2, W // 2, 128, kaiming(seed, 2, (128, 128, 3, 3), 128 * 9),
                       None, decay, th),
        CulifLayerSpec(CULIF_POOL, 128, H // 2, W // 2, 128, None, None, decay, th),
        CulifLayerSpec(CULIF_FC_REC, F, 1, 1, 128, kaiming(seed, 3, (128, F), F),
                       kaiming(seed, 4, (128, 128), 128), decay, th),
        CulifLayerSpec(CULIF_FC, 128, 1, 1, n_classes, kaiming(seed, 5, (n_classes, 128), 128), None,
                       decay, th),
    ]
    return CulifWorkload("culif7-dvs", consts, L, (2, H, W), n_classes, seed,
                         meta={"decay": decay, "th": th, "density": 0.03, "sigma_px": 12.0,
                               "vmax_px_per_step": 0.5})


def dvs_events(w: CulifWorkload, B: int) -> np.ndarray:
    """[B][C][H][W][T] in {0,1}: a Gaussian blob (sigma 12 px) moving linearly
    at up to 0.5 px/step per axis, Bernoulli events with mean density 0.03."""
    Cc, H, W = w.in_shape
    T = w.consts.T
    out = np.empty((B, Cc, H, W, T), np.float32)
    check(lib().vdttfs_synth_dvs(w.seed, B, Cc, H, W, T, w.meta["density"], w.meta["sigma_px"],
                                 w.meta["vmax_px_per_step"], C.c_void_p(out.ctypes.data), None))
    return out
