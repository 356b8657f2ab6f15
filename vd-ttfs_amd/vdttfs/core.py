"""Python host-side mirror of the reference driver surface over the C ABI.

Function names and argument meaning follow the reference programs
(T1V = task1_lenet_mnist/vdttfs_cuda/snn_timesorted_earlyexit.cu,
 T2V = task2_vgg16_cifar10/vdttfs_cuda/bench_vgg_eventdriven_timesorted_earlyexit.cu):
``update_LUTs``, ``k_bucketize``, ``k_conv_bucketed``, ``k_pooling``,
``k_layer_vmem``, ``launch_layer`` / ``launch_conv`` / ``launch_fc`` ...
Every call runs the HIP kernels of libvdttfs.so; errors raise VdttfsError.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import (Consts, CulifLayer, LayerDesc, VdttfsError, check, lib, INF_TIME,  # noqa: F401
                   LAYER_CONV, LAYER_FC, LAYER_POOL, LAYER_VMEM, ENCODE_LINEAR, ENCODE_LOG, ENCODE_TIMES,
                   READOUT_ARGMIN, READOUT_ARGMAX, CULIF_RAW_CONV, CULIF_CONV, CULIF_POOL,
                   CULIF_FC_REC, CULIF_FC, STEP_T1, STEP_T2, STEP_T3, LayerPlan, PATH_AUTO, PATH_BINS, PATH_DENSE,
                   PATH_FUSED, PATH_REG, PATH_WINDOW, POOL_FUSE_OFF, POOL_FUSE_ALL, POOL_FUSE_AUTO)


def _ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data)


def device_count() -> int:
    n = C.c_int(0)
    check(lib().vdttfs_device_count(C.byref(n)))
    return n.value


@dataclass(frozen=True)
class TaskConsts:
    """The reference's compile-time macros (T1V:12-19, T2V:12-18)."""
    T: int                 # TIME_WINDOW
    tfs: float = 0.0       # TIME_FIRE_START
    delta: int = 16        # CHUNK
    vth: float = 1.0       # VTH_INIT
    alpha_by_time: bool = False  # T2V alpha[clamp((int)t,0,T)] instead of T1V alpha[tb]
    conv_same_pad: bool = False  # T2V same padding instead of T1V valid

    @property
    def num_chunks(self) -> int:
        return (self.T + self.delta - 1) // self.delta

    def to_c(self) -> Consts:
        return Consts(self.T, self.tfs, self.delta, self.vth, int(self.alpha_by_time),
                      int(self.conv_same_pad))


# Task 1 (LeNet, T1V:12-19) and Task 2 (VGG, T2V:12-18) semantics
def task1_consts(T=80, delta=16) -> TaskConsts:
    return TaskConsts(T=T, tfs=0.0, delta=delta, vth=1.0, alpha_by_time=False, conv_same_pad=False)


def task2_consts(T=80, delta=8, tfs=40.0) -> TaskConsts:
    return TaskConsts(T=T, tfs=tfs, delta=delta, vth=1.0, alpha_by_time=True, conv_same_pad=True)


# Task 3 (CuLIF, T3V:17-21): T_TOTAL and CHUNK_SIZE; no fire start, no LUTs
def task3_consts(T=160, delta=32) -> TaskConsts:
    return TaskConsts(T=T, tfs=0.0, delta=delta, vth=1.0, alpha_by_time=False, conv_same_pad=True)


def build_luts_host(consts: TaskConsts, tc_integ, td_integ, tc_fire, td_fire):
    """update_LUTs' tables on the host (T1V:208-216, T2V:236-243)."""
    a = np.empty(consts.T + 1, np.float32)
    t = np.empty(consts.T, np.float32)
    c = consts.to_c()
    check(lib().vdttfs_build_luts_host(C.byref(c), tc_integ, td_integ, tc_fire, td_fire, _ptr(a),
                                       _ptr(t)))
    return a, t


class DeviceArray:
    """A device allocation with a numpy view of its shape/dtype."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().vdttfs_dev_alloc(ctx.handle, self.nbytes, C.byref(p)))
        self.ptr = p

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def upload(self, host: np.ndarray) -> "DeviceArray":
        h = np.ascontiguousarray(host, dtype=self.dtype)
        if h.nbytes != self.nbytes:
            raise ValueError(f"upload of {h.nbytes} bytes into {self.nbytes}-byte buffer")
        check(lib().vdttfs_h2d(self.ctx.handle, self.ptr, _ptr(h), self.nbytes))
        return self

    def download(self) -> np.ndarray:
        h = np.empty(self.shape, self.dtype)
        check(lib().vdttfs_d2h(self.ctx.handle, _ptr(h), self.ptr, self.nbytes))
        return h

    def fill(self, byte_value: int) -> "DeviceArray":
        check(lib().vdttfs_memset(self.ctx.handle, self.ptr, byte_value, self.nbytes))
        return self

    def free(self):
        if self.ptr is not None and self.ptr.value and self.ctx.handle is not None:
            check(lib().vdttfs_dev_free(self.ctx.handle, self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """A device context holding the per-task constants and a HIP stream."""

    def __init__(self, consts: TaskConsts, device: int = 0):
        self.consts = consts
        h = C.c_void_p()
        c = consts.to_c()
        check(lib().vdttfs_create(C.byref(c), device, C.byref(h)))
        self.handle = h

    def close(self):
        if self.handle is not None:
            lib().vdttfs_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- memory ----
    def empty(self, shape, dtype=np.float32) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def to_device(self, host: np.ndarray, dtype=None) -> DeviceArray:
        h = np.ascontiguousarray(host, dtype=dtype or host.dtype)
        return DeviceArray(self, h.shape, h.dtype).upload(h)

    def timer_begin(self):
        """Record a HIP event on the context stream (see timer_end)."""
        check(lib().vdttfs_timer_begin(self.handle))

    def timer_end(self) -> float:
        """Milliseconds on the context stream since timer_begin (HIP events)."""
        ms = C.c_double()
        check(lib().vdttfs_timer_end(self.handle, C.byref(ms)))
        return ms.value

    def synchronize(self):
        check(lib().vdttfs_synchronize(self.handle))

    def probe_gather(self, vec: int, footprint_bytes: int, n_ev: int = 512, waves: int = 32768,
                     reps: int = 5) -> float:
        """Milliseconds per launch of the gather-roof probe (vdttfs_probe_gather)."""
        ms = C.c_double(0.0)
        check(lib().vdttfs_probe_gather(self.handle, vec, footprint_bytes, n_ev, waves, reps, C.byref(ms)))
        return ms.value

    # ---- the reference surface ----
    def update_LUTs(self, d_lut_decay: DeviceArray, d_lut_th: DeviceArray, tc_integ, td_integ,
                    tc_fire, td_fire):
        check(lib().vdttfs_update_luts(self.handle, d_lut_decay.ptr, d_lut_th.ptr, tc_integ,
                                       td_integ, tc_fire, td_fire))

    def encode_image(self, d_img: DeviceArray, d_out: DeviceArray, tc: float, td: float):
        check(lib().vdttfs_encode_image(self.handle, d_img.ptr, d_out.ptr, d_img.size, tc, td))

    def encode_linear(self, d_img: DeviceArray, d_out: DeviceArray):
        check(lib().vdttfs_encode_linear(self.handle, d_img.ptr, d_out.ptr, d_img.size))

    def bucketize(self, d_in: DeviceArray, n_cols: int, c_in: int, d_cin: DeviceArray,
                  d_tin: DeviceArray, d_off: DeviceArray):
        check(lib().vdttfs_bucketize(self.handle, d_in.ptr, n_cols, c_in, d_cin.ptr, d_tin.ptr,
                                     d_off.ptr))

    def integrate(self, d_out, d_cin, d_tin, d_off, d_kernel, d_bias, d_alpha, d_theta, t_min, B,
                  H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, is_fc):
        check(lib().vdttfs_integrate(self.handle, d_out.ptr, d_cin.ptr, d_tin.ptr, d_off.ptr,
                                     d_kernel.ptr, d_bias.ptr, d_alpha.ptr, d_theta.ptr, t_min, B,
                                     H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, int(is_fc)))

    def layer_forward(self, d_out, d_in, d_kernel, d_bias, d_alpha, d_theta, t_min, B, H_in, W_in,
                      C_in, H_out, W_out, C_out, K_h, K_w, is_fc, count=False):
        ep = C.c_uint64(0)
        eb = C.c_uint64(0)
        check(lib().vdttfs_layer_forward(self.handle, d_out.ptr, d_in.ptr, d_kernel.ptr, d_bias.ptr,
                                         d_alpha.ptr, d_theta.ptr, t_min, B, H_in, W_in, C_in,
                                         H_out, W_out, C_out, K_h, K_w, int(is_fc),
                                         C.byref(ep) if count else None,
                                         C.byref(eb) if count else None))
        return (ep.value, eb.value) if count else None

    def layer_forward_noalloc(self, d_out, d_in, d_kernel, d_bias, d_alpha, d_theta, t_min, B, H_in, W_in,
                              C_in, H_out, W_out, C_out, K_h, K_w, is_fc):
        """vdttfs_layer_forward_noalloc: the layer path on the library's static scratch."""
        check(lib().vdttfs_layer_forward_noalloc(self.handle, d_out.ptr, d_in.ptr, d_kernel.ptr, d_bias.ptr,
                                                 d_alpha.ptr, d_theta.ptr, t_min, B, H_in, W_in, C_in, H_out,
                                                 W_out, C_out, K_h, K_w, int(is_fc)))

    def pool_min(self, d_in, d_out, B, H_in, W_in, Cc):
        check(lib().vdttfs_pool_min(self.handle, d_in.ptr, d_out.ptr, B, H_in, W_in, Cc))

    def fc_vmem(self, d_in, d_out, d_kernel, d_bias, d_alpha, B, C_in, C_out):
        check(lib().vdttfs_fc_vmem(self.handle, d_in.ptr, d_out.ptr, d_kernel.ptr, d_bias.ptr,
                                   d_alpha.ptr, B, C_in, C_out))

    def readout(self, d_out, B, Cc, argmax: bool, d_pred):
        fn = lib().vdttfs_readout_argmax if argmax else lib().vdttfs_readout_argmin
        check(fn(self.handle, d_out.ptr, B, Cc, d_pred.ptr))

    # launch wrappers (synchronous, T1V:222-240 / T2V:250-287)
    def launch_layer(self, d_in, d_out, H_in, W_in, C_in, H_out, W_out, C_out, K_h, K_w, td,
                     d_kernel, d_bias, d_alpha, d_theta, B, is_fc):
        check(lib().vdttfs_launch_layer_sync(self.handle, d_in.ptr, d_out.ptr, H_in, W_in, C_in,
                                             H_out, W_out, C_out, K_h, K_w, td, d_kernel.ptr,
                                             d_bias.ptr, d_alpha.ptr, d_theta.ptr, B, int(is_fc)))

    # CuLIF set (T3V:30-225), reference layouts
    def culif_conv1_raw(self, d_data, d_out, d_weight, N, C_in, C_out, H, W, decay, th):
        check(lib().vdttfs_culif_conv1_raw(self.handle, d_data.ptr, d_out.ptr, d_weight.ptr, N, C_in,
                                           C_out, H, W, decay, th))

    def culif_bucketize_conv(self, d_in, N, Cc, H, W, d_cin, d_tin, d_off):
        check(lib().vdttfs_culif_bucketize_conv(self.handle, d_in.ptr, N, Cc, H, W, d_cin.ptr,
                                                d_tin.ptr, d_off.ptr))

    def culif_bucketize_fc(self, d_in, N, F, d_cin, d_tin, d_off):
        check(lib().vdttfs_culif_bucketize_fc(self.handle, d_in.ptr, N, F, d_cin.ptr, d_tin.ptr,
                                              d_off.ptr))

    def culif_conv(self, d_cin, d_tin, d_off, d_out, d_weight, N, C_in, C_out, H, W, decay, th):
        check(lib().vdttfs_culif_conv(self.handle, d_cin.ptr, d_tin.ptr, d_off.ptr, d_out.ptr,
                                      d_weight.ptr, N, C_in, C_out, H, W, decay, th))

    def culif_pool(self, d_in, d_out, N, Cc, H_in, W_in, decay, th):
        check(lib().vdttfs_culif_pool(self.handle, d_in.ptr, d_out.ptr, N, Cc, H_in, W_in, decay, th))

    def culif_fc_recurrent(self, d_cin, d_tin, d_off, d_out, d_w, d_w_rec, N, in_f, out_f, decay, th):
        check(lib().vdttfs_culif_fc_recurrent(self.handle, d_cin.ptr, d_tin.ptr, d_off.ptr, d_out.ptr,
                                              d_w.ptr, d_w_rec.ptr, N, in_f, out_f, decay, th))

    def culif_fc(self, d_cin, d_tin, d_off, d_out, d_w, N, in_f, out_f, decay, th):
        check(lib().vdttfs_culif_fc(self.handle, d_cin.ptr, d_tin.ptr, d_off.ptr, d_out.ptr, d_w.ptr,
                                    N, in_f, out_f, decay, th))

    def readout_argmin_first(self, d_out, B, Cc, d_pred):
        check(lib().vdttfs_readout_argmin_first(self.handle, d_out.ptr, B, Cc, d_pred.ptr))

    def launch_pool(self, d_in, d_out, H_in, W_in, Cc, B):
        check(lib().vdttfs_launch_pool_sync(self.handle, d_in.ptr, d_out.ptr, H_in, W_in, Cc, B))

    def launch_fc_vmem(self, d_in, d_out, C_in, C_out, d_kernel, d_bias, d_alpha, B):
        check(lib().vdttfs_launch_fc_vmem_sync(self.handle, d_in.ptr, d_out.ptr, C_in, C_out,
                                               d_kernel.ptr, d_bias.ptr, d_alpha.ptr, B))


@dataclass
class Layer:
    """One row of the network table (host weights in the reference layout)."""
    kind: int
    H_in: int
    W_in: int
    C_in: int
    H_out: int
    W_out: int
    C_out: int
    K_h: int = 1
    K_w: int = 1
    kernel: np.ndarray | None = None   # HWIO (conv) / [C_in][C_out] (fc)
    bias: np.ndarray | None = None
    tc_fire: float = 16.0
    td: float = 0.0

    def to_c(self) -> LayerDesc:
        k = self.kernel
        b = self.bias
        fp = C.POINTER(C.c_float)
        return LayerDesc(self.kind, self.H_in, self.W_in, self.C_in, self.H_out, self.W_out,
                         self.C_out, self.K_h, self.K_w,
                         k.ctypes.data_as(fp) if k is not None else fp(),
                         b.ctypes.data_as(fp) if b is not None else fp(),
                         self.tc_fire, self.td)


class Net:
    """The engine: encode -> layers -> readout, weights and LUTs resident."""

    def __init__(self, ctx: Context, layers: list[Layer], B: int, img_elems: int,
                 encode_mode=ENCODE_LINEAR, tc_in=16.0, td_in=0.0, readout=READOUT_ARGMIN):
        self.ctx = ctx
        self.layers = layers
        self.B = B
        for l in layers:
            if l.kernel is not None:
                l.kernel = np.ascontiguousarray(l.kernel, np.float32)
            if l.bias is not None:
                l.bias = np.ascontiguousarray(l.bias, np.float32)
        arr = (LayerDesc * len(layers))(*[l.to_c() for l in layers])
        h = C.c_void_p()
        check(lib().vdttfs_net_create(ctx.handle, arr, len(layers), B, img_elems, encode_mode,
                                      tc_in, td_in, readout, C.byref(h)))
        self.handle = h

    def close(self):
        if self.handle is not None:
            lib().vdttfs_net_destroy(self.handle)
            self.handle = None

    def forward(self, d_img: DeviceArray, d_pred: DeviceArray | None = None):
        check(lib().vdttfs_net_forward(self.handle, d_img.ptr, d_pred.ptr if d_pred else None))

    def layer_output_ptr(self, i: int):
        """(device pointer, elements) of layer i's output map."""
        p = C.c_void_p()
        n = C.c_int64()
        check(lib().vdttfs_net_layer_output(self.handle, i, C.byref(p), C.byref(n)))
        return p, n.value

    def layer_output(self, i: int) -> np.ndarray:
        p = C.c_void_p()
        n = C.c_int64()
        check(lib().vdttfs_net_layer_output(self.handle, i, C.byref(p), C.byref(n)))
        h = np.empty(n.value, np.float32)
        check(lib().vdttfs_d2h(self.ctx.handle, _ptr(h), p, h.nbytes))
        return h

    def count(self, d_img: DeviceArray):
        n = len(self.layers)
        arrs = [(C.c_uint64 * n)() for _ in range(4)]
        check(lib().vdttfs_net_count(self.handle, d_img.ptr, *arrs))
        return [np.array(list(a), dtype=np.uint64) for a in arrs]

    def set_timing(self, on: bool):
        check(lib().vdttfs_net_set_timing(self.handle, int(on)))

    def set_graphs(self, on: bool):
        """Forwards captured into HIP graphs and replayed per (input,
        prediction) pair (vdttfs_net_set_graphs); same outputs."""
        check(lib().vdttfs_net_set_graphs(self.handle, int(on)))

    def set_pool_fusion(self, mode: int):
        """Which 2x2 pools run inside the next layer's list build
        (vdttfs_net_set_pool_fusion: POOL_FUSE_OFF, the default, _ALL or
        _AUTO); the outputs are the same."""
        check(lib().vdttfs_net_set_pool_fusion(self.handle, int(mode)))

    def set_windows(self, windows=None):
        """Per-layer integration windows T'_l (vdttfs_net_set_windows): one
        entry per layer, 0 or T for the full window, pools ignored; None resets."""
        if windows is None:
            check(lib().vdttfs_net_set_windows(self.handle, None, 0))
            return
        w = np.ascontiguousarray(windows, np.int32)
        check(lib().vdttfs_net_set_windows(self.handle, _ptr(w), int(w.size)))

    def set_plan(self, layer: int, path: int = 0, gather: int = 0, ppw: int = 0):
        """Launch plan of one layer (vdttfs_net_set_plan); all zeros restores
        the built-in choice."""
        pl = LayerPlan(path, gather, ppw)
        check(lib().vdttfs_net_set_plan(self.handle, layer, C.byref(pl)))

    def get_plan(self, layer: int) -> tuple:
        """(path, gather, ppw) the next forward uses for the layer."""
        pl = LayerPlan()
        check(lib().vdttfs_net_get_plan(self.handle, layer, C.byref(pl)))
        return pl.path, pl.gather, pl.ppw

    def read_layer_timing(self) -> np.ndarray:
        """Per-layer event ms since the last read (timing must be enabled)."""
        ms = np.zeros(len(self.layers), np.float64)
        check(lib().vdttfs_net_read_layer_timing(self.handle, _ptr(ms), len(self.layers)))
        return ms

    def read_timing(self):
        im, bm = C.c_double(), C.c_double()
        il, bl = C.c_int64(), C.c_int64()
        check(lib().vdttfs_net_read_timing(self.handle, C.byref(im), C.byref(il), C.byref(bm),
                                           C.byref(bl)))
        return im.value, il.value, bm.value, bl.value


class StepNet:
    """The step-by-step (time-driven) baseline over the same layer table as
    Net: T1S (STEP_T1) or T2S (STEP_T2) semantics (vdttfs_stepnet_*)."""

    def __init__(self, ctx: Context, layers: list[Layer], B: int, img_elems: int,
                 encode_mode=ENCODE_LINEAR, tc_in=16.0, td_in=0.0, mode=STEP_T1):
        self.ctx = ctx
        self.layers = layers
        self.B = B
        for l in layers:
            if l.kernel is not None:
                l.kernel = np.ascontiguousarray(l.kernel, np.float32)
            if l.bias is not None:
                l.bias = np.ascontiguousarray(l.bias, np.float32)
        arr = (LayerDesc * len(layers))(*[l.to_c() for l in layers])
        h = C.c_void_p()
        check(lib().vdttfs_stepnet_create(ctx.handle, arr, len(layers), B, img_elems, encode_mode,
                                          tc_in, td_in, mode, C.byref(h)))
        self.handle = h

    def close(self):
        if self.handle is not None:
            lib().vdttfs_stepnet_destroy(self.handle)
            self.handle = None

    def forward(self, d_img: DeviceArray, d_pred: DeviceArray | None = None):
        check(lib().vdttfs_stepnet_forward(self.handle, d_img.ptr, d_pred.ptr if d_pred else None))

    def output(self):
        """(last layer's [B][C] output as numpy, number of global steps)."""
        p = C.c_void_p()
        n = C.c_int64()
        steps = C.c_int()
        check(lib().vdttfs_stepnet_output(self.handle, C.byref(p), C.byref(n), C.byref(steps)))
        h = np.empty(n.value, np.float32)
        check(lib().vdttfs_d2h(self.ctx.handle, _ptr(h), p, h.nbytes))
        return h, steps.value


class CulifStepNet(StepNet):
    """The step-by-step CuLIF baseline (T3S semantics) over the same layer
    table as CulifNet (vdttfs_stepnet_create_culif); forward takes the dense
    event tensor [B][C][H][W][T], output() gives the last layer's first-spike
    steps."""

    def __init__(self, ctx: Context, layers: list, B: int):
        self.ctx = ctx
        self.layers = layers
        self.B = B
        for l in layers:
            if l.weight is not None:
                l.weight = np.ascontiguousarray(l.weight, np.float32)
            if l.weight_rec is not None:
                l.weight_rec = np.ascontiguousarray(l.weight_rec, np.float32)
        arr = (CulifLayer * len(layers))(*[l.to_c() for l in layers])
        h = C.c_void_p()
        check(lib().vdttfs_stepnet_create_culif(ctx.handle, arr, len(layers), B, C.byref(h)))
        self.handle = h


@dataclass
class CulifLayerSpec:
    """One layer of the CuLIF engine (vdttfs_culif_layer): conv weights OIHW
    [C_out][C_in][3][3], FC weights [out][in], FC_REC also [out][out]."""
    kind: int
    C_in: int
    H_in: int
    W_in: int
    C_out: int
    weight: np.ndarray | None = None
    weight_rec: np.ndarray | None = None
    decay: float = 0.5
    th: float = 1.0

    @property
    def out_shape(self):
        if self.kind in (CULIF_FC, CULIF_FC_REC):
            return (self.C_out, 1, 1)
        if self.kind == CULIF_POOL:
            return (self.C_out, self.H_in // 2, self.W_in // 2)
        return (self.C_out, self.H_in, self.W_in)

    def to_c(self) -> CulifLayer:
        fp = C.POINTER(C.c_float)
        w = self.weight.ctypes.data_as(fp) if self.weight is not None else fp()
        r = self.weight_rec.ctypes.data_as(fp) if self.weight_rec is not None else fp()
        return CulifLayer(self.kind, self.C_in, self.H_in, self.W_in, self.C_out, w, r, self.decay,
                          self.th)


class CulifNet:
    """The CuLIF engine: dense events -> layers -> readout (T3V:276-298)."""

    def __init__(self, ctx: Context, layers: list[CulifLayerSpec], B: int):
        self.ctx = ctx
        self.layers = layers
        self.B = B
        for l in layers:
            if l.weight is not None:
                l.weight = np.ascontiguousarray(l.weight, np.float32)
            if l.weight_rec is not None:
                l.weight_rec = np.ascontiguousarray(l.weight_rec, np.float32)
        arr = (CulifLayer * len(layers))(*[l.to_c() for l in layers])
        h = C.c_void_p()
        check(lib().vdttfs_culif_net_create(ctx.handle, arr, len(layers), B, C.byref(h)))
        self.handle = h

    def close(self):
        if self.handle is not None:
            lib().vdttfs_culif_net_destroy(self.handle)
            self.handle = None

    def forward(self, d_data: DeviceArray, d_pred: DeviceArray | None = None):
        check(lib().vdttfs_culif_net_forward(self.handle, d_data.ptr, d_pred.ptr if d_pred else None))

    def layer_output(self, i: int, layout: str = "nchw") -> np.ndarray:
        """Layer i's output as [B][C][H][W] (layout "nchw") or [B][H][W][C]
        ("nhwc"), whatever the engine keeps internally; any other layout
        returns the engine's own buffer."""
        p = C.c_void_p()
        n = C.c_int64()
        nhwc = C.c_int32()
        check(lib().vdttfs_culif_net_layer_output(self.handle, i, C.byref(p), C.byref(n),
                                                  C.byref(nhwc)))
        h = np.empty(n.value, np.float32)
        check(lib().vdttfs_d2h(self.ctx.handle, _ptr(h), p, h.nbytes))
        Cc, H, W = self.layers[i].out_shape
        if layout == "nhwc":
            if nhwc.value:
                return h
            return np.ascontiguousarray(h.reshape(self.B, Cc, H, W).transpose(0, 2, 3, 1)).reshape(-1)
        if nhwc.value:
            h = h.reshape(self.B, H, W, Cc).transpose(0, 3, 1, 2)
        return np.ascontiguousarray(h.reshape(self.B, Cc, H, W)) if layout == "nchw" else h

    def set_timing(self, on: bool):
        check(lib().vdttfs_culif_net_set_timing(self.handle, int(on)))

    def read_timing(self):
        """(per-layer milliseconds summed over the timed forwards, forwards)."""
        n = len(self.layers)
        ms = (C.c_double * n)()
        fw = C.c_int64()
        check(lib().vdttfs_culif_net_read_timing(self.handle, ms, C.byref(fw)))
        return np.array(list(ms)), fw.value

    def count(self, d_data: DeviceArray):
        """Per layer (eproc, ebin, n_ev, n_cols); nonzero for conv layers."""
        n = len(self.layers)
        arrs = [(C.c_uint64 * n)() for _ in range(4)]
        check(lib().vdttfs_culif_net_count(self.handle, d_data.ptr, *arrs))
        return [np.array(list(a), dtype=np.uint64) for a in arrs]
