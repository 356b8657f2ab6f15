"""ctypes declarations of libvdttfs.so (the C ABI in include/vdttfs.h).

The shared library is built in-tree by ``make -C vd-ttfs_amd`` (or
``__graft_entry__.build()``).  Loading fails loudly when it is missing: there
is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libvdttfs.so")

OK = 0
E_INVALID = -1
E_HIP = -2
E_IO = -3
E_FORMAT = -4
E_NOMEM = -5
E_UNSUPPORTED = -6
E_NODEVICE = -7

INF_TIME = 9999.0

LAYER_CONV, LAYER_FC, LAYER_POOL, LAYER_VMEM = 0, 1, 2, 3
ENCODE_LINEAR, ENCODE_LOG, ENCODE_TIMES = 0, 1, 2
READOUT_ARGMIN, READOUT_ARGMAX, READOUT_ARGMIN_FIRST = 0, 1, 2
CULIF_RAW_CONV, CULIF_CONV, CULIF_POOL, CULIF_FC_REC, CULIF_FC = 0, 1, 2, 3, 4
STEP_T1, STEP_T2, STEP_T3 = 1, 2, 3
PATH_AUTO, PATH_BINS, PATH_DENSE, PATH_FUSED, PATH_REG, PATH_WINDOW = 0, 1, 2, 3, 4, 5
POOL_FUSE_OFF, POOL_FUSE_ALL, POOL_FUSE_AUTO = 0, 1, 2


class VdttfsError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"vdttfs error {code}: {msg}")
        self.code = code


class Consts(C.Structure):
    _fields_ = [
        ("T", C.c_int32),
        ("tfs", C.c_float),
        ("delta", C.c_int32),
        ("vth", C.c_float),
        ("alpha_by_time", C.c_int32),
        ("conv_same_pad", C.c_int32),
    ]


class BlobLayer(C.Structure):
    _fields_ = [
        ("ndim", C.c_int32),
        ("shape", C.c_int32 * 4),
        ("k_h", C.c_int32),
        ("k_w", C.c_int32),
        ("c_in", C.c_int32),
        ("c_out", C.c_int32),
        ("kernel_elems", C.c_int64),
        ("kernel", C.POINTER(C.c_float)),
        ("bias_ndim", C.c_int32),
        ("bias_size", C.c_int32),
        ("bias", C.POINTER(C.c_float)),
        ("tc_ndim", C.c_int32),
        ("td_ndim", C.c_int32),
        ("tc_fire", C.c_float),
        ("td", C.c_float),
    ]


class Blob(C.Structure):
    _fields_ = [("num_layers", C.c_int32), ("layers", C.POINTER(BlobLayer))]


class DevLayer(C.Structure):
    _fields_ = [
        ("d_kernel", C.c_void_p),
        ("d_bias", C.c_void_p),
        ("tc_fire", C.c_float),
        ("td", C.c_float),
        ("k_h", C.c_int32),
        ("k_w", C.c_int32),
        ("c_in", C.c_int32),
        ("c_out", C.c_int32),
    ]


class LayerDesc(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("H_in", C.c_int32),
        ("W_in", C.c_int32),
        ("C_in", C.c_int32),
        ("H_out", C.c_int32),
        ("W_out", C.c_int32),
        ("C_out", C.c_int32),
        ("K_h", C.c_int32),
        ("K_w", C.c_int32),
        ("kernel", C.POINTER(C.c_float)),
        ("bias", C.POINTER(C.c_float)),
        ("tc_fire", C.c_float),
        ("td", C.c_float),
    ]


class LayerPlan(C.Structure):
    _fields_ = [("path", C.c_int32), ("gather", C.c_int32), ("ppw", C.c_int32)]


class CulifLayer(C.Structure):
    _fields_ = [
        ("kind", C.c_int32),
        ("C_in", C.c_int32),
        ("H_in", C.c_int32),
        ("W_in", C.c_int32),
        ("C_out", C.c_int32),
        ("weight", C.POINTER(C.c_float)),
        ("weight_rec", C.POINTER(C.c_float)),
        ("decay", C.c_float),
        ("th", C.c_float),
    ]


_vp = C.c_void_p
_i = C.c_int
_i64 = C.c_int64
_f = C.c_float
_u64p = C.POINTER(C.c_uint64)

# name -> argtypes (all return int status unless listed in _RESTYPES)
SIGNATURES = {
    "vdttfs_last_error": [],
    "vdttfs_version": [],
    "vdttfs_create": [C.POINTER(Consts), _i, C.POINTER(_vp)],
    "vdttfs_destroy": [_vp],
    "vdttfs_get_consts": [_vp, C.POINTER(Consts)],
    "vdttfs_num_chunks": [_vp],
    "vdttfs_synchronize": [_vp],
    "vdttfs_device_count": [C.POINTER(_i)],
    "vdttfs_dev_alloc": [_vp, C.c_size_t, C.POINTER(_vp)],
    "vdttfs_dev_free": [_vp, _vp],
    "vdttfs_h2d": [_vp, _vp, _vp, C.c_size_t],
    "vdttfs_d2h": [_vp, _vp, _vp, C.c_size_t],
    "vdttfs_memset": [_vp, _vp, _i, C.c_size_t],
    "vdttfs_update_luts": [_vp, _vp, _vp, _f, _f, _f, _f],
    "vdttfs_build_luts_host": [C.POINTER(Consts), _f, _f, _f, _f, _vp, _vp],
    "vdttfs_encode_image": [_vp, _vp, _vp, _i64, _f, _f],
    "vdttfs_encode_linear": [_vp, _vp, _vp, _i64],
    "vdttfs_bucketize": [_vp, _vp, _i64, _i, _vp, _vp, _vp],
    "vdttfs_integrate": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i,
                         _i, _i, _i, _i],
    "vdttfs_layer_forward": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i,
                             _i, _i, _i, _u64p, _u64p],
    "vdttfs_layer_forward_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i,
                                     _i, _i, _i],
    "vdttfs_pool_min": [_vp, _vp, _vp, _i, _i, _i, _i],
    "vdttfs_fc_vmem": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i],
    "vdttfs_readout_argmin": [_vp, _vp, _i, _i, _vp],
    "vdttfs_readout_argmax": [_vp, _vp, _i, _i, _vp],
    "vdttfs_launch_layer_sync": [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _vp, _vp,
                                 _vp, _i, _i],
    "vdttfs_launch_pool_sync": [_vp, _vp, _vp, _i, _i, _i, _i],
    "vdttfs_launch_fc_vmem_sync": [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _i],
    "vdttfs_blob_read": [C.c_char_p, C.POINTER(C.POINTER(Blob))],
    "vdttfs_blob_write": [C.c_char_p, C.POINTER(Blob)],
    "vdttfs_blob_free": [C.POINTER(Blob)],
    "vdttfs_load_weights": [_vp, C.c_char_p, C.POINTER(C.POINTER(DevLayer)), C.POINTER(_i)],
    "vdttfs_free_weights": [_vp, C.POINTER(DevLayer), _i],
    "vdttfs_net_create": [_vp, C.POINTER(LayerDesc), _i, _i, _i64, _i, _f, _f, _i, C.POINTER(_vp)],
    "vdttfs_net_destroy": [_vp],
    "vdttfs_net_forward": [_vp, _vp, _vp],
    "vdttfs_net_layer_output": [_vp, _i, C.POINTER(_vp), C.POINTER(_i64)],
    "vdttfs_stepnet_create": [_vp, C.POINTER(LayerDesc), _i, _i, _i64, _i, _f, _f, _i, C.POINTER(_vp)],
    "vdttfs_stepnet_destroy": [_vp],
    "vdttfs_stepnet_forward": [_vp, _vp, _vp],
    "vdttfs_stepnet_output": [_vp, C.POINTER(_vp), C.POINTER(_i64), C.POINTER(_i)],
    "vdttfs_stepnet_create_culif": [_vp, C.POINTER(CulifLayer), _i, _i, C.POINTER(_vp)],
    "vdttfs_net_count": [_vp, _vp, _u64p, _u64p, _u64p, _u64p],
    "vdttfs_net_set_timing": [_vp, _i],
    "vdttfs_net_set_pool_fusion": [_vp, _i],
    "vdttfs_net_set_graphs": [_vp, _i],
    "vdttfs_net_set_windows": [_vp, _vp, _i],
    "vdttfs_net_set_plan": [_vp, _i, _vp],
    "vdttfs_net_get_plan": [_vp, _i, _vp],
    "vdttfs_net_read_layer_timing": [_vp, _vp, _i],
    "vdttfs_net_read_timing": [_vp, C.POINTER(C.c_double), C.POINTER(_i64),
                               C.POINTER(C.c_double), C.POINTER(_i64)],
    "vdttfs_synth_uniform": [C.c_uint64, C.c_uint64, _vp, _i64],
    "vdttfs_synth_normal": [C.c_uint64, C.c_uint64, _vp, _i64, C.c_double],
    "vdttfs_synth_dvs": [C.c_uint64, _i, _i, _i, _i, _i, C.c_double, C.c_double, C.c_double, _vp,
                         _vp],
    "vdttfs_culif_conv1_raw": [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _f],
    "vdttfs_culif_bucketize_conv": [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp],
    "vdttfs_culif_bucketize_fc": [_vp, _vp, _i, _i, _vp, _vp, _vp],
    "vdttfs_culif_conv": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _f],
    "vdttfs_culif_pool": [_vp, _vp, _vp, _i, _i, _i, _i, _f, _f],
    "vdttfs_culif_fc_recurrent": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _f],
    "vdttfs_culif_fc": [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _f],
    "vdttfs_readout_argmin_first": [_vp, _vp, _i, _i, _vp],
    "vdttfs_culif_net_create": [_vp, C.POINTER(CulifLayer), _i, _i, C.POINTER(_vp)],
    "vdttfs_culif_net_destroy": [_vp],
    "vdttfs_culif_net_forward": [_vp, _vp, _vp],
    "vdttfs_culif_net_layer_output": [_vp, _i, C.POINTER(_vp), C.POINTER(_i64),
                                      C.POINTER(C.c_int32)],
    "vdttfs_culif_net_set_timing": [_vp, _i],
    "vdttfs_culif_net_read_timing": [_vp, C.POINTER(C.c_double), C.POINTER(_i64)],
    "vdttfs_culif_net_count": [_vp, _vp, _u64p, _u64p, _u64p, _u64p],
    "vdttfs_timer_begin": [_vp],
    "vdttfs_timer_end": [_vp, C.POINTER(C.c_double)],
    "vdttfs_probe_gather": [_vp, _i, _i64, _i, _i64, _i, C.POINTER(C.c_double)],
}

_RESTYPES = {"vdttfs_last_error": C.c_char_p, "vdttfs_version": C.c_char_p}

_lib = None


def lib() -> C.CDLL:
    """Load libvdttfs.so once; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `make -C vd-ttfs_amd` or __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPES.get(name, C.c_int)
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().vdttfs_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> int:
    if rc < 0:
        raise VdttfsError(rc, last_error())
    return rc
