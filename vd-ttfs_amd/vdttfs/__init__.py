"""vdttfs -- MI355X-native VD-TTFS inference engine (Python host mirror).

The compute path is libvdttfs.so (hand-written HIP for gfx950 behind the C
ABI declared in include/vdttfs.h); this package only marshals arguments.
"""
from ._lib import (INF_TIME, LIB_PATH, VdttfsError, lib, last_error,  # noqa: F401
                   LAYER_CONV, LAYER_FC, LAYER_POOL, LAYER_VMEM, ENCODE_LINEAR, ENCODE_LOG, ENCODE_TIMES,
                   READOUT_ARGMIN, READOUT_ARGMAX, READOUT_ARGMIN_FIRST, CULIF_RAW_CONV, CULIF_CONV,
                   CULIF_POOL, CULIF_FC_REC, CULIF_FC, STEP_T1, STEP_T2, STEP_T3, PATH_AUTO, PATH_BINS, PATH_DENSE,
                   PATH_FUSED, PATH_REG, PATH_WINDOW, POOL_FUSE_OFF, POOL_FUSE_ALL, POOL_FUSE_AUTO)
from .core import (Context, CulifLayerSpec, CulifNet, CulifStepNet, DeviceArray, Layer, Net, StepNet,  # noqa: F401
                   TaskConsts, build_luts_host, device_count, task1_consts, task2_consts,
                   task3_consts)
from . import models  # noqa: F401

__version__ = "0.1.0"
