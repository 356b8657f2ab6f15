"""vdttfs -- MI355X-native VD-TTFS inference engine (Python host mirror).

The compute path is libvdttfs.so (hand-written HIP for gfx950 behind the C
ABI declared in include/vdttfs.h); this package only marshals arguments.
"""
from ._lib import (INF_TIME, LIB_PATH, VdttfsError, lib, last_error,  # noqa: F401
                   LAYER_CONV, LAYER_FC, LAYER_POOL, LAYER_VMEM, ENCODE_LINEAR, ENCODE_LOG,
                   READOUT_ARGMIN, READOUT_ARGMAX)
from .core import (Context, DeviceArray, Layer, Net, TaskConsts, build_luts_host,  # noqa: F401
                   device_count, task1_consts, task2_consts)
from . import models  # noqa: F401

__version__ = "0.1.0"
