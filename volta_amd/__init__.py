"""volta_amd -- MI355X (gfx950) implementation of Volta's conv / matmul hot path.

The compute lives in ``libvolta_hip.so`` (HIP kernels for gfx950 behind the C ABI
of ``include/volta_hip.h``).  This package binds it with ctypes:

* :mod:`volta_amd.ops` mirrors the reference's ``RawTensor::gpu_*`` boundary
  (src/ops/gpu_ops.rs);
* :mod:`volta_amd.nn` mirrors ``Conv2d`` / ``ConvTranspose2d`` / ``Linear`` /
  ``PixelShuffle`` and ``ConvAlgo``.

There is no CPU fallback inside this package: without the built library every
call raises.
"""
from ._lib import ALGO_AUTO, ALGO_DIRECT, ALGO_IGEMM, ALGO_IM2COL, BF16, F32, LIB_PATH, VoltaHipError, check, lib
from . import ops
from .nn import ConvAlgo, Conv2d, ConvTranspose2d, Linear, PixelShuffle

__all__ = ["ops", "ConvAlgo", "Conv2d", "ConvTranspose2d", "Linear", "PixelShuffle", "VoltaHipError", "lib",
           "check", "F32", "BF16", "LIB_PATH"]
