"""ctypes binding of libvolta_hip.so (the C ABI in include/volta_hip.h).

The library is loaded from this package directory (built in-tree by
``__graft_entry__.build()``); there is no fallback implementation: if the
library is missing, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvolta_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "volta_hip.h")

VH_OK = 0
VH_ERR_NO_DEVICE = 1
VH_ERR_BAD_SHAPE = 2
VH_ERR_OOM = 3
VH_ERR_LAUNCH = 4
VH_ERR_BAD_ARG = 5
VH_ERR_UNSUPPORTED = 6
VH_ERR_CAPTURE = 7

F32 = 0
BF16 = 1

ALGO_DIRECT, ALGO_IM2COL, ALGO_IGEMM, ALGO_AUTO = 0, 1, 2, 3
POLICY_FASTEST, POLICY_GENERIC = 0, 1
UNARY_RELU = 0
OPT_SGD, OPT_SGD_MOMENTUM, OPT_ADAM = 0, 1, 2


class VoltaHipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"libvolta_hip status {status}: {message}")
        self.status = status


_I64 = ctypes.c_int64
_P = ctypes.c_void_p
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_PP = ctypes.POINTER(ctypes.c_void_p)

_CONV13 = [_I64] * 13
_LAYER11 = [_I64] * 11

# argtypes of every exported function, in header order
SIGNATURES = {
    "vh_init": [],
    "vh_last_error": [],
    "vh_alloc": [_SZ, ctypes.POINTER(_P)],
    "vh_free": [_P],
    "vh_upload": [_P, _P, _SZ, _P],
    "vh_download": [_P, _P, _SZ, _P],
    "vh_stream_sync": [_P],
    "vh_release_cache": [],
    "vh_workspace_info": [_P, _PP, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)],
    "vh_set_kernel_policy": [_INT],
    "vh_matmul": [_INT, _P, _P, _P, _I64, _I64, _I64, _P],
    "vh_matmul_backward_a": [_INT, _P, _P, _P, _I64, _I64, _I64, _P],
    "vh_matmul_backward_b": [_INT, _P, _P, _P, _I64, _I64, _I64, _P],
    "vh_im2col": [_INT, _P, _P] + [_I64] * 10 + [_P],
    "vh_col2im": [_INT, _P, _P] + [_I64] * 10 + [_P],
    "vh_direct_conv": [_INT, _P, _P, _P] + _CONV13 + [_P],
    "vh_igemm": [_INT, _P, _P, _P] + _CONV13 + [_P],
    "vh_conv_backward_input": [_INT, _P, _P, _P] + _CONV13 + [_P],
    "vh_conv_backward_weight": [_INT, _P, _P, _P] + _CONV13 + [_P],
    "vh_igemm_backward_input": [_INT, _P, _P, _P] + _CONV13 + [_P],
    "vh_igemm_backward_weight": [_INT, _P, _P, _P] + _CONV13 + [_P],
    "vh_matmul_alloc": [_INT, _P, _P, _PP, _I64, _I64, _I64, _P],
    "vh_matmul_backward_a_alloc": [_INT, _P, _P, _PP, _I64, _I64, _I64, _P],
    "vh_matmul_backward_b_alloc": [_INT, _P, _P, _PP, _I64, _I64, _I64, _P],
    "vh_im2col_alloc": [_INT, _P, _PP] + [_I64] * 10 + [_P],
    "vh_col2im_alloc": [_INT, _P, _PP] + [_I64] * 10 + [_P],
    "vh_direct_conv_alloc": [_INT, _P, _P, _PP] + _CONV13 + [_P],
    "vh_igemm_alloc": [_INT, _P, _P, _PP] + _CONV13 + [_P],
    "vh_conv_backward_input_alloc": [_INT, _P, _P, _PP] + _CONV13 + [_P],
    "vh_igemm_backward_input_alloc": [_INT, _P, _P, _PP] + _CONV13 + [_P],
    "vh_conv_backward_weight_alloc": [_INT, _P, _P, _PP] + _CONV13 + [_P],
    "vh_igemm_backward_weight_alloc": [_INT, _P, _P, _PP] + _CONV13 + [_P],
    "vh_conv_algo_auto_select": [_I64] * 5 + [_INT],
    "vh_conv_algo_select_mi355x": [_I64] * 11,
    "vh_conv2d_forward": [_INT, _INT, _P, _P, _P, _P] + _LAYER11 + [ctypes.POINTER(_INT), _P],
    "vh_conv2d_backward": [_INT, _INT, _P, _P, _P, _P, _P, _P] + _LAYER11 + [_P],
    "vh_conv_transpose2d_forward": [_INT, _P, _P, _P, _P] + _LAYER11 + [_P],
    "vh_conv_transpose2d_backward": [_INT, _P, _P, _P, _P, _P, _P] + _LAYER11 + [_P],
    "vh_linear_forward": [_INT, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "vh_linear_backward": [_INT, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "vh_pixel_shuffle": [_INT, _P, _P] + [_I64] * 5 + [_P],
    "vh_pixel_shuffle_backward": [_INT, _P, _P] + [_I64] * 5 + [_P],
    "vh_conv2d_forward_relu": [_INT, _INT, _P, _P, _P, _P] + _LAYER11 + [ctypes.POINTER(_INT), _P],
    "vh_conv2d_backward_relu": [_INT, _INT, _P, _P, _P, _P, _P, _P] + _LAYER11 + [_P],
    "vh_conv2d_backward_noalloc": [_INT, _INT, _P, _P, _P, _P, _P, _P] + _LAYER11 + [_P],
    "vh_unary": [_INT, _INT, _P, _P, _I64, _P],
    "vh_unary_backward": [_INT, _INT, _P, _P, _P, _I64, _P],
    "vh_sum_reduce": [_INT, _P, _I64, _P, _P],
    "vh_sum_backward": [_INT, ctypes.c_float, _P, _I64, _P],
    "vh_cast": [_INT, _INT, _P, _P, _I64, _P],
    "vh_nchw_to_nhwc": [_INT, _P, _P] + [_I64] * 4 + [_P],
    "vh_nhwc_to_nchw": [_INT, _P, _P] + [_I64] * 4 + [_P],
    "vh_grad_accumulate": [_INT, _P, _P, _I64, _P],
    "vh_optimizer_step": [_INT] + [ctypes.c_float] * 6 + [_P, _P, _P, _P, _I64, _P],
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/volta_hip.h."""
    text = open(HEADER_PATH).read()
    return re.findall(r"^\s*(?:int|const char\*)\s+(vh_\w+)\s*\(", text, re.M)


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        l = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "vh_last_error" else ctypes.c_int
        _lib = l
    return _lib


def check(status: int) -> None:
    if status != VH_OK:
        msg = lib().vh_last_error()
        raise VoltaHipError(status, msg.decode() if msg else "")
