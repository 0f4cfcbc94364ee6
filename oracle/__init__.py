"""CPU oracle for the Volta conv/matmul hot path -- TEST INFRASTRUCTURE ONLY.

numpy front end over ``oracle/_build/liboracle_volta.so`` (built from
``oracle/volta_oracle.c`` by ``oracle/Makefile``), a single-threaded restatement
of Volta's CPU loops.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker / CPU baseline; the product (``volta_amd``) never does.

Every function takes and returns float32 numpy arrays in the reference's
layouts (NCHW activations, OIHW Conv2d weights, IOHW ConvTranspose2d weights,
[in, out] Linear weights).  Reference citations live on the C functions.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_volta.so")
_lib = None

_FP = ctypes.POINTER(ctypes.c_float)
_DP = ctypes.POINTER(ctypes.c_double)
_SZ = ctypes.c_size_t

ALGO_DIRECT, ALGO_IM2COL, ALGO_IGEMM = 0, 1, 2


def build() -> None:
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.or_auto_select.restype = ctypes.c_int
        _lib.or_auto_select.argtypes = [_SZ] * 5 + [ctypes.c_int]
        _lib.or_sum.restype = ctypes.c_float
        _lib.or_sum.argtypes = [_FP, _SZ]
        _lib.or_sum_backward.argtypes = [ctypes.c_float, _FP, _SZ]
        _lib.or_optimizer_step.argtypes = [ctypes.c_int] + [ctypes.c_float] * 6 + [_FP, _FP, _FP, _FP, _SZ]
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_FP)


def _pn(a):
    return None if a is None else a.ctypes.data_as(_FP)


def conv_out(h: int, k: int, s: int, p: int) -> int:
    return (h + 2 * p - k) // s + 1


def auto_select(batch, channels, height, width, kernel_size, has_gpu) -> int:
    return lib().or_auto_select(batch, channels, height, width, kernel_size, int(bool(has_gpu)))


def _conv_dims(x_shape, w_shape, stride, pad):
    B, C, H, W = x_shape
    O, C2, KH, KW = w_shape
    assert C == C2
    SH, SW = stride
    PH, PW = pad
    return B, C, O, H, W, KH, KW, SH, SW, PH, PW


def direct_conv(x, w, stride=(1, 1), pad=(0, 0)):
    x, w = _f32(x), _f32(w)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x.shape, w.shape, stride, pad)
    y = np.empty((B, O, conv_out(H, KH, SH, PH), conv_out(W, KW, SW, PW)), np.float32)
    lib().or_direct_conv(_p(x), _p(w), _p(y), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)))
    return y


def direct_conv_backward_input(dy, w, x_shape, stride=(1, 1), pad=(0, 0), literal=False):
    dy, w = _f32(dy), _f32(w)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x_shape, w.shape, stride, pad)
    dx = np.empty((B, C, H, W), np.float32)
    fn = lib().or_direct_conv_backward_input_literal if literal else lib().or_direct_conv_backward_input
    fn(_p(dy), _p(w), _p(dx), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)))
    return dx


def direct_conv_backward_weight(dy, x, w_shape, stride=(1, 1), pad=(0, 0)):
    dy, x = _f32(dy), _f32(x)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x.shape, w_shape, stride, pad)
    dw = np.empty(w_shape, np.float32)
    lib().or_direct_conv_backward_weight(_p(dy), _p(x), _p(dw), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)))
    return dw


def conv_bias_grad(dy):
    dy = _f32(dy)
    B, O, HO, WO = dy.shape
    db = np.empty((O,), np.float32)
    lib().or_conv_bias_grad(_p(dy), _p(db), _SZ(B), _SZ(O), _SZ(HO), _SZ(WO))
    return db


def pad(x, ph, pw):
    x = _f32(x)
    B, C, H, W = x.shape
    xp = np.empty((B, C, H + 2 * ph, W + 2 * pw), np.float32)
    lib().or_pad(_p(x), _p(xp), *map(_SZ, (B, C, H, W, ph, pw)))
    return xp


def im2col(x, kernel, stride):
    x = _f32(x)
    B, C, H, W = x.shape
    KH, KW = kernel
    SH, SW = stride
    HO, WO = (H - KH) // SH + 1, (W - KW) // SW + 1
    col = np.empty((B * HO * WO, C * KH * KW), np.float32)
    lib().or_im2col(_p(x), _p(col), *map(_SZ, (B, C, H, W, KH, KW, SH, SW)))
    return col


def col2im(col, x_shape, kernel, stride):
    col = _f32(col)
    B, C, H, W = x_shape
    KH, KW = kernel
    SH, SW = stride
    x = np.empty((B, C, H, W), np.float32)
    lib().or_col2im(_p(col), _p(x), *map(_SZ, (B, C, H, W, KH, KW, SH, SW)))
    return x


def matmul(a, b):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().or_matmul(_p(a), _p(b), _p(c), _SZ(m), _SZ(k), _SZ(n))
    return c


def matmul_backward_a(g, b):
    g, b = _f32(g), _f32(b)
    m, n = g.shape
    k, n2 = b.shape
    assert n == n2
    da = np.empty((m, k), np.float32)
    lib().or_matmul_backward_a(_p(g), _p(b), _p(da), _SZ(m), _SZ(k), _SZ(n))
    return da


def matmul_backward_b(a, g):
    a, g = _f32(a), _f32(g)
    m, k = a.shape
    m2, n = g.shape
    assert m == m2
    db = np.empty((k, n), np.float32)
    lib().or_matmul_backward_b(_p(a), _p(g), _p(db), _SZ(m), _SZ(k), _SZ(n))
    return db


def im2col_conv_forward(x, w, stride=(1, 1), pad=(0, 0)):
    x, w = _f32(x), _f32(w)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x.shape, w.shape, stride, pad)
    y = np.empty((B, O, conv_out(H, KH, SH, PH), conv_out(W, KW, SW, PW)), np.float32)
    lib().or_im2col_conv_forward(_p(x), _p(w), _p(y), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)))
    return y


def im2col_conv_backward(dy, x, w, stride=(1, 1), pad=(0, 0)):
    dy, x, w = _f32(dy), _f32(x), _f32(w)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x.shape, w.shape, stride, pad)
    dx = np.empty(x.shape, np.float32)
    dw = np.empty(w.shape, np.float32)
    lib().or_im2col_conv_backward(_p(dy), _p(x), _p(w), _p(dx), _p(dw),
                                  *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)))
    return dx, dw


def igemm_forward(x, w, stride=(1, 1), pad=(0, 0), bug_compat=False):
    x, w = _f32(x), _f32(w)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x.shape, w.shape, stride, pad)
    y = np.empty((B, O, conv_out(H, KH, SH, PH), conv_out(W, KW, SW, PW)), np.float32)
    lib().or_igemm_forward(_p(x), _p(w), _p(y), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)),
                           ctypes.c_int(int(bug_compat)))
    return y


def igemm_backward_input(dy, w, x_shape, stride=(1, 1), pad=(0, 0), bug_compat=False):
    dy, w = _f32(dy), _f32(w)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x_shape, w.shape, stride, pad)
    dx = np.empty(tuple(x_shape), np.float32)
    lib().or_igemm_backward_input(_p(dy), _p(w), _p(dx), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)),
                                  ctypes.c_int(int(bug_compat)))
    return dx


def igemm_backward_weight(x, dy, w_shape, stride=(1, 1), pad=(0, 0), bug_compat=False):
    x, dy = _f32(x), _f32(dy)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x.shape, w_shape, stride, pad)
    dw = np.empty(tuple(w_shape), np.float32)
    lib().or_igemm_backward_weight(_p(x), _p(dy), _p(dw), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)),
                                   ctypes.c_int(int(bug_compat)))
    return dw


def convt_out(h: int, k: int, s: int, p: int) -> int:
    return (h - 1) * s + k - 2 * p


def conv_transpose_forward(x, w, bias=None, stride=(1, 1), pad=(0, 0)):
    x, w = _f32(x), _f32(w)
    B, CI, H, W = x.shape
    CI2, CO, KH, KW = w.shape
    assert CI == CI2
    SH, SW = stride
    PH, PW = pad
    y = np.empty((B, CO, convt_out(H, KH, SH, PH), convt_out(W, KW, SW, PW)), np.float32)
    b = None if bias is None else _f32(bias)
    lib().or_conv_transpose_forward(_p(x), _p(w), _pn(b), _p(y), *map(_SZ, (B, CI, CO, H, W, KH, KW, SH, SW, PH, PW)))
    return y


def conv_transpose_backward(dy, x, w, stride=(1, 1), pad=(0, 0)):
    dy, x, w = _f32(dy), _f32(x), _f32(w)
    B, CI, H, W = x.shape
    _, CO, KH, KW = w.shape
    SH, SW = stride
    PH, PW = pad
    dx = np.empty(x.shape, np.float32)
    dw = np.empty(w.shape, np.float32)
    db = np.empty((CO,), np.float32)
    lib().or_conv_transpose_backward(_p(dy), _p(x), _p(w), _p(dx), _p(dw), _p(db),
                                     *map(_SZ, (B, CI, CO, H, W, KH, KW, SH, SW, PH, PW)))
    return dx, dw, db


def linear_forward(x, w, bias=None):
    x, w = _f32(x), _f32(w)
    m, i = x.shape
    i2, o = w.shape
    assert i == i2
    y = np.empty((m, o), np.float32)
    b = None if bias is None else _f32(bias)
    lib().or_linear_forward(_p(x), _p(w), _pn(b), _p(y), _SZ(m), _SZ(i), _SZ(o))
    return y


def linear_backward(dy, x, w):
    dy, x, w = _f32(dy), _f32(x), _f32(w)
    m, i = x.shape
    _, o = w.shape
    dx = np.empty((m, i), np.float32)
    dw = np.empty((i, o), np.float32)
    db = np.empty((o,), np.float32)
    lib().or_linear_backward(_p(dy), _p(x), _p(w), _p(dx), _p(dw), _p(db), _SZ(m), _SZ(i), _SZ(o))
    return dx, dw, db


def pixel_shuffle(x, r):
    x = _f32(x)
    B, CR, H, W = x.shape
    assert CR % (r * r) == 0
    C = CR // (r * r)
    y = np.empty((B, C, H * r, W * r), np.float32)
    lib().or_pixel_shuffle(_p(x), _p(y), *map(_SZ, (B, C, H, W, r)))
    return y


def pixel_shuffle_backward(dy, r):
    dy = _f32(dy)
    B, C, HR, WR = dy.shape
    H, W = HR // r, WR // r
    dx = np.empty((B, C * r * r, H, W), np.float32)
    lib().or_pixel_shuffle_backward(_p(dy), _p(dx), *map(_SZ, (B, C, H, W, r)))
    return dx


def relu(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().or_relu(_p(x), _p(y), _SZ(x.size))
    return y


def relu_backward(g, x):
    g, x = _f32(g), _f32(x)
    dx = np.empty_like(x)
    lib().or_relu_backward(_p(g), _p(x), _p(dx), _SZ(x.size))
    return dx


def sum_all(x) -> float:
    """Volta's CPU Sum: one f32 accumulator in index order."""
    x = _f32(x)
    return float(lib().or_sum(_p(x), _SZ(x.size)))


def sum_backward(grad: float, shape):
    dx = np.empty(shape, np.float32)
    lib().or_sum_backward(ctypes.c_float(grad), _p(dx), _SZ(dx.size))
    return dx


def add(a, b):
    """gpu_add / accumulate_grad: a + b (f32)."""
    out = _f32(a).copy()
    b = _f32(b)
    lib().or_add_inplace(_p(out), _p(b), _SZ(out.size))
    return out


def optimizer_step(op, lr, param, grad, s1=None, s2=None, beta1=0.0, beta2=0.0, t=0.0, eps=0.0, weight_decay=0.0):
    """optimizer_step.wgsl on copies; returns (param, s1, s2)."""
    param = _f32(param).copy()
    grad = _f32(grad)
    s1 = np.zeros_like(param) if s1 is None else _f32(s1).copy()
    s2 = np.zeros_like(param) if s2 is None else _f32(s2).copy()
    lib().or_optimizer_step(op, lr, beta1, beta2, t, eps, weight_decay, _p(param), _p(grad), _p(s1), _p(s2),
                            _SZ(param.size))
    return param, s1, s2


def round_bf16(a) -> np.ndarray:
    """f32 values rounded to bf16 (RNE), returned as f32 (the bf16 oracle input)."""
    a = _f32(a)
    out = np.empty_like(a)
    lib().or_round_bf16(_p(a), _p(out), _SZ(a.size))
    return out


def bf16_bits(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    lib().or_f32_to_bf16_bits(_p(a), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), _SZ(a.size))
    return out


def conv_forward_f64(x, w, stride=(1, 1), pad=(0, 0)):
    x, w = _f32(x), _f32(w)
    B, C, O, H, W, KH, KW, SH, SW, PH, PW = _conv_dims(x.shape, w.shape, stride, pad)
    y = np.empty((B, O, conv_out(H, KH, SH, PH), conv_out(W, KW, SW, PW)), np.float64)
    lib().or_conv_forward_f64(_p(x), _p(w), y.ctypes.data_as(_DP), *map(_SZ, (B, C, O, H, W, KH, KW, SH, SW, PH, PW)))
    return y
