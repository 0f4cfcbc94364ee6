"""Python mirror of Volta's device-dispatch boundary (src/ops/gpu_ops.rs).

Each ``gpu_*`` function keeps the reference's name and argument order
(``gpu_ops.rs:151-861``) and calls the matching C-ABI entry of
libvolta_hip.so on torch device tensors.  Like the reference, the ``gpu_*``
functions return ``None`` instead of raising when the device path cannot run
(no GPU / CPU tensor), so a caller can keep a CPU fallback; shape errors
raise (the reference panics there).  Outputs are allocated by the callee, as
``GpuBuffer::zeros`` does in the reference.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import BF16, F32, VoltaHipError, check, lib

_DTYPES = {torch.float32: F32, torch.bfloat16: BF16}


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; libvolta_hip takes float32 or bfloat16") from None


def stream_ptr(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("libvolta_hip takes device tensors")
    if not t.is_contiguous():
        raise ValueError("libvolta_hip takes contiguous tensors")
    return t.data_ptr()


def _device_ok(*ts: torch.Tensor) -> bool:
    return all(t is not None and t.is_cuda for t in ts)


def _same_dtype(*ts: torch.Tensor) -> int:
    code = dtype_code(ts[0])
    for t in ts[1:]:
        if t is not None and t.dtype != ts[0].dtype:
            raise TypeError("all tensor arguments of one call must share a dtype")
    return code


def _call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def expect_numel(t: Optional[torch.Tensor], n: int, what: str) -> None:
    """The C ABI carries no tensor sizes: a tensor smaller than its dimensions
    say would be read or written out of bounds.  Raises VH_ERR_BAD_SHAPE (the
    reference's assert_eq! panic, kernels.rs:1129-1130) before any launch.  An
    empty problem (n == 0, e.g. batch 0) touches no memory and is not checked."""
    if t is not None and n > 0 and t.numel() != n:
        raise VoltaHipError(_lib.VH_ERR_BAD_SHAPE,
                            f"{what}: tensor holds {t.numel()} elements, the dimensions give {n}")


def _optional(fn):
    """Reference semantics: Option::None when the device path is unavailable."""

    def wrapper(*args, **kwargs):
        tensors = [a for a in args if isinstance(a, torch.Tensor)]
        if not _device_ok(*tensors):
            return None
        try:
            return fn(*args, **kwargs)
        except VoltaHipError as e:
            if e.status in (_lib.VH_ERR_NO_DEVICE, _lib.VH_ERR_OOM):
                return None
            raise

    wrapper.__name__ = fn.__name__
    wrapper.__doc__ = fn.__doc__
    return wrapper


# ---------------------------------------------------------------- matmul
@_optional
def gpu_matmul(a: torch.Tensor, b: torch.Tensor, m: int, k: int, n: int):
    """gpu_ops.rs:151 -- c[m,n] = a[m,k] . b[k,n]."""
    dt = _same_dtype(a, b)
    expect_numel(a, m * k, "gpu_matmul a")
    expect_numel(b, k * n, "gpu_matmul b")
    c = torch.empty((m, n), dtype=a.dtype, device=a.device)
    _call("vh_matmul", dt, ptr(a), ptr(b), ptr(c), m, k, n, stream_ptr(a.device))
    return c


@_optional
def gpu_matmul_backward_a(grad: torch.Tensor, b: torch.Tensor, m: int, k: int, n: int):
    """gpu_ops.rs:408 -- grad_a[m,k] = grad[m,n] . b[k,n]^T."""
    dt = _same_dtype(grad, b)
    expect_numel(grad, m * n, "gpu_matmul_backward_a grad")
    expect_numel(b, k * n, "gpu_matmul_backward_a b")
    out = torch.empty((m, k), dtype=grad.dtype, device=grad.device)
    _call("vh_matmul_backward_a", dt, ptr(grad), ptr(b), ptr(out), m, k, n, stream_ptr(grad.device))
    return out


@_optional
def gpu_matmul_backward_b(a: torch.Tensor, grad: torch.Tensor, m: int, k: int, n: int):
    """gpu_ops.rs:430 -- grad_b[k,n] = a[m,k]^T . grad[m,n]."""
    dt = _same_dtype(a, grad)
    expect_numel(a, m * k, "gpu_matmul_backward_b a")
    expect_numel(grad, m * n, "gpu_matmul_backward_b grad")
    out = torch.empty((k, n), dtype=a.dtype, device=a.device)
    _call("vh_matmul_backward_b", dt, ptr(a), ptr(grad), ptr(out), m, k, n, stream_ptr(a.device))
    return out


# ---------------------------------------------------------------- im2col / col2im
@_optional
def gpu_im2col(input, batch_size, channels, height, width, kernel_h, kernel_w, stride_h, stride_w, h_out, w_out):
    """gpu_ops.rs:515 -- (B,C,H,W) (already padded) -> (B*h_out*w_out, C*kh*kw)."""
    dt = dtype_code(input)
    expect_numel(input, batch_size * channels * height * width, "gpu_im2col input")
    col = torch.empty((batch_size * h_out * w_out, channels * kernel_h * kernel_w), dtype=input.dtype,
                      device=input.device)
    _call("vh_im2col", dt, ptr(input), ptr(col), batch_size, channels, height, width, kernel_h, kernel_w,
          stride_h, stride_w, h_out, w_out, stream_ptr(input.device))
    return col


@_optional
def gpu_col2im(col, batch_size, channels, height, width, kernel_h, kernel_w, stride_h, stride_w, h_out, w_out):
    """gpu_ops.rs:546 -- adjoint of gpu_im2col."""
    dt = dtype_code(col)
    expect_numel(col, batch_size * h_out * w_out * channels * kernel_h * kernel_w, "gpu_col2im col")
    out = torch.empty((batch_size, channels, height, width), dtype=col.dtype, device=col.device)
    _call("vh_col2im", dt, ptr(col), ptr(out), batch_size, channels, height, width, kernel_h, kernel_w,
          stride_h, stride_w, h_out, w_out, stream_ptr(col.device))
    return out


# ---------------------------------------------------------------- conv kernels
_CONV_OPERANDS = {  # which tensors each conv entry takes: x (input), w (weight), y (out_grad)
    "vh_direct_conv": "xw", "vh_igemm": "xw", "vh_conv_backward_input": "yw", "vh_igemm_backward_input": "yw",
    "vh_conv_backward_weight": "yx", "vh_igemm_backward_weight": "yx"}


def _conv_call(name, t0, t1, out_shape, dims):
    dt = _same_dtype(t0, t1)
    B, C, O, H, W, KH, KW = dims[:7]
    HO, WO = dims[11:13]
    sizes = {"x": B * C * H * W, "w": O * C * KH * KW, "y": B * O * HO * WO}
    for t, role in zip((t0, t1), _CONV_OPERANDS[name]):
        expect_numel(t, sizes[role], f"{name} {dict(x='input', w='weight', y='out_grad')[role]}")
    out = torch.empty(out_shape, dtype=t0.dtype, device=t0.device)
    _call(name, dt, ptr(t0), ptr(t1), ptr(out), *dims, stream_ptr(t0.device))
    return out


@_optional
def gpu_direct_conv(input, weight, batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w,
                    stride_h, stride_w, pad_h, pad_w, h_out, w_out):
    """gpu_ops.rs:574 (stride before pad)."""
    dims = (batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
            pad_h, pad_w, h_out, w_out)
    return _conv_call("vh_direct_conv", input, weight, (batch_size, out_channels, h_out, w_out), dims)


@_optional
def gpu_igemm(input, weight, batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w,
              stride_h, stride_w, pad_h, pad_w, h_out, w_out):
    """gpu_ops.rs:622."""
    dims = (batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
            pad_h, pad_w, h_out, w_out)
    return _conv_call("vh_igemm", input, weight, (batch_size, out_channels, h_out, w_out), dims)


@_optional
def gpu_conv_backward_input(out_grad, weight, batch_size, in_channels, out_channels, height, width, kernel_h,
                            kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out):
    """gpu_ops.rs:670."""
    dims = (batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
            pad_h, pad_w, h_out, w_out)
    return _conv_call("vh_conv_backward_input", out_grad, weight, (batch_size, in_channels, height, width), dims)


@_optional
def gpu_conv_backward_weight(out_grad, input, batch_size, in_channels, out_channels, height, width, kernel_h,
                             kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out):
    """gpu_ops.rs:718 -- note (out_grad, input)."""
    dims = (batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
            pad_h, pad_w, h_out, w_out)
    return _conv_call("vh_conv_backward_weight", out_grad, input, (out_channels, in_channels, kernel_h, kernel_w),
                      dims)


@_optional
def gpu_igemm_backward_input(out_grad, weight, batch_size, in_channels, out_channels, height, width, kernel_h,
                             kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out):
    """gpu_ops.rs:766."""
    dims = (batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
            pad_h, pad_w, h_out, w_out)
    return _conv_call("vh_igemm_backward_input", out_grad, weight, (batch_size, in_channels, height, width), dims)


@_optional
def gpu_igemm_backward_weight(out_grad, input, batch_size, in_channels, out_channels, height, width, kernel_h,
                              kernel_w, stride_h, stride_w, pad_h, pad_w, h_out, w_out):
    """gpu_ops.rs:814."""
    dims = (batch_size, in_channels, out_channels, height, width, kernel_h, kernel_w, stride_h, stride_w,
            pad_h, pad_w, h_out, w_out)
    return _conv_call("vh_igemm_backward_weight", out_grad, input,
                      (out_channels, in_channels, kernel_h, kernel_w), dims)


# ---------------------------------------------------------------- glue: ReLU, sum loss
_UNARY_OPS = {"relu": _lib.UNARY_RELU}


def _unary_code(op: str) -> int:
    try:
        return _UNARY_OPS[op]
    except KeyError:
        raise ValueError(f"unary op {op!r}: only 'relu' is on this path") from None


@_optional
def gpu_unary(input: torch.Tensor, op: str):
    """gpu_ops.rs:171 -- elementwise op (ReLU: max(x, 0), unary.rs:272)."""
    code = _unary_code(op)
    x = input.contiguous()
    y = torch.empty_like(x)
    _call("vh_unary", dtype_code(x), code, ptr(x), ptr(y), x.numel(), stream_ptr(x.device))
    return y


@_optional
def gpu_unary_backward(out_grad: torch.Tensor, x: torch.Tensor, op: str):
    """gpu_ops.rs:186 -- ReLU: out_grad where x > 0, else 0 (unary.rs:150-155)."""
    code = _unary_code(op)
    dt = _same_dtype(out_grad, x)
    if out_grad.numel() != x.numel():
        raise ValueError("gpu_unary_backward: out_grad and x differ in size")
    dx = torch.empty_like(x)
    _call("vh_unary_backward", dt, code, ptr(out_grad), ptr(x), ptr(dx), x.numel(), stream_ptr(x.device))
    return dx


@_optional
def gpu_sum_reduce(data: torch.Tensor):
    """gpu_ops.rs:118 -- the fp32 sum of every element, returned to the host."""
    out = torch.empty((1,), dtype=torch.float32, device=data.device)
    _call("vh_sum_reduce", dtype_code(data), ptr(data), data.numel(), ptr(out), stream_ptr(data.device))
    return float(out.item())


def gpu_sum_backward(grad: float, input_size: int, dtype=torch.float32, device="cuda:0"):
    """gpu_ops.rs:452 -- a buffer of `input_size` elements equal to `grad`
    (SumGradFn; the autograd seed when grad = 1).  None without a device."""
    if not torch.cuda.is_available():
        return None
    out = torch.empty((input_size,), dtype=dtype, device=device)
    try:
        _call("vh_sum_backward", _DTYPES[dtype], float(grad), ptr(out), input_size, stream_ptr(out.device))
    except VoltaHipError as e:
        if e.status in (_lib.VH_ERR_NO_DEVICE, _lib.VH_ERR_OOM):
            return None
        raise
    return out


# ---------------------------------------------------------------- the step after dW
@_optional
def gpu_add(a: torch.Tensor, b: torch.Tensor):
    """gpu_ops.rs:17 as used by accumulate_grad (autograd.rs:158-184): a + b."""
    dt = _same_dtype(a, b)
    if a.numel() != b.numel():
        raise ValueError("gpu_add: size mismatch")
    out = a.clone()
    _call("vh_grad_accumulate", dt, ptr(out), ptr(b), out.numel(), stream_ptr(a.device))
    return out


@_optional
def gpu_optimizer_step(params: torch.Tensor, grads: torch.Tensor, state1: torch.Tensor, state2: torch.Tensor,
                       op: int, lr: float, beta1: float = 0.0, beta2: float = 0.0, t: float = 0.0, eps: float = 0.0,
                       weight_decay: float = 0.0):
    """gpu_ops.rs:496 -- updates params (and the states) in place; f32 tensors."""
    for x in (params, grads, state1, state2):
        if x.dtype != torch.float32:
            raise TypeError("gpu_optimizer_step takes float32 tensors")
    _call("vh_optimizer_step", op, lr, beta1, beta2, t, eps, weight_decay, ptr(params), ptr(grads), ptr(state1),
          ptr(state2), params.numel(), stream_ptr(params.device))
    return ()


# ---------------------------------------------------------------- device storage: dtype and layout
def to_dtype(x: torch.Tensor, dtype) -> torch.Tensor:
    """Device cast f32 <-> bf16 (RNE), the library's conversion."""
    out = torch.empty(x.shape, dtype=dtype, device=x.device)
    _call("vh_cast", dtype_code(x), _DTYPES[dtype], ptr(x), ptr(out), x.numel(), stream_ptr(x.device))
    return out


def nchw_to_nhwc(x: torch.Tensor) -> torch.Tensor:
    B, C, H, W = x.shape
    out = torch.empty((B, H, W, C), dtype=x.dtype, device=x.device)
    _call("vh_nchw_to_nhwc", dtype_code(x), ptr(x), ptr(out), B, C, H, W, stream_ptr(x.device))
    return out


def nhwc_to_nchw(x: torch.Tensor) -> torch.Tensor:
    B, H, W, C = x.shape
    out = torch.empty((B, C, H, W), dtype=x.dtype, device=x.device)
    _call("vh_nhwc_to_nchw", dtype_code(x), ptr(x), ptr(out), B, C, H, W, stream_ptr(x.device))
    return out
