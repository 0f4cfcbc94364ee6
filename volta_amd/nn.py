"""Layer-level mirror of Volta's Conv2d / ConvTranspose2d / Linear / PixelShuffle.

The composition (algorithm choice, bias add, which gradients are produced)
runs in C++ inside libvolta_hip.so (``vh_conv2d_forward`` and friends); these
classes hold parameters as torch device tensors in the reference's layouts
and call it.  Gradients are explicit (``backward`` returns them) instead of
going through an autograd graph: the reference's GradFn objects
(conv.rs:139-1013, conv_transpose.rs:150-353, matmul.rs:374-680) map onto the
``backward`` methods here.
"""
from __future__ import annotations

import ctypes
import enum
import math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import ALGO_AUTO, ALGO_DIRECT, ALGO_IGEMM, ALGO_IM2COL, VoltaHipError, check, lib
from .ops import _same_dtype, expect_numel, ptr, stream_ptr


class ConvAlgo(enum.IntEnum):
    """conv.rs:11-24 -- same variants and order."""

    Direct = ALGO_DIRECT
    Im2col = ALGO_IM2COL
    IGEMM = ALGO_IGEMM
    Auto = ALGO_AUTO

    @staticmethod
    def auto_select(batch, channels, height, width, kernel_size, has_gpu) -> "ConvAlgo":
        """conv.rs:29-69, the reference's rule verbatim (computed in C++)."""
        v = lib().vh_conv_algo_auto_select(batch, channels, height, width, kernel_size, int(bool(has_gpu)))
        if v < 0:
            raise ValueError("input smaller than kernel (the reference underflows here)")
        return ConvAlgo(v)


def conv_out(h: int, k: int, s: int, p: int) -> int:
    return (h + 2 * p - k) // s + 1


class Conv2d:
    """conv.rs:129-135, 1017-1115, 1787-1927.  weight [O, C, K, K] (OIHW), bias [O]."""

    def __init__(self, in_ch: int, out_ch: int, kernel: int, stride: int = 1, padding: int = 0,
                 use_bias: bool = True, device="cuda", dtype=torch.float32, generator=None):
        fan_in = in_ch * kernel * kernel
        # Kaiming (He) normal init like RawTensor::he_initialization (tensor.rs:276-312)
        w = torch.randn((out_ch, in_ch, kernel, kernel), generator=generator) * math.sqrt(2.0 / fan_in)
        self.weight = w.to(device=device, dtype=dtype).contiguous()
        self.bias = torch.zeros(out_ch, device=device, dtype=dtype) if use_bias else None
        self.stride = (stride, stride)
        self.padding = (padding, padding)
        self.algo = ConvAlgo.Auto
        self.last_algo: Optional[ConvAlgo] = None

    def set_algo(self, algo: ConvAlgo) -> None:
        self.algo = ConvAlgo(algo)

    def get_algo(self) -> ConvAlgo:
        return self.algo

    def _dims(self, x: torch.Tensor):
        B, C, H, W = x.shape
        O, C2, KH, KW = self.weight.shape
        if C != C2:
            raise ValueError("Channel mismatch")
        return (B, C, O, H, W, KH, KW, self.stride[0], self.stride[1], self.padding[0], self.padding[1])

    def output_shape(self, x: torch.Tensor):
        B, C, O, H, W, KH, KW, SH, SW, PH, PW = self._dims(x)
        return (B, O, conv_out(H, KH, SH, PH), conv_out(W, KW, SW, PW))

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None, relu: bool = False) -> torch.Tensor:
        """relu=True: the layer followed by ReLU, fused (vh_conv2d_forward_relu)."""
        dt = _same_dtype(x, self.weight, self.bias)
        y = out if out is not None else torch.empty(self.output_shape(x), dtype=x.dtype, device=x.device)
        expect_numel(y, math.prod(self.output_shape(x)), "Conv2d.forward out")
        used = ctypes.c_int(-1)
        fn = lib().vh_conv2d_forward_relu if relu else lib().vh_conv2d_forward
        check(fn(dt, int(self.algo), ptr(x), ptr(self.weight), ptr(self.bias), ptr(y), *self._dims(x),
                 ctypes.byref(used), stream_ptr(x.device)))
        self.last_algo = ConvAlgo(used.value)
        return y

    __call__ = forward

    def backward(self, out_grad: torch.Tensor, x: torch.Tensor, input_grad: bool = True,
                 weight_grad: bool = True, algo: Optional[ConvAlgo] = None,
                 outs: Optional[Tuple] = None, relu_input: bool = False):
        """Returns (grad_input, grad_weight, grad_bias); None where not requested.
        relu_input=True: x came out of a ReLU; grad_input gets that ReLU's backward
        (zero where x <= 0), fused (vh_conv2d_backward_relu)."""
        algo = ConvAlgo(algo if algo is not None else (self.last_algo if self.last_algo is not None else self.algo))
        if algo == ConvAlgo.Auto:
            B, C, O, H, W, KH, KW, SH, SW, PH, PW = self._dims(x)
            algo = ConvAlgo(lib().vh_conv_algo_select_mi355x(B, C, O, H, W, KH, KW, SH, SW, PH, PW))
        dt = _same_dtype(out_grad, x, self.weight)
        if outs is not None:
            dx, dw, db = outs
        else:
            dx = torch.empty_like(x) if input_grad else None
            dw = torch.empty_like(self.weight) if weight_grad else None
            db = torch.empty_like(self.bias) if (self.bias is not None and weight_grad) else None
        expect_numel(out_grad, math.prod(self.output_shape(x)), "Conv2d.backward out_grad")
        expect_numel(dx, x.numel(), "Conv2d.backward grad_input")
        expect_numel(dw, self.weight.numel(), "Conv2d.backward grad_weight")
        expect_numel(db, self.weight.shape[0], "Conv2d.backward grad_bias")
        fn = lib().vh_conv2d_backward_relu if relu_input else lib().vh_conv2d_backward
        check(fn(dt, int(algo), ptr(out_grad), ptr(x), ptr(self.weight), ptr(dx), ptr(dw), ptr(db), *self._dims(x),
                 stream_ptr(x.device)))
        return dx, dw, db


class ConvTranspose2d:
    """conv_transpose.rs:21-58, 356-435.  weight [in, out, K, K] (IOHW), bias [out]."""

    def __init__(self, in_ch: int, out_ch: int, kernel: int, stride: int = 1, padding: int = 0,
                 use_bias: bool = True, device="cuda", dtype=torch.float32, generator=None):
        fan_in = out_ch * kernel * kernel  # he_initialization uses prod(shape[1..]) (tensor.rs:283-298)
        w = torch.randn((in_ch, out_ch, kernel, kernel), generator=generator) * math.sqrt(2.0 / fan_in)
        self.weight = w.to(device=device, dtype=dtype).contiguous()
        self.bias = torch.zeros(out_ch, device=device, dtype=dtype) if use_bias else None
        self.stride = (stride, stride)
        self.padding = (padding, padding)

    def _dims(self, x):
        B, CI, H, W = x.shape
        CI2, CO, KH, KW = self.weight.shape
        if CI != CI2:
            raise ValueError(f"Channel mismatch: input has {CI} channels but weight expects {CI2}")
        return (B, CI, CO, H, W, KH, KW, self.stride[0], self.stride[1], self.padding[0], self.padding[1])

    def output_shape(self, x):
        B, CI, CO, H, W, KH, KW, SH, SW, PH, PW = self._dims(x)
        return (B, CO, (H - 1) * SH + KH - 2 * PH, (W - 1) * SW + KW - 2 * PW)

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        dt = _same_dtype(x, self.weight, self.bias)
        y = out if out is not None else torch.empty(self.output_shape(x), dtype=x.dtype, device=x.device)
        expect_numel(y, math.prod(self.output_shape(x)), "ConvTranspose2d.forward out")
        check(lib().vh_conv_transpose2d_forward(dt, ptr(x), ptr(self.weight), ptr(self.bias), ptr(y),
                                                *self._dims(x), stream_ptr(x.device)))
        return y

    __call__ = forward

    def backward(self, out_grad, x, input_grad=True, weight_grad=True, outs=None):
        dt = _same_dtype(out_grad, x, self.weight)
        if outs is not None:
            dx, dw, db = outs
        else:
            dx = torch.empty_like(x) if input_grad else None
            dw = torch.empty_like(self.weight) if weight_grad else None
            db = torch.empty_like(self.bias) if (self.bias is not None and weight_grad) else None
        expect_numel(out_grad, math.prod(self.output_shape(x)), "ConvTranspose2d.backward out_grad")
        expect_numel(dx, x.numel(), "ConvTranspose2d.backward grad_input")
        expect_numel(dw, self.weight.numel(), "ConvTranspose2d.backward grad_weight")
        expect_numel(db, self.weight.shape[1], "ConvTranspose2d.backward grad_bias")
        check(lib().vh_conv_transpose2d_backward(dt, ptr(out_grad), ptr(x), ptr(self.weight), ptr(dx), ptr(dw),
                                                 ptr(db), *self._dims(x), stream_ptr(x.device)))
        return dx, dw, db


class Linear:
    """linear.rs:11-117.  weight [in, out] (xavier-uniform), bias [out]."""

    def __init__(self, in_features: int, out_features: int, use_bias: bool = True, device="cuda",
                 dtype=torch.float32, generator=None):
        bound = math.sqrt(6.0 / (in_features + out_features))  # xavier_uniform, tensor.rs:254-265
        w = (torch.rand((in_features, out_features), generator=generator) * 2 - 1) * bound
        self.weight = w.to(device=device, dtype=dtype).contiguous()
        self.bias = torch.zeros(out_features, device=device, dtype=dtype) if use_bias else None

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        dt = _same_dtype(x, self.weight, self.bias)
        m, i = x.shape
        o = self.weight.shape[1]
        if i != self.weight.shape[0]:
            raise VoltaHipError(_lib.VH_ERR_BAD_SHAPE, f"Linear: input has {i} features, weight expects "
                                                       f"{self.weight.shape[0]}")
        y = out if out is not None else torch.empty((m, o), dtype=x.dtype, device=x.device)
        expect_numel(y, m * o, "Linear.forward out")
        check(lib().vh_linear_forward(dt, ptr(x), ptr(self.weight), ptr(self.bias), ptr(y), m, i, o,
                                      stream_ptr(x.device)))
        return y

    __call__ = forward

    def backward(self, out_grad, x, input_grad=True, weight_grad=True, outs=None):
        dt = _same_dtype(out_grad, x, self.weight)
        m, i = x.shape
        o = self.weight.shape[1]
        if outs is not None:
            dx, dw, db = outs
        else:
            dx = torch.empty_like(x) if input_grad else None
            dw = torch.empty_like(self.weight) if weight_grad else None
            db = torch.empty_like(self.bias) if (self.bias is not None and weight_grad) else None
        if i != self.weight.shape[0]:
            raise VoltaHipError(_lib.VH_ERR_BAD_SHAPE, f"Linear: input has {i} features, weight expects "
                                                       f"{self.weight.shape[0]}")
        expect_numel(out_grad, m * o, "Linear.backward out_grad")
        expect_numel(dx, m * i, "Linear.backward grad_x")
        expect_numel(dw, i * o, "Linear.backward grad_weight")
        expect_numel(db, o, "Linear.backward grad_bias")
        check(lib().vh_linear_backward(dt, ptr(out_grad), ptr(x), ptr(self.weight), ptr(dx), ptr(dw), ptr(db),
                                       m, i, o, stream_ptr(x.device)))
        return dx, dw, db


class PixelShuffle:
    """pixelshuffle.rs:27-85: (B, C*r^2, H, W) -> (B, C, H*r, W*r)."""

    def __init__(self, upscale_factor: int):
        if upscale_factor <= 0:
            raise ValueError(f"PixelShuffle: upscale_factor must be positive, got {upscale_factor}")
        self.upscale_factor = upscale_factor

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, CR, H, W = x.shape
        r = self.upscale_factor
        if CR % (r * r):
            raise ValueError(f"PixelShuffle: input channels ({CR}) must be divisible by upscale_factor^2 ({r*r})")
        C = CR // (r * r)
        y = out if out is not None else torch.empty((B, C, H * r, W * r), dtype=x.dtype, device=x.device)
        check(lib().vh_pixel_shuffle(_same_dtype(x), ptr(x), ptr(y), B, C, H, W, r, stream_ptr(x.device)))
        return y

    __call__ = forward

    def backward(self, out_grad: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, C, HR, WR = out_grad.shape
        r = self.upscale_factor
        H, W = HR // r, WR // r
        dx = out if out is not None else torch.empty((B, C * r * r, H, W), dtype=out_grad.dtype,
                                                     device=out_grad.device)
        check(lib().vh_pixel_shuffle_backward(_same_dtype(out_grad), ptr(out_grad), ptr(dx), B, C, H, W, r,
                                              stream_ptr(out_grad.device)))
        return dx


class ReLU:
    """The ReLU between the config graphs' layers: forward max(x, 0)
    (unary.rs:272), backward out_grad where the forward input is positive
    (unary.rs:150-155)."""

    def forward(self, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        y = out if out is not None else torch.empty_like(x)
        check(lib().vh_unary(_same_dtype(x), _lib.UNARY_RELU, ptr(x), ptr(y), x.numel(), stream_ptr(x.device)))
        return y

    __call__ = forward

    def backward(self, out_grad: torch.Tensor, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        dx = out if out is not None else torch.empty_like(x)
        check(lib().vh_unary_backward(_same_dtype(out_grad, x), _lib.UNARY_RELU, ptr(out_grad), ptr(x), ptr(dx),
                                      x.numel(), stream_ptr(x.device)))
        return dx


def sum_loss(y: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Loss = sum of every element of y (reduce.rs:160-180), as a one-element
    fp32 device tensor (no host round trip)."""
    res = out if out is not None else torch.empty((1,), dtype=torch.float32, device=y.device)
    check(lib().vh_sum_reduce(_same_dtype(y), ptr(y), y.numel(), ptr(res), stream_ptr(y.device)))
    return res


def sum_loss_backward(y: torch.Tensor, grad: float = 1.0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dLoss/dy for the sum loss: every element = grad (SumGradFn, reduce.rs:22-45;
    grad = 1 is the autograd seed, autograd.rs:49-62)."""
    dy = out if out is not None else torch.empty_like(y)
    check(lib().vh_sum_backward(_same_dtype(y), float(grad), ptr(dy), y.numel(), stream_ptr(y.device)))
    return dy


class ConvChain:
    """The configs[0] / configs[4] graphs: a Sequential (sequential.rs) of
    Conv2d -> ReLU -> ... -> Conv2d, an optional tail layer (PixelShuffle) and the
    sum loss, with every activation and gradient buffer allocated once.

    Each ReLU is fused into the convolution that produces its input
    (vh_conv2d_forward_relu) and its backward into the next layer's input
    gradient (vh_conv2d_backward_relu).  ``acts[i]`` is layer i's input
    (``acts[0]`` the graph input, ``acts[i]`` = ReLU(conv_{i-1}) for 0 < i < L,
    ``acts[L]`` the last conv's output); ``grads[i]`` is the gradient with
    respect to conv_{i-1}'s output before its ReLU (``grads[L]`` w.r.t. the last
    output).  The first layer computes no input gradient (the graph input needs
    none)."""

    def __init__(self, specs, x: torch.Tensor, tail=None, generator=None, algo: ConvAlgo = ConvAlgo.Auto):
        """specs: (C, O, K, stride, pad) per conv layer; x: the graph input
        [N, C0, H, W] (kept); tail: a layer with forward(x, out=) / backward(g, out=)."""
        dev, dt = x.device, x.dtype
        self.convs = []
        self.acts = [x]
        shape = tuple(x.shape)
        for C, O, K, S, P in specs:
            if shape[1] != C:
                raise ValueError(f"ConvChain: layer expects {C} channels, gets {shape[1]}")
            conv = Conv2d(C, O, K, S, P, use_bias=True, device=dev, dtype=dt, generator=generator)
            conv.set_algo(algo)
            shape = (shape[0], O, conv_out(shape[2], K, S, P), conv_out(shape[3], K, S, P))
            self.convs.append(conv)
            self.acts.append(torch.empty(shape, device=dev, dtype=dt))
        self.grads = [None] + [torch.empty_like(a) for a in self.acts[1:]]
        self.wgrads = [(torch.empty_like(c.weight), torch.empty_like(c.bias)) for c in self.convs]
        self.tail = tail
        self.tail_out = self.tail_grad = None
        if tail is not None:
            self.tail_out = tail.forward(self.acts[-1])
            self.tail_grad = torch.empty_like(self.tail_out)
        self.loss = torch.empty((1,), device=dev, dtype=torch.float32)

    @property
    def output(self) -> torch.Tensor:
        return self.tail_out if self.tail is not None else self.acts[-1]

    def forward(self) -> torch.Tensor:
        """Forward of every layer and the loss; returns the one-element fp32 loss."""
        L = len(self.convs)
        for i, conv in enumerate(self.convs):
            conv.forward(self.acts[i], out=self.acts[i + 1], relu=i + 1 < L)
        if self.tail is not None:
            self.tail.forward(self.acts[-1], out=self.tail_out)
        return sum_loss(self.output, out=self.loss)

    def backward(self, grad: float = 1.0) -> None:
        """Seeds dLoss/dOutput = grad (the autograd seed for grad = 1) and runs the
        backward chain: gradients land in ``grads`` and ``wgrads``."""
        L = len(self.convs)
        if self.tail is not None:
            sum_loss_backward(self.tail_out, grad, out=self.tail_grad)
            self.tail.backward(self.tail_grad, out=self.grads[L])
        else:
            sum_loss_backward(self.acts[-1], grad, out=self.grads[L])
        for i in range(L - 1, -1, -1):
            dw, db = self.wgrads[i]
            self.convs[i].backward(self.grads[i + 1], self.acts[i], input_grad=i > 0, weight_grad=True,
                                   outs=(self.grads[i] if i > 0 else None, dw, db), relu_input=i > 0)

    def step(self) -> None:
        """One fwd+bwd training step of the graph."""
        self.forward()
        self.backward()

    def passes(self):
        """name -> callable of each pass alone (forward, input gradient, weight
        gradient of every layer, the tail, the loss and its seed), for timing."""
        L = len(self.convs)
        out = {}
        for i, conv in enumerate(self.convs):
            def fwd(i=i, conv=conv):
                conv.forward(self.acts[i], out=self.acts[i + 1], relu=i + 1 < L)

            def wgrad(i=i, conv=conv):
                conv.backward(self.grads[i + 1], self.acts[i], input_grad=False, weight_grad=True,
                              outs=(None,) + self.wgrads[i])
            out[f"L{i} fwd"] = fwd
            if i > 0:
                def dgrad(i=i, conv=conv):
                    conv.backward(self.grads[i + 1], self.acts[i], input_grad=True, weight_grad=False,
                                  outs=(self.grads[i], None, None), relu_input=True)
                out[f"L{i} dgrad"] = dgrad
            out[f"L{i} wgrad"] = wgrad
        if self.tail is not None:
            out["tail fwd"] = lambda: self.tail.forward(self.acts[-1], out=self.tail_out)
            out["tail bwd"] = lambda: self.tail.backward(self.tail_grad, out=self.grads[L])
        out["loss"] = lambda: sum_loss(self.output, out=self.loss)
        out["seed"] = lambda: sum_loss_backward(self.output, 1.0,
                                                out=self.tail_grad if self.tail is not None else self.grads[L])
        return out
