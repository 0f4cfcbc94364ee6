#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ (run from the repo root).

Each fixture is one layer of a BASELINE configuration, cut down to batch 2
(and, where the weights would be large, a spatial or output-channel crop)
so the committed data stays small while the contraction depth K = C*R*S of
the real layer is kept:

    C1  MNIST-CNN conv1 / conv2                       f32
    C2  Linear 1024 -> (cropped) out, deep-K square    f32, bf16
    C3  ResNet 3x3 layers and the 1x1 s2 projection    bf16
    C4  DCGAN ConvTranspose2d layers                   f32
    C5  super-resolution convs + PixelShuffle r=3      bf16

Inputs are seeded numpy draws (x ~ N(0,1) or U[0,1), Kaiming / N(0,0.02)
weights, a small non-zero bias, dY ~ N(0,1)); bf16 cases hold values already
rounded to bf16 (round-to-nearest-even) and their expected outputs are f32
math on those values, since Volta has no bf16 arithmetic.  Expected outputs
come from the CPU restatement of Volta's loops (oracle/), and every one is
cross-checked here against torch float64 before it is written, so a fixture
never records an oracle mistake.  Stored as compressed .npz, loadable with
numpy's default allow_pickle=False; bf16 inputs are stored as their raw
16-bit patterns (``<name>_bf16``), outputs as float32.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

# (name, dtype, B, C, O, H, W, K, S, P, x_dist)
CONV = [
    ("c1_conv1", "f32", 2, 1, 32, 16, 16, 3, 1, 1, "normal"),
    ("c1_conv2", "f32", 2, 32, 64, 10, 10, 3, 1, 1, "normal"),
    ("c3_3x3_64", "bf16", 2, 64, 64, 10, 10, 3, 1, 1, "normal"),
    ("c3_3x3_128", "bf16", 2, 128, 32, 8, 8, 3, 1, 1, "normal"),
    ("c3_3x3_256", "bf16", 2, 256, 16, 6, 6, 3, 1, 1, "normal"),
    ("c3_1x1_s2", "bf16", 2, 64, 128, 12, 12, 1, 2, 0, "normal"),
    ("c5_conv1_5x5", "bf16", 2, 3, 64, 14, 14, 5, 1, 2, "uniform"),
    ("c5_conv2", "bf16", 2, 64, 64, 8, 8, 3, 1, 1, "uniform"),
    ("c5_conv3", "bf16", 2, 64, 32, 8, 8, 3, 1, 1, "uniform"),
    ("c5_conv4", "bf16", 2, 32, 27, 8, 8, 3, 1, 1, "uniform"),
]
# (name, dtype, B, CI, CO, H, W, K, S, P)
CONVT = [
    ("c4_convt1", "f32", 2, 100, 16, 1, 1, 4, 1, 0),
    ("c4_convt2", "f32", 2, 512, 4, 4, 4, 4, 2, 1),
    ("c4_convt3", "f32", 2, 256, 8, 4, 4, 4, 2, 1),
    ("c4_convt4", "f32", 2, 128, 8, 6, 6, 4, 2, 1),
    ("c4_convt5", "f32", 2, 64, 3, 10, 10, 4, 2, 1),
]
# (name, dtype, M, IN, OUT, with_bias)
LINEAR = [
    ("c2_linear_f32", "f32", 8, 1024, 16, True),
    ("c2_linear_bf16", "bf16", 8, 1024, 16, True),
    ("c2_square_bf16", "bf16", 4, 8192, 4, False),
]
# (name, dtype, B, C*r*r, H, W, r)
SHUFFLE = [("c5_pixel_shuffle", "bf16", 2, 27, 8, 8, 3)]

TOL_VS_F64 = 1e-4  # scaled error of the f32 oracle against float64 truth


def _round(a, dt):
    import oracle

    a = np.ascontiguousarray(a, np.float32)
    return oracle.round_bf16(a) if dt == "bf16" else a


def _scaled(got, ref, scale):
    return float((np.abs(np.float64(got) - ref) / np.maximum(scale, 1e-30)).max()) if ref.size else 0.0


def _pin(name, what, got, ref64, scale64):
    e = _scaled(got, ref64, scale64)
    assert e <= TOL_VS_F64, f"{name}/{what}: oracle vs float64 scaled err {e:.3e}"


def conv_case(spec):
    import torch

    import oracle

    name, dt, B, C, O, H, W, K, S, P, dist = spec
    g = np.random.default_rng(sum(map(ord, name)))
    x = g.standard_normal((B, C, H, W)) if dist == "normal" else g.uniform(0, 1, (B, C, H, W))
    x = _round(x, dt)
    w = _round(g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K)), dt)
    b = _round(g.uniform(-0.1, 0.1, (O,)), dt)
    st, pd = (S, S), (P, P)
    y = oracle.direct_conv(x, w, st, pd) + b[None, :, None, None]
    dy = _round(g.standard_normal(y.shape), dt)
    dx = oracle.direct_conv_backward_input(dy, w, x.shape, st, pd)
    dw = oracle.direct_conv_backward_weight(dy, x, w.shape, st, pd)
    db = oracle.conv_bias_grad(dy)

    tx, tw, tb = (torch.from_numpy(np.float64(a)).requires_grad_() for a in (x, w, b))
    ty = torch.nn.functional.conv2d(tx, tw, tb, S, P)
    ty.backward(torch.from_numpy(np.float64(dy)))
    ax, aw, ab = (torch.from_numpy(np.abs(np.float64(a))).requires_grad_() for a in (x, w, b))
    sy = torch.nn.functional.conv2d(ax, aw, ab, S, P)
    sy.backward(torch.from_numpy(np.abs(np.float64(dy))))
    for what, got, ref, sc in (("y", y, ty, sy), ("dx", dx, tx.grad, ax.grad), ("dw", dw, tw.grad, aw.grad),
                               ("db", db, tb.grad, ab.grad)):
        _pin(name, what, got, ref.detach().numpy(), sc.detach().numpy())
    meta = np.array([B, C, O, H, W, K, S, P], np.int64)
    return dict(kind="conv", dtype=dt, meta=meta, x=x, w=w, b=b, dy=dy, y=y, dx=dx, dw=dw, db=db)


def convt_case(spec):
    import torch

    import oracle

    name, dt, B, CI, CO, H, W, K, S, P = spec
    g = np.random.default_rng(sum(map(ord, name)))
    x = _round(g.standard_normal((B, CI, H, W)), dt)
    w = _round(g.normal(0.0, 0.02, (CI, CO, K, K)), dt)
    b = _round(g.uniform(-0.1, 0.1, (CO,)), dt)
    st, pd = (S, S), (P, P)
    y = oracle.conv_transpose_forward(x, w, b, st, pd)
    dy = _round(g.standard_normal(y.shape), dt)
    dx, dw, db = oracle.conv_transpose_backward(dy, x, w, st, pd)

    tx, tw, tb = (torch.from_numpy(np.float64(a)).requires_grad_() for a in (x, w, b))
    ty = torch.nn.functional.conv_transpose2d(tx, tw, tb, S, P)
    ty.backward(torch.from_numpy(np.float64(dy)))
    ax, aw, ab = (torch.from_numpy(np.abs(np.float64(a))).requires_grad_() for a in (x, w, b))
    sy = torch.nn.functional.conv_transpose2d(ax, aw, ab, S, P)
    sy.backward(torch.from_numpy(np.abs(np.float64(dy))))
    for what, got, ref, sc in (("y", y, ty, sy), ("dx", dx, tx.grad, ax.grad), ("dw", dw, tw.grad, aw.grad),
                               ("db", db, tb.grad, ab.grad)):
        _pin(name, what, got, ref.detach().numpy(), sc.detach().numpy())
    meta = np.array([B, CI, CO, H, W, K, S, P], np.int64)
    return dict(kind="convt", dtype=dt, meta=meta, x=x, w=w, b=b, dy=dy, y=y, dx=dx, dw=dw, db=db)


def linear_case(spec):
    import torch

    import oracle

    name, dt, M, IN, OUT, with_bias = spec
    g = np.random.default_rng(sum(map(ord, name)))
    x = _round(g.standard_normal((M, IN)), dt)
    bound = np.sqrt(6.0 / (IN + OUT))
    w = _round(g.uniform(-bound, bound, (IN, OUT)), dt)
    b = _round(g.uniform(-1.0 / 32, 1.0 / 32, (OUT,)) if with_bias else np.zeros(OUT), dt)
    y = oracle.linear_forward(x, w, b)
    dy = _round(g.standard_normal(y.shape), dt)
    dx, dw, db = oracle.linear_backward(dy, x, w)

    tx, tw, tb = (torch.from_numpy(np.float64(a)).requires_grad_() for a in (x, w, b))
    ty = tx @ tw + tb
    ty.backward(torch.from_numpy(np.float64(dy)))
    ax, aw, ab = (torch.from_numpy(np.abs(np.float64(a))).requires_grad_() for a in (x, w, b))
    sy = ax @ aw + ab
    sy.backward(torch.from_numpy(np.abs(np.float64(dy))))
    for what, got, ref, sc in (("y", y, ty, sy), ("dx", dx, tx.grad, ax.grad), ("dw", dw, tw.grad, aw.grad),
                               ("db", db, tb.grad, ab.grad)):
        _pin(name, what, got, ref.detach().numpy(), sc.detach().numpy())
    meta = np.array([M, IN, OUT, int(with_bias)], np.int64)
    return dict(kind="linear", dtype=dt, meta=meta, x=x, w=w, b=b, dy=dy, y=y, dx=dx, dw=dw, db=db)


def shuffle_case(spec):
    import torch

    import oracle

    name, dt, B, CR, H, W, r = spec
    g = np.random.default_rng(sum(map(ord, name)))
    x = _round(g.uniform(0, 1, (B, CR, H, W)), dt)
    y = oracle.pixel_shuffle(x, r)
    dy = _round(g.standard_normal(y.shape), dt)
    dx = oracle.pixel_shuffle_backward(dy, r)
    assert np.array_equal(y, torch.nn.functional.pixel_shuffle(torch.from_numpy(x), r).numpy())
    assert np.array_equal(dx, torch.nn.functional.pixel_unshuffle(torch.from_numpy(dy), r).numpy())
    meta = np.array([B, CR, H, W, r], np.int64)
    return dict(kind="shuffle", dtype=dt, meta=meta, x=x, dy=dy, y=y, dx=dx)


def all_cases():
    for s in CONV:
        yield s[0], conv_case, s
    for s in CONVT:
        yield s[0], convt_case, s
    for s in LINEAR:
        yield s[0], linear_case, s
    for s in SHUFFLE:
        yield s[0], shuffle_case, s


def main():
    import oracle

    oracle.build()
    for name, fn, spec in all_cases():
        d = fn(spec)
        if d["dtype"] == "bf16":
            for k in ("x", "w", "b", "dy"):
                if k in d:
                    d[k + "_bf16"] = oracle.bf16_bits(d.pop(k))
        d = {k: np.asarray(v) for k, v in d.items()}
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **d)
        print(f"{name}: {sum(v.nbytes for v in d.values()) / 1024:.0f} KiB raw")


if __name__ == "__main__":
    main()
