"""GPU: the BASELINE configurations at their full sizes.

The oracle cannot run every pass at these sizes in seconds, so each full-size
launch is checked through properties that do not depend on the batch size:

* forward and input gradient are independent per image (per row for a
  product): a few images / rows of the full-size result are compared with the
  oracle run on just those images / rows;
* weight (and bias) gradients are sums over images / rows: the full-size
  kernel is run with dY zero except on a few images / rows, and the result
  must equal the oracle's gradient over those images / rows alone;
* data movement (PixelShuffle) is compared in full, bit for bit.

The launches are exactly the full-size ones (grid, tiling, split-K plan depend
only on the shapes).  Inputs follow each configuration's distributions."""
import numpy as np
import pytest
import torch

import oracle
from tests.parity import assert_parity
from volta_amd import nn as vnn
from volta_amd import ops

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def prep(a, dt):
    a = np.ascontiguousarray(a, np.float32)
    r = oracle.round_bf16(a) if dt == "bf16" else a
    return r, torch.from_numpy(r).to(DEV, DT[dt])


def scaled(fn, args, kw):
    return fn(*args, **kw), fn(*[np.abs(a) if isinstance(a, np.ndarray) else a for a in args], **kw)


def conv_full(B, C, O, H, K, S, P, dt, algo, seed, x_dist="normal", images=(0, -1), dw_images=(1, -2),
              bias=True):
    g = np.random.default_rng(seed)
    xs = (B, C, H, H)
    x, xt = prep(g.standard_normal(xs) if x_dist == "normal" else g.uniform(0, 1, xs), dt)
    w, wt = prep(g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K)), dt)
    b, bt = prep(g.uniform(-0.1, 0.1, (O,)) if bias else np.zeros(O), dt)
    conv = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=DEV, dtype=DT[dt])
    conv.weight, conv.bias = wt, bt
    conv.set_algo(algo)
    y = host(conv.forward(xt))
    HO = oracle.conv_out(H, K, S, P)
    dy, dyt = prep(g.standard_normal((B, O, HO, HO)), dt)
    dx = host(conv.backward(dyt, xt, input_grad=True, weight_grad=False)[0])
    kw = dict(stride=(S, S), pad=(P, P))
    bb = b[None, :, None, None]
    for i in images:
        xi, dyi = x[i:i + 1 if i != -1 else None], dy[i:i + 1 if i != -1 else None]
        ref, sc = scaled(oracle.direct_conv, (xi, w), kw)
        assert_parity(y[i:i + 1 if i != -1 else None], ref + bb, sc + np.abs(bb), dt, f"y[{i}]",
                      k=C * K * K + 1)
        ref, sc = scaled(oracle.direct_conv_backward_input, (dyi, w, xi.shape), kw)
        assert_parity(dx[i:i + 1 if i != -1 else None], ref, sc, dt, f"dx[{i}]", k=O * K * K)
    # weight / bias gradient through a dY that is zero outside dw_images
    sel = sorted(i % B for i in dw_images)
    dyz = np.zeros_like(dy)
    dyz[sel] = dy[sel]
    _, dw, db = conv.backward(torch.from_numpy(dyz).to(DEV, DT[dt]), xt, input_grad=False, weight_grad=True)
    # the zero images add exact zeros: K counts the products of the selected images
    ksel = len(sel) * HO * HO
    ref, sc = scaled(oracle.direct_conv_backward_weight, (dy[sel], x[sel], w.shape), kw)
    assert_parity(host(dw), ref, sc, dt, f"dw over images {sel}", k=ksel)
    ref, sc = scaled(oracle.conv_bias_grad, (dy[sel],), {})
    assert_parity(host(db), ref, sc, dt, f"db over images {sel}", k=ksel)
    return conv


# ------------------------------------------------------------------ config 3 (the bench workload)
C3 = [(64, 64, 56, 3, 1, 1), (128, 128, 28, 3, 1, 1), (256, 256, 14, 3, 1, 1), (64, 128, 56, 1, 2, 0)]


@pytest.mark.parametrize("layer", C3, ids=lambda l: "C{}O{}H{}K{}S{}".format(*l[:5]))
def test_config3_resnet_block_bf16(layer):
    C, O, H, K, S, P = layer
    conv_full(128, C, O, H, K, S, P, "bf16", vnn.ConvAlgo.IGEMM, seed=C + O + H, images=(0, 77, -1),
              dw_images=(3, 127), bias=False)


def test_config3_tail_tiles_bias_relu_bf16():
    """64@56 at N=128 runs 1568 tiles on 768 block slots (three blocks per CU,
    one LDS stage), so the last 32 tiles run in a partial final round.  The
    last images lie in those tiles: they are checked with a bias, and the
    fused-ReLU forward must equal ReLU of the plain forward bit for bit."""
    g = np.random.default_rng(11)
    B, C, O, H = 128, 64, 64, 56
    x, xt = prep(g.standard_normal((B, C, H, H)), "bf16")
    w, wt = prep(g.standard_normal((O, C, 3, 3)) * np.sqrt(2.0 / (C * 9)), "bf16")
    b, bt = prep(g.uniform(-0.5, 0.5, (O,)), "bf16")
    conv = vnn.Conv2d(C, O, 3, 1, 1, use_bias=True, device=DEV, dtype=torch.bfloat16)
    conv.weight, conv.bias = wt, bt
    conv.set_algo(vnn.ConvAlgo.IGEMM)
    y = host(conv.forward(xt))
    yr = host(conv.forward(xt, relu=True))
    # ReLU before the one rounding equals ReLU of the rounded value, bit for bit
    assert np.array_equal(yr, np.maximum(y, 0)), "fused ReLU differs from ReLU of the plain forward"
    kw = dict(stride=(1, 1), pad=(1, 1))
    bb = b[None, :, None, None]
    for i in (0, 124, 125, 126, 127):
        ref, sc = scaled(oracle.direct_conv, (x[i:i + 1], w), kw)
        assert_parity(y[i:i + 1], ref + bb, sc + np.abs(bb), "bf16", f"y[{i}]", k=C * 9 + 1)


# ------------------------------------------------------------------ config 1 (f32, whole batch vs oracle)
def test_config1_mnist_cnn_f32():
    for C, O in ((1, 32), (32, 64)):
        conv = conv_full(64, C, O, 28, 3, 1, 1, "f32", vnn.ConvAlgo.Auto, seed=O, images=(0, 31, -1),
                         dw_images=(5, 63))
        assert conv.last_algo is not None


# ------------------------------------------------------------------ config 5 (bf16, N=16, 256x256)
C5 = [(3, 64, 5, 2, "uniform"), (64, 64, 3, 1, "normal"), (64, 32, 3, 1, "normal"), (32, 27, 3, 1, "normal")]


@pytest.mark.parametrize("layer", C5, ids=lambda l: "C{}O{}K{}".format(*l[:3]))
def test_config5_superres_bf16(layer):
    C, O, K, P, dist = layer
    conv_full(16, C, O, 256, K, 1, P, "bf16", vnn.ConvAlgo.Auto, seed=C * O, x_dist=dist, images=(9,),
              dw_images=(2,))


def test_config5_pixel_shuffle_full():
    g = np.random.default_rng(3)
    for dt in ("bf16", "f32"):
        x, xt = prep(g.uniform(0, 1, (16, 27, 256, 256)), dt)
        ps = vnn.PixelShuffle(3)
        assert np.array_equal(host(ps.forward(xt)), oracle.pixel_shuffle(x, 3))
        dy, dyt = prep(g.standard_normal((16, 3, 768, 768)), dt)
        assert np.array_equal(host(ps.backward(dyt)), oracle.pixel_shuffle_backward(dy, 3))


# ------------------------------------------------------------------ config 4 (f32 ConvTranspose2d, N=128)
C4 = [(100, 512, 1, 4, 1, 0), (512, 256, 4, 4, 2, 1), (256, 128, 8, 4, 2, 1), (128, 64, 16, 4, 2, 1),
      (64, 3, 32, 4, 2, 1)]


@pytest.mark.parametrize("layer", C4, ids=lambda l: "CI{}CO{}H{}".format(*l[:3]))
def test_config4_dcgan_convtranspose_f32(layer):
    CI, CO, H, K, S, P = layer
    B = 128
    g = np.random.default_rng(CI + CO)
    x, xt = prep(g.standard_normal((B, CI, H, H)), "f32")
    w, wt = prep(g.normal(0.0, 0.02, (CI, CO, K, K)), "f32")
    b, bt = prep(g.uniform(-0.1, 0.1, (CO,)), "f32")
    ct = vnn.ConvTranspose2d(CI, CO, K, S, P, device=DEV, dtype=torch.float32)
    ct.weight, ct.bias = wt, bt
    y = host(ct.forward(xt))
    HO = oracle.convt_out(H, K, S, P)
    dy, dyt = prep(g.standard_normal((B, CO, HO, HO)), "f32")
    dx = host(ct.backward(dyt, xt)[0])
    kw = dict(stride=(S, S), pad=(P, P))
    for i in (0, 100):
        ref, sc = scaled(oracle.conv_transpose_forward, (x[i:i + 1], w, b), kw)
        assert_parity(y[i:i + 1], ref, sc, "f32", f"y[{i}]")
        ref, sc = scaled(lambda *a, **k: oracle.conv_transpose_backward(*a, **k)[0], (dy[i:i + 1], x[i:i + 1], w), kw)
        assert_parity(dx[i:i + 1], ref, sc, "f32", f"dx[{i}]")
    sel = [7, 64]
    dyz = np.zeros_like(dy)
    dyz[sel] = dy[sel]
    _, dw, db = ct.backward(torch.from_numpy(dyz).to(DEV), xt)
    for j, (name, got) in ((1, ("dw", dw)), (2, ("db", db))):
        ref, sc = scaled(lambda *a, j=j, **k: oracle.conv_transpose_backward(*a, **k)[j], (dy[sel], x[sel], w), kw)
        assert_parity(host(got), ref, sc, "f32", f"{name} over images {sel}")


# ------------------------------------------------------------------ config 2 (Linear and the square product)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_config2_linear_full(dt):
    M, IN, OUT = 4096, 1024, 4096
    g = np.random.default_rng(11)
    x, xt = prep(g.standard_normal((M, IN)), dt)
    bound = np.sqrt(6.0 / (IN + OUT))
    w, wt = prep(g.uniform(-bound, bound, (IN, OUT)), dt)
    b, bt = prep(g.uniform(-1.0 / 32, 1.0 / 32, (OUT,)), dt)
    lin = vnn.Linear(IN, OUT, device=DEV, dtype=DT[dt])
    lin.weight, lin.bias = wt, bt
    y = host(lin.forward(xt))
    dy, dyt = prep(g.standard_normal((M, OUT)), dt)
    dx = host(lin.backward(dyt, xt)[0])
    rows = [0, 1234, 4095]
    ref, sc = scaled(oracle.linear_forward, (x[rows], w, b), {})
    assert_parity(y[rows], ref, sc, dt, "y rows", k=IN + 1)
    ref, sc = scaled(lambda *a: oracle.linear_backward(*a)[0], (dy[rows], x[rows], w), {})
    assert_parity(dx[rows], ref, sc, dt, "dx rows", k=OUT)
    dyz = np.zeros_like(dy)
    dyz[rows] = dy[rows]
    _, dw, db = lin.backward(torch.from_numpy(dyz).to(DEV, DT[dt]), xt)
    for j, name, got in ((1, "dw", dw), (2, "db", db)):
        ref, sc = scaled(lambda *a, j=j: oracle.linear_backward(*a)[j], (dy[rows], x[rows], w), {})
        assert_parity(host(got), ref, sc, dt, f"{name} over rows", k=len(rows))


def test_config2_square_8192_bf16():
    n = 8192
    g = np.random.default_rng(12)
    a, at = prep(g.standard_normal((n, n)), "bf16")
    b, bt = prep(g.standard_normal((n, n)), "bf16")
    rows = [0, 5000, n - 1]
    c = host(ops.gpu_matmul(at, bt, n, n, n))
    ref, sc = scaled(oracle.matmul, (a[rows], b), {})
    assert_parity(c[rows], ref, sc, "bf16", "C rows", k=n)
    del c
    gr, grt = prep(g.standard_normal((n, n)), "bf16")
    da = host(ops.gpu_matmul_backward_a(grt, bt, n, n, n))
    ref, sc = scaled(oracle.matmul_backward_a, (gr[rows], b), {})
    assert_parity(da[rows], ref, sc, "bf16", "dA rows", k=n)
    del da
    grz = np.zeros_like(gr)
    grz[rows] = gr[rows]
    db = host(ops.gpu_matmul_backward_b(at, torch.from_numpy(grz).to(DEV, torch.bfloat16), n, n, n))
    ref, sc = scaled(oracle.matmul_backward_b, (a[rows], gr[rows]), {})
    assert_parity(db, ref, sc, "bf16", "dB over rows", k=len(rows))
