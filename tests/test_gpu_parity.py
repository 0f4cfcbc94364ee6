"""GPU parity: every hot-path entry point of libvolta_hip.so against the CPU oracle.

Inputs are seeded numpy arrays; the same arrays (bf16-rounded for bf16) go to
the oracle and, through the C ABI, to the MI355X.  Sizes keep the oracle to
seconds; full-size configurations are covered in test_gpu_fullsize.py.
"""
import numpy as np
import pytest
import torch

import oracle
import volta_amd
from volta_amd import nn as vnn
from volta_amd import ops
from tests.parity import assert_parity, k_conv_dgrad, k_conv_fwd, k_conv_wgrad

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16}


def rng(seed):
    return np.random.default_rng(seed)


def prep(a, dt):
    """numpy f32 -> (oracle input, device tensor) with identical values."""
    a = np.ascontiguousarray(a, np.float32)
    r = oracle.round_bf16(a) if dt == "bf16" else a
    return r, torch.from_numpy(r).to(DEV, DTYPES[dt])


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def ref_and_scale(fn, *args, **kw):
    """oracle result and its per-element scale S = fn(|args|) (fn is bilinear)."""
    ab = [np.abs(a) if isinstance(a, np.ndarray) else a for a in args]
    return fn(*args, **kw), fn(*ab, **kw)


def check(got, fn, args, dt, what, kw=None, extra_ref=None, extra_scale=None, k=None):
    """k: products per output element (required by the bf16 gate)."""
    ref, scale = ref_and_scale(fn, *args, **(kw or {}))
    if extra_ref is not None:
        ref = ref + extra_ref
        scale = scale + extra_scale
    return assert_parity(host(got), ref, scale, dt, what, k=k)


# ------------------------------------------------------------------ known answers
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_matmul_known_answers(dt):
    a = torch.tensor([[1, 2], [3, 4]], dtype=DTYPES[dt], device=DEV)
    b = torch.tensor([[5, 6], [7, 8]], dtype=DTYPES[dt], device=DEV)
    assert host(ops.gpu_matmul(a, b, 2, 2, 2)).ravel().tolist() == [19, 22, 43, 50]  # tests/gpu_test.rs:46-60
    a = torch.tensor([[1, 2, 3], [4, 5, 6]], dtype=DTYPES[dt], device=DEV)
    b = torch.tensor([[1, 0], [0, 1], [1, 1]], dtype=DTYPES[dt], device=DEV)
    assert host(ops.gpu_matmul(a, b, 2, 3, 2)).ravel().tolist() == [4, 5, 10, 11]  # lib.rs:4538-4547


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_linear_known_answer(dt):
    lin = vnn.Linear(2, 3, device=DEV, dtype=DTYPES[dt])
    lin.weight = torch.tensor([[1, 2, 3], [4, 5, 6]], dtype=DTYPES[dt], device=DEV)
    lin.bias = torch.tensor([10, 20, 30], dtype=DTYPES[dt], device=DEV)
    y = lin.forward(torch.ones(1, 2, dtype=DTYPES[dt], device=DEV))
    assert host(y).ravel().tolist() == [15, 27, 39]  # lib.rs:4693-4712


@pytest.mark.parametrize("algo", [vnn.ConvAlgo.Direct, vnn.ConvAlgo.Im2col, vnn.ConvAlgo.IGEMM])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_conv_all_ones_closed_form(algo, dt):
    # conv.rs:2930-2976: C=2 -> 4, 3x3, pad 1, ones 1x2x8x8 => 2 * (#valid taps)
    conv = vnn.Conv2d(2, 4, 3, 1, 1, use_bias=True, device=DEV, dtype=DTYPES[dt])
    conv.weight = torch.ones(4, 2, 3, 3, dtype=DTYPES[dt], device=DEV)
    conv.set_algo(algo)
    y = host(conv.forward(torch.ones(1, 2, 8, 8, dtype=DTYPES[dt], device=DEV)))
    taps = np.full(8, 3.0)
    taps[0] = taps[-1] = 2.0
    for o in range(4):
        assert np.array_equal(y[0, o], 2.0 * np.outer(taps, taps))


@pytest.mark.parametrize("algo", [vnn.ConvAlgo.Direct, vnn.ConvAlgo.Im2col, vnn.ConvAlgo.IGEMM])
def test_conv_ramp_window_sums(algo):
    # conv.rs:3021-3065
    conv = vnn.Conv2d(1, 1, 2, 1, 0, use_bias=False, device=DEV)
    conv.weight = torch.ones(1, 1, 2, 2, device=DEV)
    conv.set_algo(algo)
    x = torch.arange(16, dtype=torch.float32, device=DEV).reshape(1, 1, 4, 4)
    y = host(conv.forward(x))[0, 0]
    r = np.arange(16, dtype=np.float32).reshape(4, 4)
    assert np.array_equal(y, r[:-1, :-1] + r[:-1, 1:] + r[1:, :-1] + r[1:, 1:])


# ------------------------------------------------------------------ matmul family
MM_CASES = [(37, 19, 23), (128, 256, 64), (130, 70, 200), (64, 1024, 96), (256, 512, 384), (3, 5, 300),
            (200, 72, 136), (8, 40, 24), (520, 264, 392)]  # K % 8 == 0, M / N off the tile sizes


@pytest.mark.parametrize("mkn", MM_CASES)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_matmul_family(mkn, dt):
    m, k, n = mkn
    g = rng(m * 7 + n)
    a, at = prep(g.standard_normal((m, k)), dt)
    b, bt = prep(g.standard_normal((k, n)), dt)
    gr, grt = prep(g.standard_normal((m, n)), dt)
    check(ops.gpu_matmul(at, bt, m, k, n), oracle.matmul, (a, b), dt, "matmul", k=k)
    check(ops.gpu_matmul_backward_a(grt, bt, m, k, n), oracle.matmul_backward_a, (gr, b), dt, "dA", k=n)
    check(ops.gpu_matmul_backward_b(at, grt, m, k, n), oracle.matmul_backward_b, (a, gr), dt, "dB", k=m)


# m, k or n = 1: the 2-D forms of the reference's mat-vec, vec-mat and dot products
MM_EDGE = [(1, 5, 7), (6, 1, 9), (4, 8, 1), (1, 1, 1), (1, 64, 1), (300, 1, 2), (1, 300, 130), (130, 300, 1)]


@pytest.mark.parametrize("mkn", MM_EDGE)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_matmul_family_unit_dims(mkn, dt):
    m, k, n = mkn
    g = rng(m * 13 + k * 5 + n)
    a, at = prep(g.standard_normal((m, k)), dt)
    b, bt = prep(g.standard_normal((k, n)), dt)
    gr, grt = prep(g.standard_normal((m, n)), dt)
    check(ops.gpu_matmul(at, bt, m, k, n), oracle.matmul, (a, b), dt, "matmul", k=k)
    check(ops.gpu_matmul_backward_a(grt, bt, m, k, n), oracle.matmul_backward_a, (gr, b), dt, "dA", k=n)
    check(ops.gpu_matmul_backward_b(at, grt, m, k, n), oracle.matmul_backward_b, (a, gr), dt, "dB", k=m)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_matmul_vector_known_answers(dt):
    """lib.rs:4559-4605 as 2-D products: (3,2)@(2,1) = [-1,-1,-1]; (1,3)@(3,2) =
    [4,5]; (1,3)@(3,1) = 8 -- exact in both dtypes (small integers)."""
    def mm(a, b):
        a = np.asarray(a, np.float32)
        b = np.asarray(b, np.float32)
        m, k = a.shape
        n = b.shape[1]
        return host(ops.gpu_matmul(torch.from_numpy(a).to(DEV, DTYPES[dt]), torch.from_numpy(b).to(DEV, DTYPES[dt]),
                                   m, k, n))
    assert np.array_equal(mm([[1, 2], [3, 4], [5, 6]], [[1], [-1]]), np.array([[-1], [-1], [-1]], np.float32))
    assert np.array_equal(mm([[1, 2, 3]], [[1, 0], [0, 1], [1, 1]]), np.array([[4, 5]], np.float32))
    assert np.array_equal(mm([[1, 2, 3]], [[4], [-1], [2]]), np.array([[8]], np.float32))


@pytest.mark.parametrize("shape", [(9, 6, 4), (64, 100, 48), (256, 1024, 512), (200, 136, 264), (1, 7, 5)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_linear_fwd_bwd(shape, dt):
    m, i, o = shape
    g = rng(m + i + o)
    x, xt = prep(g.standard_normal((m, i)), dt)
    w, wt = prep(g.uniform(-0.5, 0.5, (i, o)), dt)
    b, bt = prep(g.uniform(-1, 1, (o,)), dt)
    dy, dyt = prep(g.standard_normal((m, o)), dt)
    lin = vnn.Linear(i, o, device=DEV, dtype=DTYPES[dt])
    lin.weight, lin.bias = wt, bt
    check(lin.forward(xt), oracle.linear_forward, (x, w, b), dt, "y", k=i + 1)
    dx, dw, db = lin.backward(dyt, xt)
    check(dx, lambda *a: oracle.linear_backward(*a)[0], (dy, x, w), dt, "dx", k=o)
    check(dw, lambda *a: oracle.linear_backward(*a)[1], (dy, x, w), dt, "dw", k=m)
    check(db, lambda *a: oracle.linear_backward(*a)[2], (dy, x, w), dt, "db", k=m)


# ------------------------------------------------------------------ Conv2d
CONV_CASES = [
    # (B, C, O, H, W, K, S, P)
    (2, 3, 8, 9, 7, 3, 1, 1),
    (2, 16, 24, 10, 12, 3, 1, 1),
    (2, 32, 64, 28, 28, 3, 1, 1),    # config 1 conv2, batch 2
    (2, 1, 32, 28, 28, 3, 1, 1),     # config 1 conv1, batch 2
    (2, 64, 128, 56, 56, 1, 2, 0),   # config 3 projection, batch 2
    (2, 64, 64, 14, 14, 3, 1, 1),
    (1, 3, 64, 32, 32, 5, 1, 2),     # config 5 conv1 shape, smaller image
    (2, 8, 4, 9, 9, 4, 2, 1),
    (3, 5, 7, 6, 5, 2, 3, 0),
    (1, 2, 3, 12, 12, 9, 1, 4),      # 81-tap window (element-wise weight relayout)
    (2, 16, 24, 11, 9, 3, 2, 1),     # stride 2, 3x3: phases with 1 and 2 taps per axis, odd sizes
    (2, 8, 16, 10, 10, 1, 2, 0),     # 1x1 stride 2: odd input phases get no taps (zeros)
    (2, 3, 16, 10, 10, 4, 2, 1),     # 3 input channels, stride 2: input gradient one lane per position
    (2, 4, 8, 9, 11, 3, 3, 2),       # 4 input channels, stride 3
    (2, 2, 8, 17, 16, 4, 2, 1),      # 4x4 stride 2 pad 1, 2 input channels: cell-wise input gradient, odd height
    (1, 4, 6, 16, 17, 4, 2, 1),      # the same with 4 input channels, odd width (a cell past the last dY column)
    (2, 16, 128, 12, 12, 3, 1, 1),   # fp32 weight gradient on 128 x 128 tiles with split K (O and C*R*S >= 128)
    (2, 3, 16, 64, 64, 4, 2, 1),     # 4x4 stride 2 from 3 channels, 32-column output rows: fp32 cell forward
    (2, 64, 32, 15, 20, 3, 1, 1),    # fp32 halo kernel from 64 channels (rows split over wave pairs), a partial band
    (3, 32, 64, 1, 8, 3, 1, 1),      # fp32 halo kernels, one-row images (the band's other rows are padding)
    (2, 32, 64, 7, 28, 3, 1, 1),     # fp32 halo kernels, exactly one 7-row band
    (2, 4, 24, 10, 16, 3, 1, 1),     # bf16 few-channel 3x3 weight gradient, (channel, tap) MFMA columns (C*S = 12)
]


def _conv_ids(c):
    return "B{}C{}O{}H{}W{}K{}S{}P{}".format(*c)


@pytest.mark.parametrize("case", CONV_CASES, ids=_conv_ids)
@pytest.mark.parametrize("algo", [vnn.ConvAlgo.Direct, vnn.ConvAlgo.Im2col, vnn.ConvAlgo.IGEMM])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_conv2d_fwd_bwd(case, algo, dt):
    B, C, O, H, W, K, S, P = case
    if algo == vnn.ConvAlgo.Direct and C * O * H * W > 2_000_000:
        B = 1  # one output element per lane: the large layers run at batch 1
    g = rng(sum(case))
    x, xt = prep(g.standard_normal((B, C, H, W)), dt)
    w, wt = prep(g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K)), dt)
    b, bt = prep(g.uniform(-1, 1, (O,)), dt)
    conv = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=DEV, dtype=DTYPES[dt])
    conv.weight, conv.bias = wt, bt
    conv.set_algo(algo)
    y = conv.forward(xt)
    assert conv.last_algo == algo
    bb = b[None, :, None, None]
    y_shape = (B, O, oracle.conv_out(H, K, S, P), oracle.conv_out(W, K, S, P))
    check(y, oracle.direct_conv, (x, w), dt, "y", dict(stride=(S, S), pad=(P, P)),
          extra_ref=bb, extra_scale=np.abs(bb), k=k_conv_fwd(C, K, K))
    dy, dyt = prep(g.standard_normal(y_shape), dt)
    dx, dw, db = conv.backward(dyt, xt)
    kwg = k_conv_wgrad(B, y_shape[2], y_shape[3])
    check(dx, oracle.direct_conv_backward_input, (dy, w, x.shape), dt, "dx", dict(stride=(S, S), pad=(P, P)),
          k=k_conv_dgrad(O, K, K))
    check(dw, oracle.direct_conv_backward_weight, (dy, x, w.shape), dt, "dw", dict(stride=(S, S), pad=(P, P)),
          k=kwg)
    check(db, oracle.conv_bias_grad, (dy,), dt, "db", k=kwg)
    if algo == vnn.ConvAlgo.Direct and dt == "f32":
        # the direct kernels keep Volta's CPU summation order and unfused
        # multiply/add (conv.rs:1370-1407, 458-505): bit-identical results
        assert np.array_equal(host(y), oracle.direct_conv(x, w, (S, S), (P, P)) + bb)
        assert np.array_equal(host(dx), oracle.direct_conv_backward_input(dy, w, x.shape, (S, S), (P, P)))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_gpu_ops_boundary_functions(dt):
    # The gpu_ops.rs-named entry points, including argument order (stride before pad).
    B, C, O, H, W, K, S, P = 2, 8, 16, 11, 9, 3, 2, 1
    HO, WO = oracle.conv_out(H, K, S, P), oracle.conv_out(W, K, S, P)
    g = rng(5)
    x, xt = prep(g.standard_normal((B, C, H, W)), dt)
    w, wt = prep(g.standard_normal((O, C, K, K)) * 0.2, dt)
    dy, dyt = prep(g.standard_normal((B, O, HO, WO)), dt)
    dims = (B, C, O, H, W, K, K, S, S, P, P, HO, WO)
    kw = dict(stride=(S, S), pad=(P, P))
    kf, kd, kwg = k_conv_fwd(C, K, K, bias=False), k_conv_dgrad(O, K, K), k_conv_wgrad(B, HO, WO)
    check(ops.gpu_direct_conv(xt, wt, *dims), oracle.direct_conv, (x, w), dt, "direct", kw, k=kf)
    check(ops.gpu_igemm(xt, wt, *dims), oracle.direct_conv, (x, w), dt, "igemm", kw, k=kf)
    check(ops.gpu_conv_backward_input(dyt, wt, *dims), oracle.direct_conv_backward_input, (dy, w, x.shape), dt,
          "direct dx", kw, k=kd)
    check(ops.gpu_igemm_backward_input(dyt, wt, *dims), oracle.direct_conv_backward_input, (dy, w, x.shape), dt,
          "igemm dx", kw, k=kd)
    check(ops.gpu_conv_backward_weight(dyt, xt, *dims), oracle.direct_conv_backward_weight, (dy, x, w.shape), dt,
          "direct dw", kw, k=kwg)
    check(ops.gpu_igemm_backward_weight(dyt, xt, *dims), oracle.direct_conv_backward_weight, (dy, x, w.shape), dt,
          "igemm dw", kw, k=kwg)
    # im2col / col2im on the padded input, exact copies (sums for col2im)
    xp = oracle.pad(x, P, P)
    xpt = torch.from_numpy(xp).to(DEV, DTYPES[dt])
    HP, WP = xp.shape[2:]
    col = ops.gpu_im2col(xpt, B, C, HP, WP, K, K, S, S, HO, WO)
    assert np.array_equal(host(col), oracle.im2col(xp, (K, K), (S, S)))
    gcol, gcolt = prep(g.standard_normal(col.shape), dt)
    back = ops.gpu_col2im(gcolt, B, C, HP, WP, K, K, S, S, HO, WO)
    check(back, oracle.col2im, (gcol, xp.shape, (K, K), (S, S)), dt, "col2im", k=K * K)


def test_bad_shape_is_an_error_not_a_crash():
    x = torch.zeros(1, 2, 5, 5, device=DEV)
    w = torch.zeros(3, 2, 3, 3, device=DEV)
    with pytest.raises(volta_amd.VoltaHipError) as e:
        ops.gpu_igemm(x, w, 1, 2, 3, 5, 5, 3, 3, 1, 1, 1, 1, 4, 5)  # h_out should be 5
    assert e.value.status == 2
    y = ops.gpu_igemm(x, w, 0, 2, 3, 5, 5, 3, 3, 1, 1, 1, 1, 5, 5)  # empty batch is a no-op
    assert y.shape == (0, 3, 5, 5)


# ------------------------------------------------------------------ stride-1 fast path vs generic
HALO_CASES = [
    # (B, C, O, H, W, K, S, P): shapes inside the bf16 halo kernel's envelope
    (3, 16, 32, 14, 14, 3, 1, 1),    # blocks span 2-3 images
    (2, 32, 128, 28, 28, 3, 1, 1),   # 128-channel tile (two wave rows)
    (2, 64, 64, 56, 56, 3, 1, 1),    # config 3 first layer, batch 2
    (1, 16, 48, 20, 24, 5, 1, 2),    # 5x5 pad 2, O not a tile multiple
    (2, 16, 16, 9, 10, 3, 1, 0),     # no padding (P = H - 2)
    (5, 32, 16, 4, 4, 3, 1, 1),      # tiny images, many per block
    (2, 48, 80, 16, 18, 1, 1, 0),    # 1x1 stride 1
    (2, 16, 16, 8, 8, 3, 1, 2),      # even padding wider than 1 (P = H + 2)
    (4, 64, 96, 12, 12, 3, 1, 1),    # O and C not multiples of the 64-wide tiles
    (2, 128, 64, 9, 9, 3, 1, 1),     # odd image size (W odd: generic fallback)
    (2, 64, 128, 56, 56, 1, 2, 0),   # config 3 projection: subsampled 1x1 path
    (3, 32, 48, 13, 11, 1, 2, 0),    # strided 1x1, odd sizes (scatter edges)
    (2, 16, 32, 12, 12, 1, 3, 0),    # stride 3
    (3, 48, 80, 16, 16, 1, 2, 0),    # strided 1x1: O, C not tile multiples
    (2, 32, 64, 15, 16, 1, 2, 0),    # strided 1x1: odd H (last cell row clipped)
    (2, 64, 64, 8, 256, 3, 1, 1),    # wide rows: weight gradient over column segments
    (1, 32, 40, 5, 200, 3, 1, 1),    # wide rows, W not a multiple of the segment width
    (1, 16, 24, 4, 300, 3, 1, 2),    # wide rows, Q = W + 2 (bias columns past W)
    (1, 20, 30, 6, 166, 3, 1, 0),    # wide rows, no padding, 2-element chunks
    (2, 27, 32, 16, 16, 3, 1, 1),    # C not a multiple of 16: partial last channel group (forward)
    (2, 32, 27, 12, 12, 3, 1, 1),    # O = 27: partial channel group in the input gradient
    (84, 17, 20, 56, 56, 3, 1, 1),   # >= 1024 blocks, two channel groups: one LDS stage, 3 blocks per CU
    (4, 18, 17, 256, 256, 3, 1, 1),  # the same over column strips (no vector epilogue)
    (2, 3, 64, 20, 24, 5, 1, 2),     # 3 input channels, 5x5: one partial group, one LDS stage
    (1, 5, 20, 8, 10, 3, 1, 1),      # C = 5 forward; input gradient over 20 = 16 + 4 channels
    (3, 48, 64, 30, 30, 3, 1, 1),    # W % 8 != 0: halo kernel for a shape the resident-weight kernel declines
    (2, 48, 64, 24, 32, 3, 1, 1),    # resident weights: three channel groups, tiles across images
    (3, 64, 40, 16, 24, 3, 1, 1),    # resident weights, O = 40: partly empty 64-row tile
    (2, 40, 24, 20, 16, 3, 1, 1),    # resident weights, C = 40: partial channel group (grouped copy)
    (1, 64, 64, 16, 16, 3, 1, 1),    # one tile per block (fewer tiles than CUs)
    (8, 3, 16, 64, 64, 5, 1, 2),     # few-channel weight gradient, 5x5: two steps per split (x rows reused)
    (16, 8, 16, 48, 32, 3, 1, 1),    # few-channel weight gradient, 3x3 pad 1: steps cross a column chunk
]


def _bf16_conv_case(case, policy):
    B, C, O, H, W, K, S, P = case
    dt = "bf16"
    volta_amd.check(volta_amd.lib().vh_set_kernel_policy(policy))
    try:
        g = rng(sum(case) + 7)
        x, xt = prep(g.standard_normal((B, C, H, W)), dt)
        w, wt = prep(g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K)), dt)
        b, bt = prep(g.uniform(-1, 1, (O,)), dt)
        conv = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=DEV, dtype=DTYPES[dt])
        conv.weight, conv.bias = wt, bt
        conv.set_algo(vnn.ConvAlgo.IGEMM)
        y = conv.forward(xt)
        bb = b[None, :, None, None]
        kw = dict(stride=(S, S), pad=(P, P))
        check(y, oracle.direct_conv, (x, w), dt, "y", kw, extra_ref=bb, extra_scale=np.abs(bb),
              k=k_conv_fwd(C, K, K))
        dy, dyt = prep(g.standard_normal(tuple(y.shape)), dt)
        dx, dw, db = conv.backward(dyt, xt)
        kwg = k_conv_wgrad(B, y.shape[2], y.shape[3])
        check(dx, oracle.direct_conv_backward_input, (dy, w, x.shape), dt, "dx", kw, k=k_conv_dgrad(O, K, K))
        check(dw, oracle.direct_conv_backward_weight, (dy, x, w.shape), dt, "dw", kw, k=kwg)
        check(db, oracle.conv_bias_grad, (dy,), dt, "db", k=kwg)
    finally:
        volta_amd.check(volta_amd.lib().vh_set_kernel_policy(volta_amd._lib.POLICY_FASTEST))


@pytest.mark.parametrize("case", HALO_CASES, ids=_conv_ids)
@pytest.mark.parametrize("policy", [volta_amd._lib.POLICY_FASTEST, volta_amd._lib.POLICY_GENERIC])
def test_conv2d_bf16_fast_and_generic_paths(case, policy):
    _bf16_conv_case(case, policy)


# 3x3 stride-1 shapes with at most 64 input and output channels: the
# resident-weight kernel takes the masked input gradient by default;
# VOLTA_HIP_WRES=1 sends every shape in its envelope there (the others fall back).
WRES_CASES = [c for c in HALO_CASES if c[5] == 3 and c[6] == 1 and c[1] <= 64 and c[2] <= 64]


@pytest.mark.parametrize("case", WRES_CASES, ids=_conv_ids)
def test_conv2d_bf16_3x3_resident_weight_kernel(case, monkeypatch):
    monkeypatch.setenv("VOLTA_HIP_WRES", "1")
    _bf16_conv_case(case, volta_amd._lib.POLICY_FASTEST)


# ------------------------------------------------------------------ ConvTranspose2d
CT_CASES = [
    # (B, CI, CO, H, W, K, S, P)
    (2, 4, 3, 4, 4, 4, 2, 1),
    (4, 100, 32, 1, 1, 4, 1, 0),     # config 4 layer 1 (512 -> 32 out channels)
    (2, 64, 32, 8, 8, 4, 2, 1),      # config 4 inner layer shape
    (2, 16, 3, 16, 16, 4, 2, 1),     # config 4 last layer (to RGB)
    (1, 5, 6, 5, 3, 3, 2, 1),
    (2, 8, 5, 5, 7, 3, 2, 0),        # stride 2, no padding, odd output sizes
    (1, 4, 6, 3, 3, 5, 3, 2),        # stride 3, 5x5
    (2, 8, 2, 5, 5, 3, 1, 1),        # 2 output channels, stride 1 (one lane per output position)
    (3, 6, 1, 4, 6, 4, 2, 1),        # 1 output channel
    (2, 16, 4, 1, 1, 3, 1, 0),       # 1x1 input: the layer is one product
    (2, 8, 1, 8, 4, 4, 2, 1),        # k4 s2 p1 to 1 channel: cell-wise kernel, one 4-wide load per dY row
    (2, 12, 4, 6, 8, 4, 2, 1),       # k4 s2 p1 to 4 channels
    (3, 10, 2, 5, 12, 4, 2, 1),      # k4 s2 p1 to 2 channels, 10 input channels (uneven split over waves)
    (2, 128, 16, 4, 4, 4, 2, 1),     # fp32 dW on 128 x 128 tiles (128 input channels x 16 x 16 taps)
    (2, 64, 3, 32, 32, 4, 2, 1),     # config 4 last layer at batch 2: fp32 dW and dB in one MFMA pass
    (2, 16, 3, 4, 32, 4, 2, 1),      # the same kernel, 4 input rows
    (1, 64, 4, 2, 64, 4, 2, 1),      # two 32-position segments per input row, 4 output channels
    (2, 8, 1, 3, 32, 4, 2, 1),       # 1 output channel, odd input height
    (2, 512, 128, 3, 4, 4, 2, 1),    # 512 x 128 weight rows: the row-wise stride-phase weight relayout
]


@pytest.mark.parametrize("case", CT_CASES, ids=_conv_ids)
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_conv_transpose2d_fwd_bwd(case, dt):
    B, CI, CO, H, W, K, S, P = case
    g = rng(sum(case) + 1)
    x, xt = prep(g.standard_normal((B, CI, H, W)), dt)
    w, wt = prep(g.normal(0, 0.02 * 10, (CI, CO, K, K)), dt)
    b, bt = prep(g.uniform(-1, 1, (CO,)), dt)
    ct = vnn.ConvTranspose2d(CI, CO, K, S, P, device=DEV, dtype=DTYPES[dt])
    ct.weight, ct.bias = wt, bt
    y = ct.forward(xt)
    kw = dict(stride=(S, S), pad=(P, P))
    check(y, oracle.conv_transpose_forward, (x, w, b), dt, "y", kw, k=CI * K * K + 1)
    dy, dyt = prep(g.standard_normal(tuple(y.shape)), dt)
    dx, dw, db = ct.backward(dyt, xt)
    ks = (CO * K * K, B * H * W, B * y.shape[2] * y.shape[3])
    for i, (name, got) in enumerate((("dx", dx), ("dw", dw), ("db", db))):
        check(got, lambda *a, i=i, **k: oracle.conv_transpose_backward(*a, **k)[i], (dy, x, w), dt, name, kw,
              k=ks[i])


# ------------------------------------------------------------------ PixelShuffle
@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 27, 8, 9, 3), (1, 12, 4, 4, 2), (2, 3, 5, 7, 1), (3, 18, 5, 24, 3),
                                   (2, 48, 6, 16, 4), (1, 8, 3, 8, 2)])
def test_pixel_shuffle_exact(shape, dt):
    B, CR, H, W, r = shape
    g = rng(CR)
    x, xt = prep(g.standard_normal((B, CR, H, W)), dt)
    ps = vnn.PixelShuffle(r)
    y = ps.forward(xt)
    assert np.array_equal(host(y), oracle.pixel_shuffle(x, r))
    dy, dyt = prep(g.standard_normal(y.shape), dt)
    assert np.array_equal(host(ps.backward(dyt)), oracle.pixel_shuffle_backward(dy, r))


# ------------------------------------------------------------------ glue: ReLU, sum loss
GLUE_SIZES = [1, 7, 8, 1000, 4099, 1 << 20]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("n", GLUE_SIZES)
def test_relu_fwd_bwd_exact(n, dt):
    g = rng(n)
    x, xt = prep(g.standard_normal(n), dt)
    special = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0], np.float32)
    if n >= 8:
        x[:5] = special
        xt[:5] = torch.from_numpy(special).to(DEV, DTYPES[dt])
    y = ops.gpu_unary(xt, "relu")
    assert np.array_equal(host(y), oracle.relu(x), equal_nan=True)
    dy, dyt = prep(g.standard_normal(n), dt)
    dx = ops.gpu_unary_backward(dyt, xt, "relu")
    assert np.array_equal(host(dx), oracle.relu_backward(dy, x))
    # unaligned views take the element path
    if n >= 16:
        yv = torch.empty(n + 1, dtype=DTYPES[dt], device=DEV)[1:]
        relu = vnn.ReLU()
        relu.forward(xt, out=yv)
        assert np.array_equal(host(yv), oracle.relu(x), equal_nan=True)


def test_unary_other_ops_are_unsupported():
    x = torch.ones(8, device=DEV)
    with pytest.raises(ValueError):
        ops.gpu_unary(x, "exp")
    y = torch.empty_like(x)
    assert volta_amd.lib().vh_unary(volta_amd.F32, 7, x.data_ptr(), y.data_ptr(), 8,
                                    torch.cuda.current_stream().cuda_stream) == volta_amd._lib.VH_ERR_UNSUPPORTED


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("n", GLUE_SIZES + [37 << 20])
def test_sum_loss_and_seed(n, dt):
    g = rng(n + 1)
    x, xt = prep(g.standard_normal(n), dt)
    got = ops.gpu_sum_reduce(xt)
    exact = float(np.sum(x.astype(np.float64)))
    scale = float(np.abs(x).sum())
    # fp32 accumulation in a fixed order: the gate's scaled error, f32 bar
    assert abs(got - exact) <= 1e-6 * scale + 1e-30, (got, exact)
    # and close to Volta's own sequential f32 sum (both within n*eps of exact)
    if n <= (1 << 20):
        assert abs(got - oracle.sum_all(x)) <= n * 2 ** -24 * scale
    # deterministic: the same value twice
    assert ops.gpu_sum_reduce(xt) == got
    # the loss's gradient / the autograd seed
    for grad in (1.0, 0.1, -3.0):
        dy = vnn.sum_loss_backward(xt, grad)
        want = oracle.round_bf16(np.full(n, grad, np.float32)) if dt == "bf16" else np.full(n, grad, np.float32)
        assert np.array_equal(host(dy), want)


def test_sum_loss_known_answers():
    # test_sum_backward_gpu (src/lib.rs:3528-3550): x = 1..6, sum 21, grad all ones
    x = torch.tensor([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]], device=DEV)
    assert host(vnn.sum_loss(x)).tolist() == [21.0]
    assert host(ops.gpu_sum_backward(1.0, 6)).tolist() == [1.0] * 6
    assert ops.gpu_sum_reduce(torch.tensor([42.0], device=DEV)) == 42.0
    assert ops.gpu_sum_reduce(torch.empty(0, device=DEV)) == 0.0


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("off", [1, 3, 8])
def test_sum_and_seed_on_offset_views(off, dt):
    # slices that start off a 16-byte boundary take the element-wise path
    n = 4099
    g = rng(off)
    x, xt = prep(g.standard_normal(n + off), dt)
    got = ops.gpu_sum_reduce(xt[off:])
    exact = float(np.sum(x[off:].astype(np.float64)))
    assert abs(got - exact) <= 1e-6 * float(np.abs(x[off:]).sum()), (got, exact)
    buf = torch.zeros(n + off + 5, dtype=DTYPES[dt], device=DEV)
    view = buf[off:off + n]
    ops._call("vh_sum_backward", ops.dtype_code(view), 0.5, ops.ptr(view), n, ops.stream_ptr(view.device))
    got = host(buf)
    assert np.all(got[:off] == 0) and np.all(got[off:off + n] == 0.5) and np.all(got[off + n:] == 0)


# ------------------------------------------------------------------ fused conv -> ReLU
RELU_CASES = [
    # (B, C, O, H, W, K, S, P)
    (2, 32, 64, 28, 28, 3, 1, 1),    # config 1 conv2 / halo kernel (bf16)
    (2, 64, 64, 20, 24, 3, 1, 1),
    (2, 64, 64, 14, 14, 3, 1, 1),    # P*Q % 8 == 4 and
    (2, 32, 64, 7, 14, 3, 1, 1),     # P*Q % 4 == 2: halo epilogue position by position
    (1, 3, 64, 24, 32, 5, 1, 2),     # config 5 conv1 shape: one partial channel group
    (2, 64, 128, 16, 16, 1, 2, 0),   # strided 1x1 (bf16 pointwise kernels: separate ReLU pass)
    (2, 16, 24, 11, 9, 3, 2, 1),     # strided 3x3: stride phases
    (2, 1, 32, 12, 12, 3, 1, 1),     # one input channel (MI355X selector: direct)
    (2, 3, 16, 16, 17, 4, 2, 1),     # k4 s2 p1, 3 input channels: masked cell-wise input gradient
    (1, 2, 8, 16, 64, 4, 2, 1),      # k4 s2 p1 to 32-column rows: fp32 cell forward with the ReLU fused
    (2, 32, 64, 9, 12, 3, 1, 1),     # fp32 halo kernel: ReLU forward, masked dX through the K-split form
    (1, 64, 32, 8, 4, 3, 1, 1),      # fp32 halo kernel, 4-column rows
]


@pytest.mark.parametrize("case", RELU_CASES, ids=_conv_ids)
@pytest.mark.parametrize("algo", [vnn.ConvAlgo.Auto, vnn.ConvAlgo.IGEMM, vnn.ConvAlgo.Im2col])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_conv2d_fused_relu_fwd_and_masked_dgrad(case, algo, dt):
    B, C, O, H, W, K, S, P = case
    g = rng(sum(case) + 11)
    # the layer input came out of a ReLU: non-negative, about half zeros
    x, xt = prep(np.maximum(g.standard_normal((B, C, H, W)), 0), dt)
    w, wt = prep(g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K)), dt)
    b, bt = prep(g.uniform(-1, 1, (O,)), dt)
    conv = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=DEV, dtype=DTYPES[dt])
    conv.weight, conv.bias = wt, bt
    conv.set_algo(algo)
    kw = dict(stride=(S, S), pad=(P, P))
    bb = b[None, :, None, None]
    ref, scale = ref_and_scale(oracle.direct_conv, x, w, **kw)
    y = conv.forward(xt, relu=True)
    got = host(y)
    assert (got >= 0).all()
    assert_parity(got, np.maximum(ref + bb, 0), scale + np.abs(bb), dt, "relu(y)", k=k_conv_fwd(C, K, K))
    dy, dyt = prep(g.standard_normal(got.shape), dt)
    dx, dw, db = conv.backward(dyt, xt, relu_input=True)
    dref, dscale = ref_and_scale(oracle.direct_conv_backward_input, dy, w, x.shape, **kw)
    mask = x > 0
    gdx = host(dx)
    assert (gdx[~mask] == 0).all()
    assert_parity(gdx, np.where(mask, dref, 0), dscale, dt, "masked dx", k=k_conv_dgrad(O, K, K))
    # the weight and bias gradients are those of the plain backward
    kwg = k_conv_wgrad(B, got.shape[2], got.shape[3])
    check(dw, oracle.direct_conv_backward_weight, (dy, x, w.shape), dt, "dw", kw, k=kwg)
    check(db, oracle.conv_bias_grad, (dy,), dt, "db", k=kwg)


@pytest.mark.parametrize("case", [c for c in RELU_CASES if c[5] == 3 and c[6] == 1 and c[1] <= 64 and c[2] <= 64]
                         + [(2, 64, 64, 20, 24, 3, 1, 1), (3, 32, 64, 16, 32, 3, 1, 1), (2, 64, 32, 24, 16, 3, 1, 1),
                            (2, 27, 32, 12, 16, 3, 1, 1)], ids=_conv_ids)
@pytest.mark.parametrize("wres", ["0", "1"])
def test_conv2d_bf16_fused_relu_both_3x3_kernels(case, wres, monkeypatch):
    monkeypatch.setenv("VOLTA_HIP_WRES", wres)
    test_conv2d_fused_relu_fwd_and_masked_dgrad(case, vnn.ConvAlgo.IGEMM, "bf16")


# ------------------------------------------------------------------ the step after dW
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_grad_accumulate_matches_oracle(dt):
    g = rng(5)
    for n in (1, 1000, 782336):
        a, at = prep(g.standard_normal(n), dt)
        b, bt = prep(g.standard_normal(n), dt)
        got = host(ops.gpu_add(at, bt))
        want = oracle.add(a, b)
        want = oracle.round_bf16(want) if dt == "bf16" else want
        assert np.array_equal(got, want)


@pytest.mark.parametrize("op", [0, 1, 2])
@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_optimizer_step_matches_oracle(op, wd):
    g = rng(op * 10 + int(wd * 100))
    n = 782336  # configs[2]'s weight count
    p0 = g.standard_normal(n).astype(np.float32)
    gr = g.standard_normal(n).astype(np.float32)
    s10 = (g.standard_normal(n) * 0.1).astype(np.float32)
    s20 = (np.abs(g.standard_normal(n)) * 0.01).astype(np.float32)
    pt, gt, s1t, s2t = (torch.from_numpy(a.copy()).to(DEV) for a in (p0, gr, s10, s20))
    kw = dict(beta1=0.9, beta2=0.999, t=3.0, eps=1e-8, weight_decay=wd)
    for step in range(2):  # two steps: the states carry over
        ops.gpu_optimizer_step(pt, gt, s1t, s2t, op, 1e-2, **kw)
        p0, s10, s20 = oracle.optimizer_step(op, 1e-2, p0, gr, s10, s20, **kw)
    got = host(pt)
    if op < 2:
        assert np.array_equal(got, p0)  # same formula and order, no contraction: bit-identical
        if op == 1:
            assert np.array_equal(host(s1t), s10)
    else:
        # Adam: sqrt / division may differ in the last bit
        assert np.abs(got - p0).max() <= 4 * np.spacing(np.abs(p0)).max()


# ------------------------------------------------------------------ device storage: dtype and layout
def test_casts_match_bf16_rne():
    g = rng(77)
    x = np.concatenate([g.standard_normal(100000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf,
                                  np.nan], np.float32)])
    xt = torch.from_numpy(x).to(DEV)
    b = ops.to_dtype(xt, torch.bfloat16)
    bits = b.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(bits[:-1], oracle.bf16_bits(x)[:-1])
    assert np.isnan(host(b)[-1])
    back = host(ops.to_dtype(b, torch.float32))
    assert np.array_equal(back[:-1], oracle.round_bf16(x)[:-1])
    assert np.array_equal(host(ops.to_dtype(xt, torch.float32)), x, equal_nan=True)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 3, 5, 7), (1, 64, 56, 56), (3, 33, 17, 9), (16, 27, 256, 256)])
def test_layout_transforms_exact(shape, dt):
    g = rng(sum(shape))
    x, xt = prep(g.standard_normal(shape), dt)
    y = ops.nchw_to_nhwc(xt)
    assert np.array_equal(host(y), np.ascontiguousarray(x.transpose(0, 2, 3, 1)))
    assert np.array_equal(host(ops.nhwc_to_nchw(y)), x)


def test_size_mismatch_is_an_error_before_launch():
    # a weight one output channel short of what the dimensions say: rejected by the wrapper
    x = torch.zeros(1, 2, 5, 5, device=DEV)
    w = torch.zeros(2, 2, 3, 3, device=DEV)
    with pytest.raises(volta_amd.VoltaHipError) as e:
        ops.gpu_igemm(x, w, 1, 2, 3, 5, 5, 3, 3, 1, 1, 1, 1, 5, 5)
    assert e.value.status == 2
    with pytest.raises(volta_amd.VoltaHipError):
        ops.gpu_matmul(torch.zeros(4, 3, device=DEV), torch.zeros(2, 5, device=DEV), 4, 3, 5)
    conv = vnn.Conv2d(2, 3, 3, 1, 1, device=DEV)
    with pytest.raises(volta_amd.VoltaHipError):
        conv.backward(torch.zeros(1, 3, 4, 4, device=DEV), x)  # out_grad of the wrong size


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_allocating_forms_match_out_parameter_entries(dt):
    """The *_alloc entries (the reference's gpu_* return a new buffer,
    gpu_ops.rs:160-168) give the same bits as the out-parameter entries, in a
    pool buffer the caller releases with vh_free."""
    import ctypes
    lib = volta_amd.lib()
    code = volta_amd.F32 if dt == "f32" else volta_amd.BF16
    st = torch.cuda.current_stream().cuda_stream
    g = rng(17)

    def alloc_call(name, shape, *args):
        p = ctypes.c_void_p()
        volta_amd.check(getattr(lib, name)(code, *args[:2], ctypes.byref(p), *args[2:], st))
        torch.cuda.synchronize()
        host_buf = np.empty(int(np.prod(shape)), np.uint16 if dt == "bf16" else np.float32)
        volta_amd.check(lib.vh_download(host_buf.ctypes.data, p.value, host_buf.nbytes, st))
        volta_amd.check(lib.vh_free(p.value))
        t = torch.from_numpy(host_buf.view(np.int16) if dt == "bf16" else host_buf)
        return (t.view(torch.bfloat16) if dt == "bf16" else t).reshape(shape)

    m, k, n = 37, 24, 40
    _, at = prep(g.standard_normal((m, k)), dt)
    _, bt = prep(g.standard_normal((k, n)), dt)
    _, grt = prep(g.standard_normal((m, n)), dt)
    cases = [("vh_matmul_alloc", ops.gpu_matmul(at, bt, m, k, n), (at.data_ptr(), bt.data_ptr(), m, k, n)),
             ("vh_matmul_backward_a_alloc", ops.gpu_matmul_backward_a(grt, bt, m, k, n),
              (grt.data_ptr(), bt.data_ptr(), m, k, n)),
             ("vh_matmul_backward_b_alloc", ops.gpu_matmul_backward_b(at, grt, m, k, n),
              (at.data_ptr(), grt.data_ptr(), m, k, n))]
    B, C, O, H, W, K, S, P = 2, 8, 16, 11, 9, 3, 2, 1
    HO, WO = oracle.conv_out(H, K, S, P), oracle.conv_out(W, K, S, P)
    _, xt = prep(g.standard_normal((B, C, H, W)), dt)
    _, wt = prep(g.standard_normal((O, C, K, K)) * 0.2, dt)
    _, dyt = prep(g.standard_normal((B, O, HO, WO)), dt)
    dims = (B, C, O, H, W, K, K, S, S, P, P, HO, WO)
    for name, fn, t0, t1 in (("vh_direct_conv", ops.gpu_direct_conv, xt, wt), ("vh_igemm", ops.gpu_igemm, xt, wt),
                             ("vh_conv_backward_input", ops.gpu_conv_backward_input, dyt, wt),
                             ("vh_igemm_backward_input", ops.gpu_igemm_backward_input, dyt, wt),
                             ("vh_conv_backward_weight", ops.gpu_conv_backward_weight, dyt, xt),
                             ("vh_igemm_backward_weight", ops.gpu_igemm_backward_weight, dyt, xt)):
        cases.append((name + "_alloc", fn(t0, t1, *dims), (t0.data_ptr(), t1.data_ptr()) + dims))
    xp = torch.from_numpy(oracle.pad(host(xt), P, P)).to(DEV, DTYPES[dt])
    HP, WP = xp.shape[2:]
    col = ops.gpu_im2col(xp, B, C, HP, WP, K, K, S, S, HO, WO)
    cases.append(("vh_im2col_alloc", col, (xp.data_ptr(), None, B, C, HP, WP, K, K, S, S, HO, WO)))
    back = ops.gpu_col2im(col, B, C, HP, WP, K, K, S, S, HO, WO)
    cases.append(("vh_col2im_alloc", back, (col.data_ptr(), None, B, C, HP, WP, K, K, S, S, HO, WO)))
    for name, ref, args in cases:
        if args[1] is None:  # one input: (input, out, dims...)
            p = ctypes.c_void_p()
            volta_amd.check(getattr(lib, name)(code, args[0], ctypes.byref(p), *args[2:], st))
            torch.cuda.synchronize()
            host_buf = np.empty(ref.numel(), np.uint16 if dt == "bf16" else np.float32)
            volta_amd.check(lib.vh_download(host_buf.ctypes.data, p.value, host_buf.nbytes, st))
            volta_amd.check(lib.vh_free(p.value))
            t = torch.from_numpy(host_buf.view(np.int16) if dt == "bf16" else host_buf)
            got = (t.view(torch.bfloat16) if dt == "bf16" else t).reshape(ref.shape)
        else:
            got = alloc_call(name, tuple(ref.shape), *args)
        assert torch.equal(got, ref.cpu()), f"{name} differs from the out-parameter entry"
