"""Pins the CPU oracle (oracle/volta_oracle.c) before anything is checked against it.

Each oracle function is tied to something that does not restate its own formula:
the reference's known-answer tests (file:line), closed forms (all-ones convs,
window sums), float64 library routines (torch CPU double), adjointness
identities, and cross-algorithm equalities that the reference's own tests assert.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as orc

RNG = np.random.default_rng(1234)


def randn(*shape):
    return RNG.standard_normal(shape).astype(np.float32)


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def close(a, b, tol):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(np.abs(b).max(), 1e-30)
    return np.abs(a - b).max() / scale <= tol


# ----------------------------------------------------------------- known answers
def test_matmul_known_answers():
    # src/lib.rs:4538-4547
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    assert orc.matmul(a, b).ravel().tolist() == [4.0, 5.0, 10.0, 11.0]
    # tests/gpu_test.rs:46-60
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    assert orc.matmul(a, b).ravel().tolist() == [19.0, 22.0, 43.0, 50.0]
    # src/lib.rs:4621-4631 (all-ones (2,3)@(3,2) -> 3 everywhere)
    assert (orc.matmul(np.ones((2, 3)), np.ones((3, 2))) == 3.0).all()
    # src/lib.rs:4592-4605 (dot: [1,2,3].[4,-1,2] = 8 as a 1x3 @ 3x1)
    assert orc.matmul(np.array([[1, 2, 3]]), np.array([[4], [-1], [2]]))[0, 0] == 8.0


def test_linear_known_answer():
    # src/lib.rs:4693-4712: W=[[1,2,3],[4,5,6]] (in=2,out=3), b=[10,20,30], x=[1,1]
    w = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    y = orc.linear_forward(np.ones((1, 2)), w, np.array([10, 20, 30], np.float32))
    assert y.ravel().tolist() == [15.0, 27.0, 39.0]


def test_transpose_known_answer():
    # src/lib.rs:4640-4647 transpose_2d_shape_and_value
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    g = orc.matmul_backward_a(np.eye(3, dtype=np.float32), x)  # I . x^T = x^T
    assert g.ravel().tolist() == [1.0, 4.0, 2.0, 5.0, 3.0, 6.0]


# ----------------------------------------------------------------- closed forms
ALGOS = {
    "direct": lambda x, w, s, p: orc.direct_conv(x, w, s, p),
    "im2col": lambda x, w, s, p: orc.im2col_conv_forward(x, w, s, p),
    "igemm": lambda x, w, s, p: orc.igemm_forward(x, w, s, p),
}


@pytest.mark.parametrize("algo", sorted(ALGOS))
def test_conv_all_ones_closed_form(algo):
    # conv.rs:2930-2976: 2->4 channels, 3x3, pad 1, all-ones 1x2x8x8 -> C * (#valid taps)
    x = np.ones((1, 2, 8, 8), np.float32)
    w = np.ones((4, 2, 3, 3), np.float32)
    y = ALGOS[algo](x, w, (1, 1), (1, 1))
    taps = np.full(8, 3.0)
    taps[0] = taps[-1] = 2.0
    expect = 2.0 * np.outer(taps, taps)
    for o in range(4):
        assert np.array_equal(y[0, o], expect)


@pytest.mark.parametrize("algo", sorted(ALGOS))
def test_conv_ramp_window_sums(algo):
    # conv.rs:3021-3065: 1x1x4x4 ramp 0..15, 2x2 all-ones kernel, no pad
    x = np.arange(16, dtype=np.float32).reshape(1, 1, 4, 4)
    w = np.ones((1, 1, 2, 2), np.float32)
    y = ALGOS[algo](x, w, (1, 1), (0, 0))[0, 0]
    r = x[0, 0]
    expect = r[:-1, :-1] + r[:-1, 1:] + r[1:, :-1] + r[1:, 1:]
    assert np.array_equal(y, expect)


def test_conv_output_shapes():
    # conv.rs:2241-2266 (H_out = (H + 2p - k)/s + 1) and conv_transpose.rs:672-698
    for (h, k, s, p) in [(28, 3, 1, 1), (56, 1, 2, 0), (7, 3, 2, 1), (32, 5, 1, 2), (9, 4, 3, 0)]:
        x = randn(1, 2, h, h)
        w = randn(3, 2, k, k)
        y = orc.direct_conv(x, w, (s, s), (p, p))
        assert y.shape[2] == (h + 2 * p - k) // s + 1
        yt = F.conv2d(t64(x), t64(w), stride=s, padding=p)
        assert y.shape == tuple(yt.shape)
    for (h, k, s, p) in [(1, 4, 1, 0), (4, 4, 2, 1), (32, 4, 2, 1)]:
        x = randn(1, 2, h, h)
        w = randn(2, 3, k, k)
        y = orc.conv_transpose_forward(x, w, None, (s, s), (p, p))
        assert y.shape == (1, 3, (h - 1) * s + k - 2 * p, (h - 1) * s + k - 2 * p)


# ----------------------------------------------------------------- auto-select table
@pytest.mark.parametrize(
    "dims,cpu,gpu",
    [
        # (B, C, H, W, K): values from conv.rs:29-69 applied to the BASELINE configs
        ((64, 1, 28, 28, 3), orc.ALGO_IM2COL, orc.ALGO_IM2COL),   # e = 389,376
        ((64, 32, 28, 28, 3), orc.ALGO_DIRECT, orc.ALGO_IGEMM),   # e = 12,460,032
        ((128, 64, 56, 56, 3), orc.ALGO_DIRECT, orc.ALGO_IGEMM),  # e = 214,990,848
        ((128, 64, 56, 56, 1), orc.ALGO_DIRECT, orc.ALGO_IGEMM),  # e = 25,690,112
        ((2, 3, 8, 8, 3), orc.ALGO_DIRECT, orc.ALGO_IM2COL),      # K<=3 && B<=4 on CPU
        ((8, 32, 30, 30, 3), orc.ALGO_IGEMM, orc.ALGO_IGEMM),     # 1e6 < e = 1,806,336 <= 5e6
        ((8, 4, 12, 12, 5), orc.ALGO_IM2COL, orc.ALGO_IM2COL),    # e = 51,200
    ],
)
def test_auto_select_table(dims, cpu, gpu):
    B, C, H, W, K = dims
    e = B * (H - K + 1) * (W - K + 1) * C * K * K
    assert orc.auto_select(B, C, H, W, K, False) == cpu, e
    assert orc.auto_select(B, C, H, W, K, True) == gpu, e


def test_auto_select_underflow_reported():
    assert orc.auto_select(1, 1, 2, 2, 3, True) == -1


# ----------------------------------------------------------------- float64 library
CONV_CASES = [
    # (B, C, O, H, W, K, S, P)
    (2, 3, 4, 7, 9, 3, 1, 1),
    (3, 2, 5, 8, 8, 3, 2, 1),
    (2, 4, 3, 9, 7, 1, 2, 0),
    (1, 3, 2, 10, 10, 5, 1, 2),
    (2, 2, 3, 6, 6, 4, 2, 1),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv_fwd_bwd_vs_torch_f64(case):
    B, C, O, H, W, K, S, P = case
    x, w = randn(B, C, H, W), randn(O, C, K, K)
    xt = t64(x).requires_grad_(True)
    wt = t64(w).requires_grad_(True)
    yt = F.conv2d(xt, wt, stride=S, padding=P)
    dy = randn(*yt.shape)
    yt.backward(t64(dy))
    for y in (orc.direct_conv(x, w, (S, S), (P, P)),
              orc.im2col_conv_forward(x, w, (S, S), (P, P)),
              orc.igemm_forward(x, w, (S, S), (P, P))):
        assert close(y, yt.detach().numpy(), 1e-5)
    assert close(orc.conv_forward_f64(x, w, (S, S), (P, P)), yt.detach().numpy(), 1e-12)
    dx_ref, dw_ref = xt.grad.numpy(), wt.grad.numpy()
    assert close(orc.direct_conv_backward_input(dy, w, x.shape, (S, S), (P, P)), dx_ref, 1e-5)
    assert close(orc.igemm_backward_input(dy, w, x.shape, (S, S), (P, P)), dx_ref, 1e-5)
    assert close(orc.direct_conv_backward_weight(dy, x, w.shape, (S, S), (P, P)), dw_ref, 1e-5)
    assert close(orc.igemm_backward_weight(x, dy, w.shape, (S, S), (P, P)), dw_ref, 1e-5)
    dx2, dw2 = orc.im2col_conv_backward(dy, x, w, (S, S), (P, P))
    assert close(dx2, dx_ref, 1e-5) and close(dw2, dw_ref, 1e-5)
    assert close(orc.conv_bias_grad(dy), dy.astype(np.float64).sum(axis=(0, 2, 3)), 1e-5)


@pytest.mark.parametrize("case", [(1, 2, 3, 5, 4, 3, 1, 1), (2, 2, 2, 6, 5, 3, 2, 1), (1, 1, 2, 4, 4, 2, 2, 0)])
def test_direct_dx_pruned_equals_literal_bitwise(case):
    # conv.rs:450-515 literally vs. the order-preserving pruned form used at scale
    B, C, O, H, W, K, S, P = case
    w = randn(O, C, K, K)
    HO, WO = orc.conv_out(H, K, S, P), orc.conv_out(W, K, S, P)
    dy = randn(B, O, HO, WO)
    a = orc.direct_conv_backward_input(dy, w, (B, C, H, W), (S, S), (P, P))
    b = orc.direct_conv_backward_input(dy, w, (B, C, H, W), (S, S), (P, P), literal=True)
    assert np.array_equal(a, b)


def test_conv_adjointness():
    # <conv(x), y> = <x, dgrad(y)> = <W, wgrad(x, y)>
    B, C, O, H, W, K, S, P = 2, 3, 4, 9, 8, 3, 2, 1
    x, w = randn(B, C, H, W), randn(O, C, K, K)
    y = orc.direct_conv(x, w, (S, S), (P, P))
    g = randn(*y.shape)
    lhs = float((y.astype(np.float64) * g).sum())
    dx = orc.direct_conv_backward_input(g, w, x.shape, (S, S), (P, P))
    dw = orc.direct_conv_backward_weight(g, x, w.shape, (S, S), (P, P))
    assert abs(lhs - float((x.astype(np.float64) * dx).sum())) < 1e-4 * max(1, abs(lhs))
    assert abs(lhs - float((w.astype(np.float64) * dw).sum())) < 1e-4 * max(1, abs(lhs))


def test_algorithms_agree_batch1_reference_tolerances():
    # conv.rs:2386-2450 (Direct vs Im2col fwd, 1e-5), 2587-2668 (grads, 1e-4),
    # 2733-2850 (iGEMM vs Direct) -- all at batch 1 in the reference.
    x, w = randn(1, 3, 10, 10), randn(4, 3, 3, 3)
    d = orc.direct_conv(x, w, (1, 1), (1, 1))
    assert np.abs(orc.im2col_conv_forward(x, w, (1, 1), (1, 1)) - d).max() < 1e-5
    assert np.abs(orc.igemm_forward(x, w, (1, 1), (1, 1), bug_compat=True) - d).max() < 1e-5
    dy = np.ones_like(d)
    dxd = orc.direct_conv_backward_input(dy, w, x.shape, (1, 1), (1, 1))
    dwd = orc.direct_conv_backward_weight(dy, x, w.shape, (1, 1), (1, 1))
    dxi, dwi = orc.im2col_conv_backward(dy, x, w, (1, 1), (1, 1))
    assert np.abs(dxi - dxd).max() < 1e-4 and np.abs(dwi - dwd).max() < 1e-4
    assert np.abs(orc.igemm_backward_input(dy, w, x.shape, (1, 1), (1, 1), True) - dxd).max() < 1e-4
    assert np.abs(orc.igemm_backward_weight(x, dy, w.shape, (1, 1), (1, 1), True) - dwd).max() < 1e-4


def test_igemm_batch_offset_bug_mapping():
    # conv.rs:1773: slot index b*O*SP + oc*SP + s_idx with s_idx = b*SP + rem.
    B, C, O, H, W = 3, 2, 5, 5, 4
    x, w = randn(B, C, H, W), randn(O, C, 3, 3)
    good = orc.igemm_forward(x, w, (1, 1), (1, 1), bug_compat=False)
    bad = orc.igemm_forward(x, w, (1, 1), (1, 1), bug_compat=True)
    SP = good.shape[2] * good.shape[3]
    total = good.size
    expect = np.zeros(total, np.float64)
    gf = good.reshape(B, O, SP)
    for b in range(B):
        for oc in range(O):
            for rem in range(SP):
                idx = b * O * SP + oc * SP + b * SP + rem
                if idx < total:
                    expect[idx] += gf[b, oc, rem]
    assert close(bad.ravel(), expect, 1e-6)
    assert np.array_equal(bad[0], good[0])  # batch 0 is unaffected
    assert not np.allclose(bad[1:], good[1:])


# ----------------------------------------------------------------- im2col / col2im
def test_im2col_col2im_adjoint_and_index_map():
    x = randn(2, 3, 6, 7)
    col = orc.im2col(x, (3, 2), (2, 1))
    HO, WO = (6 - 3) // 2 + 1, (7 - 2) // 1 + 1
    for b, oh, ow, c, kh, kw in [(0, 0, 0, 0, 0, 0), (1, 1, 5, 2, 2, 1), (1, 0, 3, 1, 1, 0)]:
        row = (b * HO + oh) * WO + ow
        assert col[row, (c * 3 + kh) * 2 + kw] == x[b, c, oh * 2 + kh, ow + kw]
    g = randn(*col.shape)
    back = orc.col2im(g, x.shape, (3, 2), (2, 1))
    lhs = float((col.astype(np.float64) * g).sum())
    rhs = float((x.astype(np.float64) * back).sum())
    assert abs(lhs - rhs) < 1e-4 * max(1.0, abs(lhs))
    # Unfold in torch is the same map (rows transposed)
    u = F.unfold(t64(x), (3, 2), stride=(2, 1))  # [B, C*kh*kw, L]
    assert close(col, u.permute(0, 2, 1).reshape(-1, 18).numpy(), 0)


# ----------------------------------------------------------------- matmul / linear
def test_matmul_family_vs_torch_f64():
    a, b = randn(37, 19), randn(19, 23)
    g = randn(37, 23)
    assert close(orc.matmul(a, b), (t64(a) @ t64(b)).numpy(), 1e-6)
    assert close(orc.matmul_backward_a(g, b), (t64(g) @ t64(b).T).numpy(), 1e-6)
    assert close(orc.matmul_backward_b(a, g), (t64(a).T @ t64(g)).numpy(), 1e-6)


def test_linear_fwd_bwd_vs_torch_f64():
    x, w, bias = randn(9, 6), randn(6, 4), randn(4)
    xt, wt, bt = (t64(v).requires_grad_(True) for v in (x, w, bias))
    yt = xt @ wt + bt
    dy = randn(9, 4)
    yt.backward(t64(dy))
    assert close(orc.linear_forward(x, w, bias), yt.detach().numpy(), 1e-6)
    dx, dw, db = orc.linear_backward(dy, x, w)
    assert close(dx, xt.grad.numpy(), 1e-6)
    assert close(dw, wt.grad.numpy(), 1e-6)
    assert close(db, bt.grad.numpy(), 1e-6)


# ----------------------------------------------------------------- ConvTranspose2d
@pytest.mark.parametrize("case", [(2, 3, 4, 1, 1, 4, 1, 0), (2, 4, 3, 4, 4, 4, 2, 1), (1, 2, 2, 5, 3, 3, 2, 1)])
def test_conv_transpose_vs_torch_f64(case):
    B, CI, CO, H, W, K, S, P = case
    x, w, bias = randn(B, CI, H, W), randn(CI, CO, K, K), randn(CO)
    xt, wt, bt = (t64(v).requires_grad_(True) for v in (x, w, bias))
    yt = F.conv_transpose2d(xt, wt, bt, stride=S, padding=P)
    dy = randn(*yt.shape)
    yt.backward(t64(dy))
    y = orc.conv_transpose_forward(x, w, bias, (S, S), (P, P))
    assert close(y, yt.detach().numpy(), 1e-5)
    dx, dw, db = orc.conv_transpose_backward(dy, x, w, (S, S), (P, P))
    assert close(dx, xt.grad.numpy(), 1e-5)
    assert close(dw, wt.grad.numpy(), 1e-5)
    assert close(db, bt.grad.numpy(), 1e-5)
    # identity: convT(x; W) == conv-dgrad(x as dY; W as OIHW) on the output grid
    y2 = orc.direct_conv_backward_input(x, w, (B, CO) + y.shape[2:], (S, S), (P, P))
    assert close(y2 + bias[None, :, None, None], y, 1e-5)


# ----------------------------------------------------------------- PixelShuffle
def test_pixel_shuffle_vs_torch():
    x = randn(2, 27, 4, 5)
    y = orc.pixel_shuffle(x, 3)
    assert np.array_equal(y, F.pixel_shuffle(torch.from_numpy(x), 3).numpy())
    dy = randn(*y.shape)
    assert np.array_equal(orc.pixel_shuffle_backward(dy, 3), F.pixel_unshuffle(torch.from_numpy(dy), 3).numpy())


# ----------------------------------------------------------------- glue: ReLU, sum loss
def test_relu_known_answers_and_special_values():
    # src/lib.rs:4332-4336 (relu_forward)
    assert orc.relu(np.array([1.0, -2.0, 0.0, 3.5], np.float32)).tolist() == [1.0, 0.0, 0.0, 3.5]
    x = np.array([np.nan, np.inf, -np.inf, -0.0, 1e-45, -1e-45], np.float32)
    y = orc.relu(x)
    # Rust f32::max(NaN, 0) = 0 (the non-NaN operand); +inf kept; subnormals kept
    assert y.tolist() == [0.0, np.inf, 0.0, 0.0, np.float32(1e-45), 0.0]
    z = randn(4096)
    assert np.array_equal(orc.relu(z), torch.relu(torch.from_numpy(z)).numpy())


def test_relu_backward_vs_autograd_and_gradcheck_points():
    # relu_gradcheck (src/lib.rs:4406-4411) points, away from 0
    x = np.array([-1.5, -0.5, 0.5, 1.5], np.float32)
    assert orc.relu_backward(np.ones(4, np.float32), x).tolist() == [0.0, 0.0, 1.0, 1.0]
    x = randn(3000)
    g = randn(3000)
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    torch.relu(xt).backward(t64(g))
    assert np.array_equal(orc.relu_backward(g, x), xt.grad.numpy().astype(np.float32))
    # at exactly 0 the reference passes no gradient (x > 0 is false)
    assert orc.relu_backward(np.ones(2, np.float32), np.array([0.0, -0.0], np.float32)).tolist() == [0.0, 0.0]


def test_sum_known_answers_and_float64_bound():
    # test_scalar_sum (src/lib.rs:2701-2712), test_sum_backward (src/lib.rs:145-151)
    assert orc.sum_all(np.array([42.0], np.float32)) == 42.0
    assert orc.sum_all(np.array([1.0, 2.0, 3.0], np.float32)) == 6.0
    assert orc.sum_backward(1.0, (3,)).tolist() == [1.0, 1.0, 1.0]
    # integers below 2^24 add exactly in f32: closed form n(n-1)/2
    assert orc.sum_all(np.arange(4096, dtype=np.float32)) == 4096 * 4095 / 2
    # one f32 accumulator in index order: within n * eps * sum|x| of the exact sum,
    # and equal to a literal Python loop in float32
    x = randn(20000)
    exact = float(np.sum(x.astype(np.float64)))
    assert abs(orc.sum_all(x) - exact) <= x.size * 2 ** -24 * float(np.abs(x).sum())
    acc = np.float32(0)
    for v in x[:2000]:
        acc = np.float32(acc + v)
    assert orc.sum_all(x[:2000]) == float(acc)
    assert np.array_equal(orc.sum_backward(2.5, (2, 3)), np.full((2, 3), 2.5, np.float32))


# ----------------------------------------------------------------- the step after dW
def test_optimizer_step_reference_known_answers():
    # tests/test_optimizers.rs:169-197 (SGD), 199-224 (weight decay)
    p, _, _ = orc.optimizer_step(0, 0.1, np.array([5.0], np.float32), np.array([2.0], np.float32))
    assert abs(p[0] - 4.8) < 1e-7
    p, _, _ = orc.optimizer_step(0, 0.1, p, np.array([2.0], np.float32))
    assert abs(p[0] - np.float32(np.float32(4.8) - np.float32(0.2))) < 1e-7
    p, _, _ = orc.optimizer_step(0, 0.1, np.array([4.0], np.float32), np.array([1.0], np.float32), weight_decay=0.1)
    assert abs(p[0] - 3.86) < 1e-7
    # tests/coverage_fill.rs:46-66 (momentum 0.9, lr 0.1, grad 0.1)
    p, v, _ = orc.optimizer_step(1, 0.1, np.array([1.0], np.float32), np.array([0.1], np.float32), beta1=0.9)
    assert abs(p[0] - 0.99) < 1e-6
    p, v, _ = orc.optimizer_step(1, 0.1, p, np.array([0.1], np.float32), s1=v, beta1=0.9)
    assert abs(p[0] - 0.971) < 1e-6


def test_optimizer_step_vs_float64_formulas():
    n = 1000
    p0, g, m0, v0 = randn(n), randn(n), randn(n) * 0.1, np.abs(randn(n)) * 0.01
    for wd in (0.0, 0.01):
        ge = g.astype(np.float64) + wd * p0.astype(np.float64)
        p, _, _ = orc.optimizer_step(0, 0.05, p0, g, weight_decay=wd)
        assert close(p, p0 - 0.05 * ge, 1e-6)
        p, v, _ = orc.optimizer_step(1, 0.05, p0, g, s1=m0, beta1=0.9, weight_decay=wd)
        ve = 0.9 * m0 - 0.05 * ge
        assert close(v, ve, 1e-6) and close(p, p0 + ve, 1e-6)
        t = 3.0
        p, m, v = orc.optimizer_step(2, 1e-3, p0, g, s1=m0, s2=v0, beta1=0.9, beta2=0.999, t=t, eps=1e-8,
                                     weight_decay=wd)
        me = 0.9 * m0 + 0.1 * ge
        vv = 0.999 * v0 + 0.001 * ge * ge
        pe = p0 - 1e-3 * (me / (1 - 0.9 ** t)) / (np.sqrt(vv / (1 - 0.999 ** t)) + 1e-8)
        assert close(m, me, 1e-6) and close(v, vv, 1e-5) and close(p, pe, 1e-6)


def test_grad_accumulate():
    a, b = randn(500), randn(500)
    assert np.array_equal(orc.add(a, b), (a + b).astype(np.float32))


# ----------------------------------------------------------------- bf16 rounding
def test_bf16_rne_matches_torch():
    vals = np.concatenate([randn(4096) * 1e3, np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875,
                                                         3.4e38, -3.4e38, 1e-40, np.inf, -np.inf], np.float32)])
    ours = orc.bf16_bits(vals)
    theirs = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    r = orc.round_bf16(vals)
    assert np.array_equal(r, torch.from_numpy(vals).to(torch.bfloat16).float().numpy())
