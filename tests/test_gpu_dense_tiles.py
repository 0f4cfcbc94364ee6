"""GPU parity of the 256 x 256 product tiles (operands copied straight into
LDS, swizzled layouts), bf16 and f32: whole outputs of every operand layout
they serve -- matmul (K-major x MN-major), its dA (K-major x K-major) and dB
(MN-major x MN-major), and the Linear forward with its bias -- at shapes that
take them (M and N multiples of 256 with at least 256 tiles, K a multiple of
128 for bf16 -- one and three turns of its two-stage loop -- and of 64 for
f32), against the CPU oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from volta_amd import nn as vnn
from volta_amd import ops
from tests.parity import assert_parity

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


TORCH_DT = {"bf16": torch.bfloat16, "f32": torch.float32}


def prep(a, dt):
    r = np.ascontiguousarray(a, np.float32)
    if dt == "bf16":
        r = oracle.round_bf16(r)
    return r, torch.from_numpy(r).to(DEV, TORCH_DT[dt])


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def check(got, fn, args, what, k, dt, extra=None):
    ref = fn(*args)
    scale = fn(*[np.abs(a) for a in args])
    if extra is not None:
        ref = ref + extra
        scale = scale + np.abs(extra)
    assert_parity(host(got), ref, scale, dt, what, k=k)


@pytest.mark.parametrize("dt,kk", [("bf16", 128), ("bf16", 384), ("f32", 64), ("f32", 384)])
def test_matmul_256_tiles(dt, kk):
    m, n = 4096, 4096
    g = np.random.default_rng(kk + 1)
    a, at = prep(g.standard_normal((m, kk)), dt)
    b, bt = prep(g.standard_normal((kk, n)), dt)
    check(ops.gpu_matmul(at, bt, m, kk, n), oracle.matmul, (a, b), f"C = A.B, K = {kk}", kk, dt)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_matmul_backward_a_256_tiles(dt):
    # dA[m][k] = G[m][n] . B[k][n]^T: M = m, N = k, contraction n
    m, k, n = 4096, 4096, 128
    g = np.random.default_rng(21)
    gr, grt = prep(g.standard_normal((m, n)), dt)
    b, bt = prep(g.standard_normal((k, n)), dt)
    check(ops.gpu_matmul_backward_a(grt, bt, m, k, n), oracle.matmul_backward_a, (gr, b), "dA", n, dt)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_matmul_backward_b_256_tiles(dt):
    # dB[k][n] = A[m][k]^T . G[m][n]: M = k, N = n, contraction m
    m, k, n = 128, 4096, 4096
    g = np.random.default_rng(22)
    a, at = prep(g.standard_normal((m, k)), dt)
    gr, grt = prep(g.standard_normal((m, n)), dt)
    check(ops.gpu_matmul_backward_b(at, grt, m, k, n), oracle.matmul_backward_b, (a, gr), "dB", m, dt)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_linear_forward_256_tiles(dt):
    m, i, o = 4096, 128, 4096
    g = np.random.default_rng(23)
    x, xt = prep(g.standard_normal((m, i)), dt)
    w, wt = prep(g.uniform(-0.5, 0.5, (i, o)), dt)
    b, bt = prep(g.uniform(-1, 1, (o,)), dt)
    lin = vnn.Linear(i, o, device=DEV, dtype=TORCH_DT[dt])
    lin.weight, lin.bias = wt, bt
    check(lin.forward(xt), oracle.matmul, (x, w), "Linear y = x.W + b", i + 1, dt, extra=b[None, :])


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_linear_backward_pair_tiles(dt):
    # dX (K-major x K-major) and dW + db (MN-major x MN-major, the column sums
    # of dY in the dW tiles) as one launch of 128 x 256 tiles: 32 + 256 tiles,
    # 16 m-tiles sharing each dW column tile's 256 bias columns
    m, i, o = 512, 2048, 4096
    g = np.random.default_rng(24)
    x, xt = prep(g.standard_normal((m, i)), dt)
    w, wt = prep(g.uniform(-0.05, 0.05, (i, o)), dt)
    dy, dyt = prep(g.standard_normal((m, o)), dt)
    lin = vnn.Linear(i, o, device=DEV, dtype=TORCH_DT[dt])
    lin.weight = wt
    dx, dw, db = lin.backward(dyt, xt)
    ref = oracle.linear_backward(dy, x, w)
    sc = oracle.linear_backward(np.abs(dy), np.abs(x), np.abs(w))
    assert_parity(host(dx), ref[0], sc[0], dt, "dX", k=o)
    assert_parity(host(dw), ref[1], sc[1], dt, "dW", k=m)
    assert_parity(host(db), ref[2], sc[2], dt, "db", k=m)
