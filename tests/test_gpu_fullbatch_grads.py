"""GPU: full-batch weight and bias gradients of the BASELINE layers with a dense dY.

`test_gpu_fullsize.py` checks the full-size weight gradients through a dY that
is zero outside a few images, so the split-K partials of most image ranges
are zero there.  Here every image contributes: dY is dense ~N(0,1) over the
whole batch and dW / db are compared with the oracle's sum over all images
(evaluated over image chunks in a thread pool, `tests/oracle_pool.py`).

configs[1]'s Linear layer (4096 rows, and a ragged 4104 x 1032 -> 4104) is
checked the same way, and its combined backward (in bf16 one launch for dX and
dW, with db as column sums inside the dW tiles) against the separate dX-only
and dW-only calls: dX and dW bit for bit, db against the oracle.

configs[2] is also run exactly as bench.py calls it: Conv2d without a bias,
so the forward gets a NULL bias and the weight gradient a NULL db (a separate
runtime path and workspace size in the weight-gradient kernel), next to the
same layer with a bias and its gradient."""
import numpy as np
import pytest
import torch

import oracle
from tests.oracle_pool import batch_sum
from tests.parity import assert_parity, k_conv_fwd, k_conv_wgrad
from volta_amd import nn as vnn

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


def oracle_wgrad(dy, x, w_shape, kw):
    return batch_sum(oracle.direct_conv_backward_weight, (dy, x), (w_shape,), kw)


def oracle_bgrad(dy):
    return batch_sum(oracle.conv_bias_grad, (dy,))


# ------------------------------------------------------------------ configs[2], N=128, bf16
C3 = [(64, 64, 56, 3, 1, 1), (128, 128, 28, 3, 1, 1), (256, 256, 14, 3, 1, 1), (64, 128, 56, 1, 2, 0)]


@pytest.mark.parametrize("layer", C3, ids=lambda l: "C{}O{}H{}K{}S{}".format(*l[:5]))
def test_config3_dense_wgrad_and_bench_calls(layer):
    C, O, H, K, S, P = layer
    B = 128
    print(f"configs[2] C{C} O{O} H{H} K{K} S{S}: dense dY over N={B}", flush=True)
    g = np.random.default_rng(1000 + C + O + H)
    x, xt = prep(g.standard_normal((B, C, H, H)), "bf16")
    w, wt = prep(g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K)), "bf16")
    HO = oracle.conv_out(H, K, S, P)
    dy, dyt = prep(g.standard_normal((B, O, HO, HO)), "bf16")
    kw = dict(stride=(S, S), pad=(P, P))
    kwg = k_conv_wgrad(B, HO, HO)
    ref_dw, sc_dw = oracle_wgrad(dy, x, w.shape, kw)

    # bench.py's calls: no bias (NULL bias pointer, NULL db)
    conv = vnn.Conv2d(C, O, K, S, P, use_bias=False, device=DEV, dtype=torch.bfloat16)
    conv.weight = wt
    conv.set_algo(vnn.ConvAlgo.IGEMM)
    y = host(conv.forward(xt))
    for i in (0, B - 1):
        ref = oracle.direct_conv(x[i:i + 1], w, **kw)
        sc = oracle.direct_conv(np.abs(x[i:i + 1]), np.abs(w), **kw)
        assert_parity(y[i:i + 1], ref, sc, "bf16", f"no-bias y[{i}]", k=k_conv_fwd(C, K, K, bias=False))
    dx_none, dw, db = conv.backward(dyt, xt, input_grad=False, weight_grad=True)
    assert dx_none is None and db is None
    assert_parity(host(dw), ref_dw, sc_dw, "bf16", "no-bias dw over the whole batch", k=kwg)

    # the same layer with a bias: dW and db over the whole batch
    convb = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=DEV, dtype=torch.bfloat16)
    convb.weight = wt
    convb.set_algo(vnn.ConvAlgo.IGEMM)
    _, dwb, dbb = convb.backward(dyt, xt, input_grad=False, weight_grad=True)
    dwb = host(dwb)
    assert_parity(dwb, ref_dw, sc_dw, "bf16", "dw (with db) over the whole batch", k=kwg)
    ref_db, sc_db = oracle_bgrad(dy)
    assert_parity(host(dbb), ref_db, sc_db, "bf16", "db over the whole batch", k=kwg)
    # requesting db does not change dW's bits
    assert np.array_equal(dwb, host(dw)), "dW differs between the calls with and without db"


# ------------------------------------------------------------------ configs[4], N=16, bf16
C5 = [(3, 64, 5, 2, "uniform"), (64, 64, 3, 1, "normal"), (64, 32, 3, 1, "normal"), (32, 27, 3, 1, "normal")]


@pytest.mark.parametrize("layer", C5, ids=lambda l: "C{}O{}K{}".format(*l[:3]))
def test_config5_dense_wgrad(layer):
    C, O, K, P, dist = layer
    B, H = 16, 256
    print(f"configs[4] C{C} O{O} K{K}: dense dY over N={B}", flush=True)
    g = np.random.default_rng(2000 + C * O)
    xs = (B, C, H, H)
    x, xt = prep(g.standard_normal(xs) if dist == "normal" else g.uniform(0, 1, xs), "bf16")
    w, wt = prep(g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K)), "bf16")
    dy, dyt = prep(g.standard_normal((B, O, H, H)), "bf16")
    conv = vnn.Conv2d(C, O, K, 1, P, use_bias=True, device=DEV, dtype=torch.bfloat16)
    conv.weight = wt
    _, dw, db = conv.backward(dyt, xt, input_grad=False, weight_grad=True, algo=vnn.ConvAlgo.Auto)
    kw = dict(stride=(1, 1), pad=(P, P))
    kwg = k_conv_wgrad(B, H, H)
    ref, sc = oracle_wgrad(dy, x, w.shape, kw)
    assert_parity(host(dw), ref, sc, "bf16", "dw over the whole batch", k=kwg)
    ref, sc = oracle_bgrad(dy)
    assert_parity(host(db), ref, sc, "bf16", "db over the whole batch", k=kwg)


# ------------------------------------------------------------------ configs[3], N=128, f32 ConvTranspose2d
C4 = [(100, 512, 1, 4, 1, 0), (512, 256, 4, 4, 2, 1), (256, 128, 8, 4, 2, 1), (128, 64, 16, 4, 2, 1),
      (64, 3, 32, 4, 2, 1)]


@pytest.mark.parametrize("layer", C4, ids=lambda l: "CI{}CO{}H{}".format(*l[:3]))
def test_config4_dense_wgrad(layer):
    CI, CO, H, K, S, P = layer
    B = 128
    print(f"configs[3] CI{CI} CO{CO} H{H}: dense dY over N={B}", flush=True)
    g = np.random.default_rng(3000 + CI + CO)
    x, xt = prep(g.standard_normal((B, CI, H, H)), "f32")
    w, wt = prep(g.normal(0.0, 0.02, (CI, CO, K, K)), "f32")
    HO = oracle.convt_out(H, K, S, P)
    dy, dyt = prep(g.standard_normal((B, CO, HO, HO)), "f32")
    ct = vnn.ConvTranspose2d(CI, CO, K, S, P, device=DEV, dtype=torch.float32)
    ct.weight = wt
    _, dw, db = ct.backward(dyt, xt, input_grad=False, weight_grad=True)
    kw = dict(stride=(S, S), pad=(P, P))
    for j, name, got in ((1, "dw", dw), (2, "db", db)):
        ref, sc = batch_sum(oracle.conv_transpose_backward, (dy, x), (w,), kw, pick=lambda r, j=j: r[j])
        assert_parity(host(got), ref, sc, "f32", f"{name} over the whole batch")


# ------------------------------------------------------------------ configs[1], N=64, f32
@pytest.mark.parametrize("C,O", [(1, 32), (32, 64)])
def test_config1_dense_wgrad(C, O):
    B, H = 64, 28
    g = np.random.default_rng(4000 + C)
    x, xt = prep(g.standard_normal((B, C, H, H)), "f32")
    w, wt = prep(g.uniform(-1, 1, (O, C, 3, 3)) * np.sqrt(6.0 / (C * 9)), "f32")
    dy, dyt = prep(g.standard_normal((B, O, H, H)), "f32")
    conv = vnn.Conv2d(C, O, 3, 1, 1, use_bias=True, device=DEV, dtype=torch.float32)
    conv.weight = wt
    _, dw, db = conv.backward(dyt, xt, input_grad=False, weight_grad=True, algo=vnn.ConvAlgo.Auto)
    kw = dict(stride=(1, 1), pad=(1, 1))
    ref, sc = oracle_wgrad(dy, x, w.shape, kw)
    assert_parity(host(dw), ref, sc, "f32", "dw over the whole batch")
    ref, sc = oracle_bgrad(dy)
    assert_parity(host(db), ref, sc, "f32", "db over the whole batch")


# ------------------------------------------------------------------ configs[1] Linear, 4096 rows
@pytest.mark.parametrize("dt,shape", [("f32", (4096, 1024, 4096)), ("bf16", (4096, 1024, 4096)),
                                      ("bf16", (4104, 1032, 4104))], ids=["f32", "bf16", "bf16-ragged"])
def test_config2_linear_dense_grads(dt, shape):
    M, IN, OUT = shape
    print(f"configs[1] Linear {dt} {shape}: dense dY over {M} rows", flush=True)
    g = np.random.default_rng(5000)
    x, xt = prep(g.standard_normal((M, IN)), dt)
    bound = np.sqrt(6.0 / (IN + OUT))
    w, wt = prep(g.uniform(-bound, bound, (IN, OUT)), dt)
    dy, dyt = prep(g.standard_normal((M, OUT)), dt)
    lin = vnn.Linear(IN, OUT, device=DEV, dtype=DT[dt])
    lin.weight = wt
    dxt, dwt, dbt = lin.backward(dyt, xt)
    dx, dw, db = host(dxt), host(dwt), host(dbt)
    both = lambda r: np.concatenate([r[1].ravel(), r[2]])  # dW and db of one chunk
    ref, sc = batch_sum(oracle.linear_backward, (dy, x), (w,), pick=both)
    n = IN * OUT
    assert_parity(dw, ref[:n].reshape(IN, OUT), sc[:n].reshape(IN, OUT), dt, "dw over all rows", k=M)
    ref_db, sc_db = ref[n:], sc[n:]
    assert_parity(db, ref_db, sc_db, dt, "db over all rows", k=M)
    rows = [0, 1, M // 2, M - 1]
    ref = oracle.linear_backward(dy[rows], x[rows], w)[0]
    sc = oracle.linear_backward(np.abs(dy[rows]), np.abs(x[rows]), np.abs(w))[0]
    assert_parity(dx[rows], ref, sc, dt, "dx rows", k=OUT)
    # the combined call equals the separate ones (dX, dW: the same MFMA order
    # per element whatever the tiling); the dW-only call's db is its own sum
    dx1 = host(lin.backward(dyt, xt, input_grad=True, weight_grad=False)[0])
    _, dw2, db2 = lin.backward(dyt, xt, input_grad=False, weight_grad=True)
    assert np.array_equal(dx, dx1), "dX of the combined backward differs from the dX-only call"
    assert np.array_equal(dw, host(dw2)), "dW of the combined backward differs from the dW-only call"
    assert_parity(host(db2), ref_db, sc_db, dt, "db of the dW-only call", k=M)
