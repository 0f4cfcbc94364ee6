"""GPU: every golden fixture (one layer of each BASELINE configuration, batch 2)
through the HIP library, compared with the fixture's expected outputs under the
scaled-error gate.  Convolutions run under every algorithm; the per-element scale
S = f(|inputs|) comes from the oracle on absolute values."""
import numpy as np
import pytest
import torch

import oracle
import volta_amd
from tests.golden_io import load, names
from tests.parity import assert_parity
from volta_amd import nn as vnn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV, DT[dt])


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def _abs(d):
    return {k: (np.abs(v) if isinstance(v, np.ndarray) and v.dtype == np.float32 else v) for k, v in d.items()}


def _conv_scales(d):
    a = _abs(d)
    m = d["meta"]
    st, pd = (int(m[6]),) * 2, (int(m[7]),) * 2
    return dict(y=oracle.direct_conv(a["x"], a["w"], st, pd) + a["b"][None, :, None, None],
                dx=oracle.direct_conv_backward_input(a["dy"], a["w"], d["x"].shape, st, pd),
                dw=oracle.direct_conv_backward_weight(a["dy"], a["x"], d["w"].shape, st, pd),
                db=oracle.conv_bias_grad(a["dy"]))


CONV = [n for n in names() if n.startswith(("c1_", "c3_", "c5_conv"))]
CONVT = [n for n in names() if n.startswith("c4_")]
LINEAR = [n for n in names() if n.startswith("c2_")]


@pytest.mark.parametrize("algo", [vnn.ConvAlgo.Direct, vnn.ConvAlgo.Im2col, vnn.ConvAlgo.IGEMM, vnn.ConvAlgo.Auto])
@pytest.mark.parametrize("name", CONV)
def test_conv_fixture(name, algo):
    d = load(name)
    dt = d["dtype"]
    B, C, O, H, W, K, S, P = map(int, d["meta"])
    conv = vnn.Conv2d(C, O, K, S, P, use_bias=True, device=DEV, dtype=DT[dt])
    conv.weight, conv.bias = dev(d["w"], dt), dev(d["b"], dt)
    conv.set_algo(algo)
    x = dev(d["x"], dt)
    y = conv.forward(x)
    dx, dw, db = conv.backward(dev(d["dy"], dt), x)
    sc = _conv_scales(d)
    HO, WO = oracle.conv_out(H, K, S, P), oracle.conv_out(W, K, S, P)
    ks = dict(y=C * K * K + 1, dx=O * K * K, dw=B * HO * WO, db=B * HO * WO)
    for k, got in (("y", y), ("dx", dx), ("dw", dw), ("db", db)):
        assert_parity(host(got), d[k], sc[k], dt, f"{name}/{algo.name}/{k}", k=ks[k])


@pytest.mark.parametrize("name", CONVT)
def test_conv_transpose_fixture(name):
    d = load(name)
    dt = d["dtype"]
    B, CI, CO, H, W, K, S, P = map(int, d["meta"])
    ct = vnn.ConvTranspose2d(CI, CO, K, S, P, device=DEV, dtype=DT[dt])
    ct.weight, ct.bias = dev(d["w"], dt), dev(d["b"], dt)
    x = dev(d["x"], dt)
    y = ct.forward(x)
    dx, dw, db = ct.backward(dev(d["dy"], dt), x)
    a = _abs(d)
    st, pd = (S, S), (P, P)
    sy = oracle.conv_transpose_forward(a["x"], a["w"], a["b"], st, pd)
    sdx, sdw, sdb = oracle.conv_transpose_backward(a["dy"], a["x"], a["w"], st, pd)
    HO, WO = d["y"].shape[2:]
    ks = dict(y=CI * K * K + 1, dx=CO * K * K, dw=B * H * W, db=B * HO * WO)
    for k, got, sc in (("y", y, sy), ("dx", dx, sdx), ("dw", dw, sdw), ("db", db, sdb)):
        assert_parity(host(got), d[k], sc, dt, f"{name}/{k}", k=ks[k])


@pytest.mark.parametrize("name", LINEAR)
def test_linear_fixture(name):
    d = load(name)
    dt = d["dtype"]
    M, IN, OUT, with_bias = map(int, d["meta"])
    lin = vnn.Linear(IN, OUT, device=DEV, dtype=DT[dt])
    lin.weight, lin.bias = dev(d["w"], dt), dev(d["b"], dt)
    x = dev(d["x"], dt)
    y = lin.forward(x)
    dx, dw, db = lin.backward(dev(d["dy"], dt), x)
    a = _abs(d)
    sy = oracle.linear_forward(a["x"], a["w"], a["b"])
    sdx, sdw, sdb = oracle.linear_backward(a["dy"], a["x"], a["w"])
    ks = dict(y=IN + 1, dx=OUT, dw=M, db=M)
    for k, got, sc in (("y", y, sy), ("dx", dx, sdx), ("dw", dw, sdw), ("db", db, sdb)):
        assert_parity(host(got), d[k], sc, dt, f"{name}/{k}", k=ks[k])


def test_pixel_shuffle_fixture():
    d = load("c5_pixel_shuffle")
    dt = d["dtype"]
    ps = vnn.PixelShuffle(int(d["meta"][4]))
    assert np.array_equal(host(ps.forward(dev(d["x"], dt))), d["y"])
    assert np.array_equal(host(ps.backward(dev(d["dy"], dt))), d["dx"])
