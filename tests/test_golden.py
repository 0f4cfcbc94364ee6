"""CPU: the golden fixtures against the oracle and against float64 torch.

The fixtures pin the GPU box, which has neither the reference nor torch's
float64 CPU path in its parity tests; here they are checked two ways:
the oracle reproduces them bit for bit (so the oracle did not drift), and
float64 torch agrees with them to the f32 bar under the scaled-error metric
(so they record the convolution / product and not an oracle mistake)."""
import numpy as np
import pytest
import torch

import oracle
from tests.golden_io import load, names
from tests.parity import TOL, scaled_err

F = torch.nn.functional


def _t(a, grad=True):
    return torch.from_numpy(np.float64(a)).requires_grad_(grad)


def _torch_pass(kind, d, absolute):
    m = d["meta"]
    f = np.abs if absolute else (lambda a: a)
    x, dy = _t(f(d["x"])), torch.from_numpy(np.float64(f(d["dy"])))
    if kind == "shuffle":
        y = F.pixel_shuffle(x, int(m[4]))
        y.backward(dy)
        return dict(y=y, dx=x.grad)
    w, b = _t(f(d["w"])), _t(f(d["b"]))
    if kind == "conv":
        y = F.conv2d(x, w, b, int(m[6]), int(m[7]))
    elif kind == "convt":
        y = F.conv_transpose2d(x, w, b, int(m[6]), int(m[7]))
    else:
        y = x @ w + b
    y.backward(dy)
    return dict(y=y, dx=x.grad, dw=w.grad, db=b.grad)


def _oracle_pass(kind, d):
    m = d["meta"]
    if kind == "conv":
        st, pd = (int(m[6]),) * 2, (int(m[7]),) * 2
        y = oracle.direct_conv(d["x"], d["w"], st, pd) + d["b"][None, :, None, None]
        return dict(y=y, dx=oracle.direct_conv_backward_input(d["dy"], d["w"], d["x"].shape, st, pd),
                    dw=oracle.direct_conv_backward_weight(d["dy"], d["x"], d["w"].shape, st, pd),
                    db=oracle.conv_bias_grad(d["dy"]))
    if kind == "convt":
        st, pd = (int(m[6]),) * 2, (int(m[7]),) * 2
        dx, dw, db = oracle.conv_transpose_backward(d["dy"], d["x"], d["w"], st, pd)
        return dict(y=oracle.conv_transpose_forward(d["x"], d["w"], d["b"], st, pd), dx=dx, dw=dw, db=db)
    if kind == "linear":
        dx, dw, db = oracle.linear_backward(d["dy"], d["x"], d["w"])
        return dict(y=oracle.linear_forward(d["x"], d["w"], d["b"]), dx=dx, dw=dw, db=db)
    r = int(m[4])
    return dict(y=oracle.pixel_shuffle(d["x"], r), dx=oracle.pixel_shuffle_backward(d["dy"], r))


def test_fixture_set_covers_every_config():
    got = names()
    assert len(got) >= 19
    for prefix in ("c1_", "c2_", "c3_", "c4_", "c5_"):
        assert any(n.startswith(prefix) for n in got), prefix


@pytest.mark.parametrize("name", names())
def test_oracle_reproduces_fixture(name):
    d = load(name)
    for k, v in _oracle_pass(d["kind"], d).items():
        assert np.array_equal(v, d[k]), f"{name}/{k}"


@pytest.mark.parametrize("name", names())
def test_fixture_matches_float64_torch(name):
    d = load(name)
    ref = _torch_pass(d["kind"], d, False)
    if d["kind"] == "shuffle":
        for k in ref:
            assert np.array_equal(ref[k].detach().numpy(), d[k]), k
        return
    scale = _torch_pass(d["kind"], d, True)
    for k in ref:
        e = scaled_err(d[k], ref[k].detach().numpy(), scale[k].detach().numpy())
        assert e <= TOL["f32"], f"{name}/{k}: {e:.3e}"
