"""CPU: the parity gate itself (tests/parity.py) must reject results with a
missing term and accept correct results computed in a different order.

Negative controls on a K = 2304 bf16 convolution (256 -> 32 channels, 3x3,
pad 1: the depth of configs[2]'s 256@14 layer): a result with one (c, r, s)
tap dropped and a result with all of input channel 0 dropped must both fail;
the correct result (float64 math on the same bf16-rounded inputs, rounded to
bf16 once, as the device rounds its fp32 sum) must pass.  Signed inputs and
ReLU'd inputs (a layer fed by a ReLU) are both covered; f32 likewise against
its 1e-4 bar."""
import numpy as np
import pytest

import oracle
from tests.parity import (assert_parity, bf16_bound_ratio, k_conv_dgrad, k_conv_fwd, k_conv_wgrad, parity_errors,
                          parity_ok, rel_err)

B, C, O, H = 1, 256, 32, 10
KK = 3
KW = dict(stride=(1, 1), pad=(1, 1))


def _case(relu_input: bool, dtype: str, seed=0):
    g = np.random.default_rng(seed)
    x = g.standard_normal((B, C, H, H)).astype(np.float32)
    if relu_input:
        x = np.maximum(x, 0)
    bound = np.sqrt(6.0 / (C * KK * KK))
    w = g.uniform(-bound, bound, (O, C, KK, KK)).astype(np.float32)
    if dtype == "bf16":
        x, w = oracle.round_bf16(x), oracle.round_bf16(w)
    ref = oracle.direct_conv(x, w, **KW)                     # Volta's f32 loop
    scale = oracle.direct_conv(np.abs(x), np.abs(w), **KW)
    return x, w, ref, scale


def _device_like(x, w, dtype):
    """float64 sum (a different order than the oracle's) rounded like the device output."""
    y = oracle.conv_forward_f64(x, w, **KW)
    return oracle.round_bf16(y.astype(np.float32)) if dtype == "bf16" else y.astype(np.float32)


@pytest.mark.parametrize("relu_input", [False, True])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_gate_accepts_correct_result(relu_input, dtype):
    x, w, ref, scale = _case(relu_input, dtype)
    got = _device_like(x, w, dtype)
    k = k_conv_fwd(C, KK, KK, bias=False)
    assert parity_ok(got, ref, scale, dtype, k=k), parity_errors(got, ref, scale, dtype, k)
    assert_parity(got, ref, scale, dtype, "correct", k=k)


@pytest.mark.parametrize("relu_input", [False, True])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("tap", [(0, 0, 0), (17, 1, 1), (255, 2, 0)])
def test_gate_rejects_one_missing_tap(tap, relu_input, dtype):
    x, w, ref, scale = _case(relu_input, dtype)
    wb = w.copy()
    wb[:, tap[0], tap[1], tap[2]] = 0.0   # one (c, r, s) term missing from every output
    got = _device_like(x, wb, dtype)
    k = k_conv_fwd(C, KK, KK, bias=False)
    assert not parity_ok(got, ref, scale, dtype, k=k), parity_errors(got, ref, scale, dtype, k)
    with pytest.raises(AssertionError):
        assert_parity(got, ref, scale, dtype, "one tap missing", k=k)


@pytest.mark.parametrize("relu_input", [False, True])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_gate_rejects_missing_channel(relu_input, dtype):
    x, w, ref, scale = _case(relu_input, dtype)
    wb = w.copy()
    wb[:, 0] = 0.0                        # all 9 taps of input channel 0 missing
    got = _device_like(x, wb, dtype)
    k = k_conv_fwd(C, KK, KK, bias=False)
    assert not parity_ok(got, ref, scale, dtype, k=k), parity_errors(got, ref, scale, dtype, k)


@pytest.mark.parametrize("relu_input", [False, True])
def test_bf16_gate_margins(relu_input):
    """The correct result sits well inside every bf16 bar; a missing tap fails the
    rounding-aware bound and north_star's relative metric by a wide margin."""
    x, w, ref, scale = _case(relu_input, "bf16")
    k = k_conv_fwd(C, KK, KK, bias=False)
    good = _device_like(x, w, "bf16")
    e = parity_errors(good, ref, scale, "bf16", k)
    assert e["bound"] <= 0.75 and e["rel"] <= 5e-3, e
    wb = w.copy()
    wb[:, 17, 1, 1] = 0.0
    bad = _device_like(x, wb, "bf16")
    assert bf16_bound_ratio(bad, ref, scale, k) > 2.0
    assert rel_err(bad, ref) > 5e-2


def test_gate_rejects_doubled_term_in_weight_gradient():
    """dW over K = B*P*Q = 200 positions: one position counted twice must fail."""
    g = np.random.default_rng(3)
    x = oracle.round_bf16(g.standard_normal((2, 16, H, H)).astype(np.float32))
    dy = oracle.round_bf16(g.standard_normal((2, 8, H, H)).astype(np.float32))
    ref = oracle.direct_conv_backward_weight(dy, x, (8, 16, 3, 3), **KW)
    scale = oracle.direct_conv_backward_weight(np.abs(dy), np.abs(x), (8, 16, 3, 3), **KW)
    k = k_conv_wgrad(2, H, H)
    good = oracle.round_bf16(ref)
    assert parity_ok(good, ref, scale, "bf16", k=k)
    dy2 = dy.copy()
    dy2[1, :, 4, 4] *= 2.0                # position (1, 4, 4) counted twice
    bad = oracle.round_bf16(oracle.direct_conv_backward_weight(dy2, x, (8, 16, 3, 3), **KW))
    assert not parity_ok(bad, ref, scale, "bf16", k=k)


def test_bf16_gate_needs_k():
    a = np.ones(4, np.float32)
    with pytest.raises(ValueError):
        assert_parity(a, a, a, "bf16", "no k")
    assert k_conv_dgrad(4, 3, 3) == 36
