"""GPU: the reference's own Conv2d GPU/CPU consistency suite
(src/nn/layers/conv.rs:3106-3480) and its output-shape cases (conv.rs:2068-2150),
plus the stride edges of the stride-phase input gradient and ConvTranspose2d.

The reference runs each consistency case with all-ones inputs and weights and a
zero bias, so its expected output is the closed form C * (number of in-bounds
taps): small integers, exact in f32 and in bf16.  Here each case runs under
every algorithm, both kernel policies and both dtypes against that closed form,
and again on seeded random data (forward, input and weight gradients) against
the oracle under the parity gate.

Stride edges: stride 4 in both axes gives exactly 16 stride phases (the phase
table's capacity), some with no taps when the kernel is smaller than the
stride; stride 5 gives 25 phases, beyond the table, which the library runs on
the generic kernel."""
import numpy as np
import pytest
import torch

import oracle
import volta_amd
from tests.parity import assert_parity, k_conv_dgrad, k_conv_fwd, k_conv_wgrad
from volta_amd import nn as vnn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DT = {"f32": torch.float32, "bf16": torch.bfloat16}
ALGOS = [vnn.ConvAlgo.Direct, vnn.ConvAlgo.Im2col, vnn.ConvAlgo.IGEMM]
POLICIES = [volta_amd._lib.POLICY_FASTEST, volta_amd._lib.POLICY_GENERIC]

# (label: reference test, B, C, O, H, W, K, S, P, bias)
REF_CASES = [
    ("1x1_3106", 1, 4, 8, 8, 8, 1, 1, 0, True),
    ("5x5_3150", 1, 3, 8, 16, 16, 5, 1, 2, True),
    ("stride2_3191", 1, 3, 8, 16, 16, 3, 2, 1, True),
    ("stride4_3232", 1, 3, 8, 32, 32, 3, 4, 1, True),
    ("pad3_3273", 1, 3, 8, 8, 8, 3, 1, 3, True),
    ("nobias_3314", 1, 3, 8, 16, 16, 3, 1, 1, False),
    ("batch1_3351", 1, 3, 8, 16, 16, 3, 1, 1, True),
    ("batch2_3351", 2, 3, 8, 16, 16, 3, 1, 1, True),
    ("batch4_3351", 4, 3, 8, 16, 16, 3, 1, 1, True),
    ("batch8_3351", 8, 3, 8, 16, 16, 3, 1, 1, True),
    ("asym_3397", 1, 3, 8, 16, 32, 3, 2, 1, True),
    ("ch1_3438", 1, 1, 1, 8, 8, 3, 1, 1, True),
    ("ch3_3438", 1, 3, 16, 16, 16, 3, 1, 1, True),
    ("ch16_3438", 1, 16, 32, 8, 8, 3, 1, 1, True),
    ("7x7_2092", 1, 3, 16, 32, 32, 7, 1, 3, True),
    ("stride3_2104", 1, 3, 8, 16, 16, 3, 3, 1, True),
    ("pad2_2128", 1, 3, 8, 8, 8, 3, 1, 2, True),
    # stride-phase edges of the input gradient (16 phases with empty ones; 25 phases)
    ("s4k3_16phases", 2, 8, 16, 33, 30, 3, 4, 1, True),
    ("s5k3_25phases", 2, 4, 6, 23, 21, 3, 5, 1, True),
    ("s4k7p3", 2, 16, 24, 29, 31, 7, 4, 3, True),
]


def _ids(c):
    return c[0]


def _taps(n, k, s, p, out):
    """in-bounds taps per output index along one axis"""
    return np.array([sum(1 for r in range(k) if 0 <= i * s + r - p < n) for i in range(out)], np.float32)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def _policy(policy):
    volta_amd.check(volta_amd.lib().vh_set_kernel_policy(policy))


@pytest.mark.parametrize("case", REF_CASES, ids=_ids)
@pytest.mark.parametrize("policy", POLICIES, ids=["fastest", "generic"])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_reference_all_ones_closed_form(case, policy, dt):
    _, B, C, O, H, W, K, S, P, bias = case
    HO, WO = oracle.conv_out(H, K, S, P), oracle.conv_out(W, K, S, P)
    want = C * np.outer(_taps(H, K, S, P, HO), _taps(W, K, S, P, WO))
    _policy(policy)
    try:
        for algo in ALGOS:
            conv = vnn.Conv2d(C, O, K, S, P, use_bias=bias, device=DEV, dtype=DT[dt])
            conv.weight = torch.ones(O, C, K, K, dtype=DT[dt], device=DEV)
            if bias:
                conv.bias = torch.zeros(O, dtype=DT[dt], device=DEV)
            conv.set_algo(algo)
            y = host(conv.forward(torch.ones(B, C, H, W, dtype=DT[dt], device=DEV)))
            assert y.shape == (B, O, HO, WO)
            assert np.array_equal(y, np.broadcast_to(want, y.shape)), f"{algo.name}: closed form differs"
    finally:
        _policy(volta_amd._lib.POLICY_FASTEST)


@pytest.mark.parametrize("case", REF_CASES, ids=_ids)
@pytest.mark.parametrize("policy", POLICIES, ids=["fastest", "generic"])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_reference_shapes_random_data(case, policy, dt):
    _, B, C, O, H, W, K, S, P, bias = case
    g = np.random.default_rng(sum(case[1:9]))
    x = g.standard_normal((B, C, H, W)).astype(np.float32)
    w = (g.standard_normal((O, C, K, K)) * np.sqrt(2.0 / (C * K * K))).astype(np.float32)
    b = g.uniform(-1, 1, (O,)).astype(np.float32) if bias else np.zeros(O, np.float32)
    if dt == "bf16":
        x, w, b = oracle.round_bf16(x), oracle.round_bf16(w), oracle.round_bf16(b)
    HO, WO = oracle.conv_out(H, K, S, P), oracle.conv_out(W, K, S, P)
    dy = g.standard_normal((B, O, HO, WO)).astype(np.float32)
    if dt == "bf16":
        dy = oracle.round_bf16(dy)
    kw = dict(stride=(S, S), pad=(P, P))
    ab = [np.abs(a) for a in (x, w, dy)]
    ref_y = oracle.direct_conv(x, w, **kw) + b[None, :, None, None]
    sc_y = oracle.direct_conv(ab[0], ab[1], **kw) + np.abs(b)[None, :, None, None]
    ref_dx = oracle.direct_conv_backward_input(dy, w, x.shape, **kw)
    sc_dx = oracle.direct_conv_backward_input(ab[2], ab[1], x.shape, **kw)
    ref_dw = oracle.direct_conv_backward_weight(dy, x, w.shape, **kw)
    sc_dw = oracle.direct_conv_backward_weight(ab[2], ab[0], w.shape, **kw)
    _policy(policy)
    try:
        for algo in ALGOS:
            conv = vnn.Conv2d(C, O, K, S, P, use_bias=bias, device=DEV, dtype=DT[dt])
            conv.weight = torch.from_numpy(w).to(DEV, DT[dt])
            if bias:
                conv.bias = torch.from_numpy(b).to(DEV, DT[dt])
            conv.set_algo(algo)
            xt = torch.from_numpy(x).to(DEV, DT[dt])
            y = conv.forward(xt)
            dx, dw, _ = conv.backward(torch.from_numpy(dy).to(DEV, DT[dt]), xt)
            what = f"{case[0]} {algo.name}"
            assert_parity(host(y), ref_y, sc_y, dt, what + " y", k=k_conv_fwd(C, K, K))
            assert_parity(host(dx), ref_dx, sc_dx, dt, what + " dx", k=k_conv_dgrad(O, K, K))
            assert_parity(host(dw), ref_dw, sc_dw, dt, what + " dw", k=k_conv_wgrad(B, HO, WO))
    finally:
        _policy(volta_amd._lib.POLICY_FASTEST)


# ConvTranspose2d at strides 4 and 5 (its forward is the strided input gradient)
CT_EDGE = [
    # (B, CI, CO, H, W, K, S, P)
    (2, 4, 3, 4, 5, 7, 5, 1),   # 25 phases: generic path
    (2, 6, 5, 3, 4, 5, 5, 0),   # kernel = stride: every phase one tap
    (1, 8, 4, 5, 3, 3, 4, 1),   # kernel < stride: empty phases
]


@pytest.mark.parametrize("case", CT_EDGE, ids=lambda c: "B{}CI{}CO{}H{}W{}K{}S{}P{}".format(*c))
@pytest.mark.parametrize("policy", POLICIES, ids=["fastest", "generic"])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_conv_transpose2d_stride_edges(case, policy, dt):
    B, CI, CO, H, W, K, S, P = case
    g = np.random.default_rng(sum(case))
    x = g.standard_normal((B, CI, H, W)).astype(np.float32)
    w = g.normal(0, 0.2, (CI, CO, K, K)).astype(np.float32)
    b = g.uniform(-1, 1, (CO,)).astype(np.float32)
    if dt == "bf16":
        x, w, b = oracle.round_bf16(x), oracle.round_bf16(w), oracle.round_bf16(b)
    kw = dict(stride=(S, S), pad=(P, P))
    _policy(policy)
    try:
        ct = vnn.ConvTranspose2d(CI, CO, K, S, P, device=DEV, dtype=DT[dt])
        ct.weight, ct.bias = torch.from_numpy(w).to(DEV, DT[dt]), torch.from_numpy(b).to(DEV, DT[dt])
        xt = torch.from_numpy(x).to(DEV, DT[dt])
        y = ct.forward(xt)
        ref = oracle.conv_transpose_forward(x, w, b, **kw)
        sc = oracle.conv_transpose_forward(np.abs(x), np.abs(w), np.abs(b), **kw)
        assert_parity(host(y), ref, sc, dt, "y", k=CI * K * K + 1)
        dy = g.standard_normal(ref.shape).astype(np.float32)
        if dt == "bf16":
            dy = oracle.round_bf16(dy)
        dx, dw, db = ct.backward(torch.from_numpy(dy).to(DEV, DT[dt]), xt)
        refs = oracle.conv_transpose_backward(dy, x, w, **kw)
        scs = oracle.conv_transpose_backward(np.abs(dy), np.abs(x), np.abs(w), **kw)
        ks = (CO * K * K, B * H * W, B * ref.shape[2] * ref.shape[3])
        for name, got, r, s, k in zip(("dx", "dw", "db"), (dx, dw, db), refs, scs, ks):
            assert_parity(host(got), r, s, dt, name, k=k)
    finally:
        _policy(volta_amd._lib.POLICY_FASTEST)
