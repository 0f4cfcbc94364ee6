"""GPU: vh_conv2d_backward_noalloc (workspace in a static device array, no
allocation) against vh_conv2d_backward, both called through the C ABI.

Both entry points run the same kernels with the same plans, and every kernel is
deterministic, so the outputs must be identical bit for bit.  Each case makes
two no-alloc calls in a row, the second on a smaller input: the scratch keeps
the first call's contents, which the second must not depend on.  A call whose
workspace exceeds the static maximum is rejected before anything is queued
(its outputs keep their sentinel contents)."""
import pytest
import torch

import volta_amd
from volta_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DT = {"f32": (torch.float32, _lib.F32), "bf16": (torch.bfloat16, _lib.BF16)}


def _tensors(dims, dt, seed):
    B, C, O, H, W, K, S, P = dims
    HO, WO = (H + 2 * P - K) // S + 1, (W + 2 * P - K) // S + 1
    g = torch.Generator().manual_seed(seed)
    tdt = DT[dt][0]
    x = torch.randn(B, C, H, W, generator=g).to(DEV, tdt)
    w = (torch.randn(O, C, K, K, generator=g) * (2.0 / (C * K * K)) ** 0.5).to(DEV, tdt)
    dy = torch.randn(B, O, HO, WO, generator=g).to(DEV, tdt)
    return x, w, dy


def _backward(name, dims, dt, algo, x, w, dy, sentinel=0.0):
    B, C, O, H, W, K, S, P = dims
    dx = torch.full_like(x, sentinel)
    dw = torch.full_like(w, sentinel)
    db = torch.full((O,), sentinel, dtype=w.dtype, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    st = getattr(volta_amd.lib(), name)(DT[dt][1], algo, dy.data_ptr(), x.data_ptr(), w.data_ptr(), dx.data_ptr(),
                                        dw.data_ptr(), db.data_ptr(), B, C, O, H, W, K, K, S, S, P, P, stream)
    torch.cuda.synchronize()
    return st, (dx, dw, db)


# (dtype, algorithm, first call, second smaller call): (B, C, O, H, W, K, S, P)
CASES = [
    ("bf16", _lib.ALGO_IGEMM, (128, 128, 128, 28, 28, 3, 1, 1), (4, 64, 64, 14, 14, 3, 1, 1)),   # configs[2] 128@28
    ("bf16", _lib.ALGO_IGEMM, (128, 64, 64, 56, 56, 3, 1, 1), (2, 64, 64, 20, 20, 3, 1, 1)),     # configs[2] 64@56
    ("bf16", _lib.ALGO_IGEMM, (128, 64, 128, 56, 56, 1, 2, 0), (2, 64, 128, 20, 20, 1, 2, 0)),   # strided 1x1
    ("f32", _lib.ALGO_IGEMM, (16, 32, 48, 30, 30, 3, 2, 1), (2, 32, 48, 11, 11, 3, 2, 1)),       # stride phases
    ("f32", _lib.ALGO_IGEMM, (8, 64, 32, 28, 28, 3, 1, 1), (2, 16, 8, 9, 9, 3, 1, 1)),            # generic split-K
    ("f32", _lib.ALGO_IM2COL, (8, 16, 32, 20, 20, 3, 1, 1), (2, 16, 32, 9, 9, 3, 1, 1)),
    ("bf16", _lib.ALGO_DIRECT, (4, 8, 16, 12, 12, 3, 1, 1), (1, 8, 16, 7, 7, 3, 1, 1)),
    # at most 4 input channels at a large batch: the input gradient needs no workspace and
    # the weight gradient only the few-channel kernel's partials (what the sizing must report)
    ("bf16", _lib.ALGO_IGEMM, (256, 3, 64, 64, 64, 5, 1, 2), (4, 3, 64, 16, 16, 5, 1, 2)),
    ("f32", _lib.ALGO_IGEMM, (512, 4, 32, 28, 28, 3, 1, 1), (2, 4, 32, 9, 9, 3, 1, 1)),
]


@pytest.mark.parametrize("dt,algo,first,second", CASES,
                         ids=[f"{c[0]}-a{c[1]}-{'x'.join(map(str, c[2][:5]))}" for c in CASES])
def test_noalloc_backward_matches_allocating_entry(dt, algo, first, second):
    for i, dims in enumerate((first, second)):
        print(f"case {dt} algo {algo} call {i} dims {dims}", flush=True)
        x, w, dy = _tensors(dims, dt, seed=sum(dims) + i)
        st, ref = _backward("vh_conv2d_backward", dims, dt, algo, x, w, dy)
        assert st == _lib.VH_OK, volta_amd.lib().vh_last_error()
        st, got = _backward("vh_conv2d_backward_noalloc", dims, dt, algo, x, w, dy, sentinel=float("nan"))
        assert st == _lib.VH_OK, volta_amd.lib().vh_last_error()
        for name, a, b in zip(("dx", "dw", "db"), got, ref):
            assert torch.equal(a, b), f"call {i} {dims}: {name} differs from vh_conv2d_backward"


def test_noalloc_rejects_oversize_before_queuing():
    # Im2col at configs[2]'s first layer needs a 462 MB column matrix
    dims = (128, 64, 64, 56, 56, 3, 1, 1)
    x, w, dy = _tensors(dims, "bf16", seed=1)
    st, outs = _backward("vh_conv2d_backward_noalloc", dims, "bf16", _lib.ALGO_IM2COL, x, w, dy, sentinel=7.0)
    assert st == _lib.VH_ERR_UNSUPPORTED
    assert b"static maximum" in volta_amd.lib().vh_last_error()
    for t in outs:
        assert bool((t == 7.0).all()), "a rejected call must not have queued any kernel"
    # the next call of the same entry point still works
    small = (2, 64, 64, 14, 14, 3, 1, 1)
    x, w, dy = _tensors(small, "bf16", seed=2)
    st, ref = _backward("vh_conv2d_backward", small, "bf16", _lib.ALGO_IGEMM, x, w, dy)
    st2, got = _backward("vh_conv2d_backward_noalloc", small, "bf16", _lib.ALGO_IGEMM, x, w, dy)
    assert st == st2 == _lib.VH_OK
    assert all(torch.equal(a, b) for a, b in zip(got, ref))
