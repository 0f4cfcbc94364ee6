"""Parity metric shared by the GPU tests, smoke() and bench.py.

Per element |got - ref| / max(|ref|, tau) with tau = 1e-3 * max|ref| (keeps
near-zero outputs from dominating), maximised over the tensor.  Bars from the
brief: <= 1e-4 for f32, <= 1e-2 for bf16.  The bf16 reference is f32 math on
bf16-rounded inputs (the reference has no bf16 arithmetic).
"""
import numpy as np

TOL = {"f32": 1e-4, "bf16": 1e-2}


def rel_err(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if ref.size == 0:
        return 0.0
    tau = 1e-3 * float(np.abs(ref).max())
    if tau == 0.0:
        return float(np.abs(got).max())
    return float((np.abs(got - ref) / np.maximum(np.abs(ref), tau)).max())


def assert_parity(got, ref, dtype: str, what: str = "") -> float:
    err = rel_err(got, ref)
    assert err <= TOL[dtype], f"{what}: max rel err {err:.3e} > {TOL[dtype]:.0e} ({dtype})"
    return err
