"""Parity metric shared by the GPU tests, smoke() and bench.py.

Every output element here is a sum of products, y_i = sum_k a_k b_k.  Two correct
fp32 evaluations of that sum in different orders (Volta's sequential loop, an
MFMA block sum, float64) differ by up to ~K * eps * sum_k |a_k b_k|, which is
arbitrarily large RELATIVE to |y_i| when the terms cancel.  The gate is therefore
the error scaled by each element's own magnitude scale

    err = max_i |got_i - ref_i| / S_i,      S_i = sum_k |a_k b_k|  (+ |bias_i|)

which equals the ordinary relative error wherever the terms do not cancel
(|y_i| = S_i) and stays meaningful where they do.  S is computed by running the
same oracle function on absolute values (the functions are bilinear).  Bars:
<= 1e-4 for f32, <= 1e-2 for bf16 (the bf16 reference is f32 math on
bf16-rounded inputs; the reference itself has no bf16 arithmetic).

`rel_err` (per element |got - ref| / max(|ref|, 1e-3 max|ref|)) is kept as a
diagnostic only: float64 truth itself misses it by ~2e-4 against Volta's f32
loop.
"""
import numpy as np

TOL = {"f32": 1e-4, "bf16": 1e-2}


def scaled_err(got, ref, scale) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.asarray(scale, np.float64)
    assert got.shape == ref.shape == scale.shape, (got.shape, ref.shape, scale.shape)
    if ref.size == 0:
        return 0.0
    return float((np.abs(got - ref) / np.maximum(scale, 1e-30)).max())


def norm_err(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.linalg.norm(ref.ravel())
    return float(np.linalg.norm((got - ref).ravel()) / (d if d > 0 else 1.0))


def rel_err(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if ref.size == 0:
        return 0.0
    tau = 1e-3 * float(np.abs(ref).max())
    if tau == 0.0:
        return float(np.abs(got).max())
    return float((np.abs(got - ref) / np.maximum(np.abs(ref), tau)).max())


def assert_parity(got, ref, scale, dtype: str, what: str = "") -> float:
    err = scaled_err(got, ref, scale)
    assert err <= TOL[dtype], (f"{what}: scaled err {err:.3e} > {TOL[dtype]:.0e} ({dtype}); "
                               f"normwise {norm_err(got, ref):.2e}")
    return err
