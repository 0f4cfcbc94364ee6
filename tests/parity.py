"""Parity metric shared by the GPU tests, smoke() and bench.py.

Every output element here is a sum of products, y_i = sum_k a_k b_k (k < K,
plus a bias term where the layer has one).  Two correct fp32 evaluations of
that sum in different orders (Volta's sequential loop, an MFMA block sum, a
split-K reduction, float64) differ by at most 2 (K - 1) u S_i with u = 2^-24
and S_i = sum_k |a_k b_k| (+ |bias_i|), which is arbitrarily large RELATIVE to
|y_i| when the terms cancel.  S is computed by running the same oracle
function on absolute values (the functions are bilinear).

f32 gate (bar 1e-4, north_star):

    scaled_err = max_i |got_i - ref_i| / S_i  <= 1e-4

which equals the ordinary relative error wherever the terms do not cancel.
The per-element relative metric |got - ref| / max(|ref|, 1e-3 max|ref|) is
not usable for f32: float64 truth itself misses it by ~2e-4 against Volta's
own f32 loop.

bf16 gate (the reference is f32 math on bf16-rounded inputs, unrounded; the
device result is rounded to bf16 once).  Three conditions, all required:

 1. rounding-aware bound, per element:
        |got_i - ref_i| <= 2^-8 |ref_i| + 8 K u S_i
    2^-8 |ref| covers the one output rounding (half a bf16 ulp), 8 K u S the
    fp32 accumulation-order difference (4x its worst case).  A missing or
    doubled term a_k b_k shows up at full size against this bound;
 2. north_star's per-element relative error with the tau floor
    (tau = 1e-3 max|ref|) <= 1e-2;
 3. scaled_err <= 1e-2.

`K` (the number of products per output element, an upper bound where it
varies) is therefore required for bf16 checks.
"""
import numpy as np

TOL = {"f32": 1e-4, "bf16": 1e-2}
U32 = 2.0 ** -24        # fp32 unit roundoff
BF16_HALF_ULP = 2.0 ** -8  # relative bound of one round-to-nearest to bf16
ACC_FACTOR = 8.0        # accumulation allowance: 8 K u S (worst case is 2 (K - 1) u S)
TINY = 1e-30            # absolute floor (flushed subnormals)


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
    """north_star's metric: max |got - ref| / max(|ref|, tau), tau = 1e-3 max|ref|."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if ref.size == 0:
        return 0.0
    tau = 1e-3 * float(np.abs(ref).max())
    if tau == 0.0:
        return float(np.abs(got).max())
    return float((np.abs(got - ref) / np.maximum(np.abs(ref), tau)).max())


def bf16_bound_ratio(got, ref, scale, k) -> float:
    """max_i |got_i - ref_i| / (2^-8 |ref_i| + 8 K u S_i): <= 1 for a correct bf16 result."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.asarray(scale, np.float64)
    assert got.shape == ref.shape == scale.shape, (got.shape, ref.shape, scale.shape)
    if ref.size == 0:
        return 0.0
    bound = BF16_HALF_ULP * np.abs(ref) + ACC_FACTOR * float(k) * U32 * scale + TINY
    return float((np.abs(got - ref) / bound).max())


def parity_errors(got, ref, scale, dtype: str, k=None) -> dict:
    """Every metric of the gate (plus the normwise error) for one comparison."""
    e = {"scaled": scaled_err(got, ref, scale), "rel": rel_err(got, ref), "norm": norm_err(got, ref)}
    if dtype == "bf16":
        if k is None:
            raise ValueError("bf16 parity needs K, the number of products per output element")
        e["bound"] = bf16_bound_ratio(got, ref, scale, k)
    return e


def parity_ok(got, ref, scale, dtype: str, k=None) -> bool:
    e = parity_errors(got, ref, scale, dtype, k)
    if dtype == "f32":
        return e["scaled"] <= TOL["f32"]
    return e["bound"] <= 1.0 and e["rel"] <= TOL["bf16"] and e["scaled"] <= TOL["bf16"]


def assert_parity(got, ref, scale, dtype: str, what: str = "", k=None) -> float:
    """Asserts the gate for `dtype`; returns the scaled error."""
    e = parity_errors(got, ref, scale, dtype, k)
    if dtype == "f32":
        assert e["scaled"] <= TOL["f32"], (f"{what}: scaled err {e['scaled']:.3e} > {TOL['f32']:.0e} (f32); "
                                           f"normwise {e['norm']:.2e}")
    else:
        assert e["bound"] <= 1.0, (f"{what}: |d| exceeds 2^-8|ref| + 8Ku S by {e['bound']:.3g}x (bf16, K={k}); "
                                   f"rel {e['rel']:.2e}, scaled {e['scaled']:.2e}, normwise {e['norm']:.2e}")
        assert e["rel"] <= TOL["bf16"], f"{what}: rel err {e['rel']:.3e} > 1e-2 (bf16); normwise {e['norm']:.2e}"
        assert e["scaled"] <= TOL["bf16"], f"{what}: scaled err {e['scaled']:.3e} > 1e-2 (bf16)"
    return e["scaled"]


# K (products per output element) of the hot-path passes, upper bounds.
def k_conv_fwd(C, KH, KW, bias=True):
    return C * KH * KW + (1 if bias else 0)


def k_conv_dgrad(O, KH, KW):
    return O * KH * KW


def k_conv_wgrad(B, HO, WO):
    return B * HO * WO
