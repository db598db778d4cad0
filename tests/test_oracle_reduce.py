"""Pins the oracle's reductions: HostArray sum/mean/max/min
(contiguous_array_ce.c:1163-1270), CudaArray argMax/argMin
(reduction_ops.cuh:319-401) and var/std (cuda_array_ce.c:1850-1940).

Checks: every reduction known-answer vector in the reference tests, closed
forms on integer-valued data (sums exact below 2^24), math.fsum bounds for
random data, numpy.nanmax/nanmin/argmax equality and hand-built tie, NaN and
-inf rows.  A dropped element, a wrong axis decode or a swapped
max/min would fail these.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_expectations.json")))


def _fill(case):
    if "data" in case:
        vals = [float(v) if isinstance(v, str) else v for v in case["data"]]
        return vals
    if "fill_rows" in case:
        return list(case["fill_rows"]) * case["shape"][0]
    return [case["fill"]] * int(np.prod(case["shape"]))


def _storage(case):
    dtype = O.NAMES[case["dtype"]]
    vals = _fill(case)
    if dtype in (O.I64, O.U64):
        arr = np.array(vals, dtype=O.NP_STORAGE[dtype])
    else:
        arr = O.to_storage(np.array(vals, dtype=np.float64), dtype)
    return arr.reshape(case["shape"]), dtype


def _expect_equal(got, expected):
    for g, e in zip(got.ravel().tolist(), expected):
        if isinstance(e, str):
            assert math.isnan(g)
        else:
            assert g == e, (g, e)


@pytest.mark.parametrize("case", GOLDEN["reduce"], ids=lambda c: c["id"])
def test_reduce_reference_vectors(case):
    x, dtype = _storage(case)
    out, rdtype = O.reduce(x, dtype, case["op"], case["axis"])
    assert rdtype == O.NAMES[case["expected_dtype"]]
    assert list(out.shape) == case["expected_shape"]
    if "expected_fill" in case:
        assert np.all(out == case["expected_fill"])
    elif "abs_tol" in case:
        assert abs(float(out[0]) - case["expected"][0]) < case["abs_tol"]
    elif rdtype == O.BOOL:
        assert out.tolist() == [bool(v) for v in case["expected"]]
    else:
        _expect_equal(out, case["expected"])


@pytest.mark.parametrize("case", GOLDEN["arg_reduce"], ids=lambda c: c["id"])
def test_arg_reduce_reference_vectors(case):
    x, dtype = _storage(case)
    out = O.arg_reduce(x, dtype, case["op"], case["axis"])
    assert list(out.shape) == case["expected_shape"]
    assert out.ravel().tolist() == case["expected"]


@pytest.mark.parametrize("case", GOLDEN["moments"], ids=lambda c: c["id"])
def test_moments_reference_vectors(case):
    x, dtype = _storage(case)
    out = O.moments(x, dtype, case["axis"], case["correction"], case["std"])
    if "expected_dtype" in case:
        assert out.dtype == np.float64
    for g, e in zip(out.ravel().tolist(), case["expected"]):
        if isinstance(e, str):
            assert math.isnan(g)
        else:
            assert round(g, case["decimals"]) == pytest.approx(e, abs=0.5 * 10 ** -case["decimals"])


def test_sum_integer_valued_rows_exact():
    rng = np.random.default_rng(11)
    x = rng.integers(-1000, 1000, size=(37, 513)).astype(np.float32)
    for axis in (0, 1, None):
        got, _ = O.reduce(x, O.F32, "sum", axis)
        ref = x.astype(np.float64).sum(axis=axis)
        assert np.array_equal(got.ravel(), np.atleast_1d(ref).astype(np.float32).ravel())


def test_sum_mean_random_within_fsum_bound():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((16, 4096)).astype(np.float32)
    got, _ = O.reduce(x, O.F32, "sum", 1)
    mean, _ = O.reduce(x, O.F32, "mean", 1)
    for r in range(16):
        exact = math.fsum(x[r].astype(np.float64))
        bound = 4096 * 2.0 ** -24 * float(np.abs(x[r]).sum())
        assert abs(float(got[r]) - exact) <= bound
        assert abs(float(mean[r]) - exact / 4096) <= bound / 4096 + 1e-7


def test_sum_sequential_float_order():
    # 2^24 + 1 + 1 ... in float: sequential accumulation loses each +1,
    # which a pairwise or double accumulation would not.
    x = np.array([2.0 ** 24] + [1.0] * 8, np.float32)
    got, _ = O.reduce(x, O.F32, "sum", None)
    assert float(got[0]) == 2.0 ** 24


def test_max_min_equal_numpy_and_skip_nan():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((64, 300)).astype(np.float32)
    x[3, 17] = np.nan
    x[5, :] = np.nan
    mx, _ = O.reduce(x, O.F32, "max", 1)
    mn, _ = O.reduce(x, O.F32, "min", 1)
    with np.errstate(all="ignore"):
        import warnings
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            ref_max = np.nanmax(x, axis=1)
            ref_min = np.nanmin(x, axis=1)
    ok = ~np.isnan(ref_max)
    assert np.array_equal(mx[ok], ref_max[ok])
    assert np.array_equal(mn[ok], ref_min[ok])
    assert mx[5] == -np.inf and mn[5] == np.inf  # all-NaN row keeps the identity


def test_argmax_matches_numpy_first_occurrence():
    rng = np.random.default_rng(14)
    x = rng.integers(-3, 4, size=(50, 77)).astype(np.float32)  # many ties
    for axis in (0, 1):
        got = O.arg_reduce(x, O.F32, "argmax", axis)
        assert np.array_equal(got, np.argmax(x, axis=axis).astype(np.int32))
        got = O.arg_reduce(x, O.F32, "argmin", axis)
        assert np.array_equal(got, np.argmin(x, axis=axis).astype(np.int32))
    got = O.arg_reduce(x, O.F32, "argmax", None)
    assert got[0] == np.argmax(x)


def test_argmax_nan_and_identity_rules():
    inf = np.inf
    nan = np.nan
    x = np.array([
        [nan, 1.0, 3.0, 3.0],      # NaN never chosen; tie -> lowest index
        [-inf, -inf, -inf, -inf],  # all identity -> 0
        [nan, nan, nan, nan],      # all NaN -> 0
        [nan, -inf, 2.0, nan],
        [-inf, nan, -inf, 5.0],
    ], np.float32)
    got = O.arg_reduce(x, O.F32, "argmax", 1)
    assert got.tolist() == [2, 0, 0, 2, 3]
    got = O.arg_reduce(-x, O.F32, "argmin", 1)
    assert got.tolist() == [2, 0, 0, 2, 3]


def test_var_matches_numpy():
    rng = np.random.default_rng(15)
    x = (rng.standard_normal((20, 1000)) * 3 + 7).astype(np.float32)
    for corr in (0, 1):
        got = O.moments(x, O.F32, 1, corr, False)
        ref = x.astype(np.float64).var(axis=1, ddof=corr)
        assert np.allclose(got, ref, rtol=1e-6, atol=0)
        got = O.moments(x, O.F32, 0, corr, True)
        ref = x.astype(np.float64).std(axis=0, ddof=corr)
        assert np.allclose(got, ref, rtol=1e-6, atol=0)


def test_empty_axis_rules():
    x = np.zeros((2, 0, 3), np.float32)
    out, _ = O.reduce(x, O.F32, "sum", 1)
    assert out.shape == (2, 3) and np.all(out == 0)
    out, _ = O.reduce(x, O.F32, "mean", 1)
    assert np.all(np.isnan(out))
    with pytest.raises(ValueError):
        O.reduce(x, O.F32, "max", 1)
    with pytest.raises(ValueError):
        O.arg_reduce(x, O.F32, "argmax", 1)
