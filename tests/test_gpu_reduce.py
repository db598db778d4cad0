"""GPU parity: pt_reduce / pt_arg_reduce / pt_moments / pt_softmax /
pt_layernorm against the CPU oracle on identical seeded bytes.

Bars (stated per test): argmax/argmin indices, max/min and integer sums are
bit-exact; fp32 sums within 1e-5 * max(|ref|, sum|x|/sqrt(n)); means, var,
softmax and layerNorm within 1e-5 relative (floored where the reference
value is near zero).
"""
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_expectations.json")))


@pytest.fixture(scope="module")
def G():
    import gpu_util
    from phptensors import _abi
    _abi.load()
    _abi.check(_abi.load().pt_init(), "init")
    return gpu_util


def _storage(case):
    dtype = O.NAMES[case["dtype"]]
    if "data" in case:
        vals = [float(v) if isinstance(v, str) else v for v in case["data"]]
    elif "fill_rows" in case:
        vals = list(case["fill_rows"]) * case["shape"][0]
    else:
        vals = [case["fill"]] * int(np.prod(case["shape"]))
    if dtype in (O.I64, O.U64):
        arr = np.array(vals, dtype=O.NP_STORAGE[dtype])
    else:
        arr = O.to_storage(np.array(vals, dtype=np.float64), dtype)
    return arr.reshape(case["shape"]), dtype


def sum_bound(x, axis):
    x64 = np.abs(x.astype(np.float64))
    n = x.shape[axis] if axis is not None else x.size
    s = x64.sum(axis=axis) if axis is not None else np.array([x64.sum()])
    return s / math.sqrt(max(n, 1))


# ------------------------------------------------------------ golden vectors
@pytest.mark.parametrize("case", GOLDEN["reduce"], ids=lambda c: c["id"])
def test_reduce_golden(G, case):
    x, dtype = _storage(case)
    got, rdt = G.reduce(x, dtype, case["op"], case["axis"])
    assert rdt == O.NAMES[case["expected_dtype"]]
    assert list(got.shape) == case["expected_shape"]
    if "expected_fill" in case:
        assert np.all(got == case["expected_fill"])
    elif "abs_tol" in case:
        assert abs(float(got[0]) - case["expected"][0]) < case["abs_tol"]
    elif rdt == O.BOOL:
        assert got.tolist() == [int(bool(v)) for v in case["expected"]]
    else:
        for g, e in zip(got.ravel().tolist(), case["expected"]):
            if isinstance(e, str):
                assert math.isnan(g)
            else:
                assert g == e


@pytest.mark.parametrize("case", GOLDEN["arg_reduce"], ids=lambda c: c["id"])
def test_arg_reduce_golden(G, case):
    x, dtype = _storage(case)
    got = G.arg_reduce(x, dtype, case["op"], case["axis"])
    assert got.ravel().tolist() == case["expected"]


@pytest.mark.parametrize("case", GOLDEN["moments"], ids=lambda c: c["id"])
def test_moments_golden(G, case):
    x, dtype = _storage(case)
    got = G.moments(x, dtype, case["axis"], case["correction"], case["std"])
    for g, e in zip(got.ravel().tolist(), case["expected"]):
        if isinstance(e, str):
            assert math.isnan(g)
        else:
            assert abs(g - e) <= 0.5e-6 + 1e-6 * abs(e)


# ------------------------------------------------------- random fp32 parity
SHAPES = [(64, 4096), (33, 1000), (7, 3, 257), (2, 8192), (128, 64), (5, 1)]


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("op", ["sum", "mean", "max", "min"])
def test_reduce_f32_lastaxis_vs_oracle(G, shape, op):
    from phptensors import synthetic
    x = synthetic.normal(shape, 0.0, 1.0, seed=100 + len(shape))
    got, _ = G.reduce(x, O.F32, op, -1)
    ref, _ = O.reduce(x, O.F32, op, -1)
    if op in ("max", "min"):
        assert np.array_equal(got, ref)  # bit-exact
    else:
        bound = sum_bound(x, -1)
        if op == "mean":
            bound = bound / shape[-1]
        tol = 1e-5 * np.maximum(np.abs(ref.astype(np.float64)), bound)
        assert np.all(np.abs(got.astype(np.float64) - ref) <= tol)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("op", ["argmax", "argmin"])
def test_arg_reduce_f32_vs_oracle(G, shape, op):
    from phptensors import synthetic
    x = synthetic.normal(shape, 0.0, 1.0, seed=200 + shape[0])
    # force ties: quantize so equal maxima occur in many rows
    xq = np.round(x * 4) / 4
    for arr in (x, xq.astype(np.float32)):
        got = G.arg_reduce(arr, O.F32, op, -1)
        ref = O.arg_reduce(arr, O.F32, op, -1)
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("reps", [300, 1024, 1100])
def test_argmax_nan_inf_rules(G, reps):
    inf, nan = np.inf, np.nan
    x = np.array([[nan, 1.0, 3.0, 3.0], [-inf, -inf, -inf, -inf], [nan] * 4,
                  [nan, -inf, 2.0, nan], [-inf, nan, -inf, 5.0]], np.float32)
    # long rows: ties spread over lanes (and over the waves of a block when
    # the row is long enough for the block-per-row kernel)
    x = np.tile(x, (1, reps))
    got = G.arg_reduce(x, O.F32, "argmax", 1)
    assert np.array_equal(got, O.arg_reduce(x, O.F32, "argmax", 1))
    got = G.arg_reduce(-x, O.F32, "argmin", 1)
    assert np.array_equal(got, O.arg_reduce(-x, O.F32, "argmin", 1))


@pytest.mark.parametrize("axis", [0, 1, 2, None])
@pytest.mark.parametrize("op", ["sum", "max", "argmax", "mean"])
def test_reduce_non_last_axis_and_global(G, axis, op):
    from phptensors import synthetic
    x = synthetic.uniform((6, 50, 37), -1.0, 1.0, seed=300)
    xi = np.round(x * 64).astype(np.float32)  # integer-valued: sums exact
    if op == "argmax":
        got = G.arg_reduce(xi, O.F32, op, axis)
        assert np.array_equal(got, O.arg_reduce(xi, O.F32, op, axis))
        return
    got, _ = G.reduce(xi, O.F32, op, axis)
    ref, _ = O.reduce(xi, O.F32, op, axis)
    if op == "mean":
        assert np.allclose(got, ref, rtol=1e-6, atol=1e-7)
    else:
        assert np.array_equal(got.ravel(), ref.ravel())


@pytest.mark.parametrize("dt", [O.F32, O.F64, O.BF16, O.F16], ids=["f32", "f64", "bf16", "f16"])
@pytest.mark.parametrize("shape,axis", [((4096, 1024), 0), ((4096, 10), 0), ((3, 700, 36), 1),
                                        ((2, 20000, 8), 1), ((1000, 3000), 0), ((64, 70000), 0),
                                        ((5, 1, 40), 1)], ids=str)
def test_column_reductions(G, dt, shape, axis):
    """Reductions along a non-last axis of a contiguous input (bias
    gradients of the MLP step are sums over axis 0): split and unsplit row
    ranges, packed and scalar columns, outer > 1.  Integer-valued inputs keep
    float sums exact, so sum/max/min are bit-exact and mean within 1 ulp."""
    from phptensors import synthetic
    x = np.round(synthetic.uniform(shape, -64.0, 64.0, seed=sum(shape))).astype(np.float32)
    x[(0,) * len(shape)] = 100.0
    xs = O.to_storage(x.astype(np.float64) if dt == O.F64 else x, dt)
    for op in ("sum", "mean", "max", "min"):
        got, rdt = G.reduce(xs, dt, op, axis)
        ref, rrdt = O.reduce(xs, dt, op, axis)
        assert rdt == rrdt, op
        if op == "mean":
            assert np.allclose(got, ref, rtol=2e-7 if dt != O.F64 else 1e-15, atol=0), op
        else:
            assert np.array_equal(got.ravel(), ref.ravel()), op


@pytest.mark.parametrize("dt", [O.F32, O.BF16], ids=["f32", "bf16"])
def test_column_nan_and_inf(G, dt):
    from phptensors import synthetic
    # NaN in a column: max/min/sum of that column follow the oracle
    y = synthetic.uniform((2048, 64), -1.0, 1.0, seed=78)
    y[100, 5] = np.nan
    y[7, 9] = np.inf
    ys = O.to_storage(y, dt)
    for op in ("max", "min", "sum"):
        got, _ = G.reduce(ys, dt, op, 0)
        ref, _ = O.reduce(ys, dt, op, 0)
        assert np.array_equal(np.isnan(got), np.isnan(ref)), op
        assert np.array_equal(np.isinf(got), np.isinf(ref)), op
        fin = np.isfinite(ref)
        if op == "sum":
            assert np.allclose(got[fin], ref[fin], rtol=1e-4, atol=1e-4), op
        else:
            assert np.array_equal(got[fin], ref[fin]), op


def test_reduce_transposed_view(G):
    from phptensors import synthetic
    base = synthetic.normal((40, 70), 0.0, 1.0, seed=301)
    # view base.T: shape (70, 40), strides (1, 70)
    for axis in (0, 1, None):
        got, _ = G.reduce(base, O.F32, "max", axis, strides=[1, 70], shape=(70, 40))
        ref, _ = O.reduce(np.ascontiguousarray(base.T), O.F32, "max", axis)
        assert np.array_equal(got.ravel(), ref.ravel())
        gi = G.arg_reduce(base, O.F32, "argmax", axis, strides=[1, 70], shape=(70, 40))
        assert np.array_equal(gi.ravel(), O.arg_reduce(np.ascontiguousarray(base.T), O.F32,
                                                       "argmax", axis).ravel())


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("op", ["sum", "max", "argmax"])
@pytest.mark.parametrize("shape", [(48, 1024), (6, 8200)], ids=str)
def test_low_precision_inputs_promote_to_f32(G, dt, op, shape):
    from phptensors import synthetic
    x = synthetic.normal(shape, 0.0, 1.0, seed=400)
    if op == "argmax":
        x = np.round(x * 8) / 8  # ties
    xs = O.to_storage(x, dt)
    if op == "argmax":
        assert np.array_equal(G.arg_reduce(xs, dt, op, 1), O.arg_reduce(xs, dt, op, 1))
        return
    got, rdt = G.reduce(xs, dt, op, 1)
    ref, rrdt = O.reduce(xs, dt, op, 1)
    assert rdt == rrdt == O.F32
    if op == "max":
        assert np.array_equal(got, ref)
    else:
        xf = O.from_storage(xs, dt)
        tol = 1e-5 * np.maximum(np.abs(ref), sum_bound(xf, 1))
        assert np.all(np.abs(got - ref) <= tol)


@pytest.mark.parametrize("dt", [O.I8, O.I32, O.I64, O.U8, O.U64, O.BOOL])
def test_integer_reductions_bit_exact(G, dt):
    from phptensors import synthetic
    info = {O.I8: (-128, 128), O.I32: (-2**31, 2**31), O.I64: (-2**62, 2**62),
            O.U8: (0, 256), O.U64: (0, 2**63), O.BOOL: (0, 2)}[dt]
    x = synthetic.integers((9, 301), info[0], info[1], seed=500).astype(O.NP_STORAGE[dt])
    for op in ("sum", "max", "min", "mean"):
        for axis in (1, 0, None):
            got, rdt = G.reduce(x, dt, op, axis)
            ref, rrdt = O.reduce(x, dt, op, axis)
            assert rdt == rrdt
            if op == "mean":
                assert np.allclose(got, ref, rtol=1e-12)
            else:
                assert np.array_equal(got.ravel(), ref.ravel()), (op, axis)


def test_f64_reductions(G):
    from phptensors import synthetic
    x = synthetic.normal((20, 999), 0.0, 1.0, seed=501).astype(np.float64)
    for op in ("sum", "mean", "max", "min"):
        got, rdt = G.reduce(x, O.F64, op, 1)
        ref, _ = O.reduce(x, O.F64, op, 1)
        assert rdt == O.F64
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    assert np.array_equal(G.arg_reduce(x, O.F64, "argmax", 1), O.arg_reduce(x, O.F64, "argmax", 1))


def test_empty_axis_rules(G):
    from phptensors._abi import InvalidArgumentException
    x = np.zeros((2, 0, 3), np.float32)
    got, _ = G.reduce(x, O.F32, "sum", 1)
    assert got.shape == (2, 3) and np.all(got == 0)
    got, _ = G.reduce(x, O.F32, "mean", 1)
    assert np.all(np.isnan(got))
    with pytest.raises(InvalidArgumentException):
        G.reduce(x, O.F32, "max", 1)
    with pytest.raises(InvalidArgumentException):
        G.arg_reduce(x, O.F32, "argmax", 1)


# ------------------------------------------------------------------- moments
@pytest.mark.parametrize("shape", [(64, 4096), (33, 1000), (3, 70001), (7, 1280), (16, 8192), (5, 2052)], ids=str)
def test_var_std_vs_oracle(G, shape):
    from phptensors import synthetic
    x = synthetic.normal(shape, 3.0, 2.0, seed=600)
    for corr in (0, 1):
        for std in (False, True):
            got = G.moments(x, O.F32, 1, corr, std)
            ref = O.moments(x, O.F32, 1, corr, std)
            assert np.allclose(got, ref, rtol=1e-5, atol=0)
    got = G.moments(x, O.F32, None, 0, False)
    assert np.allclose(got, O.moments(x, O.F32, None, 0, False), rtol=1e-5)
    got = G.moments(x, O.F32, 0, 0, False)
    assert np.allclose(got, O.moments(x, O.F32, 0, 0, False), rtol=1e-5)


def test_var_nonfinite_and_correction_errors(G):
    from phptensors._abi import InvalidArgumentException
    x = np.array([1.0, np.inf], np.float64)
    assert np.isnan(G.moments(x, O.F64)[0])
    # long rows (register-resident two-pass kernel): infinities poison too
    xl = np.ones((5, 4096), np.float32)
    xl[0, 5] = np.inf
    xl[2, 4095] = -np.inf
    xl[3, 0] = np.nan
    xl[4, 7], xl[4, 4000] = np.inf, -np.inf
    got = G.moments(xl, O.F32, 1)
    assert np.isnan(got[0]) and got[1] == 0.0
    assert np.isnan(got[2]) and np.isnan(got[3]) and np.isnan(got[4])
    with pytest.raises(InvalidArgumentException):
        G.moments(np.zeros((0, 3), np.float32), O.F32)
    with pytest.raises(InvalidArgumentException):
        G.moments(np.ones(4, np.float32), O.F32, None, 4)


# ------------------------------------------------------------ softmax / norm
@pytest.mark.parametrize("shape", [(64, 4096), (33, 1000), (8, 3), (4, 20000), (16, 8192), (7, 1280),
                                   (8, 12288)], ids=str)
def test_softmax_lastaxis_vs_oracle(G, shape):
    from phptensors import synthetic
    x = synthetic.normal(shape, 0.0, 1.0, seed=700)
    got = G.softmax(x, O.F32, -1)
    ref = O.softmax_lastaxis(x)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-12)


@pytest.mark.parametrize("case", GOLDEN["softmax"], ids=lambda c: c["id"])
def test_softmax_golden(G, case):
    x = np.array(case["data"], np.float64).reshape(case["shape"])
    if case["dtype"] == "float32":
        got = G.softmax(x.astype(np.float32), O.F32, case["axis"])
    else:  # integer input is promoted to float64 by the host before the call
        got = G.softmax(x, O.F64, case["axis"])
    d = case["decimals"]
    if "expected_index" in case:
        assert got.dtype == np.float64
        assert round(float(got.ravel()[case["expected_index"]]), d) == case["expected_value"]
    else:
        assert [round(float(v), d) for v in got.ravel()] == case["expected"]


def test_softmax_non_last_axis_and_views(G):
    from phptensors import synthetic
    x = synthetic.normal((5, 37, 11), 0.0, 2.0, seed=701)
    for axis in (0, 1, 2):
        got = G.softmax(x, O.F32, axis)
        ref = np.moveaxis(O.softmax_lastaxis(np.ascontiguousarray(np.moveaxis(x, axis, -1))), -1, axis)
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-12)
    base = synthetic.normal((30, 40), 0.0, 1.0, seed=702)
    got = G.softmax(base, O.F32, 1, strides=[1, 40], shape=(40, 30))  # base.T rows
    ref = O.softmax_lastaxis(np.ascontiguousarray(base.T))
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-12)


def test_softmax_empty_rules(G):
    from phptensors._abi import InvalidArgumentException
    assert G.softmax(np.zeros((0, 3), np.float32), O.F32).shape == (0, 3)
    with pytest.raises(InvalidArgumentException):
        G.softmax(np.zeros((2, 0), np.float32), O.F32)


@pytest.mark.parametrize("case", GOLDEN["layernorm"], ids=lambda c: c["id"])
def test_layernorm_golden(G, case):
    if "data" in case:
        x = np.array(case["data"], np.float32).reshape(case["shape"])
    else:
        x = np.full(case["shape"], case["fill"], np.float32)
    axis = case["axes"][0]
    xt = np.ascontiguousarray(np.moveaxis(x, axis, -1))
    out = G.layernorm(xt, O.F32, case["eps"], case.get("scale"), case.get("bias"))
    out = np.moveaxis(out, -1, axis)
    if "expected_first_row" in case:
        assert [round(float(v), case["decimals"]) for v in out[0]] == case["expected_first_row"]
    elif "expected_at" in case:
        idx, val = case["expected_at"]
        assert round(float(out[tuple(idx)]), case["decimals"]) == val
    else:
        assert out.ravel().tolist() == case["expected"]


@pytest.mark.parametrize("shape", [(64, 4096), (33, 1000), (4, 20000), (100, 12), (7, 1280), (8, 12288)], ids=str)
def test_layernorm_vs_oracle(G, shape):
    from phptensors import synthetic
    x = synthetic.normal(shape, 0.5, 2.0, seed=800)
    g = synthetic.normal(shape[-1:], 1.0, 0.5, seed=801)
    b = synthetic.normal(shape[-1:], 0.0, 0.5, seed=802)
    for gamma, beta in ((None, None), (g, b)):
        got = G.layernorm(x, O.F32, 1e-5, gamma, beta)
        ref = O.layernorm_lastaxis(x, 1e-5, gamma, beta)
        assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_layernorm_errors(G):
    from phptensors._abi import InvalidArgumentException
    with pytest.raises(InvalidArgumentException):
        G.layernorm(np.ones((2, 2), np.float32), O.F32, 0.0)
    with pytest.raises(InvalidArgumentException):
        G.layernorm(np.ones((2, 2), np.float32), O.F32, float("nan"))


# ------------------------------------------------- config 2 at full size
def test_config2_full_size_parity(G):
    """X[8192,4096] N(0,1): every config-2 op against the oracle."""
    from phptensors import synthetic
    x = synthetic.normal((8192, 4096), 0.0, 1.0, seed=2)
    bound = sum_bound(x, 1)
    got, _ = G.reduce(x, O.F32, "sum", 1)
    ref, _ = O.reduce(x, O.F32, "sum", 1)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-5 * np.maximum(np.abs(ref), bound))
    got, _ = G.reduce(x, O.F32, "mean", 1)
    ref, _ = O.reduce(x, O.F32, "mean", 1)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-5 * np.maximum(np.abs(ref), bound / 4096))
    got, _ = G.reduce(x, O.F32, "max", 1)
    assert np.array_equal(got, O.reduce(x, O.F32, "max", 1)[0])
    assert np.array_equal(G.arg_reduce(x, O.F32, "argmax", 1), O.arg_reduce(x, O.F32, "argmax", 1))
    assert np.allclose(G.moments(x, O.F32, 1), O.moments(x, O.F32, 1), rtol=1e-5)
    assert np.allclose(G.softmax(x, O.F32, -1), O.softmax_lastaxis(x), rtol=1e-5, atol=1e-12)
    assert np.allclose(G.layernorm(x, O.F32, 1e-5, np.ones(4096), np.zeros(4096)),
                       O.layernorm_lastaxis(x, 1e-5, np.ones(4096, np.float32),
                                            np.zeros(4096, np.float32)), rtol=1e-5, atol=1e-5)
