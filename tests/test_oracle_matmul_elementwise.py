"""Pins the oracle's matmul (contiguous_array_ce.c:1295-1343) and
elementwise restatements (:1075-1131, :1345-1447, :1021-1073).

Checks: every matmul known-answer vector of the reference tests (including
batch broadcasting and bf16/fp16 outputs), exactness on integer-valued data,
the gamma_K error bound against float64 numpy, the transposed-view integer
pattern of ca_matmul_accelerated.phpt, the no-contraction vector of
fusion_precision.phpt and agreement with numpy float32 arithmetic.  A
transposed operand, a wrong batch offset or an fma contraction fails them.
"""
import json
import os

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_expectations.json")))


@pytest.mark.parametrize("case", GOLDEN["matmul"], ids=lambda c: c["id"])
def test_matmul_reference_vectors(case):
    dtype = O.NAMES[case["dtype"]]
    a = O.to_storage(np.array(case["a"], np.float64), dtype).reshape(case["shape_a"])
    b = O.to_storage(np.array(case["b"], np.float64), dtype).reshape(case["shape_b"])
    c = O.matmul(a, b, dtype)
    assert list(c.shape) == case["expected_shape"]
    vals = O.from_storage(c, dtype).astype(np.float64).ravel()
    if "abs_tol" in case:
        assert np.all(np.abs(vals - np.array(case["expected"])) < case["abs_tol"])
    else:
        assert vals.tolist() == [float(v) for v in case["expected"]]


@pytest.mark.parametrize("threads", [2, 3, 8])
def test_threaded_matmul_gives_the_same_bits(threads):
    """or_matmul_mt (the bench's CPU baseline driver) splits the outputs over
    host threads; every output keeps or_matmul's sum, so the bits agree, for
    batch broadcasting, a strided (transposed) operand and 16-bit outputs,
    and for output counts that do not divide evenly."""
    rng = np.random.default_rng(threads)
    a = rng.standard_normal((3, 37, 51)).astype(np.float32)
    b = rng.standard_normal((1, 51, 29)).astype(np.float32)
    assert O.matmul(a, b, O.F32, threads=threads).tobytes() == O.matmul(a, b, O.F32).tobytes()
    base = rng.standard_normal((51, 37)).astype(np.float32)  # A = base^T as a view
    kw = dict(strides_a=[1, 37], shape_a=[37, 51])
    b2 = rng.standard_normal((51, 29)).astype(np.float32)
    assert (O.matmul(base, b2, O.F32, threads=threads, **kw).tobytes() ==
            O.matmul(base, b2, O.F32, **kw).tobytes())
    for dt in (O.BF16, O.F16):
        a16, b16 = O.to_storage(a.astype(np.float64), dt), O.to_storage(b.astype(np.float64), dt)
        assert O.matmul(a16, b16, dt, threads=threads).tobytes() == O.matmul(a16, b16, dt).tobytes()


def test_matmul_transposed_view_integer_pattern():
    # ca_matmul_accelerated.phpt:31-48: left^T @ right with exact integers
    rows, cols = np.meshgrid(np.arange(64), np.arange(128), indexing="ij")
    left = ((rows + cols * 2) % 7).astype(np.float32)
    right = ((rows * 3 + cols) % 5).astype(np.float32)
    # left.transpose() as a strided view: shape [128,64], strides [1,128]
    c = O.matmul(left, right, O.F32, strides_a=[1, 128], shape_a=[128, 64])
    ref = left.T.astype(np.float64) @ right.astype(np.float64)
    assert np.array_equal(c.astype(np.float64), ref)


def test_matmul_integer_valued_exact_and_error_bound():
    rng = np.random.default_rng(31)
    a = rng.integers(-8, 8, size=(3, 33, 70)).astype(np.float32)
    b = rng.integers(-8, 8, size=(3, 70, 21)).astype(np.float32)
    c = O.matmul(a, b, O.F32)
    assert np.array_equal(c.astype(np.float64), a.astype(np.float64) @ b.astype(np.float64))
    # config 1 (A[256,512] @ B[512,256], U(-1,1) from seed S1 = 1 of the
    # bench's SplitMix64 generator): within gamma_K of the float64 product
    a, b = O.config1_operands()
    c = O.matmul(a, b, O.F32).astype(np.float64)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert np.all(np.abs(c - ref) <= 512 * 2.0 ** -24 * scale)
    # the sequential fmaf order of contiguous_array_ce.c:1327-1333 (one
    # rounding per step of the exact a*b + acc), in exact rational
    # arithmetic for a sample of outputs
    from fractions import Fraction
    from test_rowdiv_rounding import rn32
    for i, j in ((0, 0), (17, 200), (255, 255), (128, 3)):
        acc = Fraction(0)
        for k in range(512):
            acc = rn32(Fraction(float(a[i, k])) * Fraction(float(b[k, j])) + acc)
        assert c[i, j] == float(acc), (i, j)


def test_matmul_bf16_output_is_rne_of_fp32_product():
    rng = np.random.default_rng(32)
    a32 = rng.standard_normal((4, 40, 24)).astype(np.float32)
    b32 = rng.standard_normal((4, 24, 16)).astype(np.float32)
    a = O.f32_to_bf16(a32)
    b = O.f32_to_bf16(b32)
    c = O.matmul(a, b, O.BF16)
    c32 = O.matmul(O.bf16_to_f32(a), O.bf16_to_f32(b), O.F32)
    assert np.array_equal(c, O.f32_to_bf16(c32))


def test_binary_no_contraction_vector():
    # fusion_precision.phpt:11-15: a + b*c rounds the product first
    a = np.array([-1.0], np.float32)
    b = np.array([1.0 + 2.0 ** -23], np.float32)
    c = np.array([1.0 - 2.0 ** -23], np.float32)
    prod = O.binary(b, O.F32, c, O.F32, "mul", O.F32)
    out = O.binary(a, O.F32, prod, O.F32, "add", O.F32)
    assert out[0] == np.float32(0.0)          # separate roundings
    assert float(np.float64(b[0]) * np.float64(c[0]) - 1.0) != 0.0  # fma would not be 0


def test_binary_matches_numpy_float32_with_broadcast():
    rng = np.random.default_rng(33)
    x = rng.uniform(-2, 2, (64, 96)).astype(np.float32)
    y = rng.uniform(-2, 2, (96,)).astype(np.float32)
    for op, fn in (("add", np.add), ("sub", np.subtract), ("mul", np.multiply),
                   ("div", np.divide)):
        got = O.binary(x, O.F32, y, O.F32, op, O.F32)
        assert np.array_equal(got, fn(x, y))
        got = O.binary(y, O.F32, x, O.F32, op, O.F32)
        assert np.array_equal(got, fn(y, x))


def test_binary_scalar_reverse_order():
    x = np.array([1.0, 2.0, 4.0], np.float32)
    assert O.binary_scalar(x, O.F32, 100.0, "sub", O.F32, reverse=True).tolist() == [99, 98, 96]
    assert O.binary_scalar(x, O.F32, 2.0, "div", O.F32).tolist() == [0.5, 1.0, 2.0]


def test_unary_tanh_close_to_float64():
    x = np.linspace(-10, 10, 200001).astype(np.float32)
    got = O.unary(x, O.F32, "tanh").astype(np.float64)
    ref = np.tanh(x.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2 * ulp + 1e-45)
    special = O.unary(np.array([0.0, -0.0, np.inf, -np.inf], np.float32), O.F32, "tanh")
    assert special.tolist() == [0.0, -0.0, 1.0, -1.0]


def test_where_bitwise_selection():
    cond = np.array([[1], [0]], np.float32)
    x = np.array([1.0, 2.0, 3.0], np.float32)
    y = np.array([[7.0, 8.0, 9.0]], np.float32)
    out = O.where(cond, O.F32, x, y, O.F32)
    assert out.tolist() == [[1, 2, 3], [7, 8, 9]]
