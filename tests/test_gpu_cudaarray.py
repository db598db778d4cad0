"""GPU parity of the CudaArray operator surface (host runtime over the C-ABI)
against the CPU oracle.  Mirrors the reference's ca_*.phpt / cudaarray_*.phpt
tests: exact for +,-,*,/ (one IEEE rounding each), comparisons, casts,
max/argmax and integer work; libm-vs-device tolerances for transcendentals."""
import zlib

import numpy as np
import pytest

import oracle_lib as O
from phptensors import CudaArray, InvalidArgumentException

pytestmark = pytest.mark.gpu

F32, F64, I32, I64, F16, BF16, BOOL, U8 = 0, 1, 4, 5, 11, 12, 10, 6


def rng(seed):
    return np.random.default_rng(seed)


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


# ----------------------------------------------------------------- transfers
@pytest.mark.parametrize("dtype,npdt", [("float32", np.float32), ("float64", np.float64),
                                        ("int8", np.int8), ("int16", np.int16),
                                        ("int32", np.int32), ("int64", np.int64),
                                        ("uint8", np.uint8), ("uint16", np.uint16),
                                        ("uint32", np.uint32), ("uint64", np.uint64),
                                        ("float16", np.float16), ("bool", np.bool_)])
def test_round_trip_bits(dtype, npdt):
    r = rng(1)
    if npdt == np.bool_:
        x = r.integers(0, 2, (7, 13)).astype(bool)
    elif np.issubdtype(npdt, np.integer):
        info = np.iinfo(npdt)
        x = r.integers(info.min, info.max, (7, 13), dtype=npdt, endpoint=True)
    else:
        x = r.standard_normal((7, 13)).astype(npdt)
    t = CudaArray.fromNumpy(x, dtype)
    assert t.getShape() == [7, 13] and t.getDtype() == dtype
    assert t.getStrides() == [13, 1]
    np.testing.assert_array_equal(t.toBits(), x.view(np.uint16) if npdt == np.float16 else x)
    np.testing.assert_array_equal(t.toNumpy(), x)
    assert t.toBuffer() == x.tobytes()


def test_bfloat16_upload_rounds_to_nearest_even():
    # matmul_low_precision.phpt:28-46 conversion vectors
    vals = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38, 1e-40, np.inf], np.float32)
    t = CudaArray.fromNumpy(vals, "bfloat16")
    np.testing.assert_array_equal(t.toBits(), O.f32_to_bf16(vals))


def test_from_buffer_round_trip():
    x = np.arange(12, dtype=np.int32).reshape(3, 4)
    t = CudaArray.fromBuffer(x.tobytes(), [3, 4], "int32")
    np.testing.assert_array_equal(t.toNumpy(), x)
    with pytest.raises(InvalidArgumentException):
        CudaArray.fromBuffer(b"\0" * 8, [3, 4], "int32")


def test_full_and_zeros():
    np.testing.assert_array_equal(CudaArray.full([3, 5], 2.5).toNumpy(), np.full((3, 5), 2.5, np.float32))
    np.testing.assert_array_equal(CudaArray.zeros([4], "int64").toNumpy(), np.zeros(4, np.int64))
    np.testing.assert_array_equal(CudaArray.ones([2, 2], "bfloat16").toBits(), np.full((2, 2), 0x3F80, np.uint16))


# ----------------------------------------------------------------- binary
@pytest.mark.parametrize("op", ["ADD", "SUB", "MUL", "DIV"])
@pytest.mark.parametrize("sa,sb", [((64, 33), (64, 33)), ((64, 33), (33,)), ((5, 1, 7), (1, 6, 7)),
                                   ((1,), (19, 3)), ((4096,), (4096,)),
                                   # 2-D float32 row kernel: row, column and scalar broadcasts
                                   ((64, 32), (32,)), ((64, 32), (64, 1)), ((32,), (64, 32)),
                                   ((3, 5, 8), (5, 8)), ((7, 12), (1, 12)), ((9, 1), (9, 16)),
                                   ((12,), (1,)), ((300, 1024), (1, 1024))])
def test_binary_f32_exact(op, sa, sb):
    r = rng(zlib.crc32(repr((op, sa, sb)).encode()))
    a = r.standard_normal(sa).astype(np.float32)
    b = (r.standard_normal(sb) + 3.0).astype(np.float32)
    got = getattr(CudaArray.fromNumpy(a), {"ADD": "add", "SUB": "subtract", "MUL": "multiply",
                                            "DIV": "divide"}[op])(CudaArray.fromNumpy(b))
    ref = O.binary(a, F32, b, F32, op, F32)
    np.testing.assert_array_equal(got.toNumpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("op,sym", [("ADD", "+"), ("SUB", "-"), ("MUL", "*"), ("DIV", "/")])
def test_scalar_and_inverse_scalar_exact(op, sym):
    r = rng(7)
    a = (r.standard_normal((33, 65)) + 4).astype(np.float32)
    t = CudaArray.fromNumpy(a)
    fwd = eval(f"t {sym} 1.7")
    inv = eval(f"1.7 {sym} t")
    np.testing.assert_array_equal(fwd.toNumpy(), O.binary_scalar(a, F32, 1.7, op, F32))
    np.testing.assert_array_equal(inv.toNumpy(), O.binary_scalar(a, F32, 1.7, op, F32, reverse=True))


@pytest.mark.parametrize("op", ["GT", "LT", "EQ", "NE", "GE", "LE", "MAXIMUM", "MINIMUM"])
def test_compare_and_extrema(op):
    r = rng(3)
    a = r.integers(-3, 4, (40, 17)).astype(np.float32)
    b = r.integers(-3, 4, (17,)).astype(np.float32)
    got = getattr(CudaArray.fromNumpy(a), op.lower())(CudaArray.fromNumpy(b))
    ref_fn = {"GT": np.greater, "LT": np.less, "EQ": np.equal, "NE": np.not_equal,
              "GE": np.greater_equal, "LE": np.less_equal, "MAXIMUM": np.maximum,
              "MINIMUM": np.minimum}[op]
    ref = ref_fn(a, b).astype(np.float32)
    assert got.getDtype() == "float32"
    np.testing.assert_array_equal(got.toNumpy(), ref)


@pytest.mark.parametrize("shape", [(6, 8), (1000, 37), (3, 4, 5, 6)], ids=str)
def test_strided_views_through_generic_kernels(shape):
    """Transposed views run the generic index-decoding kernels (32-bit
    indices at these sizes) for binary, unary, cast and where."""
    r = rng(11)
    a = r.standard_normal(shape).astype(np.float32)
    b = r.standard_normal(shape[::-1]).astype(np.float32)
    ta, tb = CudaArray.fromNumpy(a), CudaArray.fromNumpy(b).transpose()
    bt = np.ascontiguousarray(b.transpose())
    np.testing.assert_array_equal((ta + tb).toNumpy(), O.binary(a, F32, bt, F32, "ADD", F32))
    np.testing.assert_array_equal(tb.abs().toNumpy(), np.abs(bt))
    np.testing.assert_array_equal(tb.astype("float64").toNumpy(), bt.astype(np.float64))
    w = CudaArray.where(tb.gt(0), ta, tb).toNumpy()
    np.testing.assert_array_equal(w, np.where(bt > 0, a, bt))


def test_division_promotes_integers_to_float():
    # promote_types_for_arithmetic (data_types.c:495-516): DIV/POW of int32
    # operands compute in float32, int64 in float64
    ai = np.array([7, -7, 9, 1], np.int32)
    bi = np.array([2, 2, 4, -3], np.int32)
    q = CudaArray.fromNumpy(ai) / CudaArray.fromNumpy(bi)
    assert q.getDtype() == "float32"
    np.testing.assert_array_equal(q.toNumpy(), ai.astype(np.float32) / bi.astype(np.float32))
    q64 = CudaArray.fromNumpy(ai.astype(np.int64)) / CudaArray.fromNumpy(bi)
    assert q64.getDtype() == "float64"
    m = CudaArray.fromNumpy(ai) + CudaArray.fromNumpy(np.full(4, 0.5, np.float32))
    assert m.getDtype() == "float32"
    hb = CudaArray.fromNumpy(np.ones(4, np.float32), "bfloat16")
    assert (hb / hb).getDtype() == "float32"
    assert (hb + hb).getDtype() == "bfloat16"


def test_integer_arithmetic_wraps_exactly():
    a = np.array([2**31 - 1, -2**31, 100000, -7], np.int32)
    b = np.array([1, -1, 100000, 3], np.int32)
    for op, fn in (("ADD", "add"), ("SUB", "subtract"), ("MUL", "multiply")):
        got = getattr(CudaArray.fromNumpy(a), fn)(CudaArray.fromNumpy(b))
        assert got.getDtype() == "int32"
        wide = {"ADD": np.add, "SUB": np.subtract, "MUL": np.multiply}[op](a.astype(np.int64), b.astype(np.int64))
        np.testing.assert_array_equal(got.toNumpy(), wide.astype(np.int32))  # two's-complement wrap


def test_golden_broadcast_cast_promotion():
    # fusion_broadcast_cast.phpt eager equivalent: int32[2,1] + float32[1,3] * float64[3]
    a = CudaArray.fromNumpy(np.array([[1], [2]], np.int32))
    b = CudaArray.fromNumpy(np.array([[3, 4, 5]], np.float32))
    c = CudaArray.fromNumpy(np.array([2, 3, 4], np.float64))
    out = a + b * c
    assert out.getDtype() == "float64" and out.getShape() == [2, 3]
    np.testing.assert_array_equal(out.toNumpy().reshape(-1), [7, 13, 21, 8, 14, 22])


def test_power_integer_fast_path():
    x = np.array([1.5, -2.0, 3.0, 0.5], np.float32)
    t = CudaArray.fromNumpy(x)
    np.testing.assert_array_equal((t ** 2).toNumpy(), x * x)
    np.testing.assert_array_equal((t ** 3).toNumpy(), x * x * x)
    got = (t ** 0.5)
    assert np.isnan(got.toNumpy()[1])


def test_binary_shape_mismatch_raises():
    with pytest.raises(InvalidArgumentException):
        CudaArray.zeros([3, 4]) + CudaArray.zeros([5])


def test_bf16_binary_rounds_once_per_op():
    r = rng(11)
    a = r.standard_normal((128,)).astype(np.float32)
    b = r.standard_normal((128,)).astype(np.float32)
    ab = O.f32_to_bf16(a)
    bb = O.f32_to_bf16(b)
    got = CudaArray.fromNumpy(ab, "bfloat16") * CudaArray.fromNumpy(bb, "bfloat16")
    assert got.getDtype() == "bfloat16"
    ref = O.binary(ab, BF16, bb, BF16, "MUL", BF16)
    np.testing.assert_array_equal(got.toBits(), ref)


# ----------------------------------------------------------------- unary
UNARY = ["EXP", "EXPM1", "EXP2", "LOG", "LOG1P", "LOG2", "LOG10", "SQRT", "SIN", "COS", "TAN",
         "ASIN", "ACOS", "ATAN", "SINH", "COSH", "TANH", "ABS", "NEG", "FLOOR", "CEIL", "ROUND"]


@pytest.mark.parametrize("op", UNARY)
def test_unary_f32_vs_libm(op):
    r = rng(5)
    if op in ("ASIN", "ACOS"):
        x = r.uniform(-0.99, 0.99, 4099)
    elif op in ("LOG", "LOG2", "LOG10", "SQRT", "LOG1P"):
        x = r.uniform(0.01, 50, 4099)
    else:
        x = r.uniform(-4, 4, 4099)
    x = x.astype(np.float32)
    got = getattr(CudaArray.fromNumpy(x), op.lower())().toNumpy()
    ref = O.unary(x, F32, op)
    exact = op in ("ABS", "NEG", "FLOOR", "CEIL", "ROUND", "SQRT")
    d = ulp_diff(got, ref)
    # device math library vs glibc: a few ulp; sqrt and rounding ops exact
    assert d.max() <= (0 if exact else 4), (op, d.max())


def test_unary_bf16_computes_in_f32():
    x = O.f32_to_bf16(np.linspace(-3, 3, 97).astype(np.float32))
    got = CudaArray.fromNumpy(x, "bfloat16").tanh()
    assert got.getDtype() == "bfloat16"
    ref = O.unary(x, BF16, "TANH")
    assert np.abs(got.toBits().astype(np.int32) - ref.astype(np.int32)).max() <= 1


# ----------------------------------------------------------------- where / cast / views
def test_where_broadcast():
    r = rng(9)
    c = r.integers(0, 2, (6, 5)).astype(np.float32)
    x = r.standard_normal((6, 5)).astype(np.float32)
    y = r.standard_normal((5,)).astype(np.float32)
    got = CudaArray.where(CudaArray.fromNumpy(c), CudaArray.fromNumpy(x), CudaArray.fromNumpy(y))
    np.testing.assert_array_equal(got.toNumpy(), np.where(c != 0, x, y))


@pytest.mark.parametrize("src,dst", [("int32", "float32"), ("int16", "float32"), ("bfloat16", "float32"),
                                     ("float16", "float64"), ("float32", "float64"), ("int8", "int64"),
                                     ("uint8", "int16"), ("bool", "float32"), ("bool", "int32")])
def test_astype_safe_casts(src, dst):
    r = rng(4)
    x = np.round(r.standard_normal(257) * 50).astype(np.float32)
    codes = {"float32": F32, "bfloat16": BF16, "float16": F16, "int32": I32, "float64": F64, "bool": BOOL,
             "int16": 3, "int8": 2, "int64": I64, "uint8": U8}
    if src == "uint8":
        x = np.abs(x)
    xs = O.to_storage(x, codes[src])
    got = CudaArray.fromNumpy(xs, src).astype(dst)
    assert got.getDtype() == dst
    vals = O.from_storage(xs, codes[src]).astype(np.float64)
    ref = O.to_storage(vals, codes[dst])
    np.testing.assert_array_equal(got.toBits(), ref)


@pytest.mark.parametrize("src,dst", [("float32", "bfloat16"), ("float32", "float16"), ("float32", "int32"),
                                     ("float64", "float32"), ("int64", "float32"), ("float32", "bool")])
def test_astype_rejects_unsafe_casts(src, dst):
    # tensor_cast -> can_safely_cast_to (tensor.c:104-120, data_types.c:565-620)
    t = CudaArray.zeros([4], src)
    with pytest.raises(InvalidArgumentException):
        t.astype(dst)


def test_transposed_and_sliced_views():
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    t = CudaArray.fromNumpy(x)
    tt = t.transpose([2, 0, 1])
    assert tt.getShape() == [4, 2, 3]
    np.testing.assert_array_equal(tt.toNumpy(), x.transpose(2, 0, 1))
    np.testing.assert_array_equal((tt * 2).toNumpy(), x.transpose(2, 0, 1) * 2)
    s = t.slice(None, None, [1, 4, 2])
    np.testing.assert_array_equal(s.toNumpy(), x[:, :, 1:4:2])
    np.testing.assert_array_equal(t.select(1, 2).toNumpy(), x[:, 2])
    b = CudaArray.fromNumpy(np.array([1, 2, 3], np.float32)).broadcastTo([2, 3])
    np.testing.assert_array_equal(b.toNumpy(), np.broadcast_to([1, 2, 3], (2, 3)))
    np.testing.assert_array_equal(t.reshape([6, -1]).toNumpy(), x.reshape(6, 4))


# ----------------------------------------------------------------- reductions through the surface
def test_reductions_match_oracle():
    r = rng(12)
    x = r.standard_normal((96, 1000)).astype(np.float32)
    t = CudaArray.fromNumpy(x)
    s = t.sum(1).toNumpy()
    ref, _ = O.reduce(x, F32, "SUM", axis=1)
    bound = 1e-5 * np.maximum(np.abs(ref), np.abs(x).sum(1) / np.sqrt(1000))
    assert np.all(np.abs(s - ref) <= bound)
    np.testing.assert_array_equal(t.max(1).toNumpy(), O.reduce(x, F32, "MAX", axis=1)[0])
    am = t.argMax(1)
    assert am.getDtype() == "int32"
    np.testing.assert_array_equal(am.toNumpy(), O.arg_reduce(x, F32, "ARG_MAX", axis=1))
    np.testing.assert_allclose(t.var(1).toNumpy(), O.moments(x, F32, axis=1), rtol=2e-5)
    np.testing.assert_allclose(t.std(1, 1).toNumpy(), O.moments(x, F32, axis=1, correction=1, std=True),
                               rtol=2e-5)
    g = t.sum()
    assert g.getShape() in ([], [1])
    assert abs(g.item() - float(x.astype(np.float64).sum())) <= 1e-5 * np.abs(x).sum()
    np.testing.assert_allclose(t.softmax(-1).toNumpy(), O.softmax_lastaxis(x), rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(t.layerNorm([1]).toNumpy(), O.layernorm_lastaxis(x), rtol=1e-4, atol=2e-5)


def test_golden_softmax_and_layernorm():
    # cudaarray_softmax.phpt:58-62, cudaarray_layernorm.phpt:16-40,81-87
    sm = CudaArray.fromNumpy(np.array([[1, 2, 3]], np.float32)).softmax(-1).toNumpy()
    np.testing.assert_allclose(sm[0], [0.090031, 0.244728, 0.665241], atol=1e-6)
    inp = CudaArray.fromFlatArray([1.0, 2.0, 3.0, 4.0], [2, 2])
    out = inp.layerNorm([1]).toNumpy()
    assert [f"{v:.5f}" for v in out[0]] == ["-0.99998", "0.99998"]
    const = CudaArray.ones([2, 3]).layerNorm([1]).toNumpy()
    assert np.all(const == 0.0)
    scale = CudaArray.fromFlatArray([2.0, 3.0], [2])
    bias = CudaArray.fromFlatArray([0.5, -0.5], [2])
    aff = inp.layerNorm([1], 0.00001, scale, bias).toNumpy()
    assert [f"{v:.5f}" for v in aff[0]] == ["-1.49996", "2.49994"]
    perm = CudaArray.fromFlatArray([1.0, 2.0, 3.0, 4.0], [2, 1, 2]).layerNorm(
        [2, 0], 0.00001, CudaArray.fromFlatArray([1.0, 2.0, 3.0, 4.0], [2, 2])).toNumpy()
    assert f"{perm[1][0][0]:.5f}" == "0.89442"
    strided = CudaArray.fromFlatArray([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], [2, 3]).transpose().layerNorm([0]).toNumpy()
    assert f"{strided[0][0]:.5f}" == "-1.22474"
    assert CudaArray.fromFlatArray([1, 2, 3, 4], [2, 2], "int32").layerNorm([1]).getDtype() == "float64"
    assert CudaArray.fromFlatArray([1.0, 2.0], [2], "float64").layerNorm([0]).getDtype() == "float64"
    assert inp.layerNorm([1], 0.00001, CudaArray.ones([2], "float64")).getDtype() == "float64"
    for bad in (lambda: inp.layerNorm([1, -1]), lambda: inp.layerNorm([2]), lambda: inp.layerNorm([1], 0.0),
                lambda: inp.layerNorm([1], float("nan")),
                lambda: inp.layerNorm([1], 0.00001, CudaArray.ones([3])),
                lambda: inp.layerNorm([1], 0.00001, CudaArray.ones([2], "int32")),
                lambda: CudaArray.zeros([2, 0]).layerNorm([1])):
        with pytest.raises(InvalidArgumentException):
            bad()


def test_golden_variance():
    # cudaarray_variance.phpt
    x = CudaArray.fromNumpy(np.array([[1, 2, 3, 4], [2, 4, 6, 8]], np.float32))
    np.testing.assert_allclose(x.var(1).toNumpy(), [1.25, 5.0], rtol=1e-6)
    np.testing.assert_allclose(x.std(1).toNumpy()[0], 1.118034, rtol=1e-6)
    np.testing.assert_allclose(x.var(1, 1).toNumpy()[0], 1.666667, rtol=1e-6)


def test_matmul_surface():
    r = rng(21)
    a = r.integers(-4, 5, (3, 37, 41)).astype(np.float32)
    b = r.integers(-4, 5, (41, 29)).astype(np.float32)
    for dt, code in (("float32", F32), ("bfloat16", BF16), ("float16", F16)):
        ta = CudaArray.fromNumpy(O.to_storage(a, code), dt)
        tb = CudaArray.fromNumpy(O.to_storage(b, code), dt)
        got = ta.matmul(tb)
        assert got.getShape() == [3, 37, 29] and got.getDtype() == dt
        ref = O.matmul(O.to_storage(a, code), O.to_storage(b, code), code)
        np.testing.assert_array_equal(got.toBits(), ref)
    tt = CudaArray.fromNumpy(b).transpose()  # [29,41] view
    got = CudaArray.fromNumpy(a[0].T.copy()).transpose().matmul(tt.transpose())
    np.testing.assert_array_equal(got.toNumpy(), a[0] @ b)
    with pytest.raises(InvalidArgumentException):
        CudaArray.zeros([3, 4]).matmul(CudaArray.zeros([5, 6]))
    with pytest.raises(InvalidArgumentException):
        CudaArray.zeros([3, 4]).matmul(CudaArray.zeros([4, 6], "float64"))
