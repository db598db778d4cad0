"""Operator, comparison, promotion, reduction and scalar-export expectations
of the reference's own tests, restated against CudaArray on the GPU:
ca_add / ca_sub / ca_mult / ca_div (method and operator forms), ca_where,
ca_prod_reduce, ca_transfer (the CudaArray half), comparison_semantics,
integer_promotion, scalar_precision, low_precision_reductions and
ca_logarithms.

Values printed by var_dump in those tests come from
tests/golden/var_dump_expectations.json (written by
make_var_dump_expectations.py); the tables and closed forms of the
check()-style tests are transcribed beside each test with their source
lines."""
import json
import math
import os
import struct

import numpy as np
import pytest

from phptensors import CudaArray as A
from phptensors import Fusion as F
from phptensors import InvalidArgumentException

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "var_dump_expectations.json")))


def dumped(name):
    return [e["value"] for e in GOLDEN[name] if "value" in e]


# ------------------------------------------------------------ arithmetic
ARITH = [("ca_add", lambda a, b: a.add(b)), ("ca_add_overload", lambda a, b: a + b),
         ("ca_sub", lambda a, b: a.subtract(b)), ("ca_sub_overload", lambda a, b: a - b),
         ("ca_mult", lambda a, b: a.multiply(b)), ("ca_mult_overload", lambda a, b: a * b),
         ("ca_div", lambda a, b: a.divide(b)), ("ca_div_overload", lambda a, b: a / b)]


@pytest.mark.parametrize("name,op", ARITH, ids=[n for n, _ in ARITH])
def test_broadcast_arithmetic_reference(name, op):
    """tests/<name>.phpt:9-20: a row against a matrix, a matrix against a
    rank-3 tensor, and a matrix against the scalar 11, in float32; the printed
    values (float32 widened to double) must match exactly."""
    expected = dumped(name)
    a = A([4, 1, 2, 3])
    b = A([[4, 1, 2, 3], [6, 7, 8, 9]])
    assert op(a, b).toArray() == expected[0]
    a = A([[22, 32], [47, 61]])
    b = A([[[4, 1], [2, 3]], [[6, 7], [8, 9]]])
    assert op(a, b).toArray() == expected[1]
    assert op(a, 11).toArray() == expected[2]


def test_where_reference():
    """tests/ca_where.phpt:9-35"""
    expected = dumped("ca_where")
    cond = A.fromBuffer(bytes([1, 0, 1]), [3], "bool")
    x = A.fromBuffer(struct.pack("<3f", 10, 20, 30), [3])
    y = A.fromBuffer(struct.pack("<3f", 1, 2, 3), [3])
    assert A.where(cond, x, y).toArray() == expected[0]
    cond = A.fromBuffer(bytes([1, 0]), [2, 1], "bool")
    x = A.fromBuffer(struct.pack("<3I", 10, 20, 30), [1, 3], "int32")
    y = A.fromBuffer(struct.pack("<6I", 1, 2, 3, 4, 5, 6), [2, 3], "int32")
    assert A.where(cond, x, y).toArray() == expected[1]
    cond = A.fromBuffer(bytes([1, 0, 1, 0]), [2, 2], "bool").transpose()
    x = A.fromBuffer(struct.pack("<4I", 10, 20, 30, 40), [2, 2], "int32")
    y = A.fromBuffer(struct.pack("<4I", 1, 2, 3, 4), [2, 2], "int32")
    assert A.where(cond, x, y).toArray() == expected[2]
    texts = [e["text"] for e in GOLDEN["ca_where"] if "text" in e]
    assert texts == ["dtype mismatch", "shape mismatch"]
    with pytest.raises(InvalidArgumentException):
        A.where(cond, x, A([[1.0]]))
    with pytest.raises(InvalidArgumentException):
        A.where(cond, x, A.fromBuffer(struct.pack("<9I", *range(1, 10)), [3, 3], "int32"))


def test_prod_reduce_reference():
    """tests/ca_prod_reduce.phpt:9-14"""
    expected = dumped("ca_prod_reduce")
    ca = A([[[1, 2], [3, 4]], [[5, 6], [7, 8]]])
    assert ca.prod(1).toArray() == expected[0]
    assert ca.prod(0).toArray() == expected[1]
    assert ca.prod(2).toArray() == expected[2]
    assert ca.prod().toArray() == expected[3]


def test_transfer_reference():
    """tests/ca_transfer.phpt:15-16, 27-31 (the CudaArray half; HostArray is
    the CPU oracle here, not a product type)"""
    expected = dumped("ca_transfer")
    tensor = A([[1, 2], [3, 4]], "int32")
    assert tensor.toArray() == expected[0]
    host = tensor.toNumpy()
    assert host.dtype == np.int32 and host.tolist() == expected[8]
    assert A.fromNumpy(host).toArray() == expected[9]
    packed = A.fromBuffer(struct.pack("<4I", 1, 2, 3, 4), [2, 2], "int32")
    assert packed.toArray() == expected[10]


# ------------------------------------------------------------ comparisons
def _mask(values):
    if isinstance(values, list):
        return [_mask(v) for v in values]
    assert values in (0, 1, True, False), values
    return bool(values)


def _compare(left, right, expected, label):
    """comparison_semantics.phpt:25-38: eq gives `expected`, ne its negation,
    eagerly and under Fusion.run, with the same dtype."""
    for op in ("eq", "ne"):
        want = expected if op == "eq" else _mask(
            [[not v for v in row] if isinstance(row, list) else not row for row in expected])
        eager = getattr(left, op)(right)
        fused = F.run(lambda: getattr(left, op)(right))
        assert eager.getDtype() == fused.getDtype(), (label, op)
        assert _mask(eager.toArray()) == want, (label, op, "eager")
        assert _mask(fused.toArray()) == want, (label, op, "fused")


@pytest.mark.parametrize("dtype,delta", [("float32", 1e-7), ("float64", 1e-7),
                                         ("float16", 0.0009765625), ("bfloat16", 0.0078125)])
def test_comparison_semantics_floating(dtype, delta):
    """comparison_semantics.phpt:39-52: NaN never equals, +-0 are equal,
    infinities compare by sign, broadcast and strided operands."""
    nan, inf = float("nan"), float("inf")
    left = A([1, 1 + delta, nan, inf, -inf, 0.0, -0.0, 3], dtype)
    right = A([1, 1, nan, inf, inf, -0.0, 0.0, 4], dtype)
    _compare(left, right, [True, False, False, True, False, True, True, False], dtype)
    _compare(A([0, delta, nan, inf], dtype), 0, [True, False, False, False], f"{dtype} scalar")
    _compare(A([[1], [1 + delta]], dtype), A([[1, 1 + delta]], dtype),
             [[True, False], [False, True]], f"{dtype} broadcast")
    _compare(A([[1, 1 + delta], [nan, inf]], dtype).transpose(), A([[1, nan], [1, inf]], dtype),
             [[True, False], [False, True]], f"{dtype} strided")


def test_comparison_semantics_integers():
    """comparison_semantics.phpt:53-59 and the graph replay of :60-64"""
    for dtype in ["int8", "int16", "int32", "int64", "uint8", "uint16", "uint32", "uint64", "bool"]:
        _compare(A([0, 1, 1], dtype), A([0, 0, 1], dtype), [True, False, True], dtype)
    _compare(A(np.array([9007199254740992, 9007199254740993], np.int64), "int64"),
             A(np.array([9007199254740993, 9007199254740993], np.int64), "int64"),
             [False, True], "wide integers")
    _compare(A([1, 2, 3], "int32"), A([1.0, 2.5, 3.0], "float64"), [True, False, True], "mixed")
    example = A([1.0, 2.0], "float64")
    graph = F.compile(lambda a, b: [a.eq(b), a.ne(b)], [example, example])
    equal, different = graph.run(A([float("nan"), float("inf")], "float64"),
                                 A([float("nan"), float("inf")], "float64"))
    assert _mask(equal.toArray()) == [False, True] and _mask(different.toArray()) == [True, False]


# ------------------------------------------------------- integer promotion
INT_TYPES = ["int8", "int16", "int32", "int64", "uint8", "uint16", "uint32", "uint64"]
# integer_promotion.phpt:25-34: result dtype of left (row) with right (column)
PROMOTED = {
    "int8": ["int8", "int16", "int32", "int64", "int16", "int32", "int64", None],
    "int16": ["int16", "int16", "int32", "int64", "int16", "int32", "int64", None],
    "int32": ["int32", "int32", "int32", "int64", "int32", "int32", "int64", None],
    "int64": ["int64", "int64", "int64", "int64", "int64", "int64", "int64", None],
    "uint8": ["int16", "int16", "int32", "int64", "uint8", "uint16", "uint32", "uint64"],
    "uint16": ["int32", "int32", "int32", "int64", "uint16", "uint16", "uint32", "uint64"],
    "uint32": ["int64", "int64", "int64", "int64", "uint32", "uint32", "uint32", "uint64"],
    "uint64": [None, None, None, None, "uint64", "uint64", "uint64", "uint64"],
}


@pytest.mark.parametrize("left_type", INT_TYPES)
def test_integer_promotion_table(left_type):
    """integer_promotion.phpt:35-52: every integer pairing promotes to the
    table's dtype for add/multiply/maximum/minimum/eq/lt, eagerly and fused,
    or is refused when no integer type holds both ranges."""
    ops = {"add": [3, 3], "multiply": [2, 2], "maximum": [2, 2], "minimum": [1, 1],
           "eq": [0, 0], "lt": [1, 0]}
    left = A([1, 2], left_type)
    for index, right_type in enumerate(INT_TYPES):
        right = A([2, 1], right_type)
        want = PROMOTED[left_type][index]
        for op, values in ops.items():
            for fused in (False, True):
                run = (lambda: F.run(lambda: getattr(left, op)(right))) if fused else \
                      (lambda: getattr(left, op)(right))
                if want is None:
                    with pytest.raises(InvalidArgumentException):
                        run()
                    continue
                out = run()
                assert out.getDtype() == want and out.toArray() == values, \
                    (left_type, op, right_type, fused)


@pytest.mark.parametrize("fused", [False, True])
def test_integer_promotion_boundaries(fused):
    """integer_promotion.phpt:53-89"""
    run = (lambda fn: F.run(fn)) if fused else (lambda fn: fn())
    unsigned, signed = A([0, 255], "uint8"), A([-1, 127], "int8")
    assert run(lambda: unsigned + signed).toArray() == [-1, 382]
    assert run(lambda: unsigned.gt(signed)).toArray() == [1, 1]
    large, negative = A([4294967295], "uint32"), A([-1], "int32")
    assert run(lambda: large + negative).toArray() == [4294967294]
    assert run(lambda: large.gt(negative)).toArray() == [1]
    division = run(lambda: A([3], "uint32").divide(A([2], "int32")))
    assert division.getDtype() == "float64" and division.toArray() == [1.5]
    power = run(lambda: A([3], "int64").power(A([2], "int64")))
    assert power.getDtype() == "float64" and power.toArray() == [9.0]
    scalar_div = run(lambda: A([16777217], "int64") / 1)
    assert scalar_div.getDtype() == "float64" and scalar_div.toArray() == [16777217.0]
    half = run(lambda: A([16777217], "int64") + 0.5)
    assert half.getDtype() == "float64" and half.toArray() == [16777217.5]
    wide = A.fromBuffer(bytes.fromhex("ffffffffffffffff"), [1], "uint64")
    for op in ["add", "subtract", "multiply", "divide", "power", "eq", "lt", "maximum", "minimum"]:
        with pytest.raises(InvalidArgumentException):
            run(lambda: getattr(wide, op)(A([1], "int64")))
        with pytest.raises(InvalidArgumentException):
            run(lambda: getattr(wide, op)(1))
    with pytest.raises(InvalidArgumentException):
        run(lambda: 1 + wide)
    with pytest.raises(InvalidArgumentException):
        run(lambda: 1 - wide)
    with pytest.raises(InvalidArgumentException):
        run(lambda: A([127], "int8") + 128)
    with pytest.raises(InvalidArgumentException):
        run(lambda: A([1], "uint8") + -1)
    maximum = run(lambda: A([1], "uint8").maximum(-1))
    assert maximum.getDtype() == "int64" and maximum.toArray() == [1]
    zero_unsigned = A.zeros([0], "uint64")
    with pytest.raises(InvalidArgumentException):
        run(lambda: zero_unsigned + A.zeros([0], "int64"))
    with pytest.raises(InvalidArgumentException):
        run(lambda: zero_unsigned + 1)
    safe = run(lambda: A([2], "uint64") + A([3], "uint32"))
    assert safe.getDtype() == "uint64" and safe.toArray() == [5]


def test_integer_promotion_graph_replay():
    """integer_promotion.phpt:91-97"""
    graph = F.compile(lambda a, b: [a + b, a.gt(b)], [A([1], "uint8"), A([1], "int8")])
    total, mask = graph.run(A([255], "uint8"), A([-1], "int8"))
    assert total.getDtype() == "int16" and total.toArray() == [254]
    assert mask.getDtype() == "int16" and mask.toArray() == [1]


# ------------------------------------------------------- scalar precision
SCALAR_CASES = {  # scalar_precision.phpt:19-31
    "float32": [16777216.0, -2.5], "float64": [16777217.0, 9007199254740991.0],
    "float16": [1.5, -2.5], "bfloat16": [1.5, -2.5],
    "int8": [-128, 127], "int16": [-32768, 32767], "int32": [-2147483648, 2147483647],
    "int64": [-2**63, 2**63 - 1], "uint8": [0, 255], "uint16": [0, 65535],
    "uint32": [0, 4294967295], "uint64": [0, 2**63 - 1], "bool": [False, True],
}


@pytest.mark.parametrize("dtype", list(SCALAR_CASES))
def test_scalar_exports(dtype):
    """scalar_precision.phpt:32-40: exports, indexed items (also through a
    transposed view) keep the dtype's exact values."""
    expected = SCALAR_CASES[dtype]
    npdt = {"int64": np.int64, "uint64": np.uint64}.get(dtype)
    tensor = A(np.array(expected, npdt) if npdt else expected, dtype)
    assert tensor.toArray() == expected
    assert tensor.select(0, 0).item() == expected[0] and tensor.select(0, 1).item() == expected[1]
    assert type(tensor.select(0, 0).item()) is type(expected[0])
    assert tensor.slice("1:2").reshape([1]).item() == expected[1]
    strided = A(np.array([expected, expected], npdt) if npdt else [expected, expected], dtype).transpose()
    assert strided.select(0, 1).select(0, 1).item() == expected[1]


def test_uint64_exports():
    """scalar_precision.phpt:41-49: uint64 values above the signed range
    export exactly (Python integers stand in for PHP's decimal strings)."""
    data = struct.pack("<3Q", 2**63 - 1, 2**63, 2**64 - 1)
    want = [2**63 - 1, 2**63, 2**64 - 1]
    unsigned = A.fromBuffer(data, [3], "uint64")
    for tensor in (unsigned, unsigned.copy(), F.run(lambda: unsigned.slice())):
        assert tensor.toArray() == want
        for i, v in enumerate(want):
            assert tensor.select(0, i).item() == v
    assert unsigned.toBuffer() == data


@pytest.mark.parametrize("dtype,bits,smallest", [
    ("float16", [0x8000, 0x7C00, 0xFC00, 0x7E00, 0x0001], 2.0 ** -24),
    ("bfloat16", [0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x0001], 2.0 ** -133),
])
def test_half_special_exports(dtype, bits, smallest):
    """scalar_precision.phpt:63-74"""
    tensor = A.fromBuffer(struct.pack("<5H", *bits), [5], dtype)
    read = [tensor.select(0, i).item() for i in range(5)]
    assert math.copysign(1.0, read[0]) == -1.0 and read[0] == 0.0
    assert read[1] == math.inf and read[2] == -math.inf and math.isnan(read[3])
    assert read[4] == smallest


def test_fp64_scalar_arithmetic():
    """scalar_precision.phpt:75-90: fp64 subnormals and signed zero export
    exactly, and scalar arithmetic on fp64 stays in fp64, eager and fused."""
    tiny = A([2.0 ** -1074, -0.0], "float64")
    assert tiny.select(0, 0).item() == 2.0 ** -1074
    assert math.copysign(1.0, tiny.select(0, 1).item()) == -1.0
    wide = A([16777217.0, 1e200], "float64")
    for op, want in [(lambda: wide / 2, [16777217.0 / 2, 1e200 / 2]),
                     (lambda: 2 / wide, [2 / 16777217.0, 2 / 1e200]),
                     (lambda: wide ** -1, [1 / 16777217.0, 1 / 1e200])]:
        eager, fused = op(), F.run(op)
        assert eager.getDtype() == "float64" and fused.getDtype() == "float64"
        assert eager.toArray() == want and fused.toArray() == want


# ------------------------------------------------ low-precision reductions
def _close(a, b):
    return abs(a - b) < 1e-4


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_low_precision_reductions(dtype):
    """low_precision_reductions.phpt:16-104"""
    x = A.fromFlatArray([1.0, 2.0, 3.0, 4.0], [2, 2], dtype)
    outs = [x.sum(), x.mean(), x.prod(), x.min(), x.max(), x.argMax(), x.var(), x.std()]
    assert [o.getDtype() for o in outs] == ["float32"] * 5 + ["int32", "float32", "float32"]
    vals = [o.item() for o in outs]
    for got, want in zip(vals[:5], [10.0, 2.5, 24.0, 1.0, 4.0]):
        assert _close(got, want)
    assert vals[5] == 3
    assert x.all().item() is True and x.any().item() is True
    assert _close(vals[6], 1.25) and _close(vals[7], math.sqrt(1.25))
    assert x.sum(0).toArray() == [4.0, 6.0]
    graph = F.compile(lambda t: [t.sum(), t.mean(), t.prod(), t.min(), t.max(), t.all(), t.any(),
                                 t.argMax(), t.var(), t.std()], [x])
    fs, fm, fp, fmin, fmax, fall, fany, farg, fvar, fstd = graph.run(x)
    assert [t.getDtype() for t in (fs, fp, fmin, fmax, farg)] == ["float32"] * 4 + ["int32"]
    for got, want in [(fs, 10.0), (fm, 2.5), (fp, 24.0), (fmin, 1.0), (fmax, 4.0), (fvar, 1.25),
                      (fstd, math.sqrt(1.25))]:
        assert _close(got.item(), want)
    assert fall.item() is True and fany.item() is True and farg.item() == 3
    async_graph = F.compile(lambda t: t.sum(), [x], True)
    assert async_graph.getStats()["cudaGraphCompatible"] in (True, 1)
    assert _close(async_graph.runAsync(x).wait().item(), 10.0)
    tracked = A.fromFlatArray([1.0, 2.0, 3.0], [3], dtype).requiresGrad()
    tracked.sum().backward()
    assert tracked.grad().getDtype() == "float32" and tracked.grad().toArray() == [1.0, 1.0, 1.0]
    mean_tracked = A.fromFlatArray([1.0, 2.0, 3.0], [3], dtype).requiresGrad()
    mean_tracked.mean().backward()
    assert all(_close(v, 1.0 / 3.0) for v in mean_tracked.grad().toArray())


def test_all_any_semantics():
    """all/any (cuda_array_ce.c:1791-1823, AllOpT / AnyOpT
    cuda_op_functors.cuh:141-151): an element counts when it is unequal to
    zero, so NaN counts and -0.0 does not; empty axes give all = true and
    any = false; the output is bool."""
    nan = float("nan")
    x = A([[0.0, -0.0, nan], [1.0, 2.0, 3.0]])
    assert x.all(1).toArray() == [False, True] and x.any(1).toArray() == [True, True]
    assert x.all(0).toArray() == [False, False, True] and x.any(0).toArray() == [True, True, True]
    assert A([[0.0, -0.0]]).any().toArray() == [False]
    assert x.all().getDtype() == "bool" and x.all().toArray() == [False]
    for dtype in ["int8", "int32", "int64", "uint8", "uint64", "bool", "float16", "bfloat16", "float64"]:
        t = A([[0, 1, 1], [1, 1, 1]], dtype)
        assert t.all(1).toArray() == [False, True], dtype
        assert t.any(0).toArray() == [True, True, True], dtype
        assert t.transpose().all(0).toArray() == [False, True], dtype
    empty = A.zeros([2, 0])
    assert empty.all(1).toArray() == [True, True] and empty.any(1).toArray() == [False, False]
    big = np.ones((513, 1000), np.float32)
    big[200, 999] = 0.0
    t = A.fromNumpy(big)
    assert t.all().toArray() == [False] and t.any().toArray() == [True]
    assert t.all(1).toArray() == [i != 200 for i in range(513)]
    assert t.all(0).toArray() == [j != 999 for j in range(1000)]


# ------------------------------------------------------------ logarithms
def test_logarithms_reference():
    """ca_logarithms.phpt:20-58: exp2/expm1/log2/log10/log1p eager, one fused
    kernel for their sum, and their gradients."""
    x = A.fromFlatArray([1, 2, 4, 8], [4])

    def close(actual, expected, tol):
        assert len(actual) == len(expected)
        for a, e in zip(actual, expected):
            assert abs(a - e) <= tol, (a, e)

    close(x.exp2().toArray(), [2, 4, 16, 256], 1e-5)
    close(x.expm1().toArray(), [math.expm1(v) for v in (1, 2, 4, 8)], 1e-4)
    close(x.log2().toArray(), [0, 1, 2, 3], 1e-5)
    close(x.log10().toArray(), [0, math.log10(2), math.log10(4), math.log10(8)], 1e-5)
    close(A.fromFlatArray([1e-7, 1e-5], [2]).log1p().toArray(), [math.log1p(1e-7), math.log1p(1e-5)], 1e-11)
    graph = F.compile(lambda t: t.exp2() + t.expm1() + t.log2() + t.log10() + t.log1p(), [x])
    expected = x.exp2().add(x.expm1()).add(x.log2()).add(x.log10()).add(x.log1p())
    close(graph.run(x).toArray(), expected.toArray(), 1e-5)
    assert graph.getStats()["fusedKernels"] == 1
    tracked = A.fromFlatArray([1, 2, 4], [3]).requiresGrad()
    loss = tracked.exp2().sum().add(tracked.expm1().sum()).add(tracked.log2().sum()) \
        .add(tracked.log10().sum()).add(tracked.log1p().sum())
    loss.backward()
    ln2, ln10 = math.log(2), math.log(10)
    close(tracked.grad().toArray(), [
        ln2 * 2 + math.exp(1) + 1 / ln2 + 1 / ln10 + 1 / 2,
        ln2 * 4 + math.exp(2) + 1 / (2 * ln2) + 1 / (2 * ln10) + 1 / 3,
        ln2 * 16 + math.exp(4) + 1 / (4 * ln2) + 1 / (4 * ln10) + 1 / 5,
    ], 5e-5)


def test_logarithms_fused_gradient_and_trig():
    """ca_logarithms.phpt:62-125: the gradient of the logarithm sum taken
    inside Fusion.run, inverse / hyperbolic trigonometry eager, fused and
    differentiated, and fp16/bf16 fused results bitwise equal to eager."""
    def close(actual, expected, tol):
        assert len(actual) == len(expected)
        for a, e in zip(actual, expected):
            assert abs(a - e) <= tol, (a, e)

    def log_loss(t):
        return t.exp2().sum().add(t.expm1().sum()).add(t.log2().sum()).add(t.log10().sum()) \
            .add(t.log1p().sum())

    tracked = A.fromFlatArray([1, 2, 4], [3]).requiresGrad()
    log_loss(tracked).backward()
    fused_tracked = A.fromFlatArray([1, 2, 4], [3]).requiresGrad()
    seed = A.ones([1])

    def body():
        loss = log_loss(fused_tracked)
        loss.backward(seed)
        return [loss, fused_tracked.grad()]

    _, fused_gradient = F.run(body)
    close(fused_gradient.toArray(), tracked.grad().toArray(), 1e-5)

    values = [-0.5, 0.2, 0.7]
    trig = A.fromFlatArray(values, [3])
    methods = ["asin", "acos", "atan", "sinh", "cosh", "tanh"]
    for m in methods:
        close(getattr(trig, m)().toArray(), [getattr(math, m)(v) for v in values], 1e-5)
    graph = F.compile(lambda t: t.asin() + t.acos() + t.atan() + t.sinh() + t.cosh() + t.tanh(), [trig])
    expected = trig.asin().add(trig.acos()).add(trig.atan()).add(trig.sinh()).add(trig.cosh()).add(trig.tanh())
    close(graph.run(trig).toArray(), expected.toArray(), 1e-5)
    t = A.fromFlatArray(values, [3]).requiresGrad()
    loss = t.asin().sum().add(t.acos().sum().multiply(2)).add(t.atan().sum()).add(t.sinh().sum()) \
        .add(t.cosh().sum()).add(t.tanh().sum())
    loss.backward()
    close(t.grad().toArray(), [-1 / math.sqrt(1 - v * v) + 1 / (1 + v * v) + math.cosh(v) + math.sinh(v)
                                + 1 - math.tanh(v) ** 2 for v in values], 1e-5)
    for dtype in ("float16", "bfloat16"):
        low = A.fromFlatArray([0.25, 0.5], [2], dtype)

        def chain(x):
            return x.exp2() + x.log2() + x.expm1() + x.log1p() + x.asin() + x.acos() + x.atan() + \
                x.sinh() + x.cosh() + x.tanh()

        g = F.compile(chain, [low])
        assert g.run(low).toBuffer() == chain(low).toBuffer(), dtype


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_low_precision_gradient_in_compiled_plan(dtype):
    """low_precision_reductions.phpt:84-99: a plan compiled from a tracked
    input captures backward() and returns a float32 gradient; a tracked output
    that never ran backward() is refused, and so is a tracked input whose
    example was untracked (fusion.c:357, 376-387, 479-486)."""
    tracked = A.fromFlatArray([1.0, 2.0, 3.0], [3], dtype).requiresGrad()

    def body(x):
        total = x.sum()
        total.backward()
        return [total, x.grad()]

    graph = F.compile(body, [tracked])
    _, gradient = graph.run(tracked)
    assert gradient.getDtype() == "float32" and gradient.toArray() == [1.0, 1.0, 1.0]
    with pytest.raises(InvalidArgumentException):
        F.compile(lambda x: x.sum(), [tracked])
    plain = F.compile(lambda x: x.sum(), [A.fromFlatArray([1.0, 2.0, 3.0], [3], dtype)])
    with pytest.raises(InvalidArgumentException):
        plain.run(tracked)


def test_extended_operations_reference():
    """cudaarray_extended.phpt:9-25, 31-38, 95-97 and its expected lines 1-12,
    15-18, 25 and 27 (gather / scatterAdd are indexed operations outside this
    build's path and are left out)."""
    x = A([[1.0, 0.0], [3.0, 4.0]])
    assert x.maximum(0).toArray() == [[1, 0], [3, 4]]
    assert x.minimum(0).toArray() == [[0, 0], [0, 0]]
    assert x.clamp(0, 2).toArray() == [[1, 0], [2, 2]]
    assert x.all(1).toArray() == [False, True] and x.any(1).toArray() == [True, True]
    assert "%.3f %.3f" % (x.var().item(), x.std().item()) == "2.500 1.581"
    assert x.var(0).toArray() == [1, 4]
    assert A([[7.0], [8.0]]).squeeze(1).getShape() == [2]
    assert x.unsqueeze(1).getShape() == [2, 1, 2]
    assert A([[1.0, 2.0]]).broadcastTo([2, 2]).toArray() == [[1, 2], [1, 2]]
    assert A([[1.0, 2.0], [3.0, 4.0]]).transpose().unsqueeze(0).squeeze(0).toArray() == [[1, 3], [2, 4]]
    item = A.full([1], 42, "int64").item()
    assert item == 42 and isinstance(item, int)
    graph = F.compile(lambda t: t.clamp(0, 2).maximum(0.5).var(), [x])
    assert "%.3f" % graph.run(x).item() == "0.422"
    logical = F.compile(lambda t: [t.all(1), t.any(1)], [x])
    all_, any_ = logical.run(x)
    assert all_.toArray() == [False, True] and any_.toArray() == [True, True]
    broadcast = F.compile(lambda t: t.broadcastTo([2, 2]).sum(0), [A([1.0, 2.0])])
    assert broadcast.run(A([1.0, 2.0])).toArray() == [2, 4]
    with pytest.raises(InvalidArgumentException):
        x.var(1, 2)
    tracked = A([-1.0, 0.5, 3.0]).requiresGrad()
    tracked.clamp(0, 2).sum().backward()
    assert tracked.grad().toArray() == [0, 1, 0]
