"""Cast, copy and mixed-dtype arithmetic contract of CudaArray, restating
tests/host_array_numeric_cuda.phpt, tests/host_array_copy_cast.phpt and
tests/ca_astype.phpt.

The reference checks its GPU against HostArray; here the expected bytes come
from numpy casts of small values that every dtype holds exactly (so any
rounding rule gives the same bits), bf16 patterns from the oracle's converter,
and the accepted/rejected cast pairs from the table the reference's own test
spells out (host_array_copy_cast.phpt:14-28)."""
import struct

import numpy as np
import pytest

import oracle_lib as O
from phptensors import CudaArray, InvalidArgumentException, RuntimeException

pytestmark = pytest.mark.gpu

DTYPES = ["float32", "float64", "float16", "bfloat16", "int8", "int16", "int32", "int64",
          "uint8", "uint16", "uint32", "uint64", "bool"]
NP = {"float32": np.float32, "float64": np.float64, "float16": np.float16, "int8": np.int8,
      "int16": np.int16, "int32": np.int32, "int64": np.int64, "uint8": np.uint8,
      "uint16": np.uint16, "uint32": np.uint32, "uint64": np.uint64, "bool": np.bool_}

# host_array_copy_cast.phpt:14-28: the safe-cast targets of each storage dtype
ALLOWED = {
    "float32": ["float32", "float64"],
    "float64": ["float64"],
    "float16": ["float16", "float32", "float64"],
    "bfloat16": ["bfloat16", "float32", "float64"],
    "int8": ["int8", "int16", "int32", "int64", "float32", "float64"],
    "int16": ["int16", "int32", "int64", "float32", "float64"],
    "int32": ["int32", "int64", "float32", "float64"],
    "int64": ["int64", "float64"],
    "uint8": ["uint8", "uint16", "uint32", "uint64", "int16", "int32", "int64", "float32", "float64"],
    "uint16": ["uint16", "uint32", "uint64", "int32", "int64", "float32", "float64"],
    "uint32": ["uint32", "uint64", "int64", "float32", "float64"],
    "uint64": ["uint64", "float64"],
    "bool": ["bool", "int8", "int16", "int32", "int64", "uint8", "uint16", "uint32", "uint64",
             "float32", "float64"],
}


def values_for(dtype):
    """host_array_numeric_cuda.phpt:23-24"""
    if "float" in dtype:
        return [-1.5, 0.0, 3.25]
    if dtype.startswith("int"):
        return [-7, 0, 3]
    return [0, 1, 3]


def storage_bytes(values, dtype):
    """Little-endian storage of exactly representable values."""
    if dtype == "bfloat16":
        return O.f32_to_bf16(np.asarray(values, np.float32)).astype("<u2").tobytes()
    return np.asarray(values).astype(NP[dtype]).tobytes()


def upload(values, dtype):
    return CudaArray.fromBuffer(storage_bytes(values, dtype), [len(values)], dtype)


def numeric(values, dtype):
    """The values as the storage dtype holds them (bool keeps 0/1)."""
    if dtype == "bool":
        return [1 if v else 0 for v in values]
    return values


@pytest.mark.parametrize("src", DTYPES)
def test_cast_decisions_and_bytes(src):
    """host_array_numeric_cuda.phpt:21-50: every (from, to) pair is either
    rejected or produces the target's bytes of the same logical values."""
    vals = values_for(src)
    gpu = upload(vals, src)
    assert gpu.copy().toBuffer() == storage_bytes(vals, src)
    held = numeric(vals, src)
    for dst in DTYPES:
        if dst not in ALLOWED[src]:
            with pytest.raises((InvalidArgumentException, RuntimeException)):
                gpu.astype(dst)
            continue
        out = gpu.astype(dst)
        assert out.getDtype() == dst and out.getShape() == [3], (src, dst)
        assert out.toBuffer() == storage_bytes(held, dst), (src, dst)


@pytest.mark.parametrize("src", DTYPES)
def test_broadcast_views_copy_and_cast(src):
    """host_array_numeric_cuda.phpt:42-50: a row broadcast to [2,3] has a zero
    stride, copies and casts by its logical contents, and an empty broadcast
    copies to empty rows."""
    vals = values_for(src)
    rows = CudaArray.fromBuffer(storage_bytes(vals, src), [1, 3], src)
    view = rows.select(0, 0).broadcastTo([2, 3])
    assert view.getStrides() == [0, 1]
    held = numeric(vals, src)
    assert view.copy().toBuffer() == storage_bytes(held * 2, src)
    assert view.astype("float64").toBuffer() == np.asarray(held * 2, np.float64).tobytes()
    empty = CudaArray.ones([1], src).broadcastTo([2, 0])
    assert empty.copy().getShape() == [2, 0] and empty.copy().toArray() == [[], []]


@pytest.mark.parametrize("dtype,data", [
    ("int64", struct.pack("<2q", -2**63, 2**63 - 1)),
    ("uint64", bytes.fromhex("ffffffffffffffff")),
])
def test_integer_boundary_casts(dtype, data):
    """host_array_numeric_cuda.phpt:52-56 and host_array_copy_cast.phpt:57-63:
    64-bit boundaries widen to the nearest float64 (numpy's conversion)."""
    n = len(data) // 8
    gpu = CudaArray.fromBuffer(data, [n], dtype)
    assert gpu.copy().toBuffer() == data
    expected = np.frombuffer(data, NP[dtype]).astype(np.float64).tobytes()
    assert gpu.astype("float64").toBuffer() == expected
    assert gpu.astype(dtype).toBuffer() == data


@pytest.mark.parametrize("a,b", [("float32", "float32"), ("float32", "float64"),
                                 ("float64", "float32"), ("float64", "float64")])
def test_mixed_float_broadcast_arithmetic(a, b):
    """host_array_numeric_cuda.phpt:59-70: [[8],[16]] against [2,4,8] in all
    four float pairings; the result is the wider dtype and every value is
    exact."""
    x = CudaArray.fromNumpy(np.array([[8], [16]], NP[a]))
    y = CudaArray.fromNumpy(np.array([2, 4, 8], NP[b]))
    out_dt = "float64" if "float64" in (a, b) else "float32"
    hx = np.array([[8], [16]], NP[out_dt])
    hy = np.array([2, 4, 8], NP[out_dt])
    for method, ref in [("add", hx + hy), ("subtract", hx - hy), ("multiply", hx * hy),
                        ("divide", hx / hy)]:
        got = getattr(x, method)(y)
        assert got.getDtype() == out_dt and got.getShape() == [2, 3], method
        assert got.toBuffer() == ref.astype(NP[out_dt]).tobytes(), method


def test_scalar_rounding_and_operand_order():
    """host_array_numeric_cuda.phpt:71-76: an integer scalar rounds to float32
    before the add (-16777216 + 16777217 gives 0), and scalar-left operations
    keep their operand order."""
    gpu = CudaArray.fromNumpy(np.array([-16777216], np.float32)).broadcastTo([2, 3])
    host = np.full((2, 3), -16777216, np.float32)
    assert (gpu + 16777217).toBuffer() == (host + np.float32(16777217)).tobytes()
    assert (gpu + 16777217).toArray() == [[0.0] * 3] * 2
    for got, ref in [(0 / gpu, np.float32(0) / host), (2 - gpu, np.float32(2) - host),
                     (2 * gpu, np.float32(2) * host), (2 / gpu, np.float32(2) / host)]:
        assert got.getDtype() == "float32"
        assert got.toBuffer() == ref.astype(np.float32).tobytes()


def test_empty_axis_arithmetic():
    """host_array_numeric_cuda.phpt:77-80"""
    out = CudaArray.zeros([2, 0, 3]) + CudaArray.ones([1, 3])
    assert out.getShape() == [2, 0, 3] and out.toArray() == [[], []]


def test_astype_reference_cases():
    """tests/ca_astype.phpt: a same-dtype cast stays valid after its source is
    released, int64 widens to float64, and float64 to int32 is refused."""
    original = CudaArray.fromNumpy(np.array([1, 2], np.float32))
    alias = original.astype("float32")
    del original
    assert alias.toArray() == [1.0, 2.0]
    assert CudaArray.fromNumpy(np.array([1], np.int64)).astype("float64").toArray() == [1.0]
    with pytest.raises(InvalidArgumentException):
        CudaArray.fromNumpy(np.array([1.0])).astype("int32")


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_special_values_widen(dtype):
    """host_array_copy_cast.phpt:64-70: NaN, infinities, -0.0 and 1.5 copy bit
    for bit and widen to float64 as IEEE values."""
    vals = [float("nan"), float("inf"), float("-inf"), -0.0, 1.5]
    if dtype == "bfloat16":
        data = O.f32_to_bf16(np.asarray(vals, np.float32)).astype("<u2").tobytes()
    else:
        data = np.asarray(vals, NP[dtype]).tobytes()
    gpu = CudaArray.fromBuffer(data, [5], dtype)
    assert gpu.copy().toBuffer() == data
    wide = np.frombuffer(gpu.astype("float64").toBuffer(), np.float64)
    assert np.isnan(wide[0]) and wide[1] == np.inf and wide[2] == -np.inf
    assert struct.pack("<d", wide[3]) == struct.pack("<d", -0.0) and wide[4] == 1.5
