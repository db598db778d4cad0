"""tests/ca_transfer_fast.phpt restated: construction from nested lists for
every storage dtype, raw-byte and flat round trips, strided views packed on
the device (a 8192x12 transpose, sparse columns, stepped transposes), 64-bit
exactness, input validation (ragged, too deep, non-numeric, bad flat
shapes), Fusion exports, and transfers larger than any staging window.
PHP references, key/hole handling and constructor re-initialisation are
PHP-array features and are left out."""
import struct

import numpy as np
import pytest

from phptensors import CudaArray as A
from phptensors import Fusion as F
from phptensors import InvalidArgumentException, RuntimeException

pytestmark = pytest.mark.gpu

DTYPES = ["float32", "float64", "int8", "int16", "int32", "int64", "uint8", "uint16", "uint32",
          "uint64", "bool"]


@pytest.mark.parametrize("dtype", DTYPES)
def test_construct_and_pack(dtype):
    """ca_transfer_fast.phpt:12-34"""
    data = [[[0, 1, 2], [3, 4, 5]], [[6, 7, 8], [9, 10, 11]]]

    def convert(v):
        return bool(v) if dtype == "bool" else float(v) if dtype.startswith("float") else v

    expected = [[[convert(v) for v in row] for row in plane] for plane in data]
    tensor = A(data, dtype)
    assert tensor.toArray() == expected
    assert A.fromNumpy(tensor.toNumpy(), dtype).toArray() == expected
    assert A.fromBuffer(tensor.toBuffer(), [2, 2, 3], dtype).toArray() == expected
    assert A.fromFlatArray(list(range(12)), [2, 2, 3], dtype).toArray() == expected
    view = tensor.slice("1:, :, ::2").transpose()
    assert A.fromBuffer(view.toBuffer(), view.getShape(), dtype).toArray() == view.toArray()
    row_bytes = tensor.toBuffer()
    size = len(row_bytes) // 12
    large = A.fromBuffer(row_bytes * 8192, [8192, 12], dtype).transpose()
    want = b"".join(row_bytes[i * size:(i + 1) * size] * 8192 for i in range(12))
    assert large.toBuffer() == want
    scalar = tensor.slice("1, 1, 2")
    assert scalar.toArray() == [convert(11)]
    assert A.fromBuffer(scalar.toBuffer(), [1], dtype).toArray() == [convert(11)]


def test_precision_and_validation():
    """ca_transfer_fast.phpt:35-79"""
    assert A(np.array([9007199254740993, 2**63 - 1], np.int64), "int64").toArray() == \
        [9007199254740993, 2**63 - 1]
    assert A([1.000000000000001], "float64").toArray() == [1.000000000000001]
    assert A([1, 2.5, True, False]).toArray() == [1.0, 2.5, 1.0, 0.0]
    for data in ([], [[], []], [[[], []], [[], []]]):
        t = A(data)
        assert t.toArray() == data and t.toBuffer() == b""
    assert A.fromFlatArray([], [2, 0]).toArray() == [[], []]
    deep = [1]
    for _ in range(10):
        deep = [deep]
    for bad in ([[[1, 2], [3]], [[1], [2, 3]]], [1, [2]], [[1], 2], [None], ["1"], [object()], [[], [1]], deep):
        with pytest.raises(InvalidArgumentException):
            A(bad)
    for data, shape in (([1, 2], [3]), ([1, 2], []), ([[1, 2]], [2]), ([1], [-1]), ([1], [2**63 - 1, 3])):
        with pytest.raises(InvalidArgumentException):
            A.fromFlatArray(data, shape)


def test_strided_packing_and_fusion_export():
    """ca_transfer_fast.phpt:80-112"""
    large = A.fromFlatArray(list(range(65536)), [256, 256], "int64")
    column = large.slice(":, 7")
    expected = [i * 256 + 7 for i in range(256)]
    assert column.toArray() == expected
    assert A.fromBuffer(column.toBuffer(), [256], "int64").toArray() == expected
    stepped = large.slice("1::2, 3::2").transpose()
    expected = [[i * 256 + j for i in range(1, 256, 2)] for j in range(3, 256, 2)]
    assert stepped.toArray() == expected
    assert A.fromBuffer(stepped.toBuffer(), stepped.getShape(), "int64").toArray() == expected
    bits = A(np.array([2**63 - 1, 9007199254740993], np.int64), "int64")
    assert bits.toBuffer() == struct.pack("<2q", 2**63 - 1, 9007199254740993)
    precise = A.full([256, 256], 1.000000000000001, "float64")
    assert precise.slice("::2, ::2").toBuffer() == struct.pack("<d", 1.000000000000001) * (128 * 128)
    boolean = A.fromBuffer(b"\0\1" * 32768, [256, 256], "bool").transpose()
    assert boolean.toBuffer() == (b"\0" * 256 + b"\1" * 256) * 128
    fused = F.run(lambda: large + 1)
    assert fused.toBuffer() == A(np.arange(1, 65537, dtype=np.int64), "int64").toBuffer()
    with pytest.raises(RuntimeException):
        F.compile(lambda x: x.toBuffer(), [large])


def test_transfers_beyond_staging_windows():
    """ca_transfer_fast.phpt:113-142"""
    elements = 2 * 2049 * 2049
    pattern = np.arange(1024, dtype=np.uint32).astype("<u4")
    data = np.resize(pattern, elements).astype("<i4").tobytes()
    streamed = A.fromBuffer(data, [2, 2049, 2049], "int32")
    out = streamed.toArray()
    assert len(out) == 2 and len(out[1]) == 2049 and len(out[1][2048]) == 2049
    for index in (0, 8388607, 8388608, 8388609, elements - 1):
        plane, rest = divmod(index, 2049 * 2049)
        row, col = divmod(rest, 2049)
        assert out[plane][row][col] == index % 1024
    del out, streamed
    flat = A.full([8388613], 2.5)
    out = flat.toArray()
    assert len(out) == 8388613 and out[8388608] == 2.5 and out[8388612] == 2.5
    assert A(out).toBuffer() == flat.toBuffer()
    row = [1.25] * 1048580
    nested = A([row, row], "float64")
    assert nested.toBuffer() == struct.pack("<d", 1.25) * (2 * 1048580)
    bad = [row, row[:-1] + [None]]
    with pytest.raises(InvalidArgumentException):
        A(bad, "float64")
