"""CudaArray serialization parity with tests/cuda_array_serialization.phpt:
malformed payloads are rejected with InvalidArgumentException and leave the
live tensor untouched; every dtype, empty and rank-zero tensors round-trip
through the payload (and through pickle, Python's serialize()); snapshots
carry no gradients; views refuse to serialize (cuda_array_ce.c:276-280)."""
import pickle

import pytest

from phptensors import CudaArray
from phptensors._abi import InvalidArgumentException, RuntimeException

pytestmark = pytest.mark.gpu

PHP_INT_MAX = 2 ** 63 - 1
DTYPES = ["float32", "float64", "float16", "bfloat16", "int8", "int16", "int32", "int64",
          "uint8", "uint16", "uint32", "uint64", "bool"]


def ser(t):
    return getattr(t, "__serialize")()


def unser(t, payload):
    return getattr(t, "__unserialize")(payload)


def test_malformed_payloads_preserve_existing_storage():
    tensor = CudaArray([[1, 2], [3, 4]], "float64")
    payload = ser(tensor)
    assert payload["__cuda_array_v1"] == "1" and payload["dtype"] == "float64"
    assert payload["shape"] == [2, 2] and payload["total_elements"] == 4 and payload["element_size"] == 8
    invalid = [
        {"__cuda_array_v1": "2"}, {"__cuda_array_v1": True},
        {"ndims": -1}, {"ndims": PHP_INT_MAX}, {"ndims": "2"},
        {"shape": [2, "2"]}, {"shape": [2, -2]}, {"shape": {2: 2, 3: 2}},
        {"shape": [2147483647, 2147483647, 2147483647], "ndims": 3},
        {"shape": [0, 2147483647, 2147483647, 2147483647], "ndims": 4},
        {"dtype": "unknown"}, {"dtype": "float64\0invalid"},
        {"total_elements": -1}, {"total_elements": 3},
        {"element_size": 1}, {"element_size": PHP_INT_MAX},
        {"data": payload["data"][1:]}, {"data": payload["data"] + b"\0"},
    ]
    for i, overrides in enumerate(invalid):
        with pytest.raises(InvalidArgumentException):
            unser(tensor, {**payload, **overrides})
        assert ser(tensor) == payload, i
        assert tensor.toArray() == [[1.0, 2.0], [3.0, 4.0]], i
    for key in ["__cuda_array_v1", "ndims", "shape", "dtype", "total_elements", "element_size", "data"]:
        bad = dict(payload)
        del bad[key]
        with pytest.raises(InvalidArgumentException):
            unser(tensor, bad)
        assert ser(tensor) == payload, key


@pytest.mark.parametrize("dtype", DTYPES)
def test_round_trips_every_dtype_and_empty_shapes(dtype):
    tensor = CudaArray([[1, 2], [3, 4]], "float64")
    source = CudaArray([[1, 2], [3, 4]], dtype)
    restored = pickle.loads(pickle.dumps(source))
    assert restored.toBuffer() == source.toBuffer()
    assert restored.getDtype() == dtype and restored.getShape() == [2, 2]
    unser(tensor, ser(source))
    assert tensor.toBuffer() == source.toBuffer() and tensor.getDtype() == dtype
    for shape in ([0], [2, 0]):
        empty = CudaArray.fromBuffer(b"", shape, dtype)
        copy = pickle.loads(pickle.dumps(empty))
        assert copy.getShape() == shape and copy.toBuffer() == b""


def test_rank_zero_and_gradient_free_snapshots():
    scalar = CudaArray([7.0]).select(0, 0) + 1
    restored = pickle.loads(pickle.dumps(scalar))
    assert restored.getShape() == [] and restored.item() == 8.0
    tracked = CudaArray([2.0, 3.0]).requiresGrad()
    (tracked * 2).sum().backward()
    payload = ser(tracked)
    with pytest.raises(InvalidArgumentException):
        unser(tracked, {**payload, "__cuda_array_v1": "2"})
    assert tracked.grad().toArray() == [2.0, 2.0]
    snapshot = pickle.loads(pickle.dumps(tracked))
    assert snapshot.grad() is None
    with pytest.raises(InvalidArgumentException):
        snapshot.sum().backward()


def test_views_refuse_to_serialize_and_backward_checks_its_seed():
    base = CudaArray([[1.0, 2.0], [3.0, 4.0]])
    for view in (base.transpose(), base.select(0, 1), base.reshape([4])):
        with pytest.raises(RuntimeException):
            ser(view)
    # autograd_backward argument checks (autograd.c:1712-1733)
    x = CudaArray([1.0, 2.0]).requiresGrad()
    y = x * 3
    with pytest.raises(InvalidArgumentException):
        y.backward()                                   # non-scalar without a seed
    with pytest.raises(InvalidArgumentException):
        y.backward(CudaArray([1.0, 1.0, 1.0]))         # seed shape mismatch
    with pytest.raises(InvalidArgumentException):
        y.backward(CudaArray([1.0, 1.0], "float64"))   # seed dtype mismatch
    y.backward(CudaArray([1.0, 2.0]))
    assert x.grad().toArray() == [3.0, 6.0]
