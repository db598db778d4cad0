"""tests/cuda_shape_boundaries.phpt restated (the ArrayAccess writes and
concat cases are PHP surface outside this build's path): oversized indices,
axes and extents are refused, not narrowed; virtual broadcast sizes beyond
2^32 keep full precision in shape, size and strides; reductions whose output
count or index range does not fit are refused; empty views keep their
strides; nested offset views keep their footprint."""
import pytest

from phptensors import CudaArray as A
from phptensors import Fusion as F
from phptensors import InvalidArgumentException

pytestmark = pytest.mark.gpu

LARGE = [4294967296, 4294967297, 4294966297, 2**63 - 1, -2**63]


def test_oversized_arguments_rejected():
    """cuda_shape_boundaries.phpt:22-38"""
    one = A([7])
    matrix = A([[1, 2], [3, 4]])
    for large in LARGE:
        with pytest.raises(InvalidArgumentException):
            one.select(0, large)
        assert one.slice([0, large]).toArray() == ([7.0] if large > 0 else [])
        with pytest.raises(InvalidArgumentException):
            one.reshape([large])
        with pytest.raises(InvalidArgumentException):
            one.sum(large)
        with pytest.raises(InvalidArgumentException):
            one.argMax(large)
        with pytest.raises(InvalidArgumentException):
            matrix.transpose([large, 1])
        with pytest.raises(InvalidArgumentException):
            F.run(lambda: one.sum(large))
    assert one.toArray() == [7.0]
    assert matrix.sum(-1).toArray() == [3.0, 7.0]


def test_virtual_sizes_keep_precision():
    """cuda_shape_boundaries.phpt:39-59"""
    one = A([7])
    wide = one.broadcastTo([2147483647, 2])
    assert wide.getSize() == 4294967294
    assert wide.getStrides() == [0, 0]
    assert wide.select(0, 2147483646).toArray() == [7.0, 7.0]
    with pytest.raises(InvalidArgumentException):
        wide.argMax()
    with pytest.raises(InvalidArgumentException):
        F.run(lambda: wide.argMax())
    empty = A.zeros([0, 2147483647, 2])
    assert empty.getStrides() == [4294967294, 2, 1]
    result = empty + one
    assert result.getShape() == empty.getShape() and result.getSize() == 0
    assert result.getStrides() == empty.getStrides()
    suffix = A.zeros([2147483647, 2147483647, 2147483647, 0])
    for op in (lambda: suffix.sum(3), lambda: suffix.argMax(3), lambda: suffix.var(3),
               lambda: F.run(lambda: suffix.sum(3))):
        with pytest.raises(InvalidArgumentException):
            op()
    assert suffix.sum(0).getSize() == 0
    assert suffix.slice().getShape() == suffix.getShape()
    assert suffix.getSize() == 0


def test_offset_views_and_empty_slices():
    """cuda_shape_boundaries.phpt:64-70"""
    matrix = A([[1, 2], [3, 4]])
    assert matrix.slice("1, :").slice("1").reshape([1]).toArray() == [4.0]
    byte = A([7], "int8")
    single = byte.broadcastTo([1, 1, 1, 1, 1, 2147483647, 2147483647])
    empty = F.run(lambda: single.slice("1:1,1:1,1:1,1:1,1:1,:,:"))
    assert empty.getShape() == [0, 0, 0, 0, 0, 2147483647, 2147483647]
