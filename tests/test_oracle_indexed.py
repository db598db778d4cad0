"""Pins the oracle's gather / scatter-add (oracle/hostarray.c or_gather,
or_scatter_add, restating indexed_ops.cu:108-204) against the textbook
routines they reduce to, numpy.take_along_axis and numpy.add.at, and against
the reference's own expectations (tests/cudaarray_extended.phpt:27-31,
tests/indexed_low_precision.phpt:12-60)."""
import numpy as np
import pytest

import oracle_lib as O


@pytest.mark.parametrize("shape,axis,dtype", [((5, 7), 0, O.F32), ((5, 7), 1, O.F64), ((3, 4, 6), 2, O.I32),
                                              ((3, 4, 6), 0, O.I64), ((2, 3, 4, 5), 1, O.U8), ((9,), 0, O.I16)])
def test_gather_matches_take_along_axis(shape, axis, dtype):
    r = np.random.default_rng(sum(shape) + axis)
    x = (r.standard_normal(shape) * 100).astype(O.NP_STORAGE[dtype])
    ishape = list(shape)
    ishape[axis] = 11
    idx = r.integers(0, shape[axis], ishape).astype(np.int32)
    got = O.gather(x, dtype, idx, axis)
    np.testing.assert_array_equal(got, np.take_along_axis(x, idx, axis))


def test_gather_copies_bits():
    # NaN payloads and signed zeros are copied, not re-rounded
    x = np.array([np.float32(-0.0), np.float32(np.nan), np.float32(1.5)], np.float32)
    x[1] = np.frombuffer(np.uint32(0x7fc12345).tobytes(), np.float32)[0]
    got = O.gather(x, O.F32, np.array([1, 0, 2, 1], np.int32), 0)
    assert got.view(np.uint32).tolist() == [0x7fc12345, 0x80000000, 0x3fc00000, 0x7fc12345]


@pytest.mark.parametrize("shape,axis,dtype", [((6, 5), 0, O.F64), ((4, 3, 8), 2, O.F64), ((7,), 0, O.F64)])
def test_scatter_add_matches_add_at(shape, axis, dtype):
    r = np.random.default_rng(len(shape) * 10 + axis)
    x = r.integers(-5, 6, shape).astype(np.float64)
    ishape = list(shape)
    ishape[axis] = 9
    idx = r.integers(0, shape[axis], ishape).astype(np.int32)
    upd = r.integers(-3, 4, ishape).astype(np.float64)
    expect = x.copy()
    # np.add.at along an axis: the full index tuple of every update
    coords = list(np.indices(ishape))
    coords[axis] = idx
    np.add.at(expect, tuple(coords), upd)
    np.testing.assert_array_equal(O.scatter_add(x, dtype, idx, upd, axis), expect)


def test_reference_vectors():
    # cudaarray_extended.phpt:27-31 ([[30,10],[50,50]] and [[2,0,1],[0,7,0]])
    src = np.array([[10.0, 20.0, 30.0], [40.0, 50.0, 60.0]], np.float32)
    idx = np.array([2, 0, 1, 1], np.int32).reshape(2, 2)
    assert O.gather(src, O.F32, idx, 1).tolist() == [[30.0, 10.0], [50.0, 50.0]]
    upd = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    assert O.scatter_add(np.zeros((2, 3), np.float32), O.F32, idx, upd, 1).tolist() == [[2.0, 0.0, 1.0],
                                                                                        [0.0, 7.0, 0.0]]
    # transposed source gathered along axis 0 (cudaarray_extended.phpt:64-66)
    tidx = np.array([2, 0, 1, 2, 0, 1], np.int32).reshape(3, 2)
    assert O.gather(np.ascontiguousarray(src.T), O.F32, tidx, 0).tolist() == [[30.0, 40.0], [20.0, 60.0],
                                                                               [10.0, 50.0]]
    # indexed_low_precision.phpt: [1,2,3] gathered at [2,0] -> [3,1] (float16 / bfloat16 bits)
    for dt in (O.F16, O.BF16):
        x = O.to_storage(np.array([1.0, 2.0, 3.0], np.float32), dt)
        got = O.from_storage(O.gather(x, dt, np.array([2, 0], np.int32), 0), dt)
        assert got.tolist() == [3.0, 1.0]
    # scatterAdd of [1,2,3] at [2,0,2] into zeros -> [2,0,4]
    assert O.scatter_add(np.zeros(3, np.float32), O.F32, np.array([2, 0, 2], np.int32),
                         np.array([1.0, 2.0, 3.0], np.float32), 0).tolist() == [2.0, 0.0, 4.0]


def test_out_of_range_index_is_reported():
    src = np.arange(6, dtype=np.float32).reshape(2, 3)
    with pytest.raises(O.OracleIndexError) as e:
        O.gather(src, O.F32, np.array([[3, 0]], np.int32).repeat(2, 0), 1)
    assert e.value.index == 3
    with pytest.raises(O.OracleIndexError):
        O.scatter_add(src, O.F32, np.array([[0, -1]], np.int32).repeat(2, 0), np.ones((2, 2), np.float32), 1)
