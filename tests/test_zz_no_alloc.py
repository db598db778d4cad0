"""pt_reduce_noalloc (no counterpart in the reference; for callers that
cannot allocate): through the C-ABI it must give pt_reduce's results bit for
bit -- same kernels, scratch from the library's static per-device buffer --
on two calls in a row, the second with a smaller input, on calls that
alternate between two streams with no synchronization between them (each
call's stream waits for the previous call's kernels, so they do not race on
the shared buffer), and refuse a reduction whose scratch exceeds the static
buffer with a clear error."""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
from phptensors import _abi as A
from phptensors import synthetic

pytestmark = pytest.mark.gpu


def _run(fn, x, op, axis, shape=None, strides=None):
    lib = A.load()
    shape = list(x.shape) if shape is None else shape
    strides = [int(s // x.itemsize) for s in x.strides] if strides is None else strides
    nout = 1 if axis < 0 else int(np.prod([e for d, e in enumerate(shape) if d != axis]))
    rdt = lib.pt_reduce_result_dtype(O.F32, A.OP[op])
    dev = A.to_device(x)
    out = A.DeviceBuffer(max(1, nout) * 8)
    st = fn(dev.ptr, out.ptr, O.F32, A.OP[op], A.ints(shape), A.sizes(strides), len(shape), axis, 0, None)
    A.synchronize()
    if st != 0:
        return st, None
    return st, out.download(np.float64 if rdt == O.F64 else np.float32, (max(1, nout),))


@pytest.mark.parametrize("op", ["sum", "max", "mean"])
def test_noalloc_matches_pt_reduce_twice(op):
    lib = A.load()
    A.check(lib.pt_init(), "init")
    for shape, axis, seed in (((4096, 2048), -1, 1), ((333, 77), -1, 2), ((4096, 1024), 0, 3), ((50, 130), 0, 4),
                              ((512, 4096), 1, 5), ((7, 9), 1, 6)):
        x = synthetic.normal(shape, 0.0, 1.0, seed=seed)
        st0, ref = _run(lib.pt_reduce, x, op, axis)
        st1, got = _run(lib.pt_reduce_noalloc, x, op, axis)
        assert st0 == 0 and st1 == 0, A.last_error()
        assert got.tobytes() == ref.tobytes(), (shape, axis, op)


def test_noalloc_calls_on_two_streams_do_not_race():
    """Eight global sums and column sums (both take scratch: partials of the
    two-level global pass, row-slice partials of the column split) issued
    alternately on two streams without waiting in between; every result
    equals pt_reduce's bit for bit."""
    lib = A.load()
    A.check(lib.pt_init(), "init")
    streams = [ctypes.c_void_p(), ctypes.c_void_p()]
    for s in streams:
        A.check(lib.pt_stream_create(ctypes.byref(s)), "stream")
    cases = []
    for i in range(8):
        shape, axis = (((4096, 2048), -1) if i % 2 == 0 else ((4096, 1024), 0))
        x = synthetic.normal(shape, 0.0, 1.0, seed=100 + i)
        nout = 1 if axis < 0 else shape[1]
        dev = A.to_device(x)
        out = A.DeviceBuffer(nout * 4)
        cases.append((x, shape, axis, nout, dev, out))
    A.synchronize()
    try:
        for i, (x, shape, axis, nout, dev, out) in enumerate(cases):
            st = lib.pt_reduce_noalloc(dev.ptr, out.ptr, O.F32, A.OP["sum"], A.ints(list(shape)),
                                       A.sizes([shape[1], 1]), 2, axis, 0, streams[i % 2])
            assert st == 0, A.last_error()
        for s in streams:
            A.check(lib.pt_stream_synchronize(s), "stream sync")
        for x, shape, axis, nout, dev, out in cases:
            st0, ref = _run(lib.pt_reduce, x, "sum", axis)
            assert st0 == 0
            assert out.download(np.float32, (nout,)).tobytes() == ref.tobytes(), (shape, axis)
    finally:
        for s in streams:
            lib.pt_stream_destroy(s)


def test_noalloc_refuses_scratch_beyond_the_static_buffer():
    lib = A.load()
    # a column sum of [4096, 16384] splits its 4096 rows into 32 slices whose
    # float32 partials take 32 * 16384 * 4 = 2 MiB: more than the 1 MiB
    # static buffer holds
    big = np.ones((4096, 16384), np.float32)
    st, _ = _run(lib.pt_reduce_noalloc, big, "sum", 0)
    assert st == 1
    assert b"static scratch" in lib.pt_last_error()
    st0, ref = _run(lib.pt_reduce, big, "sum", 0)
    assert st0 == 0 and np.all(ref == 4096.0)
    # and the library keeps working afterwards
    x = synthetic.normal((1024, 1024), 0.0, 1.0, seed=9)
    st0, ref = _run(lib.pt_reduce, x, "sum", -1)
    st1, got = _run(lib.pt_reduce_noalloc, x, "sum", -1)
    assert st0 == 0 and st1 == 0 and got.tobytes() == ref.tobytes()
