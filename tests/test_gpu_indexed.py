"""GPU parity of CudaArray::gather / scatterAdd (pt_gather, pt_scatter_add,
pt_index_validate; reference src/backends/cuda/indexed_ops.cu and
ca_private.c:885-1007): bit-exact against the oracle on random shapes,
axes, dtypes and strided views, and the reference's own expectations from
tests/cudaarray_extended.phpt:27-160 and tests/indexed_low_precision.phpt,
eager and inside Fusion plans (one synchronization per execution, no graph
capture, no async execution, validation errors raised after the run)."""
import numpy as np
import pytest

import oracle_lib as O
from phptensors import CudaArray, Fusion, InvalidArgumentException
from phptensors._abi import RuntimeException

pytestmark = pytest.mark.gpu

DT = {"float32": O.F32, "float64": O.F64, "int32": O.I32, "int64": O.I64, "uint8": O.U8, "int16": O.I16,
      "float16": O.F16, "bfloat16": O.BF16, "bool": O.BOOL}


def idx_array(values, shape):
    return CudaArray.fromFlatArray(list(values), list(shape), "int32")


@pytest.mark.parametrize("shape,axis,dtype", [((64, 96), 1, "float32"), ((64, 96), 0, "float64"),
                                              ((8, 16, 33), 2, "int32"), ((8, 16, 33), 1, "bfloat16"),
                                              ((5, 6, 7, 8), 0, "float16"), ((300,), 0, "int64"),
                                              ((40, 50), 1, "uint8"), ((3, 4096), 1, "int16")])
def test_gather_bit_exact_vs_oracle(shape, axis, dtype):
    r = np.random.default_rng(len(shape) * 7 + axis)
    code = DT[dtype]
    if dtype in ("float16", "bfloat16"):
        x = O.to_storage(r.standard_normal(shape).astype(np.float32), code)
    else:
        x = (r.standard_normal(shape) * 50).astype(O.NP_STORAGE[code])
    ishape = list(shape)
    ishape[axis] = 13
    idx = r.integers(0, shape[axis], ishape).astype(np.int32)
    got = CudaArray.fromNumpy(x, dtype).gather(CudaArray.fromNumpy(idx, "int32"), axis)
    assert got.getDtype() == dtype and got.getShape() == ishape
    assert got.toBits().tobytes() == O.gather(x, code, idx, axis).tobytes()


def test_gather_strided_views_and_negative_axis():
    r = np.random.default_rng(3)
    base = r.standard_normal((48, 40)).astype(np.float32)
    x = CudaArray.fromNumpy(base).transpose()            # [40, 48], strided
    ibase = r.integers(0, 48, (40, 6)).astype(np.int32)
    i_t = CudaArray.fromNumpy(np.ascontiguousarray(ibase.T), "int32").transpose()  # strided indices
    got = x.gather(i_t, -1).toNumpy()
    np.testing.assert_array_equal(got, O.gather(np.ascontiguousarray(base.T), O.F32, ibase, 1))


def test_scatter_add_vs_oracle_exact():
    # integer-valued updates make every order of the atomic adds exact
    r = np.random.default_rng(5)
    for dtype, code in (("float32", O.F32), ("float64", O.F64)):
        x = r.integers(-8, 9, (32, 24)).astype(O.NP_STORAGE[code])
        idx = r.integers(0, 24, (32, 50)).astype(np.int32)
        upd = r.integers(-4, 5, (32, 50)).astype(O.NP_STORAGE[code])
        got = CudaArray.fromNumpy(x, dtype).scatterAdd(CudaArray.fromNumpy(idx, "int32"),
                                                       CudaArray.fromNumpy(upd, dtype), 1)
        assert got.getDtype() == dtype
        np.testing.assert_array_equal(got.toNumpy(), O.scatter_add(x, code, idx, upd, 1))


def test_large_gather_bit_exact():
    # 64 Mi outputs gathered from a [8192, 2048] input: every 512th output row (and the last) checked
    r = np.random.default_rng(8)
    x = r.standard_normal((8192, 2048)).astype(np.float32)
    idx = r.integers(0, 2048, (8192, 8192)).astype(np.int32)
    got = CudaArray.fromNumpy(x).gather(CudaArray.fromNumpy(idx, "int32"), 1).toNumpy()
    rows = np.r_[0:8192:512, 8191]
    np.testing.assert_array_equal(got[rows], O.gather(x[rows], O.F32, idx[rows], 1))


def test_reference_eager_vectors_and_errors():
    """cudaarray_extended.phpt:27-31, 82-86 and its expected lines
    [[30,10],[50,50]] / [[2,0,1],[0,7,0]] / InvalidArgumentException x2."""
    source = CudaArray([[10.0, 20.0, 30.0], [40.0, 50.0, 60.0]])
    indices = idx_array([2, 0, 1, 1], [2, 2])
    assert source.gather(indices, 1).toArray() == [[30.0, 10.0], [50.0, 50.0]]
    base = CudaArray.zeros([2, 3])
    updates = CudaArray([[1.0, 2.0], [3.0, 4.0]])
    assert base.scatterAdd(indices, updates, 1).toArray() == [[2.0, 0.0, 1.0], [0.0, 7.0, 0.0]]
    # cudaarray_extended.phpt:82 passes [1, 2] indices (an error either way)
    with pytest.raises(InvalidArgumentException):
        source.gather(idx_array([3, 0], [1, 2]), 1)
    with pytest.raises(InvalidArgumentException, match=r"gather indices must be within \[0, 3\)"):
        source.gather(idx_array([3, 0, 1, 1], [2, 2]), 1)
    with pytest.raises(InvalidArgumentException):
        source.gather(indices, 3)
    with pytest.raises(InvalidArgumentException, match="int32 indices"):
        source.gather(CudaArray.fromFlatArray([1, 0], [1, 2], "int64"), 1)
    with pytest.raises(InvalidArgumentException, match="scatterAdd indices must be within"):
        base.scatterAdd(idx_array([0, -1, 1, 1], [2, 2]), updates, 1)


def test_reference_fusion_plans():
    """cudaarray_extended.phpt:44-105: gather / scatterAdd plans give the
    eager results with one synchronization per run, report asyncCompatible
    false and no graph capture, chain two gathers on one synchronization,
    raise the first invalid index after the run (and reset its status), and
    refuse runAsync with RuntimeException."""
    source = CudaArray([[10.0, 20.0, 30.0], [40.0, 50.0, 60.0]])
    indices = idx_array([2, 0, 1, 1], [2, 2])
    base = CudaArray.zeros([2, 3])
    updates = CudaArray([[1.0, 2.0], [3.0, 4.0]])
    gather_graph = Fusion.compile(lambda x, i: x.gather(i, 1), [source, indices])
    syncs = gather_graph.getStats()["synchronizations"]
    assert gather_graph.run(source, indices).toArray() == [[30.0, 10.0], [50.0, 50.0]]
    assert gather_graph.getStats()["synchronizations"] - syncs == 1
    scatter_graph = Fusion.compile(lambda x, i, u: x.scatterAdd(i, u, 1), [base, indices, updates])
    syncs = scatter_graph.getStats()["synchronizations"]
    assert scatter_graph.run(base, indices, updates).toArray() == [[2.0, 0.0, 1.0], [0.0, 7.0, 0.0]]
    assert scatter_graph.getStats()["synchronizations"] - syncs == 1
    assert gather_graph.getStats()["asyncCompatible"] in (0, False)
    assert not gather_graph.getStats()["cudaGraphCompatible"]
    assert not scatter_graph.getStats()["cudaGraphCompatible"]
    # fusion_plan.c:505-509 and fusion.c:747-754: an indexed plan is neither
    # stream- nor graph-compatible, so it reports the "native" backend, also
    # when a graph was requested
    for st in (gather_graph.getStats(), scatter_graph.getStats()):
        assert st["backend"] == "native"
        assert st["incompatibility"] == "indexed-operation"
        assert st["cudaGraphIncompatibility"] == "indexed-operation"
    requested = Fusion.compile(lambda x, i: x.gather(i, 1), [source, indices], cudaGraph=True)
    assert requested.run(source, indices).toArray() == [[30.0, 10.0], [50.0, 50.0]]
    assert requested.getStats()["backend"] == "native"
    assert requested.getStats()["cudaGraphRequested"] == 1
    transposed = source.transpose()
    tidx = idx_array([2, 0, 1, 2, 0, 1], [3, 2])
    tgraph = Fusion.compile(lambda x, i: x.gather(i, 0), [transposed, tidx])
    assert tgraph.run(transposed, tidx).toArray() == [[30.0, 40.0], [20.0, 60.0], [10.0, 50.0]]
    selector = idx_array([1, 0, 0, 1], [2, 2])
    chain = Fusion.compile(lambda x, i, j: x.gather(i, 1).gather(j, 1), [source, indices, selector])
    syncs = chain.getStats()["synchronizations"]
    assert chain.run(source, indices, selector).toArray() == [[10.0, 30.0], [50.0, 50.0]]
    assert chain.getStats()["synchronizations"] - syncs == 1
    bad = idx_array([3, 0, 1, 1], [2, 2])
    with pytest.raises(InvalidArgumentException, match=r"gather indices must be within \[0, 3\)"):
        gather_graph.run(source, bad)
    assert gather_graph.run(source, indices).toArray() == [[30.0, 10.0], [50.0, 50.0]]
    with pytest.raises(InvalidArgumentException, match=r"scatterAdd indices must be within \[0, 3\)"):
        scatter_graph.run(base, bad, updates)
    assert scatter_graph.run(base, indices, updates).toArray() == [[2.0, 0.0, 1.0], [0.0, 7.0, 0.0]]
    # fusion.c:565-569
    with pytest.raises(RuntimeException, match="runAsync requires a stream-compatible plan: indexed-operation"):
        gather_graph.runAsync(source, indices)
    with pytest.raises(RuntimeException, match="runAsync requires a stream-compatible plan: indexed-operation"):
        scatter_graph.runAsync(base, indices, updates)


def test_reference_gradients():
    """cudaarray_extended.phpt:106-160: gather and scatterAdd gradients,
    eager and recorded in Fusion, including a strided input."""
    g_idx = idx_array([2, 0], [1, 2])
    tracked = CudaArray([[1.0, 2.0, 3.0]]).requiresGrad()
    tracked.gather(g_idx, 1).sum().backward()
    assert tracked.grad().toArray() == [[1.0, 0.0, 1.0]]

    ftracked = CudaArray([[1.0, 2.0, 3.0]]).requiresGrad()

    def body(x, i):
        loss = x.gather(i, 1).sum()
        loss.backward()
        return [loss, x.grad()]
    _, grad = Fusion.compile(body, [ftracked, g_idx]).run(ftracked, g_idx)
    assert grad.toArray() == [[1.0, 0.0, 1.0]]

    s_idx = idx_array([2, 0, 1, 2], [2, 2])
    strided = CudaArray([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]).transpose().requiresGrad()
    strided.gather(s_idx, 0).sum().backward()
    assert strided.grad().toArray() == [[0.0, 1.0], [1.0, 0.0], [1.0, 1.0]]

    fstrided = CudaArray([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]).transpose().requiresGrad()

    def sbody(x, i):
        loss = x.gather(i, 0).sum()
        loss.backward()
        return [loss, x.grad()]
    _, sgrad = Fusion.compile(sbody, [fstrided, s_idx]).run(fstrided, s_idx)
    assert sgrad.toArray() == [[0.0, 1.0], [1.0, 0.0], [1.0, 1.0]]

    upd = CudaArray([[5.0, 6.0]]).requiresGrad()
    CudaArray.zeros([1, 3]).requiresGrad().scatterAdd(g_idx, upd, 1).sum().backward()
    assert upd.grad().toArray() == [[1.0, 1.0]]

    fbase = CudaArray.zeros([1, 3]).requiresGrad()
    fupd = CudaArray([[5.0, 6.0]]).requiresGrad()

    def ubody(x, i, u):
        loss = x.scatterAdd(i, u, 1).sum()
        loss.backward()
        return [loss, u.grad()]
    _, ugrad = Fusion.compile(ubody, [fbase, g_idx, fupd]).run(fbase, g_idx, fupd)
    assert ugrad.toArray() == [[1.0, 1.0]]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_reference_low_precision(dtype):
    """tests/indexed_low_precision.phpt: gather keeps the dtype (eager and
    Fusion, same bytes), gradients are float32, scatterAdd returns float32."""
    x = CudaArray.fromFlatArray([1.0, 2.0, 3.0], [3], dtype)
    i = idx_array([2, 0], [2])
    eager = x.gather(i)
    assert eager.getDtype() == dtype and eager.toArray() == [3.0, 1.0]
    fused = Fusion.compile(lambda a, b: a.gather(b), [x, i]).run(x, i)
    assert fused.getDtype() == dtype and fused.toBuffer() == eager.toBuffer()
    tracked = CudaArray.fromFlatArray([1.0, 2.0, 3.0], [3], dtype).requiresGrad()
    single = idx_array([2], [1])
    tracked.gather(single).backward()
    assert tracked.grad().getDtype() == "float32" and tracked.grad().toArray() == [0.0, 0.0, 1.0]
    sidx = idx_array([2, 0, 2], [3])
    scattered = CudaArray.zeros([3], dtype).scatterAdd(sidx, CudaArray.fromFlatArray([1.0, 2.0, 3.0], [3], dtype))
    assert scattered.getDtype() == "float32" and scattered.toArray() == [2.0, 0.0, 4.0]
    tb = CudaArray.zeros([3], dtype).requiresGrad()
    tu = CudaArray.fromFlatArray([1.0, 2.0, 3.0], [3], dtype).requiresGrad()
    tb.scatterAdd(sidx, tu).sum().backward()
    assert tb.grad().getDtype() == "float32" and tb.grad().toArray() == [1.0, 1.0, 1.0]
    assert tu.grad().getDtype() == "float32" and tu.grad().toArray() == [1.0, 1.0, 1.0]
