"""Fusion lifecycle expectations of the reference's own tests, restated on
the GPU: fusion_async.phpt (concurrent runAsync executions, native plans
from a HIP graph), fusion_errors.phpt (misuse raises the reference's
exception classes and leaves eager work intact), fusion_lifetime.phpt
(bounded replays, views, a rejected replay that recovers), fusion_cache.phpt
(compiled-module cache keyed by source and layout, bounded, clearable) and
fusion_low_precision.phpt (fp16/bf16 fused results bitwise equal to eager,
float32 gradients).

Parts that exercise PHP-only machinery are left out and named where they
fall: element assignment through ArrayAccess, Fibers, device reset and the
16 MiB memory-pool INI limit behind the out-of-memory case."""
import gc

import pytest

from phptensors import CudaArray as A
from phptensors import Fusion as F
from phptensors import InvalidArgumentException, RuntimeException

pytestmark = pytest.mark.gpu


def test_async_executions_reference():
    """fusion_async.phpt:9-51"""
    a, b = A([1, 2, 3]), A([4, 5, 6])
    graph = F.compile(lambda x, y: (x * y + 1).sqrt(), [a, b])
    first = graph.runAsync(a, b)
    second = graph.runAsync(b, b)
    assert graph.getStats()["pending"] == 2
    assert isinstance(first.isFinished(), bool)
    expected_first = (a * b + 1).sqrt().toArray()
    expected_second = (b * b + 1).sqrt().toArray()
    del a, b
    gc.collect()
    result = first.wait()
    assert result.toArray() == expected_first
    assert first.wait() is result
    assert first.isFinished()
    assert second.wait().toArray() == expected_second
    assert graph.getStats()["pending"] == 0
    assert graph.getStats()["executions"] == 2
    a = A([2, 3, 4])
    pending = graph.runAsync(a, a)
    del graph, pending
    gc.collect()
    assert a.toArray() == [2.0, 3.0, 4.0]
    native = F.compile(lambda x: (x + 1).sum() * 2, [a], cudaGraph=True)
    stats = native.getStats()
    assert stats["backend"] == "cuda-graph"
    assert stats.get("incompatibility") in (None, "", "none")
    assert native.runAsync(a).wait().toArray() == [24.0]
    assert native.run(a).toArray() == [24.0]
    power = F.compile(lambda x: x.power(2) + 1, [a])
    assert power.runAsync(a).wait().toArray() == (a.power(2) + 1).toArray()


def test_errors_reference():
    """fusion_errors.phpt:9-36 (the in-place assignment and Fiber cases are
    PHP-only and left out)"""
    a = A([1, 2])
    with pytest.raises(RuntimeException):
        F.run(lambda: F.run(lambda: a + 1))
    with pytest.raises(RuntimeException):
        F.compile(lambda x: x.toArray(), [a])
    with pytest.raises(InvalidArgumentException):
        F.run(lambda: 123)
    with pytest.raises(InvalidArgumentException):
        F.run(lambda: a + A([1, 2, 3]))
    escaped = []

    def aborts():
        escaped.append(a * 2)
        raise LookupError("abort")

    with pytest.raises(LookupError):
        F.run(aborts)
    with pytest.raises(RuntimeException):
        escaped[0].toArray()
    graph = F.compile(lambda x: x * 2, [a])
    with pytest.raises(InvalidArgumentException):
        graph.run()
    with pytest.raises(InvalidArgumentException):
        graph.run(A([1, 2, 3]))
    with pytest.raises(InvalidArgumentException):
        graph.run(A([1, 2], "float64"))
    assert (a + 1).toArray() == [2.0, 3.0]
    assert F.run(lambda: a * 2).toArray() == [2.0, 4.0]


def test_lifetime_reference():
    """fusion_lifetime.phpt:11-56 (the out-of-memory case needs the
    reference's 16 MiB pool limit and is left out)"""
    a = A.ones([4096])

    def expression(x):
        for _ in range(130):
            x = x + 1
        return x

    stream = F.compile(expression, [a])
    graph = F.compile(expression, [a], cudaGraph=True)
    stream.run(a)
    graph.run(a)
    for _ in range(100):
        one = stream.runAsync(a)
        two = stream.runAsync(a)
        assert one.wait().select(0, 0).item() == 131.0
        assert two.wait().select(0, 0).item() == 131.0
        assert graph.run(a).select(0, 0).item() == 131.0
        del one, two
    assert stream.getStats()["pending"] == 0 and graph.getStats()["pending"] == 0
    for _ in range(25):
        view = F.run(lambda: (A([[1, 2], [3, 4]]) + 1).transpose())
        assert view.toArray() == [[2.0, 4.0], [3.0, 5.0]]
        del view
    matrix = A([[1, 2], [3, 4]])
    reduce = F.compile(lambda x: x.sum() * 2, [matrix.select(0, 1)])
    for _ in range(25):
        assert reduce.run(matrix.select(0, 1)).toArray() == [14.0]
    assert matrix.select(0, 1).reshape([1, 2]).toArray() == [[3.0, 4.0]]
    assert matrix.toArray() == [[1.0, 2.0], [3.0, 4.0]]
    with pytest.raises(InvalidArgumentException):
        graph.run(A.ones([8]))
    assert graph.run(a).select(0, 0).item() == 131.0


def test_cache_reference():
    """fusion_cache.phpt:9-37"""
    F.clearCache()
    a, b = A([[1, 2], [3, 4]]), A([[5, 6], [7, 8]])
    first = F.compile(lambda x: x * 2 + 1, [a])
    second = F.compile(lambda x: x * 2 + 1, [b])
    assert not first.getStats()["cacheHit"]
    assert second.getStats()["cacheHit"]
    assert F.getCacheStats()["compilations"] == 1
    layout = F.compile(lambda x: x * 2 + 1, [a.transpose()])
    assert not layout.getStats()["cacheHit"]
    before = F.getCacheStats()["compilations"]
    F.run(lambda: a * 2 + 1)
    F.run(lambda: b * 2 + 1)
    assert F.getCacheStats()["compilations"] == before
    for i in range(20):
        g = F.compile(lambda x: x + i, [a])
        assert g.run(a).toArray()[0][0] == 1.0 + i
    stats = F.getCacheStats()
    assert stats["entries"] <= stats["maxEntries"]
    assert stats["bytes"] <= stats["maxBytes"]
    assert stats["evictions"] > 0
    F.clearCache()
    assert first.run(b).toArray() == [[11.0, 13.0], [15.0, 17.0]]
    assert F.getCacheStats()["entries"] == 0


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_low_precision_reference(dtype):
    """fusion_low_precision.phpt:14-84"""
    x = A.fromFlatArray([0.5, 1.25, 2.0], [3], dtype)
    y = A.fromFlatArray([1.0, 0.25, 2.0], [3], dtype)
    eager = x.sin() * 2 + y
    fused = F.compile(lambda u, v: u.sin() * 2 + v, [x, y]).run(x, y)
    assert eager.getDtype() == dtype and fused.getDtype() == dtype
    assert fused.toBuffer() == eager.toBuffer()
    assert F.run(lambda: 2 - x).toBuffer() == (2 - x).toBuffer()
    column = A.fromFlatArray([1.0, 2.0], [2, 1], dtype)
    row = A.fromFlatArray([0.25, 0.5, 0.75], [1, 3], dtype)
    assert F.compile(lambda u, v: u + v, [column, row]).run(column, row).toBuffer() == (column + row).toBuffer()
    tracked = A.fromFlatArray([1.0, 2.0], [2], dtype).requiresGrad()
    (tracked * tracked).backward(A.fromFlatArray([1.0, 1.0], [2], dtype))
    assert tracked.grad().getDtype() == "float32" and tracked.grad().toArray() == [2.0, 4.0]
    fused_tracked = A.fromFlatArray([1.0, 2.0], [2], dtype).requiresGrad()
    seed = A.fromFlatArray([1.0, 1.0], [2], dtype)

    def product_body():
        product = fused_tracked * fused_tracked
        product.backward(seed)
        return [product, fused_tracked.grad()]

    product, gradient = F.run(product_body)
    assert product.getDtype() == dtype
    assert gradient.getDtype() == "float32" and gradient.toArray() == [2.0, 4.0]
    condition = A.fromFlatArray([True, False, True], [3], "bool")
    when_true = A.fromFlatArray([1.0, 2.0, 3.0], [3], dtype)
    when_false = A.fromFlatArray([4.0, 5.0, 6.0], [3], dtype)
    eager_where = A.where(condition, when_true, when_false)
    fused_where = F.compile(lambda m, u, v: A.where(m, u, v),
                            [condition, when_true, when_false]).run(condition, when_true, when_false)
    assert fused_where.getDtype() == dtype and fused_where.toBuffer() == eager_where.toBuffer()
    seed3 = A.ones([3], dtype)
    t_true = A.fromFlatArray([1.0, 2.0, 3.0], [3], dtype).requiresGrad()
    t_false = A.fromFlatArray([4.0, 5.0, 6.0], [3], dtype).requiresGrad()
    A.where(condition, t_true, t_false).backward(seed3)
    f_true = A.fromFlatArray([1.0, 2.0, 3.0], [3], dtype).requiresGrad()
    f_false = A.fromFlatArray([4.0, 5.0, 6.0], [3], dtype).requiresGrad()

    def where_body():
        out = A.where(condition, f_true, f_false)
        out.backward(seed3)
        return [out, f_true.grad(), f_false.grad()]

    _, g_true, g_false = F.run(where_body)
    assert g_true.toArray() == t_true.grad().toArray() and g_false.toArray() == t_false.grad().toArray()


def test_low_precision_where_condition():
    """fusion_low_precision.phpt:86-92: a float16 mask selects by nonzero."""
    mask = A.fromFlatArray([0, 1], [2], "float16")
    when_true, when_false = A([10.0, 20.0]), A([30.0, 40.0])
    where = A.where(mask, when_true, when_false)
    assert where.toArray() == [30.0, 20.0]
    assert F.run(lambda: A.where(mask, when_true, when_false)).toBuffer() == where.toBuffer()
