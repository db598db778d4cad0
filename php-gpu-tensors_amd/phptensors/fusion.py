"""Fusion, FusionGraph and FusionExecution (stubs/cuda.stub.php:55-93).

Fusion.run(callback) records the callback's CudaArray operations into a DAG
and executes the fused plan once (src/fusion.c:250-310); Fusion.compile
records once against example inputs and returns a FusionGraph that replays
the plan, optionally from a captured HIP graph (src/fusion.c:312-418,
599-692).  All recording, planning, code generation (hipRTC for gfx950) and
execution happen in the host runtime; this module only carries handles and
the callback's result structure.
"""
import ctypes

from . import _host
from . import autograd as AG
from .cuda_array import CudaArray
from ._abi import InvalidArgumentException, RuntimeException  # noqa: F401


def _flatten(result):
    """Tensors of a callback result, in order, and a rebuild function.  The
    result is a CudaArray or a (nested) list, tuple or dict of them, as the
    reference's output arrays may nest (fusion_boundaries.phpt:22-26)."""
    if isinstance(result, CudaArray):
        return [result], lambda ts: ts[0]
    if isinstance(result, (list, tuple, dict)):
        items = list(result.items()) if isinstance(result, dict) else list(enumerate(result))
        if not items and not isinstance(result, dict):
            return [], lambda ts: type(result)()
        parts = []
        tensors = []
        for key, value in items:
            sub, rebuild = _flatten(value)
            parts.append((key, len(sub), rebuild))
            tensors.extend(sub)

        def rebuild_all(ts):
            pos, out = 0, []
            for key, count, rb in parts:
                out.append((key, rb(ts[pos:pos + count])))
                pos += count
            if isinstance(result, dict):
                return dict(out)
            return type(result)(v for _, v in out)

        return tensors, rebuild_all
    raise InvalidArgumentException("Fusion callbacks must return a CudaArray or an array of CudaArray")


def _handles(tensors):
    arr = (ctypes.c_void_p * max(1, len(tensors)))()
    for i, t in enumerate(tensors):
        arr[i] = t._h
    return arr


class Fusion:
    """Scoped elementwise fusion; eager operators remain the default."""

    @staticmethod
    def run(callback, enabled=True):
        if not enabled:
            return callback()
        lib = _host.load()
        if lib.phpt_fusion_begin(0) != 0:
            _host.raise_error("Fusion::run")
        try:
            result = callback()
        except BaseException:
            lib.phpt_fusion_abort()
            raise
        try:
            outs, _ = _flatten(result) if result is not None else ([], None)
        except BaseException:
            lib.phpt_fusion_abort()
            raise
        if lib.phpt_fusion_run_once(_handles(outs), len(outs)) != 0:
            _host.raise_error("Fusion::run")
        return result

    @staticmethod
    def compile(callback, inputs, cudaGraph=False):
        lib = _host.load()
        inputs = list(inputs)
        for t in inputs:
            if not isinstance(t, CudaArray):
                raise InvalidArgumentException("Fusion::compile inputs must be CudaArray values")
        if lib.phpt_fusion_begin(1) != 0:
            _host.raise_error("Fusion::compile")
        tracked = [bool(t._rg) for t in inputs]
        try:
            placeholders = [CudaArray._wrap(lib.phpt_fusion_input(t._h, i)) for i, t in enumerate(inputs)]
            # placeholders keep the examples' requiresGrad (fusion.c:357)
            for ph, rg in zip(placeholders, tracked):
                ph._rg = rg
            result = callback(*placeholders)
            outs, rebuild = _flatten(result)
            # a tracked output must have run backward() inside the callback
            # (fusion.c:376-387)
            if any(AG.needs_grad(t) for t in outs):
                raise InvalidArgumentException(
                    "Fusion::compile() cannot detach tracked outputs implicitly; call backward() inside "
                    "the callback or detach() the output explicitly")
        except BaseException:
            lib.phpt_fusion_abort()
            raise
        g = lib.phpt_fusion_end(_handles(outs), len(outs), 1 if cudaGraph else 0)
        if not g:
            _host.raise_error("Fusion::compile")
        graph = FusionGraph(g, rebuild, len(inputs))
        graph._tracked = tracked
        return graph

    @staticmethod
    def getCacheStats():
        return _host.parse_kv(_host.load().phpt_fusion_cache_stats())

    @staticmethod
    def clearCache():
        _host.load().phpt_fusion_clear_cache()


class FusionGraph:
    """Plan specialised for the example inputs' shapes, dtypes and strides."""

    def __init__(self, handle, rebuild, ninputs):
        self._g = handle
        self._rebuild = rebuild
        self._ninputs = ninputs
        self._tracked = [False] * ninputs

    def _check_tracking(self, inputs):
        """An input may not enable gradients its example lacked at capture
        (fusion.c:479-486)."""
        for i, (t, rg) in enumerate(zip(inputs, self._tracked)):
            if isinstance(t, CudaArray) and t._rg and not rg:
                raise InvalidArgumentException(
                    f"FusionGraph input {i} enables gradients absent from capture; enable requiresGrad() "
                    "before compile and capture backward(), or detach() the input")

    def __del__(self):
        g = getattr(self, "_g", None)
        if g and _host._lib is not None:
            _host._lib.phpt_graph_release(g)
            self._g = None

    def _outputs(self, count):
        return (ctypes.c_void_p * max(1, count))()

    def run(self, *inputs):
        self._check_tracking(inputs)
        lib = _host.load()
        n = lib.phpt_graph_num_outputs(self._g)
        outs = self._outputs(n)
        if lib.phpt_graph_run(self._g, _handles(inputs), len(inputs), outs, n) < 0:
            _host.raise_error("FusionGraph::run")
        return self._rebuild([CudaArray._wrap(outs[i]) for i in range(n)])

    def replay(self, count, *inputs):
        """Replay `count` times back to back, synchronize once and return the
        last execution's outputs as run() does (throughput measurement; not
        part of the reference API).  Each execution drops the one before it,
        so all reuse the plan's buffers."""
        lib = _host.load()
        n = lib.phpt_graph_num_outputs(self._g)
        outs = self._outputs(n)
        if lib.phpt_graph_replay(self._g, _handles(inputs), len(inputs), int(count), outs, n) < 0:
            _host.raise_error("FusionGraph::replay")
        return self._rebuild([CudaArray._wrap(outs[i]) for i in range(n)])

    def runAsync(self, *inputs):
        self._check_tracking(inputs)
        lib = _host.load()
        e = lib.phpt_graph_run_async(self._g, _handles(inputs), len(inputs))
        if not e:
            _host.raise_error("FusionGraph::runAsync")
        return FusionExecution(self, e)

    def getStats(self):
        return _host.parse_kv(_host.load().phpt_graph_stats(self._g))

    def getSource(self):
        return _host.load().phpt_graph_source(self._g).decode()

    def getPlan(self):
        """One dict per step (fusion.c:775-795): step, root, kind ('fused' or
        'native'), reason, inputs, outputs; fused steps also name their
        kernel and its variant (vector / scalar)."""
        steps = []
        for part in _host.load().phpt_graph_plan(self._g).decode().split(";"):
            if not part:
                continue
            entry = {}
            for kv in part.split(","):
                k, _, v = kv.partition("=")
                entry[k] = int(v) if k in ("step", "root", "inputs", "outputs") else v
            steps.append(entry)
        return steps

    def setProfiling(self, enabled):
        if _host.load().phpt_graph_set_profiling(self._g, 1 if enabled else 0) != 0:
            _host.raise_error("FusionGraph::setProfiling")


class FusionExecution:
    """One submitted runAsync; wait() synchronises on it and returns its
    outputs (fusion.c:561-692).  The graph stays alive while it is held."""

    def __init__(self, graph, handle):
        self._graph = graph
        self._e = handle
        self._result = None

    def wait(self):
        if self._result is None:
            lib = _host.load()
            n = lib.phpt_graph_num_outputs(self._graph._g)
            outs = self._graph._outputs(n)
            if lib.phpt_execution_wait(self._e, outs, n) < 0:
                _host.raise_error("FusionExecution::wait")
            self._result = self._graph._rebuild([CudaArray._wrap(outs[i]) for i in range(n)])
        return self._result

    def isFinished(self):
        if self._result is not None:
            return True
        rc = _host.load().phpt_execution_is_finished(self._e)
        if rc < 0:
            _host.raise_error("FusionExecution::isFinished")
        return rc == 1

    def __del__(self):
        try:
            if self._e and _host._lib is not None:
                _host._lib.phpt_execution_release(self._e)
                self._e = None
        except Exception:
            pass
