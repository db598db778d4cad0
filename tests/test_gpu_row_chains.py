"""Row chains of compiled Fusion plans (host/fusion.cpp): a run of plan steps
that each work row by row on short rows -- fused elementwise steps whose
reads of the run's own values stay inside the output row, and native
last-axis float32 reductions -- executed by one generated kernel with a wave
per row.  The chained plan must give the eager kernels' results bit for bit
(the same node functions; each reduction in the native row kernel's order),
report the same getPlan and getSource as the same graph run step by step
(PT_FUSION_ROW_CHAINS=0, in a child process), and leave steps that read a
chained value across rows out of the chain."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from phptensors import CudaArray, Fusion

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def loss_rows(s, lab):
    """Softmax cross-entropy per row with the pieces its backward reads:
    row max, shifted scores, exp, row sums, log, target, mean and min."""
    rows = s.getShape()[0]
    m = s.max(1).reshape([rows, 1])
    sh = s - m
    e = sh.exp()
    z = e.sum(1).reshape([rows, 1])
    p = e / z
    t = (sh * lab).sum(1).reshape([rows, 1])
    per_row = z.log() - t
    hit = s.eq(m)
    share = hit / hit.sum(1).reshape([rows, 1])
    return [p, per_row, p.mean(1), sh.min(1), share, (e * 0.5 + 1.0).prod(1)]


def scores(rows, cols, seed, ties=False, nan_row=None):
    rng = np.random.default_rng(seed)
    s = rng.normal(0.0, 3.0, (rows, cols)).astype(np.float32)
    if ties:
        s[::3, : min(3, cols)] = 9.0  # several maxima per row
    if nan_row is not None:
        s[nan_row, cols // 2] = np.nan
    lab = np.zeros((rows, cols), np.float32)
    lab[np.arange(rows), rng.integers(0, cols, rows)] = 1.0
    return s, lab


def assert_bitwise(got, want):
    """Bit for bit, except that a NaN matches any NaN: the compiler may give
    a NaN either sign (an a - b may become a + (-b)), in any kernel."""
    assert len(got) == len(want)
    for g, w in zip(got, want):
        assert g.getShape() == w.getShape()
        gv, wv = g.toNumpy(), w.toNumpy()
        gn, wn = np.isnan(gv), np.isnan(wv)
        np.testing.assert_array_equal(gn, wn)
        assert gv[~gn].tobytes() == wv[~wn].tobytes()


@pytest.mark.parametrize("rows,cols", [(4096, 10), (4096, 12), (333, 64), (64, 100), (130, 256), (2, 1)])
def test_chained_loss_rows_match_eager_bitwise(rows, cols):
    s, lab = scores(rows, cols, rows + cols, ties=True, nan_row=1)
    st, lt = CudaArray.fromNumpy(s), CudaArray.fromNumpy(lab)
    graph = Fusion.compile(loss_rows, [st, lt])
    stats = graph.getStats()
    assert stats["rowChains"] >= 1 and stats["rowChainSteps"] >= 6
    for _ in range(2):  # the eager measuring run, then the captured graph
        assert_bitwise(graph.run(st, lt), loss_rows(st, lt))
    assert graph.getStats()["rowChainFallbacks"] == 0
    # rebinding: other values of the same shapes
    s2, lab2 = scores(rows, cols, 7 * rows + cols)
    s2t, l2t = CudaArray.fromNumpy(s2), CudaArray.fromNumpy(lab2)
    assert_bitwise(graph.run(s2t, l2t), loss_rows(s2t, l2t))


def test_rows_longer_than_a_chain_takes_run_step_by_step():
    s, lab = scores(64, 300, 3)
    st, lt = CudaArray.fromNumpy(s), CudaArray.fromNumpy(lab)
    graph = Fusion.compile(loss_rows, [st, lt])
    assert graph.getStats()["rowChains"] == 0
    assert_bitwise(graph.run(st, lt), loss_rows(st, lt))


def across_rows(s):
    """w = row sums; v reads w along its columns too (w[j] at (i, j)), so
    the kernel of u and v cannot join the chain that produces w."""
    rows = s.getShape()[0]
    w = (s * 2.0).sum(1)
    u = s - w.reshape([rows, 1])
    v = u + w.reshape([1, rows])
    return [u.max(1), v, v.sum(1)]


def test_values_read_across_rows_stay_out_of_the_chain():
    s = np.random.default_rng(4).normal(0.0, 1.0, (96, 96)).astype(np.float32)
    st = CudaArray.fromNumpy(s)
    graph = Fusion.compile(across_rows, [st])
    for _ in range(2):
        assert_bitwise(graph.run(st), across_rows(st))
    # the kernel of u and v reads w across rows: the steps up to w form one
    # chain, and that kernel starts another one, after w is complete
    stats = graph.getStats()
    assert (stats["rowChains"], stats["rowChainSteps"]) == (2, 5)


_CHILD = r"""
import json, os, sys
import numpy as np
sys.path[:0] = [sys.argv[1], os.path.join(os.path.dirname(sys.argv[1]), "php-gpu-tensors_amd")]
import test_gpu_row_chains as T
from phptensors import CudaArray, Fusion
s, lab = T.scores(4096, 10, 11, ties=True)
st, lt = CudaArray.fromNumpy(s), CudaArray.fromNumpy(lab)
g = Fusion.compile(T.loss_rows, [st, lt])
outs = g.run(st, lt)
outs = g.run(st, lt)
print(json.dumps({"plan": g.getPlan(), "source": g.getSource(), "stats": g.getStats(),
                  "bits": [o.toBits().tobytes().hex() for o in outs]}))
"""


def _child(chains):
    env = dict(os.environ, PT_FUSION_ROW_CHAINS="1" if chains else "0")
    proc = subprocess.run([sys.executable, "-c", _CHILD, HERE], capture_output=True, text=True, timeout=300,
                          env=env, cwd=os.path.dirname(HERE))
    assert proc.returncode == 0, proc.stderr[-2000:]
    return json.loads(proc.stdout.strip().splitlines()[-1])


def test_chains_leave_plan_and_source_unchanged():
    on, off = _child(True), _child(False)
    assert on["stats"]["rowChains"] >= 1 and off["stats"]["rowChains"] == 0
    assert on["plan"] == off["plan"]
    assert on["source"] == off["source"]
    assert on["bits"] == off["bits"]
    for key in ("fusedKernels", "boundaries", "executionSteps", "intermediateBuffers", "graphLaunches"):
        assert on["stats"][key] == off["stats"][key], key
