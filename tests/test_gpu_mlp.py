"""GPU parity of the config-5 path: reverse-mode gradients of the CudaArray
operations it uses, the functional AdamW step, and the whole MLP training
step (eager and recorded by Fusion.compile) against the float64 oracle
(oracle/mlp_ref.py)."""
import os
import sys

import numpy as np
import pytest

from phptensors import CudaArray, Fusion, InvalidArgumentException
from phptensors import mlp
from phptensors.optimizer import Optimizer

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import mlp_ref as R  # noqa: E402

pytestmark = pytest.mark.gpu


def f32(t):
    return t.toNumpy().astype(np.float64)


# ------------------------------------------------------------- autograd units
def test_square_sum_gradient_and_adamw_closed_form():
    # optimizer.phpt:44-63
    p = CudaArray.fromFlatArray([2.0], [1]).requiresGrad()
    opt = Optimizer.adamW(0.1, 0.9, 0.999, 1e-8, 0.1)
    state = opt.initState([p])
    opt.zeroGrad([p])
    (p * p).sum().backward()
    assert p.grad().toNumpy()[0] == 4.0
    step = opt.step([p], [p.grad()], state, None, [False])
    assert abs(step["parameters"][0].item() - 1.9) < 1e-5
    assert abs(step["state"]["firstMoment"][0].item() - 0.4) < 1e-6
    assert abs(step["state"]["secondMoment"][0].item() - 0.016) < 1e-7
    assert abs(step["state"]["beta1Power"].item() - 0.9) < 1e-7
    assert abs(step["state"]["beta2Power"].item() - 0.999) < 1e-7
    step = opt.step([p], [p.grad()], state, None, [True])
    assert abs(step["parameters"][0].item() - 1.88) < 1e-5
    assert p.item() == 2.0  # functional: the input parameter is unchanged


def test_sgd_closed_form():
    p = CudaArray.fromFlatArray([2.0], [1]).requiresGrad()
    sgd = Optimizer.sgd(0.1, 0.9)
    st = sgd.initState([p])
    (p * p).sum().backward()
    out = sgd.step([p], [p.grad()], st)
    assert abs(out["parameters"][0].item() - 1.6) < 1e-6
    assert out["state"]["velocity"][0].item() == 4.0


def test_optimizer_reference_remaining_cases():
    """optimizer.phpt:32-105: float64 state and update keep float64, a
    Fusion-compiled SGD step over a tracked parameter (backward inside the
    callback), a mismatched gradient shape and an invalid beta are refused."""
    sgd = Optimizer.sgd(0.1, 0.9)
    dp = CudaArray.fromFlatArray([2.0], [1], "float64").requiresGrad()
    dstate = sgd.initState([dp])
    assert dstate["velocity"][0].getDtype() == "float64"
    sgd.zeroGrad([dp])
    (dp * dp).sum().backward()
    dstep = sgd.step([dp], [dp.grad()], dstate)
    assert dstep["parameters"][0].getDtype() == "float64"
    fp = CudaArray.fromFlatArray([2.0], [1]).requiresGrad()
    fstate = sgd.initState([fp])
    rate = CudaArray.fromFlatArray([0.1], [1])

    def body(parameter, velocity, r):
        sgd.zeroGrad([parameter])
        (parameter * parameter).sum().backward()
        return sgd.step([parameter], [parameter.grad()], {"velocity": [velocity]}, r)

    graph = Fusion.compile(body, [fp, fstate["velocity"][0], rate])
    fstep = graph.run(fp, fstate["velocity"][0], rate)
    assert abs(fstep["parameters"][0].item() - 1.6) < 1e-5
    assert abs(fstep["state"]["velocity"][0].item() - 4.0) < 1e-5
    p = CudaArray.fromFlatArray([2.0], [1]).requiresGrad()
    with pytest.raises(InvalidArgumentException):
        sgd.step([p], [CudaArray.fromFlatArray([1.0, 2.0], [2])], sgd.initState([p]))
    with pytest.raises(InvalidArgumentException):
        Optimizer.adamW(0.1, 1.0)


@pytest.mark.parametrize("kind", ["adamW", "sgd"])
def test_nan_gradient_keeps_parameter_and_state(kind):
    """optimizer.c:424-469: where a gradient is NaN the parameter and its
    state keep their old values; infinite gradients still update."""
    opt = Optimizer.adamW(0.1, 0.9, 0.999, 1e-8, 0.1) if kind == "adamW" else Optimizer.sgd(0.1, 0.9, 0.01)
    p = CudaArray.fromFlatArray([1.0, 2.0, 3.0], [3])
    state = opt.initState([p])
    if kind == "adamW":
        state["firstMoment"] = [CudaArray.fromFlatArray([0.5, 0.5, 0.5], [3])]
    else:
        state["velocity"] = [CudaArray.fromFlatArray([0.5, 0.5, 0.5], [3])]
    g = CudaArray.fromFlatArray([float("nan"), 1.0, float("inf")], [3])
    out = opt.step([p], [g], state)
    newp = out["parameters"][0].toArray()
    assert newp[0] == 1.0 and newp[1] != 2.0
    if kind == "adamW":
        m = out["state"]["firstMoment"][0].toArray()
        assert m[0] == 0.5 and m[1] != 0.5 and m[2] == float("inf")
        assert out["state"]["secondMoment"][0].toArray()[0] == 0.0
    else:
        v = out["state"]["velocity"][0].toArray()
        assert v[0] == 0.5 and abs(v[1] - 1.45) < 1e-6 and v[2] == float("inf")
        # weight decay enters the step, not the velocity (optimizer.c:644-660)
        assert abs(newp[1] - (2.0 - 0.1 * (1.45 + 2.0 * 0.01))) < 1e-6


def test_max_gradient_shared_among_ties():
    x = CudaArray.fromNumpy(np.array([[1.0, 3.0, 3.0, 2.0], [5.0, 1.0, 0.0, 5.0]], np.float32)).requiresGrad()
    x.max(1).sum().backward()
    np.testing.assert_allclose(x.grad().toNumpy(), [[0, 0.5, 0.5, 0], [0.5, 0, 0, 0.5]])


def test_broadcast_matmul_where_exp_log_gradients():
    rng = np.random.default_rng(3)
    a = rng.uniform(-1, 1, (5, 4)).astype(np.float32)
    w = rng.uniform(-1, 1, (4, 3)).astype(np.float32)
    b = rng.uniform(-1, 1, (1, 3)).astype(np.float32)
    ta, tw, tb = (CudaArray.fromNumpy(v).requiresGrad() for v in (a, w, b))
    z = ta.matmul(tw) + tb
    h = CudaArray.where(z.gt(0), z, CudaArray.zeros([1]))
    loss = (h.exp() + 1.0).log().sum()
    loss.backward()
    # float64 reference of the same expression
    z64 = a.astype(np.float64) @ w + b
    hm = z64 > 0
    hh = np.where(hm, z64, 0.0)
    dh = np.exp(hh) / (np.exp(hh) + 1.0)
    dz = np.where(hm, dh, 0.0)
    np.testing.assert_allclose(f32(tw.grad()), a.T.astype(np.float64) @ dz, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(f32(tb.grad()), dz.sum(0, keepdims=True), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(f32(ta.grad()), dz @ w.T.astype(np.float64), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------- MLP step
def make(rows, layers, seed):
    params = mlp.init_parameters(layers, seed)
    x, y = mlp.synthetic_batch(rows, layers[0], layers[-1], seed)
    return params, CudaArray.fromNumpy(x), CudaArray.fromNumpy(y), x, y


def check_step(layers, rows, seed, params, out, x, y, grads_gpu=None):
    """Loss within 1e-5 relative.  Every entry of every gradient (recovered
    from the first moment, (1 - beta1) * clipped gradient after one step,
    within 3 u) against the north-star GEMM bar 1e-4 * sqrt(K) * (|A||B|)_ij
    of tests/mlp_bounds.py, plus the explicit allowance of the ReLU
    pre-activations within float32 rounding of zero; every updated
    parameter against the allowance that bar implies for the AdamW step.
    No entry is excused otherwise."""
    import mlp_bounds as MB
    p_np = [f32(p) for p in params]
    zeros = [np.zeros_like(p) for p in p_np]
    loss, grads, p2, m2, v2, b1p, b2p = R.train_step(x, y, p_np, zeros, zeros, 1.0, 1.0, 1e-3, mlp.DECAY_MASK)
    _, _, allow, flips1, flips2 = MB.grad_bounds(x, y, p_np)
    assert abs(out["loss"].item() - loss) <= 1e-5 * abs(loss)
    # clipping to +-5 (train_step's grads) is 1-Lipschitz: the allowances of
    # the unclipped gradients carry over
    pallow = MB.param_bounds(p_np, grads, allow)
    for i in range(6):
        g_gpu = f32(out["state"]["firstMoment"][i]) / 0.1
        err = np.abs(g_gpu - grads[i])
        lim = allow[i] + 3 * MB.U * np.abs(grads[i])
        assert np.all(err <= lim), (i, int((err > lim).sum()), float(np.max(err / np.maximum(lim, 1e-300))))
        got = f32(out["parameters"][i])
        err = np.abs(got - p2[i])
        assert np.all(err <= pallow[i]), (i, int((err > pallow[i]).sum()))
    assert abs(out["state"]["beta1Power"].item() - b1p) < 1e-7
    assert abs(out["state"]["beta2Power"].item() - b2p) < 1e-7
    return flips1, flips2


@pytest.mark.parametrize("layers,rows", [((32, 24, 16, 10), 64), ((784, 128, 64, 10), 256)])
def test_eager_training_step_vs_oracle(layers, rows):
    params, xt, yt, x, y = make(rows, layers, 7)
    opt = Optimizer.adamW()
    state = opt.initState(params)
    out = mlp.train_batch(xt, yt, params, opt, state, CudaArray.full([1], 1e-3))
    check_step(layers, rows, 7, params, out, x, y)


def test_compiled_training_step_matches_eager_and_replays():
    layers, rows = (64, 48, 32, 10), 128
    params, xt, yt, x, y = make(rows, layers, 9)
    opt = Optimizer.adamW()
    state = opt.initState(params)
    rate = CudaArray.full([1], 1e-3)
    eager = mlp.train_batch(xt, yt, params, opt, state, rate)
    inputs = mlp.training_inputs(xt, yt, rate, params, state)
    graph = mlp.compile_training_plan(inputs, opt)
    p1, s1, loss1 = mlp.unpack_step(graph.run(*inputs))
    np.testing.assert_allclose(loss1.toNumpy(), eager["loss"].toNumpy(), rtol=1e-6)
    for a, b in zip(p1, eager["parameters"]):
        np.testing.assert_allclose(a.toNumpy(), b.toNumpy(), rtol=1e-6, atol=1e-7)
    for a, b in zip(s1["secondMoment"], eager["state"]["secondMoment"]):
        np.testing.assert_allclose(a.toNumpy(), b.toNumpy(), rtol=1e-5, atol=1e-12)
    # several replays: the loss goes down and the plan is reused
    losses = [loss1.item()]
    params_, state_ = p1, s1
    for _ in range(4):
        p_, s_, l_ = mlp.unpack_step(graph.run(*mlp.training_inputs(xt, yt, rate, params_, state_)))
        params_, state_ = p_, s_
        losses.append(l_.item())
    assert losses[-1] < losses[0]
    st = graph.getStats()
    assert st["executions"] == 5
    # the first run sizes the natives' workspace eagerly; later runs capture
    # the whole plan (natives included) into a HIP graph
    assert st["cudaGraphCompatible"] == 1
    assert st["graphLaunches"] == 4
    kinds = [s["kind"] for s in graph.getPlan()]
    assert kinds.count("native") >= 9  # forward + backward GEMMs and reductions


def test_compiled_step_graph_replays_match_eager():
    """Replays of the captured step (natives inside the graph, scratch in
    the plan's workspace) give the eager step's results on every replay."""
    layers, rows = (784, 1024, 1024, 10), 512
    params, xt, yt, x, y = make(rows, layers, 11)
    opt = Optimizer.adamW()
    state = opt.initState(params)
    rate = CudaArray.full([1], 1e-3)
    eager = mlp.train_batch(xt, yt, params, opt, state, rate)
    inputs = mlp.training_inputs(xt, yt, rate, params, state)
    graph = mlp.compile_training_plan(inputs, opt)
    for rep in range(3):
        graph.replay(2, *inputs)
        p1, s1, loss1 = mlp.unpack_step(graph.run(*inputs))
        np.testing.assert_allclose(loss1.toNumpy(), eager["loss"].toNumpy(), rtol=1e-6)
        for a, b in zip(p1, eager["parameters"]):
            np.testing.assert_allclose(a.toNumpy(), b.toNumpy(), rtol=1e-6, atol=1e-7)
        for a, b in zip(s1["firstMoment"], eager["state"]["firstMoment"]):
            np.testing.assert_allclose(a.toNumpy(), b.toNumpy(), rtol=1e-5, atol=1e-10)
    assert graph.getStats()["graphLaunches"] >= 6


def test_config5_full_size_step():
    layers, rows = (784, 1024, 1024, 10), 4096
    params, xt, yt, x, y = make(rows, layers, 5)
    opt = Optimizer.adamW()
    state = opt.initState(params)
    out = mlp.train_batch(xt, yt, params, opt, state, CudaArray.full([1], 1e-3))
    check_step(layers, rows, 5, params, out, x, y)


def test_config5_compiled_plan_full_size_vs_oracle():
    """The step bench.py times (config 5): mlp.compile_training_plan at batch
    4096, 784-1024-1024-10, replayed from its HIP graph (natives inside,
    three branches), checked against the float64 oracle like the eager step
    (examples/08_gpu_classifier.php:117-161), and bitwise against the eager
    step on the same inputs."""
    layers, rows = (784, 1024, 1024, 10), 4096
    params, xt, yt, x, y = make(rows, layers, 5)
    opt = Optimizer.adamW()
    state = opt.initState(params)
    rate = CudaArray.full([1], 1e-3)
    inputs = mlp.training_inputs(xt, yt, rate, params, state)
    graph = mlp.compile_training_plan(inputs, opt)
    graph.replay(2, *inputs)
    p1, s1, loss1 = mlp.unpack_step(graph.run(*inputs))
    stats = graph.getStats()
    assert stats["graphLaunches"] >= 2
    # the loss chain's [4096, 10] steps run as row chains
    assert stats["rowChains"] >= 1 and stats["rowChainSteps"] >= 8 and stats["rowChainFallbacks"] == 0
    # the plan's scratch arena holds every native's scratch side by side (a
    # region is not reused within a replay): split-K partials of dW2 (8 x
    # 1024 x 1024 fp32, 33.5 MB), dW1 (9 x 784 x 1024, 28.9 MB) and dW3
    # (1.3 MB) plus the column-reduction partials of the bias gradients
    assert 0 < stats["workspaceBytes"] <= 80 << 20
    out = {"loss": loss1, "parameters": p1, "state": s1}
    check_step(layers, rows, 5, params, out, x, y)
    eager = mlp.train_batch(xt, yt, params, opt, state, rate)
    assert loss1.toBits().tobytes() == eager["loss"].toBits().tobytes()
    for a, b in zip(p1, eager["parameters"]):
        assert a.toBits().tobytes() == b.toBits().tobytes()
    for key in ("firstMoment", "secondMoment"):
        for a, b in zip(s1[key], eager["state"][key]):
            assert a.toBits().tobytes() == b.toBits().tobytes()


def test_training_plan_groups_adamw_updates_like_the_reference():
    """tests/classifier_training.phpt:41-49: the training plan of a
    784-512-256-10 model keeps one fused dependent-output group per
    parameter (six) and at most 24 fused kernels."""
    layers = (784, 512, 256, 10)
    params, xt, yt, x, y = make(128, layers, 3)
    opt = Optimizer.adamW()
    inputs = mlp.training_inputs(xt, yt, CudaArray.full([1], 1e-3), params, opt.initState(params))
    graph = mlp.compile_training_plan(inputs, opt)
    plan = graph.getPlan()
    groups = [s for s in plan if s["reason"] == "dependent-outputs"]
    assert len(groups) == 6
    assert graph.getStats()["fusedKernels"] <= 24
    assert all(s["outputs"] <= 4 for s in plan)


# ------------------------------------------- AdamW under Fusion (reference)
def _adamw_inputs(parameters, gradients, state, rate):
    return [rate, state["beta1Power"], state["beta2Power"], *parameters, *gradients,
            *state["firstMoment"], *state["secondMoment"]]


def _adamw_tensors(result):
    st = result["state"]
    return [*result["parameters"], *st["firstMoment"], *st["secondMoment"], st["beta1Power"], st["beta2Power"]]


@pytest.mark.parametrize("dtype,tol", [("float32", 1e-6), ("float64", 1e-12)])
@pytest.mark.parametrize("cuda_graph", [False, True])
def test_adamw_fusion_outputs_reference(dtype, tol, cuda_graph):
    """tests/optimizer_fusion_outputs.phpt:33-115 restated: clipped AdamW
    recorded by Fusion.compile groups each weight with its two moments,
    matches the eager step over twelve replays (variable and zero rates,
    signed clipping boundaries, a strided gradient), keeps earlier outputs
    and inputs intact, replays asynchronously, rejects a changed gradient
    shape, and propagates NaN / clips infinities as the eager step does."""
    from phptensors._abi import InvalidArgumentException
    opt = Optimizer.adamW(0.001, 0.8, 0.95, 1e-6, 0.02)
    params = [CudaArray.full([4, 8], 0.25, dtype), CudaArray.full([1, 8], -0.5, dtype)]
    initial_bytes = [p.toBuffer() for p in params]
    state = opt.initState(params)
    ref_params, ref_state = params, state
    values = [-8.0, -5.0, -4.99, -0.0, 1e-7, 4.99, 5.0, 8.0]
    grads = [CudaArray.fromFlatArray(values * 4, [8, 4], dtype).transpose(),
             CudaArray.fromFlatArray(values, [1, 8], dtype)]
    rate = CudaArray.full([1], 0.001, dtype)

    def body(rate, b1p, b2p, *tensors):
        p, g, m, v = tensors[0:2], list(tensors[2:4]), tensors[4:6], tensors[6:8]
        for i, gr in enumerate(g):
            gr = CudaArray.where(gr.gt(5.0), CudaArray.full([1], 5.0, gr.getDtype()), gr)
            g[i] = CudaArray.where(gr.lt(-5.0), CudaArray.full([1], -5.0, gr.getDtype()), gr)
        return opt.step(list(p), g, {"firstMoment": list(m), "secondMoment": list(v),
                                     "beta1Power": b1p, "beta2Power": b2p}, rate, [True, False])

    graph = Fusion.compile(body, _adamw_inputs(params, grads, state, rate), cudaGraph=cuda_graph)
    grouped = [s for s in graph.getPlan() if s["kind"] == "fused" and s["outputs"] >= 3]
    assert len(grouped) >= 2 and graph.getStats()["fusedKernels"] <= 12

    def check(actual, expected):
        for i, (a, e) in enumerate(zip(_adamw_tensors(actual), _adamw_tensors(expected))):
            d = (a - e).abs().max().item()
            assert np.isfinite(d) and d <= tol, (i, d)

    saved = saved_bytes = None
    for step in range(12):
        rate = CudaArray.full([1], 0.0 if step == 3 else 0.002 / (step + 1), dtype)
        sign = -1.0 if step % 2 else 1.0
        signed = [(grads[0].transpose() * sign).transpose(), grads[1] * sign]
        expected = body(*_adamw_inputs(ref_params, signed, ref_state, rate))
        actual = graph.run(*_adamw_inputs(params, signed, state, rate))
        check(actual, expected)
        if step == 0:
            saved = actual
            saved_bytes = [t.toBuffer() for t in _adamw_tensors(actual)]
        params, state = actual["parameters"], actual["state"]
        ref_params, ref_state = expected["parameters"], expected["state"]
    assert [t.toBuffer() for t in _adamw_tensors(saved)] == saved_bytes
    assert [p.toBuffer() for p in ref_params] != initial_bytes
    pending = graph.runAsync(*_adamw_inputs(params, grads, state, rate))
    expected = body(*_adamw_inputs(params, grads, state, rate))
    check(pending.wait(), expected)
    with pytest.raises(InvalidArgumentException):
        graph.run(*_adamw_inputs(params, [CudaArray.zeros([1], dtype), grads[1]], state, rate))
    check(graph.run(*_adamw_inputs(params, grads, state, rate)), expected)
    special = [float("nan"), float("inf"), float("-inf"), -5.0, 5.0, 0.0, 1.0, -1.0]
    nonfinite = [CudaArray.fromFlatArray(special * 4, [8, 4], dtype).transpose(),
                 CudaArray.fromFlatArray(special, [1, 8], dtype)]
    expected = body(*_adamw_inputs(params, nonfinite, state, rate))
    actual = graph.run(*_adamw_inputs(params, nonfinite, state, rate))
    for a, e in zip(_adamw_tensors(actual), _adamw_tensors(expected)):
        av, ev = a.toNumpy().ravel(), e.toNumpy().ravel()
        assert np.array_equal(np.isnan(av), np.isnan(ev))
        fin = np.isfinite(ev)
        assert np.array_equal(av[np.isinf(ev)], ev[np.isinf(ev)])
        assert np.all(np.abs(av[fin] - ev[fin]) <= tol)
