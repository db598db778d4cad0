"""Pinning of the MLP training-step oracle (oracle/mlp_ref.py): analytic
gradients against central finite differences, AdamW against the closed-form
values of the reference's optimizer.phpt, and the loss against its closed
form."""
import math
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import mlp_ref as R  # noqa: E402


def tiny(seed=0):
    rng = np.random.default_rng(seed)
    layers = (6, 5, 4, 3)
    params = []
    for a, b in zip(layers[:-1], layers[1:]):
        params.append(rng.uniform(-1, 1, (a, b)))
        params.append(rng.uniform(-0.2, 0.2, (1, b)))
    x = rng.uniform(-1, 1, (7, 6))
    y = np.zeros((7, 3))
    y[np.arange(7), rng.integers(0, 3, 7)] = 1.0
    return x, y, params


def test_gradients_match_finite_differences():
    x, y, params = tiny()
    scale = 1.0 / x.shape[0]
    _, grads = R.loss_and_grads(x, y, params, scale)
    h = 1e-6
    for pi, p in enumerate(params):
        num = np.zeros_like(p)
        for idx in np.ndindex(p.shape):
            old = p[idx]
            p[idx] = old + h
            lp = R.cross_entropy(R.predict(x, params)[0], y)
            p[idx] = old - h
            lm = R.cross_entropy(R.predict(x, params)[0], y)
            p[idx] = old
            num[idx] = (lp - lm) / (2 * h) * scale
        assert np.allclose(grads[pi], num, rtol=1e-5, atol=1e-8), pi


def test_max_shift_gradient_sums_to_zero_per_row():
    # the max term cancels when labels are one-hot: d_scores equals softmax - labels
    x, y, params = tiny(1)
    scores, _ = R.predict(x, params)
    e = np.exp(scores - scores.max(1, keepdims=True))
    p = e / e.sum(1, keepdims=True)
    _, grads = R.loss_and_grads(x, y, params, 1.0)
    h2 = R.predict(x, params)[1][3]
    assert np.allclose(grads[4], h2.T @ (p - y), rtol=1e-12, atol=1e-12)


def test_adamw_closed_form():
    # optimizer.phpt:44-63: p = 2, gradient of p^2 = 4, lr 0.1, wd 0.1
    p = [np.array([2.0])]
    g = [np.array([4.0])]
    z = [np.zeros(1)]
    out_p, m, v, b1p, b2p = R.adamw(p, g, z, z, 1.0, 1.0, 0.1, weight_decay=0.1, mask=[False])
    assert abs(out_p[0][0] - 1.9) < 1e-8  # eps = 1e-8 in the denominator
    assert abs(m[0][0] - 0.4) < 1e-12 and abs(v[0][0] - 0.016) < 1e-12
    assert abs(b1p - 0.9) < 1e-12 and abs(b2p - 0.999) < 1e-12
    out_p, *_ = R.adamw(p, g, z, z, 1.0, 1.0, 0.1, weight_decay=0.1, mask=[True])
    assert abs(out_p[0][0] - 1.88) < 1e-8


def test_loss_closed_form_for_constant_scores():
    rows, classes = 9, 10
    scores = np.full((rows, classes), 3.25)
    y = np.zeros((rows, classes))
    y[:, 4] = 1.0
    assert abs(R.cross_entropy(scores, y) - rows * math.log(classes)) < 1e-9


def test_clip():
    assert np.array_equal(R.clip(np.array([-7.0, -5.0, 0.5, 5.0, 9.0])), [-5.0, -5.0, 0.5, 5.0, 5.0])


# ------------------------------------------- the float32 step's tolerances
def _fp32_step(x, y, params, mistake=None):
    """The config-5 composition computed in numpy float32 (an independent
    float32 evaluation standing in for the GPU step), optionally with a
    planted mistake, returning the six gradients in float64."""
    f = np.float32
    w1, b1, w2, b2, w3, b3 = (p.astype(f) for p in params)
    x, y = x.astype(f), y.astype(f)
    rows = f(x.shape[0])
    z1 = x @ w1 + b1
    h1 = np.where(z1 > 0, z1, f(0))
    z2 = h1 @ w2 + b2
    h2 = np.where(z2 > 0, z2, f(0))
    s = h2 @ w3 + b3
    e = np.exp(s - s.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    ds = (p - y) / rows
    dh2 = ds @ w3.T
    dz2 = np.where(z2 > 0, dh2, f(0))
    dh1 = dz2 @ w2.T
    dz1 = dh1 if mistake == "relu-mask" else np.where(z1 > 0, dh1, f(0))
    grads = [x.T @ dz1, dz1.sum(axis=0, keepdims=True), h1.T @ dz2, dz2.sum(axis=0, keepdims=True),
             h2.T @ ds, ds.sum(axis=0, keepdims=True)]
    if mistake == "scale":
        grads[2] = grads[2] * f(1.1)
    if mistake == "transpose":
        grads[4] = (h2.T @ ds[::-1]).astype(f)
    return [g.astype(np.float64) for g in grads]


def test_fp32_step_tolerances_hold_and_catch_planted_mistakes():
    """The per-entry allowances of tests/mlp_bounds.py contain an
    independent float32 evaluation of the step on every entry, and reject it
    when a mistake is planted in it: a dropped ReLU mask in layer 1's
    backward, a 10 % scale on dW2, and the rows of d_scores reversed in
    dW3."""
    import mlp_bounds as MB
    rng = np.random.default_rng(12)
    layers, rows = (64, 128, 96, 10), 512
    params = []
    for a, b in zip(layers[:-1], layers[1:]):
        params.append(rng.uniform(-math.sqrt(6 / a), math.sqrt(6 / a), (a, b)).astype(np.float32).astype(np.float64))
        params.append(np.zeros((1, b)))
    x = rng.uniform(0, 1, (rows, layers[0])).astype(np.float32).astype(np.float64)
    y = np.zeros((rows, layers[-1]))
    y[np.arange(rows), rng.integers(0, layers[-1], rows)] = 1.0
    loss, ref, allow, unc1, unc2 = MB.grad_bounds(x, y, params)
    got = _fp32_step(x, y, params)
    for i in range(6):
        assert np.all(np.abs(got[i] - ref[i]) <= allow[i]), i
    for mistake, layer in (("relu-mask", 0), ("scale", 2), ("transpose", 4)):
        bad = _fp32_step(x, y, params, mistake)
        assert np.any(np.abs(bad[layer] - ref[layer]) > allow[layer]), mistake
