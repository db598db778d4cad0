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
