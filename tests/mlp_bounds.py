"""Per-entry tolerances for the float32 MLP training step (config 5)
against the float64 oracle (oracle/mlp_ref.py): test infrastructure.

Every gradient is a product of the step's operands, checked entry by entry
against the north-star GEMM bar 1e-4 * sqrt(K) * (|A||B|)_ij (a bias
gradient is the product with a ones vector), with |A|, |B| taken from the
oracle's float64 operands, plus the errors its operands bring from upstream
(dA B + A dB).  Those come from probabilistic rounding error analysis
(Higham & Mary 2019): a float32 sum of n products errs by about
sqrt(n) u (|A||B|)_ij (u = 2^-24); such scales propagate from layer to
layer as a root sum of squares (independent roundings), and lambda = 8 of
them bound an error with probability above 1 - 1e-13.  They matter where an activation
is small against the terms it cancels from, such as a neuron that is active
on a few rows only.  ReLU passes forward errors on unchanged (it is
1-Lipschitz), but its backward mask can flip: a pre-activation whose
float64 value is within its rounding bound of zero may take the other branch
in float32.  Those entries are identified explicitly, and the full effect of
the other branch (the upstream gradient the entry passes or blocks) is added
to the allowance of exactly the gradient entries it reaches, through layer
2's input gradient as well.  The AdamW update of a first step
is lr * g / (|g| + eps) (the bias corrections cancel); its allowance comes
from the gradient's through the derivative eps / (|g| + eps)^2, capped at 2
(a flipped sign), from the float32 bias corrections, and 8 u of |p| for its
own roundings.
"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import mlp_ref as R  # noqa: E402

U = 2.0 ** -24
LAMBDA = 8.0


def _scale(n, mag):
    """Scale of the float32 rounding error of a sum of n products of
    magnitude mag: about sqrt(n) u |A||B| (a few standard deviations of the
    random-walk model), plus 2 u for the rest of the expression."""
    return (np.sqrt(n) + 2.0) * U * mag


def _rss(err, w):
    """Scale of the error a product with weights w inherits from independent
    operand errors err: the root of the sum of squares."""
    return np.sqrt((err * err) @ (w * w))


def grad_bounds(x, labels, params):
    """(loss, reference gradients, per-entry allowances, number of
    ReLU entries of layers 1 and 2 that may take the other branch)."""
    x = np.asarray(x, np.float64)
    labels = np.asarray(labels, np.float64)
    params = [np.asarray(p, np.float64) for p in params]
    rows, k1 = x.shape
    k2, k3 = params[2].shape[0], params[4].shape[0]
    it = {}
    loss, grads = R.loss_and_grads(x, labels, params, 1.0 / rows, it)
    w1, b1, w2, b2, w3, b3 = (np.abs(p) for p in params)
    ax = np.abs(x)
    lam = LAMBDA
    bar = lambda k, mag: 1e-4 * np.sqrt(k) * mag  # noqa: E731  the north-star GEMM bar
    # forward error scales of the pre-activations (ReLU passes them on: it
    # is 1-Lipschitz); lambda times them are the flip thresholds
    t1 = _scale(k1, ax @ w1 + b1)
    t2 = _scale(k2, np.abs(it["h1"]) @ w2 + b2) + _rss(t1, w2)
    ts = _scale(k3, np.abs(it["h2"]) @ w3 + b3) + _rss(t2, w3)
    flip1 = np.abs(it["z1"]) <= lam * t1
    flip2 = np.abs(it["z2"]) <= lam * t2
    # backward: softmax cross-entropy seeded with 1/rows, |dp_i| <= 2 p_i
    # max_j |ds_j| plus 64 u p_i for its exp / sum / division roundings
    s = it["scores"]
    pr = np.exp(s - s.max(axis=1, keepdims=True))
    pr /= pr.sum(axis=1, keepdims=True)
    e_ds = (2.0 * ts.max(axis=1, keepdims=True) + 64 * U) * (pr + labels) / rows
    ds = np.abs(it["d_scores"])
    e_dh2 = _scale(k3, ds @ w3.T) + _rss(e_ds, w3.T)
    e_dz2 = np.where((it["z2"] > 0) | flip2, e_dh2, 0.0)
    e_dh1 = _scale(k2, np.abs(it["dz2"]) @ w2.T) + _rss(e_dz2, w2.T)
    e_dz1 = np.where((it["z1"] > 0) | flip1, e_dh1, 0.0)
    # the other branch of a ReLU within rounding of zero: dz may be dh or 0
    f_dz2 = np.where(flip2, np.abs(it["dh2"]), 0.0)
    f_dh1 = f_dz2 @ w2.T
    f_dz1 = np.where(flip1, np.abs(it["dh1"]) + f_dh1, np.where(it["z1"] > 0, f_dh1, 0.0))
    dz2 = np.abs(it["dz2"]) + f_dz2
    dz1 = np.abs(it["dz1"]) + f_dz1
    h1, h2 = np.abs(it["h1"]), np.abs(it["h2"])
    ones = np.ones((1, rows))
    inherit = lambda a, ea, b, eb: lam * np.sqrt((ea * ea).T @ (b * b) + (a * a).T @ (eb * eb))  # noqa: E731
    allow = [bar(rows, ax.T @ dz1) + inherit(ax, 0 * ax, dz1, e_dz1) + ax.T @ f_dz1,
             bar(rows, ones @ dz1) + inherit(ones.T, 0 * ones.T, dz1, e_dz1) + ones @ f_dz1,
             bar(rows, h1.T @ dz2) + inherit(h1, t1, dz2, e_dz2) + (h1 + lam * t1).T @ f_dz2,
             bar(rows, ones @ dz2) + inherit(ones.T, 0 * ones.T, dz2, e_dz2) + ones @ f_dz2,
             bar(rows, h2.T @ ds) + inherit(h2, t2, ds, e_ds),
             bar(rows, ones @ ds) + inherit(ones.T, 0 * ones.T, ds, e_ds)]
    return loss, grads, allow, int(flip1.sum()), int(flip2.sum())


def param_bounds(params, grads, allow, lr=1e-3, eps=1e-8, beta1=0.9, beta2=0.999):
    """Allowances of the parameters after the first AdamW step.  Besides the
    gradient's allowance, the bias corrections c = 1 - beta^t are formed in
    float32 from the float32 beta powers, as the reference's tensors hold
    them (optimizer.c:471-607): one rounding of beta^t is u * beta^t / c of
    c (6e-5 for c2 = 1 - 0.999), which reaches the update through m / c1
    and, halved, through sqrt(v / c2)."""
    rel = U * (2 * beta1 / (1 - beta1) + beta2 / (1 - beta2) + 16)
    out = []
    for p, g, e in zip(params, grads, allow):
        p = np.asarray(p, np.float64)
        ag = np.abs(g)
        df = np.minimum(2.0, eps * e / (np.maximum(ag - e, 0.0) + eps) ** 2)
        out.append(lr * (df + rel) + 8 * U * np.abs(p) + 1e-12)
    return out
