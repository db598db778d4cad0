"""CPU ORACLE -- test infrastructure only.

numpy (float64) restatement of the MLP classifier training step of the
reference (examples/08_gpu_classifier.php:117-161): forward (predict),
softmax cross-entropy (crossEntropy), the gradients reverse-mode autograd
produces for them (src/autograd.c: matmul :1539-1585, broadcast add,
where, max with the gradient shared among ties :945-1003, exp, log, sum),
gradient clipping to [-5, 5] and the functional AdamW step
(src/optimizer.c:471-607).  Only tests/ and bench.py's cpu_baseline leg use
it, as the checker / CPU baseline; the product never imports it.

Pinning: the analytic gradients are checked against central finite
differences of the same loss (tests/test_oracle_mlp.py); AdamW against the
closed-form values of tests/optimizer.phpt:51-63; the loss against its
closed form for constant scores (rows * log(classes)).
"""
import numpy as np


def predict(x, params):
    w1, b1, w2, b2, w3, b3 = params
    z1 = x @ w1 + b1
    h1 = np.where(z1 > 0, z1, 0.0)
    z2 = h1 @ w2 + b2
    h2 = np.where(z2 > 0, z2, 0.0)
    return h2 @ w3 + b3, (z1, h1, z2, h2)


def cross_entropy(scores, labels):
    shifted = scores - scores.max(axis=1, keepdims=True)
    logz = np.log(np.exp(shifted).sum(axis=1, keepdims=True))
    target = (shifted * labels).sum(axis=1, keepdims=True)
    return float((logz - target).sum())


def loss_and_grads(x, labels, params, scale, intermediates=None):
    """Loss and d(loss * scale)/d(params) (backward seeded with `scale`).
    A dict passed as `intermediates` receives the forward and backward
    values (z1, h1, z2, h2, scores, d_scores, dh2, dz2, dh1, dz1)."""
    w1, b1, w2, b2, w3, b3 = params
    scores, (z1, h1, z2, h2) = predict(x, params)
    loss = cross_entropy(scores, labels)
    m = scores.max(axis=1, keepdims=True)
    shifted = scores - m
    e = np.exp(shifted)
    p = e / e.sum(axis=1, keepdims=True)
    # d/dshifted of sum(logz - target), times the seed
    d_shifted = (p - labels) * scale
    # max reduction: minus the row sum of d_shifted, shared among the maxima
    hit = (scores == m).astype(np.float64)
    d_scores = d_shifted - hit / hit.sum(axis=1, keepdims=True) * d_shifted.sum(axis=1, keepdims=True)
    gw3 = h2.T @ d_scores
    gb3 = d_scores.sum(axis=0, keepdims=True)
    dh2 = d_scores @ w3.T
    dz2 = np.where(z2 > 0, dh2, 0.0)
    gw2 = h1.T @ dz2
    gb2 = dz2.sum(axis=0, keepdims=True)
    dh1 = dz2 @ w2.T
    dz1 = np.where(z1 > 0, dh1, 0.0)
    gw1 = x.T @ dz1
    gb1 = dz1.sum(axis=0, keepdims=True)
    if intermediates is not None:
        intermediates.update(z1=z1, h1=h1, z2=z2, h2=h2, scores=scores, d_scores=d_scores, dh2=dh2, dz2=dz2,
                             dh1=dh1, dz1=dz1)
    return loss, [gw1, gb1, gw2, gb2, gw3, gb3]


def clip(g, bound=5.0):
    return np.where(g > bound, bound, np.where(g < -bound, -bound, g))


def adamw(params, grads, first, second, beta1_power, beta2_power, lr,
          beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, mask=None):
    """optimizer.c:471-607 in float64: returns new params, moments, powers."""
    mask = mask if mask is not None else [True] * len(params)
    b1p = beta1_power * beta1
    b2p = beta2_power * beta2
    c1 = 1.0 - b1p
    c2 = 1.0 - b2p
    out_p, out_m, out_v = [], [], []
    for i, (p, g) in enumerate(zip(params, grads)):
        m = first[i] * beta1 + g * (1.0 - beta1)
        v = second[i] * beta2 + g * g * (1.0 - beta2)
        upd = (m / c1) / (np.sqrt(v / c2) + eps) * lr
        if weight_decay > 0.0 and mask[i]:
            newp = p * (1.0 - lr * weight_decay) - upd
        else:
            newp = p - upd
        # a NaN gradient keeps the old value (optimizer.c:424-469)
        keep = np.isnan(g)
        out_p.append(np.where(keep, p, newp))
        out_m.append(np.where(keep, first[i], m))
        out_v.append(np.where(keep, second[i], v))
    return out_p, out_m, out_v, b1p, b2p


def train_step(x, labels, params, first, second, beta1_power, beta2_power, lr, mask):
    """One full step: returns (loss, clipped grads, params', m', v', b1p', b2p')."""
    x = np.asarray(x, np.float64)
    labels = np.asarray(labels, np.float64)
    params = [np.asarray(p, np.float64) for p in params]
    loss, grads = loss_and_grads(x, labels, params, 1.0 / x.shape[0])
    grads = [clip(g) for g in grads]
    p2, m2, v2, b1p, b2p = adamw(params, grads, [np.asarray(m, np.float64) for m in first],
                                 [np.asarray(v, np.float64) for v in second],
                                 beta1_power, beta2_power, lr, mask=mask)
    return loss, grads, p2, m2, v2, b1p, b2p
