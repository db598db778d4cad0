"""The MLP classifier training step of examples/08_gpu_classifier.php
(predict :117-124, crossEntropy :126-134, trainBatch :137-161), written
against the CudaArray / Optimizer surface so that it runs eagerly or is
recorded whole by Fusion.compile and replayed.

Config 5 shape: X[4096,784] float32 U(0,1), one-hot labels [4096,10],
784 -> 1024 -> ReLU -> 1024 -> ReLU -> 10, Kaiming-uniform weights
(U(-sqrt(6/fan_in), sqrt(6/fan_in))) from a fixed seed, zero biases,
AdamW(lr 1e-3) with weight decay on the weights only, gradients clipped to
[-5, 5].
"""
import math

import numpy as np

from . import synthetic
from .cuda_array import CudaArray
from .fusion import Fusion


def init_parameters(layers=(784, 1024, 1024, 10), seed=5):
    """[W1, b1, W2, b2, W3, b3]: W ~ U(+-sqrt(6/fan_in)) [fan_in, fan_out], b = 0 [1, fan_out]."""
    params = []
    for i, (fan_in, fan_out) in enumerate(zip(layers[:-1], layers[1:])):
        bound = math.sqrt(6.0 / fan_in)
        w = synthetic.uniform((fan_in, fan_out), -bound, bound, seed=seed * 100 + i)
        params.append(CudaArray.fromNumpy(w))
        params.append(CudaArray.zeros([1, fan_out]))
    return params


def synthetic_batch(rows=4096, features=784, classes=10, seed=5):
    """X U(0,1) and one-hot labels of integer classes U[0, classes)."""
    x = synthetic.uniform((rows, features), 0.0, 1.0, seed=seed * 1000 + 1)
    cls = synthetic.integers((rows,), 0, classes, seed=seed * 1000 + 2)
    y = np.zeros((rows, classes), np.float32)
    y[np.arange(rows), cls] = 1.0
    return x, y


def predict(features, parameters, zero):
    w1, b1, w2, b2, w3, b3 = parameters
    h1 = features.matmul(w1) + b1
    h1 = CudaArray.where(h1.gt(0), h1, zero)
    h2 = h1.matmul(w2) + b2
    h2 = CudaArray.where(h2.gt(0), h2, zero)
    return h2.matmul(w3) + b3


def cross_entropy(scores, labels):
    """Sum over rows of logsumexp(scores) - score of the target (stable shift)."""
    rows = scores.getShape()[0]
    shifted = scores - scores.max(1).reshape([rows, 1])
    log_partition = shifted.exp().sum(1).reshape([rows, 1]).log()
    target = (shifted * labels).sum(1).reshape([rows, 1])
    return (log_partition - target).sum(0)


DECAY_MASK = [True, False, True, False, True, False]


def train_batch(features, labels, parameters, optimizer, state, learning_rate, clip=5.0):
    """One training step; returns {'loss', 'parameters', 'state'}."""
    zero = CudaArray.zeros([1])
    one = CudaArray.ones([1])
    upper = CudaArray.full([1], clip)
    lower = CudaArray.full([1], -clip)
    optimizer.zeroGrad(parameters)
    for p in parameters:
        p.requiresGrad()
    loss = cross_entropy(predict(features, parameters, zero), labels)
    # gradients averaged over the batch
    loss.backward(one / float(features.getShape()[0]))
    grads = []
    for p in parameters:
        g = p.grad()
        g = CudaArray.where(g.gt(clip), upper, g)
        grads.append(CudaArray.where(g.lt(-clip), lower, g))
    out = optimizer.step(parameters, grads, state, learning_rate, DECAY_MASK)
    for p in parameters:
        p.requiresGrad(False)
        p.zeroGrad()
    return {"loss": loss.detach(), "parameters": out["parameters"], "state": out["state"]}


def training_inputs(features, labels, rate, parameters, state):
    return [features, labels, rate, state["beta1Power"], state["beta2Power"],
            *parameters, *state["firstMoment"], *state["secondMoment"]]


def compile_training_plan(inputs, optimizer, cuda_graph=True):
    """Fusion.compile of the whole training step (examples/08: compileTrainingPlan)."""
    def body(features, labels, rate, beta1_power, beta2_power, *tensors):
        params, first, second = list(tensors[0:6]), list(tensors[6:12]), list(tensors[12:18])
        state = {"firstMoment": first, "secondMoment": second,
                 "beta1Power": beta1_power, "beta2Power": beta2_power}
        r = train_batch(features, labels, params, optimizer, state, rate)
        st = r["state"]
        return [*r["parameters"], *st["firstMoment"], *st["secondMoment"],
                st["beta1Power"], st["beta2Power"], r["loss"]]
    return Fusion.compile(body, inputs, cudaGraph=cuda_graph)


def unpack_step(outputs):
    """Outputs of a compiled step -> (parameters, state, loss)."""
    params = list(outputs[0:6])
    state = {"firstMoment": list(outputs[6:12]), "secondMoment": list(outputs[12:18]),
             "beta1Power": outputs[18], "beta2Power": outputs[19]}
    return params, state, outputs[20]


def step_flops(rows=4096, layers=(784, 1024, 1024, 10)):
    """Forward (3 GEMMs) + backward (dW1, dW2, dH1, dW3, dH2) GEMM FLOP."""
    fwd = sum(2 * rows * a * b for a, b in zip(layers[:-1], layers[1:]))
    bwd_w = sum(2 * rows * a * b for a, b in zip(layers[:-1], layers[1:]))
    bwd_x = sum(2 * rows * a * b for a, b in zip(layers[1:-1], layers[2:]))
    return fwd + bwd_w + bwd_x
