"""PhpTensors\\Optimizer: functional AdamW and SGD steps over CudaArray
(stubs/cuda.stub.php:709-730, src/optimizer.c).

Every update is an expression of CudaArray operations in the order the
reference evaluates them (optimizer_adamw_step, optimizer.c:471-607), so a
step inside Fusion.compile is recorded and fused like any other code, and the
per-operation float32 rounding matches the reference's eager kernels.
"""
import math

from ._abi import InvalidArgumentException
from .cuda_array import CudaArray


class Optimizer:
    def __init__(self, kind, learning_rate, momentum, beta1, beta2, epsilon, weight_decay):
        self.kind = kind
        self.learningRate = learning_rate
        self.momentum = momentum
        self.beta1 = beta1
        self.beta2 = beta2
        self.epsilon = epsilon
        self.weightDecay = weight_decay

    @staticmethod
    def _nonneg(value, name, allow_zero=True):
        if not math.isfinite(value) or value < 0 or (value == 0 and not allow_zero):
            raise InvalidArgumentException(f"{name} must be a finite non-negative value")

    @classmethod
    def adamW(cls, learningRate=0.001, beta1=0.9, beta2=0.999, epsilon=1e-8, weightDecay=0.01):
        """optimizer.c:151-176 (argument validation as there)."""
        cls._nonneg(learningRate, "learningRate")
        cls._nonneg(epsilon, "epsilon")
        cls._nonneg(weightDecay, "weightDecay")
        for b in (beta1, beta2):
            if not math.isfinite(b) or b < 0.0 or b >= 1.0:
                raise InvalidArgumentException("beta1 and beta2 must be finite values in [0, 1)")
        return cls("adamW", learningRate, 0.0, beta1, beta2, epsilon, weightDecay)

    @classmethod
    def sgd(cls, learningRate=0.01, momentum=0.0, weightDecay=0.0):
        cls._nonneg(learningRate, "learningRate")
        cls._nonneg(momentum, "momentum")
        cls._nonneg(weightDecay, "weightDecay")
        return cls("sgd", learningRate, momentum, 0.9, 0.999, 1e-8, weightDecay)

    def initState(self, parameters):
        """Zeroed moments (and unit beta powers) in each parameter's dtype."""
        if self.kind == "adamW":
            dt = parameters[0].getDtype() if parameters else "float32"
            return {"firstMoment": [CudaArray.zeros(p.getShape(), p.getDtype()) for p in parameters],
                    "secondMoment": [CudaArray.zeros(p.getShape(), p.getDtype()) for p in parameters],
                    "beta1Power": CudaArray.ones([1], dt), "beta2Power": CudaArray.ones([1], dt)}
        return {"velocity": [CudaArray.zeros(p.getShape(), p.getDtype()) for p in parameters]}

    def zeroGrad(self, parameters):
        for p in parameters:
            p.zeroGrad()

    def step(self, parameters, gradients, state, learningRate=None, weightDecayMask=None):
        if len(parameters) != len(gradients):
            raise InvalidArgumentException("One gradient per parameter is required")
        for p, g in zip(parameters, gradients):
            if g is not None and g.getShape() != p.getShape():
                raise InvalidArgumentException("Gradient shape does not match its parameter")
        mask = weightDecayMask if weightDecayMask is not None else [True] * len(parameters)
        lr = self.learningRate if learningRate is None else learningRate
        if self.kind == "adamW":
            return self._adamw(parameters, gradients, state, lr, mask)
        return self._sgd(parameters, gradients, state, lr, mask)

    def _adamw(self, parameters, gradients, state, lr, mask):
        b1, b2, eps, wd = self.beta1, self.beta2, self.epsilon, self.weightDecay
        # shared terms (optimizer.c:505-514)
        b1p = state["beta1Power"] * b1
        b2p = state["beta2Power"] * b2
        c1 = (b1p - 1.0) * -1.0
        c2 = (b2p - 1.0) * -1.0
        out_p, out_m, out_v = [], [], []
        for i, (p, g) in enumerate(zip(parameters, gradients)):
            m0, v0 = state["firstMoment"][i], state["secondMoment"][i]
            if g is None:
                out_p.append(p)
                out_m.append(m0)
                out_v.append(v0)
                continue
            m = m0 * b1 + g * (1.0 - b1)
            v = v0 * b2 + (g * g) * (1.0 - b2)
            upd = (m / c1) / ((v / c2).sqrt() + eps) * lr
            if wd > 0.0 and mask[i]:
                decay = ((lr * wd) - 1.0) * -1.0 if isinstance(lr, CudaArray) else 1.0 - lr * wd
                newp = p * decay - upd
            else:
                newp = p - upd
            out_p.append(newp)
            out_m.append(m)
            out_v.append(v)
        return {"parameters": out_p,
                "state": {"firstMoment": out_m, "secondMoment": out_v, "beta1Power": b1p, "beta2Power": b2p}}

    def _sgd(self, parameters, gradients, state, lr, mask):
        mom, wd = self.momentum, self.weightDecay
        out_p, out_v = [], []
        for i, (p, g) in enumerate(zip(parameters, gradients)):
            vel = state["velocity"][i]
            if g is None:
                out_p.append(p)
                out_v.append(vel)
                continue
            if wd > 0.0 and mask[i]:
                g = g + p * wd
            v = vel * mom + g if mom > 0.0 else g
            out_p.append(p - v * lr)
            out_v.append(v)
        return {"parameters": out_p, "state": {"velocity": out_v}}
