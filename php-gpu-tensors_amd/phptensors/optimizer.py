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
        """Optimizer::step (optimizer.c:730-800): equally long CudaArray lists,
        each gradient of its parameter's shape and dtype, a boolean decay mask
        per parameter; the rate is a CudaArray or, when omitted, the
        optimizer's own."""
        parameters, gradients = list(parameters), list(gradients)
        if len(parameters) != len(gradients) or not all(
                isinstance(t, CudaArray) for t in parameters + gradients):
            raise InvalidArgumentException("parameters and gradients must be equally sized CudaArray lists")
        for p, g in zip(parameters, gradients):
            if g.getShape() != p.getShape():
                raise InvalidArgumentException("Each gradient must have the same shape as its parameter")
            if g.getDtype() != p.getDtype():
                raise InvalidArgumentException("Each gradient must have the same dtype as its parameter")
        if weightDecayMask is not None:
            mask = list(weightDecayMask)
            if len(mask) != len(parameters):
                raise InvalidArgumentException("weightDecayMask must match the parameter count")
            if not all(isinstance(m, bool) for m in mask):
                raise InvalidArgumentException("weightDecayMask entries must be booleans")
        else:
            mask = [True] * len(parameters)
        lr = self.learningRate if learningRate is None else learningRate
        if self.kind == "adamW":
            return self._adamw(parameters, gradients, state, lr, mask)
        return self._sgd(parameters, gradients, state, lr, mask)

    @staticmethod
    def _selected(g, updated, original, detach):
        """Where the gradient is NaN the old value is kept (where(g == g, ...),
        optimizer.c:424-469); updated parameters are detached from the graph."""
        out = CudaArray.where(g.eq(g), updated, original)
        return out.detach() if detach else out

    def _adamw(self, parameters, gradients, state, lr, mask):
        """optimizer_adamw_step (optimizer.c:471-607), operation by operation."""
        b1, b2, eps, wd = self.beta1, self.beta2, self.epsilon, self.weightDecay
        b1p = state["beta1Power"] * b1
        b2p = state["beta2Power"] * b2
        c1 = (b1p - 1.0) * -1.0
        c2 = (b2p - 1.0) * -1.0
        out_p, out_m, out_v = [], [], []
        for i, (p, g) in enumerate(zip(parameters, gradients)):
            m0, v0 = state["firstMoment"][i], state["secondMoment"][i]
            m = m0 * b1 + g * (1.0 - b1)
            v = v0 * b2 + (g * g) * (1.0 - b2)
            upd = (m / c1) / ((v / c2).sqrt() + eps) * lr
            if wd > 0.0 and mask[i]:
                decay = ((lr * wd) - 1.0) * -1.0 if isinstance(lr, CudaArray) else 1.0 - lr * wd
                newp = p * decay - upd
            else:
                newp = p - upd
            out_p.append(self._selected(g, newp, p, True))
            out_m.append(self._selected(g, m, m0, False))
            out_v.append(self._selected(g, v, v0, False))
        return {"parameters": out_p,
                "state": {"firstMoment": out_m, "secondMoment": out_v, "beta1Power": b1p, "beta2Power": b2p}}

    def _sgd(self, parameters, gradients, state, lr, mask):
        """optimizer_sgd_step (optimizer.c:609-676): the velocity g + v·momentum
        is the new state; weight decay enters the step only."""
        mom, wd = self.momentum, self.weightDecay
        out_p, out_v = [], []
        for i, (p, g) in enumerate(zip(parameters, gradients)):
            vel0 = state["velocity"][i]
            vel = g + vel0 * mom
            direction = vel + p * wd if (wd > 0.0 and mask[i]) else vel
            newp = p - direction * lr
            out_p.append(self._selected(g, newp, p, True))
            out_v.append(self._selected(g, vel, vel0, False))
        return {"parameters": out_p, "state": {"velocity": out_v}}
