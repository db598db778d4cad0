"""Reverse-mode differentiation for the CudaArray operations of the MLP
training path (requiresGrad / backward / grad / detach).

Each differentiable CudaArray operation whose operand requires a gradient
records a node: its parents and a function from the upstream gradient to the
parents' gradients.  backward() walks the graph in reverse topological order
and accumulates gradients on the leaves.  The gradient formulas follow
src/autograd.c: matmul (:1539-1585, upstream @ B^T and A^T @ upstream over
transposed views), broadcast operands reduced back to their shape,
reductions (:900-1003: sum expands, max shares the upstream gradient equally
among the maxima), where, exp, log, reshape.  Every gradient is itself a
CudaArray expression, so inside a Fusion scope the backward pass is recorded
into the plan like the forward pass.
"""


class Node:
    __slots__ = ("parents", "backward", "op")

    def __init__(self, parents, backward, op):
        self.parents = parents
        self.backward = backward
        self.op = op


_recording = [True]


def needs_grad(t):
    return t is not None and (t._rg or t._node is not None)


def active(*ts):
    """True when an operation on `ts` must record a node."""
    return _recording[0] and any(needs_grad(t) for t in ts if t is not None and hasattr(t, "_rg"))


def record(out, parents, backward, op):
    """Attach a node to `out` when any parent requires a gradient."""
    if _recording[0] and any(needs_grad(p) for p in parents):
        out._node = Node(parents, backward, op)
    return out


def reduce_to(g, shape):
    """Sum a broadcast gradient back to `shape` (leading and extent-1 dims)."""
    gshape = g.getShape()
    shape = list(shape)
    if gshape == shape:
        return g
    lead = len(gshape) - len(shape)
    out = g
    # leading dimensions
    for _ in range(lead):
        out = out.sum(0)
    cur = out.getShape()
    for d, (have, want) in enumerate(zip(cur, shape)):
        if want == 1 and have != 1:
            keep = out.getShape()
            out = out.sum(d)
            keep[d] = 1
            out = out.reshape(keep)
    if out.getShape() != shape:
        out = out.reshape(shape)
    return out


def expand_reduced(g, in_shape, axis):
    """Upstream gradient of a reduction along `axis` (None: global) broadcast
    back over the reduced input shape."""
    if axis is None:
        return g.reshape([1] * len(in_shape)).broadcastTo(in_shape)
    keep = list(in_shape)
    keep[axis] = 1
    return g.reshape(keep).broadcastTo(in_shape)


def backward(root, gradient=None):
    """Accumulate d(root)/d(leaf) into every leaf that requires a gradient."""
    from .cuda_array import CudaArray
    order, seen = [], set()

    def visit(t):
        if id(t) in seen:
            return
        seen.add(id(t))
        if t._node is not None:
            for p in t._node.parents:
                if needs_grad(p):
                    visit(p)
        order.append(t)

    visit(root)
    # fp16 / bf16 roots propagate float32 gradients (autograd.c:1741-1764)
    low = root.getDtype() in ("float16", "bfloat16")
    if gradient is None:
        gradient = CudaArray.ones(root.getShape(), "float32" if low else root.getDtype())
    elif low:
        gradient = gradient.astype("float32")
    grads = {id(root): gradient}
    _recording[0] = False  # gradients carry no history of their own
    try:
        _walk(order, grads)
    finally:
        _recording[0] = True


def _walk(order, grads):
    for t in reversed(order):
        g = grads.pop(id(t), None)
        if g is None:
            continue
        if t._node is None:
            if t._rg:
                t._grad = g if t._grad is None else t._grad + g
            continue
        pg = t._node.backward(g)
        for p, gp in zip(t._node.parents, pg):
            if gp is None or not needs_grad(p):
                continue
            grads[id(p)] = gp if id(p) not in grads else grads[id(p)] + gp
