"""Helpers for GPU parity tests: run one C-ABI entry point on host arrays."""
import numpy as np

from phptensors import _abi as A

NP = {A.FLOAT32: np.float32, A.FLOAT64: np.float64, A.INT8: np.int8, A.INT16: np.int16,
      A.INT32: np.int32, A.INT64: np.int64, A.UINT8: np.uint8, A.UINT16: np.uint16,
      A.UINT32: np.uint32, A.UINT64: np.uint64, A.BOOL: np.uint8, A.FLOAT16: np.uint16,
      A.BFLOAT16: np.uint16}


def elem_strides(a):
    return [s // a.itemsize for s in a.strides]


def out_shape(shape, axis):
    if axis is None or axis < 0:
        return (1,)
    return tuple(s for d, s in enumerate(shape) if d != axis) or (1,)


def reduce(x, dtype, op, axis=None, strides=None, shape=None, base=None):
    """pt_reduce over x (a contiguous storage array, optionally read through
    explicit shape/strides to form a view)."""
    lib = A.load()
    shape = tuple(x.shape if shape is None else shape)
    strides = elem_strides(x) if strides is None else strides
    rdt = lib.pt_reduce_result_dtype(dtype, A.OP[op])
    ax = -1 if axis is None else axis % len(shape)
    oshape = out_shape(shape, None if axis is None else ax)
    dx = A.to_device(x)
    dy = A.DeviceBuffer(max(1, int(np.prod(oshape)) * A.DTYPE_SIZES[rdt]))
    A.check(lib.pt_reduce(dx.ptr, dy.ptr, dtype, A.OP[op], A.ints(shape), A.sizes(strides),
                          len(shape), ax, 0 if base is None else base, None), op)
    return dy.download(NP[rdt], oshape), rdt


def arg_reduce(x, dtype, op, axis=None, strides=None, shape=None):
    lib = A.load()
    shape = tuple(x.shape if shape is None else shape)
    strides = elem_strides(x) if strides is None else strides
    ax = -1 if axis is None else axis % len(shape)
    oshape = out_shape(shape, None if axis is None else ax)
    dx = A.to_device(x)
    dy = A.DeviceBuffer(max(1, int(np.prod(oshape)) * 4))
    A.check(lib.pt_arg_reduce(dx.ptr, dy.ptr, dtype, A.OP[op], A.ints(shape), A.sizes(strides),
                              len(shape), ax, 0, None), op)
    return dy.download(np.int32, oshape)


def moments(x, dtype, axis=None, correction=0, std=False, strides=None, shape=None):
    lib = A.load()
    shape = tuple(x.shape if shape is None else shape)
    strides = elem_strides(x) if strides is None else strides
    rdt = A.FLOAT32 if dtype in (A.FLOAT32, A.FLOAT16, A.BFLOAT16) else A.FLOAT64
    ax = -1 if axis is None else axis % len(shape)
    oshape = out_shape(shape, None if axis is None else ax)
    dx = A.to_device(x)
    dy = A.DeviceBuffer(max(1, int(np.prod(oshape)) * A.DTYPE_SIZES[rdt]))
    A.check(lib.pt_moments(dx.ptr, dy.ptr, dtype, rdt, A.ints(shape), A.sizes(strides),
                           len(shape), ax, correction, int(std), None), "moments")
    return dy.download(NP[rdt], oshape)


def softmax(x, dtype, axis=-1, strides=None, shape=None):
    lib = A.load()
    shape = tuple(x.shape if shape is None else shape)
    strides = elem_strides(x) if strides is None else strides
    odt = A.FLOAT32 if dtype in (A.FLOAT32, A.FLOAT16, A.BFLOAT16) else A.FLOAT64
    dx = A.to_device(x)
    dy = A.DeviceBuffer(max(1, int(np.prod(shape)) * A.DTYPE_SIZES[odt]))
    A.check(lib.pt_softmax(dx.ptr, dy.ptr, dtype, odt, A.ints(shape), A.sizes(strides),
                           len(shape), axis % len(shape), None), "softmax")
    return dy.download(NP[odt], shape)


def layernorm(x, dtype, eps=1e-5, gamma=None, beta=None, compute=A.FLOAT32):
    lib = A.load()
    n = x.shape[-1]
    rows = x.size // n
    dx = A.to_device(x)
    npc = np.float32 if compute == A.FLOAT32 else np.float64
    dy = A.DeviceBuffer(max(1, x.size * np.dtype(npc).itemsize))
    dg = A.to_device(np.asarray(gamma, npc)) if gamma is not None else None
    db = A.to_device(np.asarray(beta, npc)) if beta is not None else None
    A.check(lib.pt_layernorm(dx.ptr, dy.ptr, dtype, compute, rows, n, eps,
                             dg.ptr if dg else None, db.ptr if db else None, None), "layernorm")
    return dy.download(npc, x.shape)
