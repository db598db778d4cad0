"""ctypes bindings for the CPU oracle (oracle/lib/liboracle.so).

Test infrastructure only: the oracle is the checker for the HIP path and the
CPU baseline of bench.py; product code never imports this module.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
LIB_PATH = os.path.join(ORACLE_DIR, "lib", "liboracle.so")

# dtype codes follow the reference's dtype_t numbering (src/data_types.h:8-25)
F32, F64, I8, I16, I32, I64, U8, U16, U32, U64, BOOL, F16, BF16 = range(13)
NP_STORAGE = {
    F32: np.float32, F64: np.float64, I8: np.int8, I16: np.int16, I32: np.int32,
    I64: np.int64, U8: np.uint8, U16: np.uint16, U32: np.uint32, U64: np.uint64,
    BOOL: np.uint8, F16: np.uint16, BF16: np.uint16,
}
NAMES = {
    "float32": F32, "float64": F64, "int8": I8, "int16": I16, "int32": I32,
    "int64": I64, "uint8": U8, "uint16": U16, "uint32": U32, "uint64": U64,
    "bool": BOOL, "float16": F16, "bfloat16": BF16,
}
class _OpTable(dict):
    """Operation codes of include/pt_hip.h; names are case-insensitive."""

    def __getitem__(self, key):
        return dict.__getitem__(self, key.lower())


OP = _OpTable({
    "add": 0, "sub": 1, "mul": 2, "div": 3, "exp": 5, "expm1": 6, "sqrt": 7,
    "log": 8, "log1p": 9, "exp2": 10, "log2": 11, "log10": 12, "asin": 13,
    "acos": 14, "atan": 15, "sinh": 16, "cosh": 17, "tanh": 18, "sin": 19,
    "cos": 20, "tan": 21, "abs": 22, "neg": 23, "ceil": 26, "floor": 27,
    "round": 28, "sum": 35, "mean": 36, "max": 37, "min": 38,
    "argmax": 42, "argmin": 43, "arg_max": 42, "arg_min": 43,
})

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.or_f32_to_bf16.restype = ctypes.c_uint16
        _lib.or_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.or_f32_to_f16.restype = ctypes.c_uint16
        _lib.or_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.or_bf16_to_f32.restype = ctypes.c_float
        _lib.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.or_f16_to_f32.restype = ctypes.c_float
        _lib.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.or_reduce_result_dtype.restype = ctypes.c_int
        _lib.or_layernorm_f32.argtypes = [
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_float,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _ints(values):
    values = list(values)
    return (ctypes.c_int * max(1, len(values)))(*values)


def _sizes(values):
    values = list(values)
    return (ctypes.c_size_t * max(1, len(values)))(*values)


def _check(status, what):
    if status != 0:
        raise ValueError(f"oracle {what} rejected its arguments (status {status})")


# ---- dtype conversions ---------------------------------------------------

def f32_to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_n(_p(x), _p(out), ctypes.c_size_t(x.size))
    return out


def bf16_to_f32(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().or_bf16_to_f32_n(_p(bits), _p(out), ctypes.c_size_t(bits.size))
    return out


def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_n(_p(x), _p(out), ctypes.c_size_t(x.size))
    return out


def f16_to_f32(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().or_f16_to_f32_n(_p(bits), _p(out), ctypes.c_size_t(bits.size))
    return out


def to_storage(values, dtype):
    """Host bytes of `values` stored as `dtype` (RNE for half types)."""
    if dtype == BF16:
        return f32_to_bf16(np.asarray(values, np.float32))
    if dtype == F16:
        return f32_to_f16(np.asarray(values, np.float32))
    if dtype == BOOL:
        return (np.asarray(values) != 0).astype(np.uint8)
    return np.ascontiguousarray(np.asarray(values).astype(NP_STORAGE[dtype]))


def from_storage(arr, dtype):
    if dtype == BF16:
        return bf16_to_f32(arr)
    if dtype == F16:
        return f16_to_f32(arr)
    return arr


# ---- reductions ----------------------------------------------------------

def reduce(x, dtype, op, axis=None):
    """HostArray sum/mean/max/min (contiguous input of storage dtype)."""
    x = np.ascontiguousarray(x)
    shape = x.shape
    code = OP[op]
    rdtype = lib().or_reduce_result_dtype(dtype, code)
    if axis is None:
        out_shape = (1,)
    else:
        axis = axis % len(shape)
        out_shape = tuple(s for d, s in enumerate(shape) if d != axis) or (1,)
    out = np.zeros(out_shape, NP_STORAGE[rdtype])
    _check(lib().or_reduce(_p(x), dtype, _ints(shape), len(shape),
                           -1 if axis is None else axis, code, _p(out)), op)
    return out, rdtype


def arg_reduce(x, dtype, op, axis=None):
    x = np.ascontiguousarray(x)
    shape = x.shape
    if axis is None:
        out_shape = (1,)
    else:
        axis = axis % len(shape)
        out_shape = tuple(s for d, s in enumerate(shape) if d != axis) or (1,)
    out = np.zeros(out_shape, np.int32)
    _check(lib().or_arg_reduce(_p(x), dtype, _ints(shape), len(shape),
                               -1 if axis is None else axis, OP[op], _p(out)), op)
    return out


def moments(x, dtype, axis=None, correction=0, std=False):
    x = np.ascontiguousarray(x)
    shape = x.shape
    rdtype = F32 if dtype in (F32, F16, BF16) else F64
    if axis is None:
        out_shape = (1,)
    else:
        axis = axis % len(shape)
        out_shape = tuple(s for d, s in enumerate(shape) if d != axis) or (1,)
    out = np.zeros(out_shape, NP_STORAGE[rdtype])
    _check(lib().or_moments(_p(x), dtype, _ints(shape), len(shape),
                            -1 if axis is None else axis, int(correction),
                            int(bool(std)), _p(out)), "moments")
    return out


def softmax_lastaxis(x):
    x = np.ascontiguousarray(x)
    n = x.shape[-1] if x.ndim else 1
    rows = x.size // n if n else 0
    out = np.empty_like(x)
    fn = lib().or_softmax_f32 if x.dtype == np.float32 else lib().or_softmax_f64
    _check(fn(_p(x), ctypes.c_size_t(rows), ctypes.c_size_t(n), _p(out)), "softmax")
    return out


def layernorm_lastaxis(x, eps=1e-5, gamma=None, beta=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty_like(x)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    b = None if beta is None else np.ascontiguousarray(beta, dtype=np.float32)
    _check(lib().or_layernorm_f32(_p(x), rows, n, eps, _p(g), _p(b), _p(out)),
           "layernorm")
    return out


# ---- matmul / elementwise ------------------------------------------------

def matmul_shape(sa, sb):
    batch_a, batch_b = list(sa[:-2]), list(sb[:-2])
    nd = max(len(batch_a), len(batch_b))
    batch_a = [1] * (nd - len(batch_a)) + batch_a
    batch_b = [1] * (nd - len(batch_b)) + batch_b
    batch = []
    for x, y in zip(batch_a, batch_b):
        if x != y and x != 1 and y != 1:
            raise ValueError("incompatible batch dims")
        batch.append(y if x == 1 else x)
    return tuple(batch) + (sa[-2], sb[-1])


def matmul(a, b, dtype, strides_a=None, strides_b=None, shape_a=None, shape_b=None, threads=1):
    """HostArray matmul over storage arrays (optionally strided views given
    as a base buffer plus element strides); threads > 1 splits the outputs
    over host threads (or_matmul_mt: the same per-output sums)."""
    shape_a = tuple(shape_a if shape_a is not None else a.shape)
    shape_b = tuple(shape_b if shape_b is not None else b.shape)
    if strides_a is None:
        a = np.ascontiguousarray(a)
        strides_a = [s // a.itemsize for s in a.strides]
    if strides_b is None:
        b = np.ascontiguousarray(b)
        strides_b = [s // b.itemsize for s in b.strides]
    shape_c = matmul_shape(shape_a, shape_b)
    c = np.zeros(shape_c, NP_STORAGE[dtype])
    if threads > 1:
        _check(lib().or_matmul_mt(_p(a), _ints(shape_a), _sizes(strides_a), len(shape_a),
                                  _p(b), _ints(shape_b), _sizes(strides_b), len(shape_b),
                                  dtype, _p(c), _ints(shape_c), len(shape_c), int(threads)), "matmul")
        return c
    _check(lib().or_matmul(_p(a), _ints(shape_a), _sizes(strides_a), len(shape_a),
                           _p(b), _ints(shape_b), _sizes(strides_b), len(shape_b),
                           dtype, _p(c), _ints(shape_c), len(shape_c)), "matmul")
    return c


def binary(a, dtype_a, b, dtype_b, op, dtype_out):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    shape = np.broadcast_shapes(a.shape, b.shape)
    out = np.zeros(shape, NP_STORAGE[dtype_out])
    _check(lib().or_binary(_p(a), dtype_a, _ints(a.shape), a.ndim,
                           _p(b), dtype_b, _ints(b.shape), b.ndim, OP[op],
                           _p(out), dtype_out, _ints(shape), len(shape)), op)
    return out


def binary_scalar(a, dtype_a, scalar, op, dtype_out, reverse=False):
    a = np.ascontiguousarray(a)
    out = np.zeros(a.shape, NP_STORAGE[dtype_out])
    _check(lib().or_binary_scalar(_p(a), dtype_a, ctypes.c_size_t(a.size),
                                  ctypes.c_double(scalar), OP[op], int(reverse),
                                  _p(out), dtype_out), op)
    return out


def unary(x, dtype, op):
    x = np.ascontiguousarray(x)
    out = np.zeros(x.shape, x.dtype)
    _check(lib().or_unary(_p(x), dtype, ctypes.c_size_t(x.size), OP[op], _p(out)), op)
    return out


def where(cond, dtype_c, x, y, dtype_xy):
    cond = np.ascontiguousarray(cond)
    x = np.ascontiguousarray(x)
    y = np.ascontiguousarray(y)
    shape = np.broadcast_shapes(cond.shape, x.shape, y.shape)
    out = np.zeros(shape, x.dtype)
    _check(lib().or_where(_p(cond), dtype_c, _ints(cond.shape), cond.ndim,
                          _p(x), _ints(x.shape), x.ndim, _p(y), _ints(y.shape), y.ndim,
                          dtype_xy, _p(out), _ints(shape), len(shape)), "where")
    return out


class OracleIndexError(ValueError):
    """An index outside [0, axis size); `index` is the first one met."""

    def __init__(self, index):
        super().__init__(f"index {index} out of range")
        self.index = index


def gather(x, dtype, indices, axis):
    """CudaArray::gather semantics (indexed_ops.cu:108-133) on contiguous
    storage arrays; raises OracleIndexError for an out-of-range index."""
    x = np.ascontiguousarray(x)
    idx = np.ascontiguousarray(indices, dtype=np.int32)
    out = np.zeros(idx.shape, x.dtype)
    bad = ctypes.c_int32(0)
    st = lib().or_gather(_p(x), dtype, _ints(x.shape), _p(idx), _ints(idx.shape), x.ndim, axis % x.ndim,
                         _p(out), ctypes.byref(bad))
    if st != 0:
        if idx.ndim == x.ndim and all(a == b for d, (a, b) in enumerate(zip(x.shape, idx.shape))
                                      if d != axis % x.ndim):
            raise OracleIndexError(bad.value)
        _check(st, "gather")
    return out


def scatter_add(x, dtype, indices, updates, axis):
    """CudaArray::scatterAdd semantics (indexed_ops.cu:135-204): a copy of x
    with updates added at the indexed positions, in flat index order."""
    x = np.ascontiguousarray(x)
    idx = np.ascontiguousarray(indices, dtype=np.int32)
    upd = np.ascontiguousarray(updates, dtype=x.dtype)
    out = np.zeros_like(x)
    bad = ctypes.c_int32(0)
    st = lib().or_scatter_add(_p(x), dtype, _ints(x.shape), _p(idx), _ints(idx.shape), _p(upd), x.ndim,
                              axis % x.ndim, _p(out), ctypes.byref(bad))
    if st != 0:
        raise OracleIndexError(bad.value)
    return out


def config1_operands():
    """A[256,512] and B[512,256] fp32 U(-1,1)
    from seed S1 = 1 of the SplitMix64 generator (phptensors/synthetic.py):
    one stream of 2 * 131072 values, A first, then B."""
    from phptensors import synthetic
    ab = synthetic.uniform((2 * 256 * 512,), -1.0, 1.0, seed=1)
    return ab[:256 * 512].reshape(256, 512).copy(), ab[256 * 512:].reshape(512, 256).copy()
