"""CudaArray: the reference's PhpTensors\\CudaArray surface for the hot path,
over the host runtime (host/phpt_host.h) and the gfx950 C-ABI.

Method names, argument meaning and exception types follow
stubs/cuda.stub.php (CudaArray, :410-620 of that file) so that a test written
against the PHP class reads the same here.  Every operation runs on the GPU;
when the HIP libraries are not built, the first call raises RuntimeException.
"""
import ctypes
import numbers

import numpy as np

from . import _abi, _host
from . import autograd as AG
from ._abi import InvalidArgumentException, RuntimeException  # noqa: F401

GLOBAL_AXIS = -1000

# include/pt_hip.h dtype codes and the names the reference prints
DTYPES = {
    "float32": 0, "float64": 1, "int8": 2, "int16": 3, "int32": 4, "int64": 5,
    "uint8": 6, "uint16": 7, "uint32": 8, "uint64": 9, "bool": 10,
    "float16": 11, "bfloat16": 12,
}
DTYPE_NAMES = {v: k for k, v in DTYPES.items()}
NUMPY_OF = {
    0: np.float32, 1: np.float64, 2: np.int8, 3: np.int16, 4: np.int32, 5: np.int64,
    6: np.uint8, 7: np.uint16, 8: np.uint32, 9: np.uint64, 10: np.bool_,
    11: np.float16, 12: np.uint16,   # bfloat16 travels as its 16-bit pattern
}
CODE_OF_NUMPY = {np.dtype(v): k for k, v in NUMPY_OF.items() if k not in (12,)}
# host storage of element bit patterns (both 16-bit float types as uint16)
BITS_OF = dict(NUMPY_OF)
BITS_OF[11] = np.uint16

# include/pt_hip.h operation codes (operation_type_t of the reference)
OP = dict(ADD=0, SUB=1, MUL=2, DIV=3, POW=4, EXP=5, EXPM1=6, SQRT=7, LOG=8, LOG1P=9,
          EXP2=10, LOG2=11, LOG10=12, ASIN=13, ACOS=14, ATAN=15, SINH=16, COSH=17,
          TANH=18, SIN=19, COS=20, TAN=21, ABS=22, NEG=23, CEIL=26, FLOOR=27, ROUND=28,
          GT=29, LT=30, EQ=31, NE=32, GE=33, LE=34, SUM=35, MEAN=36, MAX=37, MIN=38,
          PROD=39, ARG_MAX=42, ARG_MIN=43, MAXIMUM=54, MINIMUM=55, ALL=57, ANY=58)


def dtype_code(dtype):
    if dtype is None:
        return DTYPES["float32"]
    if isinstance(dtype, int):
        return dtype
    code = _host.load().phpt_dtype_from_name(str(dtype).encode())
    if code < 0:
        raise InvalidArgumentException(f"Unknown dtype '{dtype}'")
    return code


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x):
    """Round-to-nearest-even float32 -> bfloat16 bit pattern (data_types.c:96-131)."""
    x = np.asarray(x, dtype=np.float32)
    u = np.ascontiguousarray(x).view(np.uint32).reshape(x.shape)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def _scalar_args(value):
    if isinstance(value, (bool, np.bool_)):
        return 0.0, int(bool(value)), 2
    if isinstance(value, numbers.Integral):
        return 0.0, int(value), 1
    if isinstance(value, numbers.Real):
        return float(value), 0, 0
    raise InvalidArgumentException(f"Unsupported scalar operand of type {type(value).__name__}")


INT32_MIN, INT32_MAX = -2**31, 2**31 - 1


def _int32(v, what="value"):
    """An extent, index or axis for the C boundary: values outside int32 are
    refused rather than narrowed (tests/cuda_shape_boundaries.phpt:23-36)."""
    v = int(v)
    if not INT32_MIN <= v <= INT32_MAX:
        raise InvalidArgumentException(f"{what} {v} is out of range")
    return v


def _ints(seq):
    seq = [_int32(v, "dimension") for v in seq]
    return (ctypes.c_int * max(1, len(seq)))(*seq), len(seq)


LN2 = 0.69314718055994530942
LN10 = 2.30258509299404568402


def _unary_backward(op, x, out):
    """Derivative of each unary operation (autograd.c:1306-1480): logarithms
    route NaN outside their domain (x < 0, or x < -1 for log1p); rounding has
    a zero gradient."""
    def outside(ga, bound):
        return CudaArray.where(x.lt(bound), CudaArray.full([1], float("nan"), ga.getDtype()), ga)

    if op == OP["EXP"]:
        return lambda g: [g * out]
    if op == OP["EXPM1"]:
        return lambda g: [g * x.exp()]
    if op == OP["EXP2"]:
        return lambda g: [g * (out * LN2)]
    if op == OP["LOG"]:
        return lambda g: [outside(g / x, 0.0)]
    if op == OP["LOG1P"]:
        return lambda g: [outside(g / (x + 1.0), -1.0)]
    if op == OP["LOG2"]:
        return lambda g: [outside(g / (x * LN2), 0.0)]
    if op == OP["LOG10"]:
        return lambda g: [outside(g / (x * LN10), 0.0)]
    if op == OP["ASIN"]:
        return lambda g: [g / (1.0 - x * x).sqrt()]
    if op == OP["ACOS"]:
        return lambda g: [-(g / (1.0 - x * x).sqrt())]
    if op == OP["ATAN"]:
        return lambda g: [g / (x * x + 1.0)]
    if op == OP["SINH"]:
        return lambda g: [g * x.cosh()]
    if op == OP["COSH"]:
        return lambda g: [g * x.sinh()]
    if op == OP["TANH"]:
        return lambda g: [g * (1.0 - out * out)]
    if op == OP["SQRT"]:
        return lambda g: [g / (out * 2.0)]
    if op == OP["SIN"]:
        return lambda g: [g * x.cos()]
    if op == OP["COS"]:
        return lambda g: [g * -x.sin()]
    if op == OP["TAN"]:
        return lambda g: [g / (x.cos() * x.cos())]
    if op == OP["ABS"]:
        def abs_back(g):
            zero = g * 0.0
            return [CudaArray.where(x.gt(0.0), g, CudaArray.where(x.lt(0.0), -g, zero))]
        return abs_back
    if op == OP["NEG"]:
        return lambda g: [-g]
    if op in (OP["CEIL"], OP["FLOOR"], OP["ROUND"]):
        return lambda g: [g * 0.0]
    return None


def _nested_array(data):
    """Nested lists of numbers (or a numpy array) as a rectangular numeric
    array of rank at most 10; ragged, non-numeric or deeper input raises
    InvalidArgumentException, as the reference's constructor does."""
    if isinstance(data, np.ndarray):
        arr = data
    else:
        try:
            arr = np.asarray(data)
        except (ValueError, TypeError) as exc:
            raise InvalidArgumentException(f"CudaArray input must be a rectangular numeric array: {exc}")
    if arr.dtype.kind not in "biuf":
        raise InvalidArgumentException("CudaArray input must hold numbers or booleans only")
    if arr.ndim > 10:
        raise InvalidArgumentException("CudaArray input is nested deeper than 10 dimensions")
    return arr


def _bound(text):
    text = text.strip()
    return None if text == "" else int(text)


def _parse_selector(text):
    """One selector of a slice() expression: "i", ":", "a:b", "a:b:c"."""
    text = text.strip()
    if ":" not in text:
        if text == "":
            raise InvalidArgumentException("slice() selector is empty")
        return ("index", int(text))
    parts = text.split(":")
    if len(parts) > 3:
        raise InvalidArgumentException(f"slice() selector '{text}' has too many ':'")
    parts += [""] * (3 - len(parts))
    return ("range", tuple(_bound(p) for p in parts))


def _selector(sel):
    if sel is None:
        return ("range", (None, None, None))
    if isinstance(sel, (bool, np.bool_)):
        raise InvalidArgumentException("slice() selectors cannot be booleans")
    if isinstance(sel, (int, np.integer)):
        return ("index", int(sel))
    if isinstance(sel, (list, tuple)):
        if not 1 <= len(sel) <= 3:
            raise InvalidArgumentException("slice() ranges are [start, stop] or [start, stop, step]")
        vals = [None if v is None else int(v) for v in sel] + [None] * (3 - len(sel))
        return ("range", tuple(vals))
    raise InvalidArgumentException(f"Unsupported slice() selector {sel!r}")


class CudaArray:
    """GPU tensor handle (src/tensor.h tensor_t behind a CudaArray object)."""

    __slots__ = ("_h", "_rg", "_node", "_grad", "__weakref__")

    def __init__(self, data=None, dtype="float32"):
        self._h = None
        self._rg = False
        self._node = None
        self._grad = None
        if data is None:
            return
        self._h = _from_numpy(_nested_array(data), dtype_code(dtype))

    @classmethod
    def _wrap(cls, handle, what=""):
        _host.check_handle(handle, what)
        obj = cls.__new__(cls)
        obj._h = handle
        obj._rg = False
        obj._node = None
        obj._grad = None
        return obj

    def __del__(self):
        h = getattr(self, "_h", None)
        if h and _host._lib is not None:
            _host._lib.phpt_release(h)
            self._h = None

    # ------------------------------------------------------------ factories
    @classmethod
    def fromNumpy(cls, arr, dtype=None):
        """Upload a host array (HostArray::toGpu -> tensor_factory.c:301-326).
        float16 / bfloat16 input is given either as uint16 bit patterns or as
        values (rounded to nearest even)."""
        arr = np.asarray(arr)
        code = dtype_code(dtype) if dtype is not None else CODE_OF_NUMPY.get(arr.dtype)
        if code is None:
            raise InvalidArgumentException(f"Unsupported host dtype {arr.dtype}")
        return cls._wrap(_from_numpy(arr, code), "fromNumpy")

    @classmethod
    def fromFlatArray(cls, values, shape, dtype="float32"):
        """A flat list of numbers laid out in `shape` (non-negative extents
        whose product is the list's length)."""
        arr = _nested_array(values)
        if arr.ndim > 1:
            raise InvalidArgumentException("fromFlatArray() expects a flat list of values")
        shape = [int(d) for d in shape]
        if any(d < 0 for d in shape) or int(np.prod(shape, dtype=object)) != arr.size:
            raise InvalidArgumentException(
                f"fromFlatArray() shape {shape} does not hold {arr.size} values")
        return cls.fromNumpy(arr.reshape(shape), dtype)

    @classmethod
    def fromBuffer(cls, data, shape, dtype="float32"):
        """Raw little-endian element bytes (cuda_array_ce.c:151-187)."""
        code = dtype_code(dtype)
        arr = np.frombuffer(bytes(data), dtype=NUMPY_OF[code])
        n = int(np.prod(shape)) if len(shape) else 1
        if arr.size != n:
            raise InvalidArgumentException(
                f"Buffer holds {arr.size} elements, shape needs {n}")
        return cls._wrap(_from_bits(arr.reshape(shape), code), "fromBuffer")

    @classmethod
    def full(cls, shape, value, dtype="float32"):
        v, iv, kind = _scalar_args(value)
        sh, n = _ints(shape)
        return cls._wrap(_host.load().phpt_full(sh, n, dtype_code(dtype), v, iv, kind), "full")

    @classmethod
    def zeros(cls, shape, dtype="float32"):
        return cls.full(shape, 0, dtype)

    @classmethod
    def ones(cls, shape, dtype="float32"):
        return cls.full(shape, 1, dtype)

    @classmethod
    def where(cls, condition, x, y):
        out = cls._wrap(_host.load().phpt_where(condition._h, x._h, y._h), "where")
        if AG.active(x, y):
            def back(g):
                zero = g * 0.0
                gx = AG.reduce_to(CudaArray.where(condition, g, zero), x.getShape()) if AG.needs_grad(x) else None
                gy = AG.reduce_to(CudaArray.where(condition, zero, g), y.getShape()) if AG.needs_grad(y) else None
                return [gx, gy]
            AG.record(out, [x, y], back, "where")
        return out

    # ------------------------------------------------------------ metadata
    def getShape(self):
        lib = _host.load()
        nd = lib.phpt_ndims(self._h)
        buf = (ctypes.c_int * max(1, nd))()
        lib.phpt_shape(self._h, buf)
        return [buf[i] for i in range(nd)]

    @property
    def shape(self):
        return tuple(self.getShape())

    def getStrides(self):
        lib = _host.load()
        nd = lib.phpt_ndims(self._h)
        buf = (ctypes.c_size_t * max(1, nd))()
        lib.phpt_strides(self._h, buf)
        return [buf[i] for i in range(nd)]

    def getNdims(self):
        return _host.load().phpt_ndims(self._h)

    def getSize(self):
        return int(_host.load().phpt_size(self._h))

    def count(self):
        return self.getSize()

    def getDtype(self):
        return DTYPE_NAMES[_host.load().phpt_dtype(self._h)]

    dtype = getDtype

    def dtypeCode(self):
        return _host.load().phpt_dtype(self._h)

    def isLazy(self):
        return bool(_host.load().phpt_is_lazy(self._h))

    # ------------------------------------------------------------ transfers
    def toBits(self):
        """Element bit patterns in a numpy array (float16 / bfloat16 as uint16)."""
        code = self.dtypeCode()
        out = np.empty(self.shape, dtype=BITS_OF[code])
        if _host.load().phpt_to_host(self._h, out.ctypes.data_as(ctypes.c_void_p), out.nbytes) != 0:
            _host.raise_error("toHost")
        return out

    def toNumpy(self):
        """Values in numpy (bfloat16 widened to float32)."""
        bits = self.toBits()
        code = self.dtypeCode()
        if code == DTYPES["bfloat16"]:
            return bf16_bits_to_f32(bits)
        if code == DTYPES["float16"]:
            return bits.view(np.float16)
        return bits

    def toArray(self):
        """Nested lists; a rank-0 tensor exports as a one-element list, as the
        reference's toArray() does (tests/slice.phpt:22-24)."""
        values = self.toNumpy().tolist()
        return [values] if self.getNdims() == 0 else values

    def toBuffer(self):
        """Raw element bytes, row-major (cuda_array_ce.c:2943-2951)."""
        return self.toBits().tobytes()

    def item(self):
        if self.getSize() != 1:
            raise InvalidArgumentException("item() requires a tensor with exactly one element")
        return self.toNumpy().reshape(-1)[0].item()

    # ------------------------------------------------------------ elementwise
    def _binary(self, other, op, reverse=False):
        lib = _host.load()
        if isinstance(other, CudaArray):
            a, b = (other, self) if reverse else (self, other)
            out = CudaArray._wrap(lib.phpt_binary(a._h, b._h, op))
            if AG.active(a, b):
                _record_binary(out, a, b, op)
            return out
        v, iv, kind = _scalar_args(other)
        out = CudaArray._wrap(lib.phpt_scalar_op(self._h, v, iv, kind, op, 1 if reverse else 0))
        if AG.active(self):
            _record_scalar(out, self, other, op, reverse)
        return out

    def add(self, other):
        return self._binary(other, OP["ADD"])

    def subtract(self, other):
        return self._binary(other, OP["SUB"])

    def multiply(self, other):
        return self._binary(other, OP["MUL"])

    def divide(self, other):
        return self._binary(other, OP["DIV"])

    def power(self, other):
        return self._binary(other, OP["POW"])

    def maximum(self, other):
        return self._binary(other, OP["MAXIMUM"])

    def minimum(self, other):
        return self._binary(other, OP["MINIMUM"])

    def gt(self, other):
        return self._binary(other, OP["GT"])

    def lt(self, other):
        return self._binary(other, OP["LT"])

    def eq(self, other):
        return self._binary(other, OP["EQ"])

    def ne(self, other):
        return self._binary(other, OP["NE"])

    def ge(self, other):
        return self._binary(other, OP["GE"])

    def le(self, other):
        return self._binary(other, OP["LE"])

    def clamp(self, min=None, max=None):
        out = self
        if min is not None:
            out = out.maximum(min)
        if max is not None:
            out = out.minimum(max)
        return out if out is not self else self.copy()

    __add__ = add
    __sub__ = subtract
    __mul__ = multiply
    __truediv__ = divide
    __pow__ = power

    def __radd__(self, other):
        return self._binary(other, OP["ADD"], reverse=True)

    def __rsub__(self, other):
        return self._binary(other, OP["SUB"], reverse=True)

    def __rmul__(self, other):
        return self._binary(other, OP["MUL"], reverse=True)

    def __rtruediv__(self, other):
        return self._binary(other, OP["DIV"], reverse=True)

    def __rpow__(self, other):
        return self._binary(other, OP["POW"], reverse=True)

    def __neg__(self):
        return self.neg()

    def __matmul__(self, other):
        return self.matmul(other)

    def _unary(self, op):
        out = CudaArray._wrap(_host.load().phpt_unary(self._h, op))
        if AG.active(self):
            back = _unary_backward(op, self, out)
            if back is None:
                raise InvalidArgumentException("Backward is not implemented for this unary operation")
            AG.record(out, [self], back, "unary")
        return out

    def sqrt(self): return self._unary(OP["SQRT"])
    def exp(self): return self._unary(OP["EXP"])
    def expm1(self): return self._unary(OP["EXPM1"])
    def exp2(self): return self._unary(OP["EXP2"])
    def log(self): return self._unary(OP["LOG"])
    def log1p(self): return self._unary(OP["LOG1P"])
    def log2(self): return self._unary(OP["LOG2"])
    def log10(self): return self._unary(OP["LOG10"])
    def sin(self): return self._unary(OP["SIN"])
    def cos(self): return self._unary(OP["COS"])
    def tan(self): return self._unary(OP["TAN"])
    def asin(self): return self._unary(OP["ASIN"])
    def acos(self): return self._unary(OP["ACOS"])
    def atan(self): return self._unary(OP["ATAN"])
    def sinh(self): return self._unary(OP["SINH"])
    def cosh(self): return self._unary(OP["COSH"])
    def tanh(self): return self._unary(OP["TANH"])
    def abs(self): return self._unary(OP["ABS"])
    def neg(self): return self._unary(OP["NEG"])
    def floor(self): return self._unary(OP["FLOOR"])
    def ceil(self): return self._unary(OP["CEIL"])
    def round(self): return self._unary(OP["ROUND"])

    def astype(self, dtype):
        return CudaArray._wrap(_host.load().phpt_astype(self._h, dtype_code(dtype)))

    def copy(self):
        return CudaArray._wrap(_host.load().phpt_copy(self._h))

    # ------------------------------------------------------------ reductions
    @staticmethod
    def _axis(axis):
        return GLOBAL_AXIS if axis is None else _int32(axis, "axis")

    def _reduce(self, axis, op):
        out = CudaArray._wrap(_host.load().phpt_reduce(self._h, self._axis(axis), op))
        if AG.active(self):
            _record_reduce(out, self, axis, op)
        return out

    def sum(self, axis=None): return self._reduce(axis, OP["SUM"])
    def mean(self, axis=None): return self._reduce(axis, OP["MEAN"])
    def max(self, axis=None): return self._reduce(axis, OP["MAX"])
    def min(self, axis=None): return self._reduce(axis, OP["MIN"])
    def prod(self, axis=None): return self._reduce(axis, OP["PROD"])

    def all(self, axis=None):
        """bool: every element along axis is unequal to zero (cuda_array_ce.c:1791-1806);
        a discrete output, so no gradient is recorded."""
        return CudaArray._wrap(_host.load().phpt_reduce(self._h, self._axis(axis), OP["ALL"]))

    def any(self, axis=None):
        """bool: some element along axis is unequal to zero (cuda_array_ce.c:1808-1823)."""
        return CudaArray._wrap(_host.load().phpt_reduce(self._h, self._axis(axis), OP["ANY"]))

    def argMax(self, axis=None):
        return CudaArray._wrap(_host.load().phpt_reduce_arg(self._h, self._axis(axis), OP["ARG_MAX"]))

    def argMin(self, axis=None):
        return CudaArray._wrap(_host.load().phpt_reduce_arg(self._h, self._axis(axis), OP["ARG_MIN"]))

    def var(self, axis=None, correction=0):
        return CudaArray._wrap(_host.load().phpt_variance(self._h, self._axis(axis), int(correction), 0))

    def std(self, axis=None, correction=0):
        return CudaArray._wrap(_host.load().phpt_variance(self._h, self._axis(axis), int(correction), 1))

    def softmax(self, axis=-1):
        return CudaArray._wrap(_host.load().phpt_softmax(self._h, int(axis)))

    def layerNorm(self, axes, epsilon=1e-5, scale=None, bias=None):
        ax, n = _ints(axes)
        return CudaArray._wrap(_host.load().phpt_layernorm(
            self._h, ax, n, float(epsilon), scale._h if scale is not None else None,
            bias._h if bias is not None else None))

    def matmul(self, other):
        if not isinstance(other, CudaArray):
            raise InvalidArgumentException("matmul() expects a CudaArray operand")
        out = CudaArray._wrap(_host.load().phpt_matmul(self._h, other._h))
        if AG.active(self, other):
            a, b = self, other

            def back(g):
                # upstream @ B^T and A^T @ upstream over transposed views (autograd.c:1539-1585)
                ga = AG.reduce_to(g.matmul(b.swapaxes(-1, -2)), a.getShape()) if AG.needs_grad(a) else None
                gb = AG.reduce_to(a.swapaxes(-1, -2).matmul(g), b.getShape()) if AG.needs_grad(b) else None
                return [ga, gb]
            AG.record(out, [a, b], back, "matmul")
        return out

    # ------------------------------------------------------------ indexed
    def gather(self, indices, axis=0):
        """out[c] = self[c with c[axis] := indices[c]] (int32 indices of the
        same rank, cuda_array_ce.c:2423-2442); the gradient scatters the
        upstream gradient back (autograd.c:1631-1646), in float32 for
        float16 / bfloat16 inputs."""
        if not isinstance(indices, CudaArray):
            raise InvalidArgumentException("gather() expects CudaArray indices")
        out = CudaArray._wrap(_host.load().phpt_gather(self._h, indices._h, int(axis)), "gather")
        if AG.active(self):
            src = self
            ax = int(axis) % self.getNdims()

            def back(g):
                zdt = "float32" if src.getDtype() in ("float16", "bfloat16") else src.getDtype()
                return [CudaArray.zeros(src.getShape(), zdt).scatterAdd(indices, g, ax)]
            AG.record(out, [self], back, "gather")
        return out

    def scatterAdd(self, indices, updates, axis=0):
        """A copy of self with updates[c] added at c with c[axis] :=
        indices[c] (cuda_array_ce.c:2444-2465); float16 / bfloat16 run and
        return float32.  Gradients: the input's is the upstream gradient,
        the updates' its gather (autograd.c:1648-1652)."""
        if not isinstance(indices, CudaArray) or not isinstance(updates, CudaArray):
            raise InvalidArgumentException("scatterAdd() expects CudaArray indices and updates")
        out = CudaArray._wrap(_host.load().phpt_scatter_add(self._h, indices._h, updates._h, int(axis)),
                              "scatterAdd")
        if AG.active(self, updates):
            ax = int(axis) % self.getNdims()

            def back(g):
                return [g, g.gather(indices, ax) if AG.needs_grad(updates) else None]
            AG.record(out, [self, updates], back, "scatterAdd")
        return out

    # ------------------------------------------------------------ views
    def reshape(self, shape):
        sh, n = _ints(shape)
        out = CudaArray._wrap(_host.load().phpt_reshape(self._h, sh, n))
        if AG.active(self):
            src = self.getShape()
            AG.record(out, [self], lambda g: [g.reshape(src)], "reshape")
        return out

    def flatten(self):
        return self.reshape([-1])

    def transpose(self, axis=None):
        nd = self.getNdims()
        if axis is not None and any(not -nd <= int(a) < nd for a in axis):
            raise InvalidArgumentException(f"transpose() axes {list(axis)} are out of range for rank {nd}")
        perm = list(range(nd))[::-1] if axis is None else [int(a) % nd for a in axis]
        p, n = _ints(perm)
        out = CudaArray._wrap(_host.load().phpt_transpose(self._h, p, n))
        if AG.active(self):
            inv = [0] * nd
            for i, a in enumerate(perm):
                inv[a] = i
            AG.record(out, [self], lambda g: [g.transpose(inv)], "transpose")
        return out

    @property
    def T(self):
        return self.transpose()

    def swapaxes(self, axis1, axis2):
        nd = self.getNdims()
        perm = list(range(nd))
        a1, a2 = axis1 % nd if nd else 0, axis2 % nd if nd else 0
        perm[a1], perm[a2] = perm[a2], perm[a1]
        return self.transpose(perm)

    def broadcastTo(self, shape):
        sh, n = _ints(shape)
        out = CudaArray._wrap(_host.load().phpt_broadcast_to(self._h, sh, n))
        if AG.active(self):
            src = self.getShape()
            AG.record(out, [self], lambda g: [AG.reduce_to(g, src)], "broadcast")
        return out

    def slice(self, *selectors):
        """CudaArray::slice(int|string|array|null ...$selectors)
        (stubs/cuda.stub.php:441-444): a view with one selector per leading
        axis.  An int is an index and drops its axis; [start, stop(, step)]
        or "start:stop:step" is an exclusive-stop range with a positive step
        (negative bounds count from the end, bounds clip to the axis, empty
        parts take their defaults); None or ":" keeps the axis whole; a
        string may hold several comma-separated selectors."""
        parsed = []
        for sel in selectors:
            if isinstance(sel, str):
                parsed.extend(_parse_selector(part) for part in sel.split(","))
            else:
                parsed.append(_selector(sel))
        if len(parsed) > self.getNdims():
            raise InvalidArgumentException(
                f"slice() got {len(parsed)} selectors for a tensor of rank {self.getNdims()}")
        out, axis = self, 0
        for kind, value in parsed:
            if kind == "index":
                out = out.select(axis, value)
                continue
            start, stop, step = value
            n = out.getShape()[axis]
            start = 0 if start is None else start
            stop = n if stop is None else stop
            step = 1 if step is None else step
            if step <= 0:
                raise InvalidArgumentException("slice() steps must be positive")
            start = max(-n, min(start, n))
            stop = max(-n, min(stop, n))
            out = out._slice_axis(axis, start, stop, step)
            axis += 1
        if out is self:  # no selectors: the whole tensor as a view
            out = CudaArray._wrap(_host.load().phpt_retain(self._h))
        return out

    def _slice_axis(self, axis, start, stop, step=1):
        return CudaArray._wrap(_host.load().phpt_slice(self._h, int(axis), int(start), int(stop), int(step)))

    def select(self, axis, index):
        return CudaArray._wrap(_host.load().phpt_select(self._h, _int32(axis, "axis"), _int32(index, "index")))

    def unsqueeze(self, axis):
        shape = self.getShape()
        axis = axis + len(shape) + 1 if axis < 0 else axis
        shape.insert(axis, 1)
        return self.reshape(shape)

    def squeeze(self, axis=None):
        shape = self.getShape()
        if axis is None:
            new = [s for s in shape if s != 1]
        else:
            axis = axis % len(shape)
            if shape[axis] != 1:
                raise InvalidArgumentException("Cannot squeeze an axis whose size is not 1")
            new = shape[:axis] + shape[axis + 1:]
        return self.reshape(new)

    # ------------------------------------------------------------ autograd
    def requiresGrad(self, requiresGrad=True):
        """Mark a leaf for gradient accumulation (returns self)."""
        if requiresGrad and self.getDtype() not in ("float32", "float64", "float16", "bfloat16"):
            raise InvalidArgumentException("Only floating tensors can require gradients")
        self._rg = bool(requiresGrad)
        return self

    def backward(self, gradient=None, retainGraph=False):
        """autograd_backward (autograd.c:1710-1735): argument checks, then
        the reverse walk."""
        if not AG.needs_grad(self):
            raise InvalidArgumentException("backward() requires a tensor marked with requiresGrad()")
        if self.getDtype() not in ("float32", "float64", "float16", "bfloat16"):
            raise InvalidArgumentException(
                "backward() is only supported for float32, float64, float16 and bfloat16 tensors")
        if gradient is None and self.getSize() != 1:
            raise InvalidArgumentException(
                "A gradient seed is required when backward() is called on a non-scalar tensor")
        if gradient is not None and (gradient.getShape() != self.getShape()
                                     or gradient.getDtype() != self.getDtype()):
            raise InvalidArgumentException("The backward gradient seed must match the tensor shape and dtype")
        AG.backward(self, gradient)
        if not retainGraph:
            self._node = None

    def grad(self):
        return self._grad

    def zeroGrad(self):
        self._grad = None

    def detach(self):
        """Same values, no history (a new handle on the same storage)."""
        return CudaArray._wrap(_host.load().phpt_retain(self._h))

    def __repr__(self):
        return f"CudaArray(shape={self.getShape()}, dtype={self.getDtype()})"


def _from_bits(arr, code):
    # np.ascontiguousarray would turn a rank-0 array into shape (1,)
    arr = np.asarray(arr)
    if not arr.flags.c_contiguous:
        arr = arr.copy(order="C")
    sh, n = _ints(arr.shape)
    return _host.load().phpt_from_host(arr.ctypes.data_as(ctypes.c_void_p), code, sh, n)


def _from_numpy(arr, code):
    arr = np.asarray(arr)
    if code in (DTYPES["bfloat16"], DTYPES["float16"]) and arr.dtype == np.uint16:
        h = _from_bits(arr, code)          # 16-bit patterns as given
    elif code == DTYPES["bfloat16"]:
        h = _from_bits(f32_to_bf16_bits(arr.astype(np.float32)), code)
    else:
        h = _from_bits(arr.astype(NUMPY_OF[code], copy=False), code)
    return _host.check_handle(h, "upload")


# ------------------------------------------------------------ gradient recorders
def _record_binary(out, a, b, op):
    if op == OP["ADD"]:
        back = lambda g: [AG.reduce_to(g, a.getShape()) if AG.needs_grad(a) else None,  # noqa: E731
                          AG.reduce_to(g, b.getShape()) if AG.needs_grad(b) else None]
    elif op == OP["SUB"]:
        back = lambda g: [AG.reduce_to(g, a.getShape()) if AG.needs_grad(a) else None,  # noqa: E731
                          AG.reduce_to(-g, b.getShape()) if AG.needs_grad(b) else None]
    elif op == OP["MUL"]:
        back = lambda g: [AG.reduce_to(g * b, a.getShape()) if AG.needs_grad(a) else None,  # noqa: E731
                          AG.reduce_to(g * a, b.getShape()) if AG.needs_grad(b) else None]
    elif op == OP["DIV"]:
        back = lambda g: [AG.reduce_to(g / b, a.getShape()) if AG.needs_grad(a) else None,  # noqa: E731
                          AG.reduce_to(-(g * a) / (b * b), b.getShape()) if AG.needs_grad(b) else None]
    elif op in (OP["GT"], OP["LT"], OP["EQ"], OP["NE"], OP["GE"], OP["LE"]):
        return  # comparisons carry no gradient
    else:
        raise InvalidArgumentException("Backward is not implemented for this binary operation")
    AG.record(out, [a, b], back, "binary")


def _record_scalar(out, a, s, op, reverse):
    if op == OP["ADD"]:
        back = lambda g: [g]  # noqa: E731
    elif op == OP["SUB"]:
        back = (lambda g: [-g]) if reverse else (lambda g: [g])  # noqa: E731
    elif op == OP["MUL"]:
        back = lambda g: [g * s]  # noqa: E731
    elif op == OP["DIV"]:
        back = (lambda g: [-(g * s) / (a * a)]) if reverse else (lambda g: [g / s])  # noqa: E731
    elif op == OP["POW"] and not reverse:
        # x ** s: g * (x ** (s - 1) * s); zero for s == 0 (autograd.c:1256-1280)
        if float(s) == 0.0:
            back = lambda g: [g * 0.0]  # noqa: E731
        else:
            back = lambda g: [g * ((a.astype(g.getDtype()) ** (float(s) - 1.0)) * s)]  # noqa: E731
    elif op in (OP["MAXIMUM"], OP["MINIMUM"]):
        # the tensor side takes the gradient where it wins, half of it at a
        # tie with the scalar (autograd.c:1282-1296)
        def back(g):
            wins = a.ge(s) if op == OP["MAXIMUM"] else a.le(s)
            zeros = g * 0.0
            return [CudaArray.where(a.eq(s), g * 0.5, CudaArray.where(wins, g, zeros))]
    elif op in (OP["GT"], OP["LT"], OP["EQ"], OP["NE"], OP["GE"], OP["LE"]):
        return
    else:
        raise InvalidArgumentException("Backward is not implemented for this scalar operation")
    AG.record(out, [a], back, "scalar")


def _record_reduce(out, a, axis, op):
    shape = a.getShape()
    ax = None if axis is None else axis % len(shape)
    if op == OP["SUM"]:
        back = lambda g: [AG.expand_reduced(g, shape, ax)]  # noqa: E731
    elif op == OP["MEAN"]:
        n = a.getSize() if ax is None else shape[ax]
        back = lambda g: [AG.expand_reduced(g / float(n), shape, ax)]  # noqa: E731
    elif op in (OP["MAX"], OP["MIN"]):
        def back(g):
            # the upstream gradient is shared equally among the extrema
            # (autograd.c:945-1003)
            hit = a.eq(AG.expand_reduced(out, shape, ax)).astype(g.getDtype())
            counts = hit.sum() if ax is None else hit.sum(ax)
            share = AG.expand_reduced(g / counts, shape, ax)
            return [CudaArray.where(hit, share, share * 0.0)]
    else:
        raise InvalidArgumentException("Backward is not implemented for this reduction")
    AG.record(out, [a], back, "reduce")


# ------------------------------------------------------------ serialization
# CudaArray::__serialize / __unserialize (cuda_array_ce.c:270-366): a
# versioned payload of metadata and the raw row-major element bytes.  The
# validation of a payload restates tensor_import_serialized_shape
# (tensor_import.c:90-123) and the size checks of :337-352; a payload that
# fails any check raises InvalidArgumentException and leaves the target
# unchanged.  Snapshots carry values only, never gradients or history.
_SERIAL_VERSION = "__cuda_array_v1"
_MAX_DIMS = 10
_LONG_MAX = 2 ** 63 - 1
_INT_MAX = 2 ** 31 - 1


def _is_long(v):
    return isinstance(v, int) and not isinstance(v, bool)


def _serialize(self):
    lib = _host.load()
    if lib.phpt_is_view(self._h):
        raise RuntimeException("Cannot serialize non-contiguous CudaArray views")
    code = lib.phpt_dtype(self._h)
    return {_SERIAL_VERSION: "1", "ndims": self.getNdims(), "dtype": DTYPE_NAMES[code],
            "total_elements": self.getSize(), "element_size": np.dtype(BITS_OF[code]).itemsize,
            "shape": self.getShape(), "data": self.toBuffer()}


def _payload_tensor(data):
    if not isinstance(data, dict):
        raise InvalidArgumentException("Invalid serialized CudaArray payload")
    version = data.get(_SERIAL_VERSION)
    if not isinstance(version, str) or version != "1":
        raise InvalidArgumentException("Invalid serialized CudaArray payload")
    nd, dt, shape = data.get("ndims"), data.get("dtype"), data.get("shape")
    raw, total, esize = data.get("data"), data.get("total_elements"), data.get("element_size")
    if (not _is_long(nd) or not isinstance(dt, str) or not isinstance(shape, (list, tuple))
            or not isinstance(raw, (bytes, bytearray)) or not _is_long(total) or not _is_long(esize)):
        raise InvalidArgumentException("Malformed serialized CudaArray payload")
    if "\0" in dt or dt not in DTYPES:
        raise InvalidArgumentException(f"Invalid serialized CudaArray dtype: {dt.split(chr(0))[0]}")
    code = DTYPES[dt]
    if nd < 0 or nd > _MAX_DIMS or len(shape) != nd:
        raise InvalidArgumentException("Invalid serialized tensor shape")
    for d in shape:
        if not _is_long(d) or d < 0 or d > _INT_MAX:
            raise InvalidArgumentException("Invalid serialized tensor dimension")
    elements = 1
    for d in reversed(shape):
        if elements > _LONG_MAX or (d and elements > _LONG_MAX // d):
            raise InvalidArgumentException("Serialized tensor shape or strides exceed supported limits")
        elements *= d
    width = np.dtype(BITS_OF[code]).itemsize
    if total < 0 or total != elements or esize != width:
        raise InvalidArgumentException("Invalid serialized CudaArray size metadata")
    if len(raw) != elements * width:
        raise InvalidArgumentException(
            f"Serialized CudaArray data size mismatch: expected {elements * width} bytes, got {len(raw)}")
    return CudaArray.fromBuffer(bytes(raw), list(shape), dt)


def _unserialize(self, data):
    fresh = _payload_tensor(data)
    old = self._h
    self._h, fresh._h = fresh._h, old
    self._rg = False
    self._node = None
    self._grad = None


def _reduce(self):
    return (_payload_tensor, (_serialize(self),))


setattr(CudaArray, "__serialize", _serialize)
setattr(CudaArray, "__unserialize", _unserialize)
CudaArray.__reduce__ = _reduce
