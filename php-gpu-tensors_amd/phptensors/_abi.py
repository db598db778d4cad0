"""ctypes view of the C-ABI in include/pt_hip.h (lib/libpt_hip.so).

This is the userland side of the boundary, the role PHP's Zend glue plays
for the reference: plain pointers, sizes and the reference's dtype/op
codes.  Loading fails loudly when the HIP library has not been built;
there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_DIR = os.path.join(PKG, "lib")
DEVICE_LIB = os.path.join(LIB_DIR, "libpt_hip.so")

# status codes
PT_OK, PT_ERR_INVALID, PT_ERR_RUNTIME, PT_ERR_UNSUPPORTED, PT_ERR_NOMEM, PT_ERR_COMPILE, \
    PT_ERR_NO_DEVICE = range(7)

# dtype codes (reference src/data_types.h:8-25)
FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, UINT8, UINT16, UINT32, UINT64, BOOL, \
    FLOAT16, BFLOAT16 = range(13)
DTYPE_NAMES = ["float32", "float64", "int8", "int16", "int32", "int64", "uint8", "uint16",
               "uint32", "uint64", "bool", "float16", "bfloat16"]
DTYPE_CODES = {n: i for i, n in enumerate(DTYPE_NAMES)}
DTYPE_SIZES = [4, 8, 1, 2, 4, 8, 1, 2, 4, 8, 1, 2, 2]

# op codes (reference src/operations_strctures.h:4-67)
OP = dict(
    add=0, sub=1, mul=2, div=3, pow=4, exp=5, expm1=6, sqrt=7, log=8, log1p=9, exp2=10,
    log2=11, log10=12, asin=13, acos=14, atan=15, sinh=16, cosh=17, tanh=18, sin=19,
    cos=20, tan=21, abs=22, neg=23, ceil=26, floor=27, round=28, gt=29, lt=30, eq=31,
    ne=32, ge=33, le=34, sum=35, mean=36, max=37, min=38, prod=39, argmax=42, argmin=43,
    maximum=54, minimum=55,
)

c_int_p = ctypes.POINTER(ctypes.c_int)
c_size_p = ctypes.POINTER(ctypes.c_size_t)
vp = ctypes.c_void_p


class PtScalar(ctypes.Structure):
    class _V(ctypes.Union):
        _fields_ = [("f64", ctypes.c_double), ("f32", ctypes.c_float),
                    ("i64", ctypes.c_int64), ("u64", ctypes.c_uint64),
                    ("u16", ctypes.c_uint16)]
    _fields_ = [("v", _V), ("dtype", ctypes.c_int)]


class PtDeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64),
                ("compute_units", ctypes.c_int), ("clock_khz", ctypes.c_int),
                ("memory_clock_khz", ctypes.c_int), ("memory_bus_width", ctypes.c_int),
                ("total_memory", ctypes.c_size_t), ("lds_per_block", ctypes.c_size_t),
                ("warp_size", ctypes.c_int), ("max_threads_per_block", ctypes.c_int),
                ("l2_cache_bytes", ctypes.c_int)]


class PtBackendInfo(ctypes.Structure):
    _fields_ = [("last_matmul", ctypes.c_char * 32)] + [
        (name, ctypes.c_uint64) for name in (
            "mfma_gemm_calls", "generic_gemm_calls", "row_reduce_calls",
            "column_reduce_calls", "strided_reduce_calls", "global_reduce_calls",
            "fused_row_calls", "elementwise_calls", "rtc_compiles", "graph_launches",
            "staged_copies")]


# name -> (restype, argtypes); every function declared in include/pt_hip.h
SIGNATURES = {
    "pt_init": (ctypes.c_int, []),
    "pt_device_count": (ctypes.c_int, [c_int_p]),
    "pt_device_set": (ctypes.c_int, [ctypes.c_int]),
    "pt_device_get": (ctypes.c_int, [c_int_p]),
    "pt_device_info_get": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(PtDeviceInfo)]),
    "pt_device_synchronize": (ctypes.c_int, []),
    "pt_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "pt_last_error": (ctypes.c_char_p, []),
    "pt_version": (ctypes.c_int, [c_int_p, c_int_p]),
    "pt_stream_create": (ctypes.c_int, [ctypes.POINTER(vp)]),
    "pt_stream_destroy": (ctypes.c_int, [vp]),
    "pt_stream_synchronize": (ctypes.c_int, [vp]),
    "pt_stream_query": (ctypes.c_int, [vp, c_int_p]),
    "pt_stream_wait_event": (ctypes.c_int, [vp, vp]),
    "pt_default_stream": (vp, []),
    "pt_stream_set_current": (ctypes.c_int, [vp]),
    "pt_event_create": (ctypes.c_int, [ctypes.POINTER(vp)]),
    "pt_event_destroy": (ctypes.c_int, [vp]),
    "pt_event_record": (ctypes.c_int, [vp, vp]),
    "pt_event_synchronize": (ctypes.c_int, [vp]),
    "pt_event_query": (ctypes.c_int, [vp, c_int_p]),
    "pt_event_elapsed_ms": (ctypes.c_int, [vp, vp, ctypes.POINTER(ctypes.c_float)]),
    "pt_mem_init": (ctypes.c_int, [ctypes.c_size_t]),
    "pt_alloc": (ctypes.c_int, [ctypes.POINTER(vp), ctypes.c_size_t, vp]),
    "pt_free": (ctypes.c_int, [vp, vp]),
    "pt_mem_info": (ctypes.c_int, [c_size_p, c_size_p, c_size_p]),
    "pt_memcpy_h2d": (ctypes.c_int, [vp, vp, ctypes.c_size_t, vp]),
    "pt_memcpy_d2h": (ctypes.c_int, [vp, vp, ctypes.c_size_t, vp]),
    "pt_memcpy_d2d": (ctypes.c_int, [vp, vp, ctypes.c_size_t, vp]),
    "pt_memset": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_size_t, vp]),
    "pt_host_alloc_pinned": (ctypes.c_int, [ctypes.POINTER(vp), ctypes.c_size_t]),
    "pt_host_free_pinned": (ctypes.c_int, [vp]),
    "pt_reduce": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, c_int_p, c_size_p,
                                 ctypes.c_int, ctypes.c_int, ctypes.c_size_t, vp]),
    "pt_reduce_result_dtype": (ctypes.c_int, [ctypes.c_int, ctypes.c_int]),
    "pt_reduce_noalloc": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, c_int_p, c_size_p,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_size_t, vp]),
    "pt_arg_reduce": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, c_int_p, c_size_p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_size_t, vp]),
    "pt_moments": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, c_int_p, c_size_p,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]),
    "pt_softmax": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, c_int_p, c_size_p,
                                  ctypes.c_int, ctypes.c_int, vp]),
    "pt_layernorm": (ctypes.c_int, [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_size_t,
                                    ctypes.c_size_t, ctypes.c_double, vp, vp, vp]),
    "pt_matmul": (ctypes.c_int, [vp, vp, vp, ctypes.c_int, c_int_p, c_size_p, ctypes.c_int,
                                 c_int_p, c_size_p, ctypes.c_int, c_int_p, ctypes.c_int, vp]),
    "pt_matmul_tune": (ctypes.c_int, [vp, vp, vp, ctypes.c_int, c_int_p, c_size_p, ctypes.c_int,
                                      c_int_p, c_size_p, ctypes.c_int, c_int_p, ctypes.c_int, c_int_p,
                                      ctypes.POINTER(ctypes.c_float), ctypes.c_int, c_int_p, c_int_p, vp]),
    "pt_matmul_set_precision": (ctypes.c_int, [ctypes.c_int]),
    "pt_matmul_precision_name": (ctypes.c_char_p, []),
    "pt_matmul_set_tile": (ctypes.c_int, [ctypes.c_int]),
    "pt_matmul_set_schedule": (ctypes.c_int, [ctypes.c_int]),
    "pt_backend_info_get": (ctypes.c_int, [ctypes.POINTER(PtBackendInfo)]),
    "pt_backend_info_reset": (ctypes.c_int, []),
    "pt_broadcast": (ctypes.c_int, [vp, ctypes.c_int, c_size_p, ctypes.c_size_t,
                                    vp, ctypes.c_int, c_size_p, ctypes.c_size_t,
                                    vp, ctypes.c_int, ctypes.c_int,
                                    c_int_p, ctypes.c_int, vp]),
    "pt_scalar": (ctypes.c_int, [vp, ctypes.c_int, c_size_p, ctypes.c_size_t,
                                 ctypes.POINTER(PtScalar), ctypes.c_int, vp, ctypes.c_int,
                                 ctypes.c_int, c_int_p, ctypes.c_int, vp]),
    "pt_unary": (ctypes.c_int, [vp, ctypes.c_int, c_size_p, ctypes.c_size_t, vp, ctypes.c_int,
                                c_int_p, ctypes.c_int, vp]),
    "pt_cast": (ctypes.c_int, [vp, ctypes.c_int, c_size_p, ctypes.c_size_t, vp, ctypes.c_int,
                               c_int_p, ctypes.c_int, vp]),
    "pt_where": (ctypes.c_int, [vp, ctypes.c_int, c_size_p, vp, c_size_p, vp, c_size_p,
                                ctypes.c_int, vp, c_int_p, ctypes.c_int, vp]),
    "pt_index_validate": (ctypes.c_int, [vp, c_int_p, c_size_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, vp, vp]),
    "pt_gather": (ctypes.c_int, [vp, ctypes.c_int, c_int_p, c_size_p, ctypes.c_size_t, vp, c_int_p, c_size_p,
                                 ctypes.c_size_t, ctypes.c_int, ctypes.c_int, vp, vp, vp]),
    "pt_scatter_add": (ctypes.c_int, [vp, c_int_p, c_size_p, ctypes.c_size_t, vp, c_size_p, ctypes.c_size_t,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, c_size_p, vp,
                                      vp]),
    "pt_fill": (ctypes.c_int, [vp, ctypes.c_int, ctypes.c_size_t, ctypes.POINTER(PtScalar), vp]),
    "pt_rtc_compile": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(vp),
                                      ctypes.c_char_p, ctypes.c_size_t]),
    "pt_module_function": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.POINTER(vp)]),
    "pt_module_unload": (ctypes.c_int, [vp]),
    "pt_launch": (ctypes.c_int, [vp, ctypes.c_uint, ctypes.c_uint, ctypes.POINTER(vp), vp]),
    "pt_graph_begin_capture": (ctypes.c_int, [vp]),
    "pt_graph_end_capture": (ctypes.c_int, [vp, ctypes.POINTER(vp)]),
    "pt_graph_end_capture_update": (ctypes.c_int, [vp, vp]),
    "pt_graph_launch": (ctypes.c_int, [vp, vp]),
    "pt_graph_destroy": (ctypes.c_int, [vp]),
    "pt_graph_node_count": (ctypes.c_int, [vp, c_size_p]),
    "pt_workspace_begin": (ctypes.c_int, [vp, ctypes.c_size_t]),
    "pt_workspace_end": (ctypes.c_int, [c_size_p]),
}


class InvalidArgumentException(ValueError):
    """Mirrors PhpTensors\\InvalidArgumentException."""


class RuntimeException(RuntimeError):
    """Mirrors PhpTensors\\RuntimeException."""


_lib = None


def load(path=DEVICE_LIB):
    """Load the HIP backend; raises when it is missing (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeException(
            f"HIP backend {path} is not built; run php-gpu-tensors_amd/build.py")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error():
    msg = load().pt_last_error()
    return msg.decode() if msg else ""


def check(status, what=""):
    if status == PT_OK:
        return
    msg = last_error()
    text = f"{what}: {msg}" if what else msg
    if status == PT_ERR_INVALID:
        raise InvalidArgumentException(text)
    raise RuntimeException(f"{text} ({load().pt_status_string(status).decode()})")


def ints(values):
    values = [int(v) for v in values]
    return (ctypes.c_int * max(1, len(values)))(*values)


def sizes(values):
    values = [int(v) for v in values]
    return (ctypes.c_size_t * max(1, len(values)))(*values)


def scalar(value, dtype):
    s = PtScalar()
    s.dtype = dtype
    if dtype == FLOAT64:
        s.v.f64 = float(value)
    elif dtype == FLOAT32:
        s.v.f32 = float(value)
    elif dtype in (FLOAT16, BFLOAT16):
        s.v.u16 = int(value)  # caller passes the bit pattern
    elif dtype in (UINT8, UINT16, UINT32, UINT64, BOOL):
        s.v.u64 = int(value)
    else:
        s.v.i64 = int(value)
    return s


class DeviceBuffer:
    """An owning device allocation from the stream-ordered pool."""

    def __init__(self, nbytes, stream=None):
        self.nbytes = int(nbytes)
        self.stream = stream
        ptr = vp()
        check(load().pt_alloc(ctypes.byref(ptr), self.nbytes, stream), "pt_alloc")
        self.ptr = ptr.value

    def free(self):
        if self.ptr:
            load().pt_free(self.ptr, self.stream)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, array):
        import numpy as np
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes
        check(load().pt_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, self.stream), "upload")

    def download(self, dtype, shape):
        import numpy as np
        out = np.empty(shape, dtype)
        if out.nbytes:
            check(load().pt_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, self.stream),
                  "download")
        return out


def matmul(a_buf, b_buf, c_buf, dtype, shape_a, strides_a, shape_b, strides_b, shape_c,
           stream=None):
    """pt_matmul on device buffers (pointers) with explicit views."""
    check(load().pt_matmul(a_buf, b_buf, c_buf, dtype, ints(shape_a), sizes(strides_a),
                           len(shape_a), ints(shape_b), sizes(strides_b), len(shape_b),
                           ints(shape_c), len(shape_c), stream), "matmul")


def to_device(array, stream=None):
    import numpy as np
    a = np.ascontiguousarray(array)
    buf = DeviceBuffer(max(a.nbytes, 1), stream)
    if a.nbytes:
        buf.upload(a)
    return buf


def synchronize():
    check(load().pt_device_synchronize(), "synchronize")


def device_info():
    info = PtDeviceInfo()
    check(load().pt_device_info_get(0, ctypes.byref(info)), "device info")
    return info


def backend_info():
    info = PtBackendInfo()
    check(load().pt_backend_info_get(ctypes.byref(info)), "backend info")
    return info
