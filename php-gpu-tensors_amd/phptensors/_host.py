"""ctypes view of the host runtime C API (host/phpt_host.h, lib/libphptensors_host.so)."""
import ctypes
import os

from . import _abi

HOST_LIB = os.path.join(_abi.LIB_DIR, "libphptensors_host.so")

T = ctypes.c_void_p          # phpt_tensor*
G = ctypes.c_void_p          # phpt_graph*
ip = ctypes.POINTER(ctypes.c_int)
sp = ctypes.POINTER(ctypes.c_size_t)
vp = ctypes.c_void_p
c_i64 = ctypes.c_int64

SIGNATURES = {
    "phpt_error_kind": (ctypes.c_int, []),
    "phpt_error_message": (ctypes.c_char_p, []),
    "phpt_clear_error": (None, []),
    "phpt_from_host": (T, [vp, ctypes.c_int, ip, ctypes.c_int]),
    "phpt_full": (T, [ip, ctypes.c_int, ctypes.c_int, ctypes.c_double, c_i64, ctypes.c_int]),
    "phpt_to_host": (ctypes.c_int, [T, vp, ctypes.c_size_t]),
    "phpt_retain": (T, [T]),
    "phpt_release": (None, [T]),
    "phpt_dtype": (ctypes.c_int, [T]),
    "phpt_ndims": (ctypes.c_int, [T]),
    "phpt_shape": (None, [T, ip]),
    "phpt_strides": (None, [T, sp]),
    "phpt_size": (ctypes.c_size_t, [T]),
    "phpt_is_lazy": (ctypes.c_int, [T]),
    "phpt_is_view": (ctypes.c_int, [T]),
    "phpt_dtype_from_name": (ctypes.c_int, [ctypes.c_char_p]),
    "phpt_dtype_name": (ctypes.c_char_p, [ctypes.c_int]),
    "phpt_reshape": (T, [T, ip, ctypes.c_int]),
    "phpt_transpose": (T, [T, ip, ctypes.c_int]),
    "phpt_broadcast_to": (T, [T, ip, ctypes.c_int]),
    "phpt_slice": (T, [T, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "phpt_select": (T, [T, ctypes.c_int, ctypes.c_int]),
    "phpt_binary": (T, [T, T, ctypes.c_int]),
    "phpt_scalar_op": (T, [T, ctypes.c_double, c_i64, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "phpt_unary": (T, [T, ctypes.c_int]),
    "phpt_reduce": (T, [T, ctypes.c_int, ctypes.c_int]),
    "phpt_reduce_arg": (T, [T, ctypes.c_int, ctypes.c_int]),
    "phpt_variance": (T, [T, ctypes.c_int, ctypes.c_long, ctypes.c_int]),
    "phpt_softmax": (T, [T, ctypes.c_int]),
    "phpt_layernorm": (T, [T, ip, ctypes.c_int, ctypes.c_double, T, T]),
    "phpt_matmul": (T, [T, T]),
    "phpt_tune_matmul": (T, [T, T, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_float), ctypes.c_int,
                             ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "phpt_where": (T, [T, T, T]),
    "phpt_gather": (T, [T, T, ctypes.c_longlong]),
    "phpt_scatter_add": (T, [T, T, T, ctypes.c_longlong]),
    "phpt_astype": (T, [T, ctypes.c_int]),
    "phpt_copy": (T, [T]),
    "phpt_fusion_begin": (ctypes.c_int, [ctypes.c_int]),
    "phpt_fusion_active": (ctypes.c_int, []),
    "phpt_fusion_abort": (None, []),
    "phpt_fusion_input": (T, [T, ctypes.c_int]),
    "phpt_fusion_end": (G, [ctypes.POINTER(T), ctypes.c_int, ctypes.c_int]),
    "phpt_fusion_run_once": (ctypes.c_int, [ctypes.POINTER(T), ctypes.c_int]),
    "phpt_graph_run": (ctypes.c_int, [G, ctypes.POINTER(T), ctypes.c_int, ctypes.POINTER(T), ctypes.c_int]),
    "phpt_graph_replay": (ctypes.c_int, [G, ctypes.POINTER(T), ctypes.c_int, ctypes.c_int, ctypes.POINTER(T),
                                         ctypes.c_int]),
    "phpt_device_pointer": (ctypes.c_void_p, [T]),
    "phpt_graph_run_async": (ctypes.c_void_p, [G, ctypes.POINTER(T), ctypes.c_int]),
    "phpt_execution_wait": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(T), ctypes.c_int]),
    "phpt_execution_is_finished": (ctypes.c_int, [ctypes.c_void_p]),
    "phpt_execution_release": (None, [ctypes.c_void_p]),
    "phpt_graph_num_outputs": (ctypes.c_int, [G]),
    "phpt_graph_source": (ctypes.c_char_p, [G]),
    "phpt_graph_stats": (ctypes.c_char_p, [G]),
    "phpt_graph_plan": (ctypes.c_char_p, [G]),
    "phpt_graph_set_profiling": (None, [G, ctypes.c_int]),
    "phpt_graph_release": (None, [G]),
    "phpt_fusion_cache_stats": (ctypes.c_char_p, []),
    "phpt_fusion_clear_cache": (None, []),
}

_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    _abi.load()  # the device backend first (no CPU fallback)
    if not os.path.exists(HOST_LIB):
        raise _abi.RuntimeException(f"host runtime {HOST_LIB} is not built")
    lib = ctypes.CDLL(HOST_LIB)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def raise_error(what=""):
    lib = load()
    kind = lib.phpt_error_kind()
    msg = (lib.phpt_error_message() or b"").decode()
    text = msg or what or "operation failed"
    if kind == 1:
        raise _abi.InvalidArgumentException(text)
    raise _abi.RuntimeException(text)


def check_handle(h, what=""):
    if not h:
        raise_error(what)
    return h


def parse_kv(text):
    out = {}
    for part in text.decode().split(";"):
        if not part:
            continue
        k, _, v = part.partition("=")
        if v == "null":
            out[k] = None
            continue
        try:
            out[k] = int(v)
        except ValueError:
            out[k] = v
    return out
