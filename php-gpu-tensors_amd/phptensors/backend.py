"""The reference's global backend functions for the matmul path
(cuda_get_backend_info, cuda_set_matmul_precision, cuda_tune_matmul;
src/cuda.c over matmul_kernels.h:31-38 and backend_info.h:7-16), over the
gfx950 C-ABI.  Names and dictionary keys follow the reference so that its
tests read the same; the backend names are this build's (MFMA kernels
instead of cuBLAS)."""
import ctypes

from . import _abi, _host
from ._abi import InvalidArgumentException, RuntimeException  # noqa: F401
from .cuda_array import CudaArray

PRECISIONS = {"fp32-strict": 0, "tf32": 1}
MAX_CANDIDATES = 16


def cuda_get_backend_info():
    """Matmul precision, the kind of the last matmul and the call counters."""
    info = _abi.backend_info()
    out = {"precision": _abi.load().pt_matmul_precision_name().decode(),
           "lastMatmul": info.last_matmul.decode()}
    for name, _ in info._fields_[1:]:
        head, *rest = name.split("_")
        out[head + "".join(w.capitalize() for w in rest)] = int(getattr(info, name))
    return out


def cuda_set_matmul_precision(precision):
    """'fp32-strict' (default) or 'tf32'.  gfx950 has no TF32 MFMA, so 'tf32'
    raises RuntimeException as on a device without TF32; an unknown name
    raises InvalidArgumentException.  The mode is unchanged on error."""
    if precision not in PRECISIONS:
        raise InvalidArgumentException(f"Unknown matmul precision '{precision}'")
    _abi.check(_abi.load().pt_matmul_set_precision(PRECISIONS[precision]), "cuda_set_matmul_precision")


def cuda_tune_matmul(a, b):
    """Time every MFMA tile configuration for a @ b, keep the fastest for this
    problem (later matmuls of the same shape and layout use it) and describe
    the sweep as cuda_tune_matmul does: backend, precision, candidateCount,
    selectedCandidate and per-candidate {tile, medianMs, workspaceBytes,
    selected}.  Problems with M*N*K below 1e7 raise InvalidArgumentException."""
    if not isinstance(a, CudaArray) or not isinstance(b, CudaArray):
        raise InvalidArgumentException("cuda_tune_matmul expects two CudaArray operands")
    tiles = (ctypes.c_int * MAX_CANDIDATES)()
    times = (ctypes.c_float * MAX_CANDIDATES)()
    count, selected = ctypes.c_int(0), ctypes.c_int(-1)
    handle = _host.load().phpt_tune_matmul(a._h, b._h, tiles, times, MAX_CANDIDATES,
                                           ctypes.byref(count), ctypes.byref(selected))
    product = CudaArray._wrap(handle, "cuda_tune_matmul")
    candidates = [{"tile": int(tiles[i]), "medianMs": float(times[i]), "workspaceBytes": 0,
                   "selected": i == selected.value} for i in range(count.value)]
    return {"backend": "mfma", "precision": _abi.load().pt_matmul_precision_name().decode(),
            "candidateCount": count.value, "selectedCandidate": selected.value,
            "candidates": candidates, "product": product}
