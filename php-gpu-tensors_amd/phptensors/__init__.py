"""PhpTensors on MI355X: the reference's CudaArray / Fusion surface over the
gfx950 C-ABI (include/pt_hip.h)."""
from . import _abi  # noqa: F401
from ._abi import InvalidArgumentException, RuntimeException  # noqa: F401
