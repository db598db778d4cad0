"""PhpTensors on MI355X: the reference's CudaArray / Fusion surface over the
gfx950 C-ABI (include/pt_hip.h) and the host runtime (host/phpt_host.h)."""
from . import _abi  # noqa: F401
from ._abi import InvalidArgumentException, RuntimeException  # noqa: F401
from .cuda_array import CudaArray  # noqa: F401
from .fusion import Fusion, FusionExecution, FusionGraph  # noqa: F401
