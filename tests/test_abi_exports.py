"""CPU-side checks of the C-ABI library: it loads without a GPU and exports
every function declared in include/pt_hip.h (no compute calls)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(ROOT, "include")


def declared_functions(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pt_[a-z0-9_]+)\s*\(", text)))


def test_device_library_exports_every_declared_symbol():
    from phptensors import _abi
    lib = ctypes.CDLL(_abi.DEVICE_LIB)
    names = declared_functions(os.path.join(HEADER_DIR, "pt_hip.h"))
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes table covers the same set
    assert sorted(_abi.SIGNATURES) == names


def test_status_strings_without_device():
    from phptensors import _abi
    lib = _abi.load()
    assert lib.pt_status_string(0) == b"success"
    assert lib.pt_status_string(1) == b"invalid argument"
    n = ctypes.c_int(-1)
    assert lib.pt_device_count(ctypes.byref(n)) == 0
    assert n.value >= 0


def test_host_runtime_exports_every_declared_symbol():
    from phptensors import _host
    header = os.path.join(ROOT, "php-gpu-tensors_amd", "host", "phpt_host.h")
    text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(phpt_[a-z0-9_]+)\s*\(", text)))
    assert len(names) > 40
    lib = ctypes.CDLL(_host.HOST_LIB)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_host.SIGNATURES) == names


def test_host_runtime_dtype_names_without_device():
    from phptensors import _host
    lib = _host.load()
    assert lib.phpt_dtype_from_name(b"bfloat16") == 12
    assert lib.phpt_dtype_from_name(b"float32") == 0
    assert lib.phpt_dtype_from_name(b"nope") == -1
    assert lib.phpt_dtype_name(11) == b"float16"
