"""Build step for the MI355X backend (gfx950 only).

Compiles the HIP sources of csrc/ into lib/libpt_hip.so (the C-ABI declared
in include/pt_hip.h) and the host runtime of host/ into
lib/libphptensors_host.so.  Always rebuilds when called; outputs stay in the
source tree so they travel with it.
"""
import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "lib", "obj")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # a*b+c stays two rounded operations, as in the reference's separate ops
    "-ffp-contract=off",
    # packed fp32 VALU ops disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("build failed: " + " ".join(cmd))
    return proc


def _compile_hip(src):
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    return obj


def build_device():
    os.makedirs(OBJ, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(_compile_hip, sources))
    out = os.path.join(LIB, "libpt_hip.so")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", out + ".tmp", *objs,
          "-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(out + ".tmp", out)
    return out


def build_host():
    sources = sorted(glob.glob(os.path.join(HERE, "host", "*.cpp")))
    if not sources:
        return None
    out = os.path.join(LIB, "libphptensors_host.so")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-I", os.path.join(ROOT, "include"), "-o", out + ".tmp", *sources,
          "-L", LIB, "-lpt_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(out + ".tmp", out)
    return out


def build():
    os.makedirs(LIB, exist_ok=True)
    dev = build_device()
    host = build_host()
    return dev, host


if __name__ == "__main__":
    print(build())
