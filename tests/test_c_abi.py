"""The boundary consumed from C: tests/c_abi/pt_reduce_driver.c is compiled
as C99 with warnings as errors against include/pt_hip.h and linked against
libpt_hip.so (CPU), then run on the GPU, where its sum / max / argmax along
axis 1 (the ca_private.c:236-342 sequence: allocate, upload, reduce, check
status, download) are compared with the oracle on the same seeded bytes."""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as O
from phptensors import synthetic

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(ROOT, "php-gpu-tensors_amd", "lib")
DRIVER = os.path.join(ROOT, "tests", "c_abi", "pt_reduce_driver.c")


def build_driver(out_dir):
    exe = os.path.join(out_dir, "pt_reduce_driver")
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", os.path.join(ROOT, "include"),
           DRIVER, "-o", exe, "-L", LIB_DIR, "-lpt_hip", "-Wl,-rpath," + LIB_DIR]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return exe


def test_driver_compiles_as_c99_and_links(tmp_path):
    assert os.path.exists(os.path.join(LIB_DIR, "libpt_hip.so")), "build the library first"
    exe = build_driver(str(tmp_path))
    assert os.access(exe, os.X_OK)


@pytest.mark.gpu
def test_driver_reductions_vs_oracle(tmp_path):
    exe = build_driver(str(tmp_path))
    rows, cols = 256, 4096
    x = synthetic.normal((rows, cols), 0.0, 1.0, seed=2)
    x[7, 100] = x[7, 3000] = 50.0            # a tie: argmax takes the lower index
    src, dst = tmp_path / "x.f32", tmp_path / "out.bin"
    x.tofile(src)
    print(f"c_abi driver: [{rows},{cols}] seed 2", flush=True)
    proc = subprocess.run([exe, str(rows), str(cols), str(src), str(dst)], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 0, proc.stderr
    raw = np.fromfile(dst, dtype=np.uint8)
    assert raw.size == rows * 12
    got_sum = raw[:rows * 4].view(np.float32)
    got_max = raw[rows * 4:rows * 8].view(np.float32)
    got_arg = raw[rows * 8:].view(np.int32)
    ref_sum, _ = O.reduce(x, O.F32, "sum", 1)
    ref_max, _ = O.reduce(x, O.F32, "max", 1)
    ref_arg = O.arg_reduce(x, O.F32, "argmax", 1)
    bound = np.abs(x.astype(np.float64)).sum(axis=1) / np.sqrt(cols)
    assert np.all(np.abs(got_sum.astype(np.float64) - ref_sum) <= 1e-5 * np.maximum(np.abs(ref_sum), bound))
    assert got_max.tobytes() == ref_max.tobytes()
    assert got_arg.tobytes() == ref_arg.tobytes()
    assert got_arg[7] == 100
