"""GPU parity: pt_matmul (MFMA kernels) against the CPU oracle (HostArray
matmul restatement) on identical seeded bytes.

Bars: integer-valued inputs give exact fp32 sums, so those outputs are
bit-exact (also for bf16/fp16 outputs, which round the exact fp32 sum to
nearest even).  Random fp32: |d| <= 1e-4 * sqrt(K) * (|A||B|)_ij.  Random
bf16/fp16: |d| <= 1e-2 * max(|ref|, (|A||B|)_ij / sqrt(K)) against the
oracle's fp32-accumulated, RNE-rounded product.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                     "reference_expectations.json")))
DTS = {"float32": O.F32, "float16": O.F16, "bfloat16": O.BF16}


@pytest.fixture(scope="module")
def A():
    from phptensors import _abi
    _abi.check(_abi.load().pt_init(), "init")
    yield _abi
    _abi.load().pt_matmul_set_tile(-1)


def run(A, a, b, dtype, shape_a=None, strides_a=None, shape_b=None, strides_b=None):
    """a, b: contiguous storage arrays; optional view shape/strides (elements)."""
    shape_a = tuple(a.shape if shape_a is None else shape_a)
    shape_b = tuple(b.shape if shape_b is None else shape_b)
    strides_a = [s // a.itemsize for s in a.strides] if strides_a is None else strides_a
    strides_b = [s // b.itemsize for s in b.strides] if strides_b is None else strides_b
    shape_c = O.matmul_shape(shape_a, shape_b)
    da, db = A.to_device(a), A.to_device(b)
    esz = 4 if dtype == O.F32 else 2
    dc = A.DeviceBuffer(max(1, int(np.prod(shape_c)) * esz))
    A.matmul(da.ptr, db.ptr, dc.ptr, dtype, shape_a, strides_a, shape_b, strides_b, shape_c)
    return dc.download(O.NP_STORAGE[dtype], shape_c)


def ref(a, b, dtype, **kw):
    return O.matmul(a, b, dtype, **kw)


@pytest.mark.parametrize("case", GOLDEN["matmul"], ids=lambda c: c["id"])
def test_matmul_golden(A, case):
    dt = DTS[case["dtype"]]
    a = O.to_storage(np.array(case["a"], np.float64), dt).reshape(case["shape_a"])
    b = O.to_storage(np.array(case["b"], np.float64), dt).reshape(case["shape_b"])
    c = run(A, a, b, dt)
    assert list(c.shape) == case["expected_shape"]
    vals = O.from_storage(c, dt).astype(np.float64).ravel()
    if "abs_tol" in case:
        assert np.all(np.abs(vals - np.array(case["expected"])) < case["abs_tol"])
    else:
        assert vals.tolist() == [float(v) for v in case["expected"]]


SHAPES = [(1, 64, 64, 64), (2, 256, 128, 64), (3, 100, 70, 33), (1, 512, 256, 512),
          (4, 128, 384, 96), (1, 1, 300, 5), (2, 65, 1, 257), (1, 33, 17, 1),
          (1, 196, 100, 64), (2, 132, 260, 128)]


def smalln_expected(b_, m, n, k):
    """The small-N kernel's eligibility (pt_gemm_smalln.hip): N <= 16,
    k-contiguous A, M*K >= 2^18 and one 16-row block per CU (256)."""
    return n <= 16 and m * k >= 1 << 18 and ((m + 15) // 16) * b_ >= 256


def _ints(shape, seed, lo=-8, hi=8):
    from phptensors import synthetic
    return synthetic.integers(shape, lo, hi, seed=seed).astype(np.float32)


@pytest.mark.parametrize("tile", [-1, 0, 1, 2, 3, 5, 8, 9, 10, 11, 12, 13])
@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("bmnk", SHAPES, ids=str)
def test_matmul_integer_exact(A, bmnk, dt, tile):
    b_, m, n, k = bmnk
    A.load().pt_matmul_set_tile(tile)
    try:
        a32 = _ints((b_, m, k), seed=m * 7 + k)
        b32 = _ints((b_, k, n), seed=n * 5 + k + 1)
        a, b = O.to_storage(a32, dt), O.to_storage(b32, dt)
        got = run(A, a, b, dt)
        assert np.array_equal(got, ref(a, b, dt))
    finally:
        A.load().pt_matmul_set_tile(-1)


@pytest.mark.parametrize("tile", [-1, 0, 1, 3, 5, 9, 10, 11])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("bmnk", [(2, 512, 512, 256), (1, 256, 768, 96), (1, 300, 260, 130)], ids=str)
def test_matmul_fp32_tiles_layouts(A, bmnk, layout, tile):
    """fp32 tiles over every operand layout: transposed A and row-major B stage
    k-major in LDS, where the row blocks of a wave interleave for wide
    fragment reads.  Exact on integer-valued operands, whole and edge tiles."""
    b_, m, n, k = bmnk
    A.load().pt_matmul_set_tile(tile)
    try:
        a = _ints((b_, m, k), seed=m + 11 * k)
        b = _ints((b_, k, n), seed=n + 13 * k)
        expect = ref(a, b, O.F32)
        kw = {}
        a_in, b_in = a, b
        if layout[0] == "T":   # A as the transposed view of a [b, k, m] buffer
            a_in = np.ascontiguousarray(np.swapaxes(a, 1, 2))
            kw.update(shape_a=(b_, m, k), strides_a=[m * k, 1, m])
        if layout[1] == "T":   # B as the transposed view of a [b, n, k] buffer
            b_in = np.ascontiguousarray(np.swapaxes(b, 1, 2))
            kw.update(shape_b=(b_, k, n), strides_b=[n * k, 1, k])
        assert np.array_equal(run(A, a_in, b_in, O.F32, **kw), expect)
    finally:
        A.load().pt_matmul_set_tile(-1)


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("bmnk", [(1, 1024, 10, 4096), (1, 4096, 10, 1024), (3, 40, 24, 3000),
                                  (1, 64, 64, 8192), (2, 65, 1, 257)], ids=str)
def test_matmul_split_k(A, bmnk, dt):
    """Few output tiles over a long K: the K range is split over workgroups
    whose fp32 partials are summed in order and rounded once.  Integer inputs
    keep every partial exact, so the result is bit-exact; random inputs stay
    within the fp32 / low-precision bars of the module docstring."""
    from phptensors import synthetic
    b_, m, n, k = bmnk
    a = O.to_storage(_ints((b_, m, k), seed=k + 3, lo=-3, hi=3), dt)
    b = O.to_storage(_ints((b_, k, n), seed=k + 4, lo=-3, hi=3), dt)
    assert np.array_equal(run(A, a, b, dt), ref(a, b, dt))
    path = A.backend_info().last_matmul.decode()
    if dt == O.F32 and smalln_expected(b_, m, n, k):
        assert path == "mfma-fp32-smalln"   # the streaming small-N kernel
    else:
        assert path.endswith("splitk")
    a = O.to_storage(synthetic.normal((b_, m, k), 0.0, 1.0, seed=k + 5), dt)
    b = O.to_storage(synthetic.normal((b_, k, n), 0.0, 1.0, seed=k + 6), dt)
    got = O.from_storage(run(A, a, b, dt), dt).astype(np.float64)
    r = O.from_storage(ref(a, b, dt), dt).astype(np.float64)
    scale = np.abs(O.from_storage(a, dt).astype(np.float64)) @ np.abs(O.from_storage(b, dt).astype(np.float64))
    if dt == O.F32:
        tol = 1e-4 * math.sqrt(k) * scale
    else:
        tol = 1e-2 * np.maximum(np.abs(r), scale / math.sqrt(k))
    assert np.all(np.abs(got - r) <= tol)


def _ring_eligible(m, n, k, layout):
    """The fp32 ring kernel's conditions (pt_gemm_f32ring.hip) for these
    aligned, packed operands: K a multiple of 16 (a last half step of 32 is
    zero-filled), and a transposed (m- or n-contiguous) operand needs its M
    or N a multiple of 4."""
    a_rc, b_rc = layout[0] == "T", layout[1] == "N"
    return k % 16 == 0 and (not a_rc or m % 4 == 0) and (not b_rc or n % 4 == 0)


@pytest.mark.parametrize("layout", ["NN", "NT", "TN", "TT"])
@pytest.mark.parametrize("bmnk", [(2, 256, 384, 128), (1, 300, 260, 96), (1, 784, 1024, 4096),
                                  (3, 130, 258, 64), (1, 128, 129, 32), (1, 1024, 1024, 2048),
                                  (2, 256, 256, 130), (1, 512, 1024, 784), (2, 132, 260, 16),
                                  (1, 1024, 1024, 2064), (1, 300, 260, 80)], ids=str)
def test_matmul_fp32_ring(A, bmnk, layout):
    """Tile 38, the fp32 LDS-ring kernel: every operand layout (A k- or
    m-contiguous, B n- or k-contiguous), whole and edge tiles (rows past M
    and columns past N load clamped packs and are not stored), batches, and
    split-K over long K with few tiles, and K ending half-way through a
    32-k step (784, 80, 16; 2064 split four ways, whose last chunk ends so),
    where the loads past the operand's end read zeros and the half step's
    upper slices are zeroed.  Integer-valued operands keep every sum exact,
    so outputs are bit-exact against numpy's float64 product.  Shapes the
    kernel does not take (K % 16 != 0, a transposed operand whose M or N is
    not a multiple of 4) run the 8-wave 128x128 kernel instead and must
    agree too."""
    from phptensors import synthetic
    b_, m, n, k = bmnk
    A.load().pt_matmul_set_tile(38)
    try:
        a = _ints((b_, m, k), seed=m + 3 * k, lo=-4, hi=4)
        b = _ints((b_, k, n), seed=n + 5 * k, lo=-4, hi=4)
        expect = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
        kw = {}
        a_in, b_in = a, b
        if layout[0] == "T":   # A as the transposed view of a [b, k, m] buffer
            a_in = np.ascontiguousarray(np.swapaxes(a, 1, 2))
            kw.update(shape_a=(b_, m, k), strides_a=[m * k, 1, m])
        if layout[1] == "T":   # B as the transposed view of a [b, n, k] buffer
            b_in = np.ascontiguousarray(np.swapaxes(b, 1, 2))
            kw.update(shape_b=(b_, k, n), strides_b=[n * k, 1, k])
        assert np.array_equal(run(A, a_in, b_in, O.F32, **kw), expect)
        path = A.backend_info().last_matmul.decode()
        assert path.startswith("mfma-fp32-ring") == _ring_eligible(m, n, k, layout), path
        if m * n * b_ <= 1024 * 1024 and k >= 2048:
            assert path.endswith("splitk"), path
        # random operands: the fp32 bar of the module docstring
        a = synthetic.normal((b_, m, k), 0.0, 1.0, seed=k + 7).astype(np.float32)
        b = synthetic.normal((b_, k, n), 0.0, 1.0, seed=k + 8).astype(np.float32)
        a_in, b_in = a, b
        if layout[0] == "T":
            a_in = np.ascontiguousarray(np.swapaxes(a, 1, 2))
        if layout[1] == "T":
            b_in = np.ascontiguousarray(np.swapaxes(b, 1, 2))
        got = run(A, a_in, b_in, O.F32, **kw).astype(np.float64)
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        assert np.all(np.abs(got - a64 @ b64) <= 1e-4 * math.sqrt(k) * (np.abs(a64) @ np.abs(b64)))
    finally:
        A.load().pt_matmul_set_tile(-1)


def test_matmul_fp32_ring_two_stages():
    """The ring kernel's 2-stage form (64 KiB of LDS, two workgroups per CU,
    every load of a step landed at its barrier), selected for whole and
    split-K products by PT_F32R_STAGES / PT_F32R_SPLIT_STAGES, which are read
    once per process: the fp32 ring cases above in a child process."""
    import subprocess
    import sys
    env = dict(os.environ, PT_F32R_STAGES="2", PT_F32R_SPLIT_STAGES="2")
    proc = subprocess.run([sys.executable, "-m", "pytest", os.path.abspath(__file__), "-q", "-x",
                           "-p", "no:cacheprovider", "-k", "test_matmul_fp32_ring and not two_stages"],
                          capture_output=True, text=True, timeout=600, env=env,
                          cwd=os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-2000:]
    assert " passed" in proc.stdout and "failed" not in proc.stdout


@pytest.mark.parametrize("dt", [O.BF16, O.F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("layout", ["NN", "NT", "TN"])
@pytest.mark.parametrize("bmnk", [(1, 512, 256, 512), (2, 256, 512, 128), (3, 256, 256, 64),
                                  (1, 256, 256, 96), (2, 768, 256, 192)], ids=str)
def test_matmul_direct_lds_kernel(A, dt, layout, bmnk):
    """Tile 8 (direct-to-LDS kernel, swizzled LDS, transpose reads for
    row-major B): exact on integer-valued operands for row-major and
    transposed B; shapes it does not take (K % 64 != 0, transposed A) run the
    fallback tile and must agree too."""
    A.load().pt_matmul_set_tile(8)
    try:
        b_, m, n, k = bmnk
        a32 = _ints((b_, m, k), seed=m + k)
        b32 = _ints((b_, k, n), seed=n + 2 * k)
        a, b = O.to_storage(a32, dt), O.to_storage(b32, dt)
        expect = ref(a, b, dt)
        kw = {}
        a_in, b_in = a, b
        if layout == "NT":   # B as the transposed view of a [b, n, k] buffer
            b_in = np.ascontiguousarray(np.swapaxes(b, 1, 2))
            kw.update(shape_b=(b_, k, n), strides_b=[n * k, 1, k])
        if layout == "TN":   # A as the transposed view of a [b, k, m] buffer
            a_in = np.ascontiguousarray(np.swapaxes(a, 1, 2))
            kw.update(shape_a=(b_, m, k), strides_a=[m * k, 1, m])
        got = run(A, a_in, b_in, dt, **kw)
        assert np.array_equal(got, expect)
    finally:
        A.load().pt_matmul_set_tile(-1)


@pytest.mark.parametrize("tile", list(range(14, 38)))
@pytest.mark.parametrize("dt", [O.BF16, O.F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("layout", ["NN", "NT"])
@pytest.mark.parametrize("bmnk", [(2, 512, 256, 512), (1, 256, 512, 384), (3, 256, 256, 128),
                                  (1, 256, 256, 96), (1, 512, 384, 256)], ids=str)
def test_matmul_ring_kernel(A, tile, dt, layout, bmnk):
    """Tiles 14-37 (k_gemm_ring: K step x stages x tile width x schedule x
    waves; 32-36: the ping-pong kernel k_gemm_pp; 37: k_gemm_wl):
    exact on integer-valued operands for row-major and k-contiguous B,
    including K-step counts that are not a multiple of the stage count
    (384 / 32 = 12 steps on the 5-stage ring, 128 / 32 = 4 < 5 steps) and
    shapes the ring does not take (K = 96, N = 384 for 256-wide tiles),
    which run the fallback tiles."""
    A.load().pt_matmul_set_tile(tile)
    try:
        b_, m, n, k = bmnk
        a = O.to_storage(_ints((b_, m, k), seed=m + 3 * k), dt)
        b = O.to_storage(_ints((b_, k, n), seed=n + 5 * k), dt)
        expect = ref(a, b, dt)
        kw = {}
        b_in = b
        if layout == "NT":
            b_in = np.ascontiguousarray(np.swapaxes(b, 1, 2))
            kw.update(shape_b=(b_, k, n), strides_b=[n * k, 1, k])
        assert np.array_equal(run(A, a, b_in, dt, **kw), expect)
    finally:
        A.load().pt_matmul_set_tile(-1)


@pytest.mark.parametrize("layout", ["NN", "TN", "NT"])
@pytest.mark.parametrize("bmnk", [(1, 4096, 10, 1024), (1, 1024, 10, 4096), (2, 333, 7, 2500),
                                  (16, 333, 7, 2500), (1, 100, 16, 3000), (40, 100, 16, 3000),
                                  (3, 517, 1, 700), (8, 517, 1, 700), (1, 64, 8, 4096), (64, 64, 8, 4096),
                                  (1, 16, 10, 65536)], ids=str)
def test_matmul_smalln(A, bmnk, layout):
    """fp32 products with N <= 16 and k-contiguous A run the small-N kernel
    (pt_gemm_smalln.hip: eight waves over interleaved 16-k groups, B in LDS
    chunks of 1024 k rows, so K = 2500, 3000 and 4096 run several chunks)
    when they have a 16-row block per CU; a transposed A (TN) and the short,
    long-K shapes (1024 x 4096, 64 x 4096, 16 x 65536 in one batch) keep the
    MFMA split-K path.  Integer inputs: bit-exact; random inputs: the fp32
    bar of the module docstring.  Ragged M (333, 517, 100) and N = 1, 7, 8,
    10, 16 cover the column padding and the clamped rows."""
    from phptensors import synthetic
    b_, m, n, k = bmnk
    for trial in ("ints", "normal"):
        if trial == "ints":
            a = _ints((b_, m, k), seed=m + k, lo=-3, hi=3)
            b = _ints((b_, k, n), seed=n + k, lo=-3, hi=3)
        else:
            a = synthetic.normal((b_, m, k), 0.0, 1.0, seed=m + k + 1).astype(np.float32)
            b = synthetic.normal((b_, k, n), 0.0, 1.0, seed=n + k + 1).astype(np.float32)
        expect = ref(a, b, O.F32)
        kw = {}
        a_in, b_in = a, b
        if layout == "TN":   # A as the transposed view of a [b, k, m] buffer
            a_in = np.ascontiguousarray(np.swapaxes(a, 1, 2))
            kw.update(shape_a=(b_, m, k), strides_a=[m * k, 1, m])
        if layout == "NT":   # B as the transposed view of a [b, n, k] buffer
            b_in = np.ascontiguousarray(np.swapaxes(b, 1, 2))
            kw.update(shape_b=(b_, k, n), strides_b=[n * k, 1, k])
        got = run(A, a_in, b_in, O.F32, **kw)
        path = A.backend_info().last_matmul.decode()
        if layout == "TN" or not smalln_expected(b_, m, n, k):
            assert path.startswith("mfma-fp32") and "smalln" not in path
        else:
            assert path == "mfma-fp32-smalln"
        if trial == "ints":
            assert np.array_equal(got, expect)
        else:
            scale = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
            assert np.all(np.abs(got.astype(np.float64) - expect.astype(np.float64)) <= 1e-4 * math.sqrt(k) * scale)


def test_matmul_smalln_forced_tile(A):
    """A forced tile bypasses the small-N kernels (the tile sweeps measure
    the MFMA kernels on these shapes too)."""
    A.load().pt_matmul_set_tile(2)
    try:
        a = _ints((1, 1024, 512), seed=3)
        b = _ints((1, 512, 10), seed=4)
        assert np.array_equal(run(A, a, b, O.F32), ref(a, b, O.F32))
        assert A.backend_info().last_matmul.decode().startswith("mfma-fp32")
    finally:
        A.load().pt_matmul_set_tile(-1)


def test_matmul_direct_lds_batch_broadcast(A):
    A.load().pt_matmul_set_tile(8)
    try:
        a = O.to_storage(_ints((1, 256, 128), seed=7), O.BF16)
        b = O.to_storage(_ints((4, 128, 256), seed=8), O.BF16)
        assert np.array_equal(run(A, a, b, O.BF16), ref(a, b, O.BF16))
        a4 = O.to_storage(_ints((4, 256, 128), seed=9), O.BF16)
        b2 = O.to_storage(_ints((128, 512), seed=10), O.BF16)
        assert np.array_equal(run(A, a4, b2, O.BF16), ref(a4, b2, O.BF16))
    finally:
        A.load().pt_matmul_set_tile(-1)


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("layout", ["NN", "TN", "NT", "TT"])
@pytest.mark.parametrize("mnk", [(96, 160, 72), (100, 132, 64), (196, 1024, 256)], ids=str)
def test_matmul_transposed_views(A, dt, layout, mnk):
    """A and/or B passed as transposed strided views (no copy).  Whole K
    steps with ragged M/N run the edge tiles with clamped rows (the last two
    shapes); a ragged K runs every tile checked (the first)."""
    m, n, k = mnk
    a32 = _ints((m, k), seed=1)
    b32 = _ints((k, n), seed=2)
    a, b = O.to_storage(a32, dt), O.to_storage(b32, dt)
    expect = ref(a, b, dt)
    if layout[0] == "T":
        at = np.ascontiguousarray(a.T)            # storage [k, m]
        va = dict(shape_a=(m, k), strides_a=[1, m])
        a_in = at
    else:
        a_in, va = a, {}
    if layout[1] == "T":
        bt = np.ascontiguousarray(b.T)            # storage [n, k]
        vb = dict(shape_b=(k, n), strides_b=[1, k])
        b_in = bt
    else:
        b_in, vb = b, {}
    got = run(A, a_in, b_in, dt, **va, **vb)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("dt", [O.F32, O.BF16], ids=["f32", "bf16"])
def test_matmul_batch_broadcast(A, dt):
    # [1,64,64] @ [8,64,64] and [2,1,48,32] @ [1,3,32,40]
    for sa, sb in (((1, 64, 64), (8, 64, 64)), ((2, 1, 48, 32), (1, 3, 32, 40)),
                   ((64, 64), (5, 64, 64)), ((4, 64, 32), (32, 16))):
        a = O.to_storage(_ints(sa, seed=3), dt)
        b = O.to_storage(_ints(sb, seed=4), dt)
        assert np.array_equal(run(A, a, b, dt), ref(a, b, dt))


def test_matmul_accelerated_known_answers(A):
    # ca_matmul_accelerated.phpt:9-29
    row = np.ones((1, 100000), np.float32)
    col = np.ones((100000, 1), np.float32)
    assert run(A, row, col, O.F32)[0, 0] == 100000.0
    ones = np.ones((64, 128), np.float32)
    got = run(A, ones, ones, O.F32, shape_a=(128, 64), strides_a=[1, 128])
    assert got.shape == (128, 128) and np.all(got == 64.0)
    batch = np.ones((8, 64, 64), np.float32)
    assert np.all(run(A, batch, batch, O.F32) == 64.0)
    multi = np.ones((2, 4, 64, 64), np.float32)
    assert np.all(run(A, multi, multi, O.F32) == 64.0)


@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16], ids=["f32", "bf16", "f16"])
def test_matmul_random_within_tolerance(A, dt):
    from phptensors import synthetic
    b_, m, n, k = 2, 256, 384, 1024
    a32 = synthetic.normal((b_, m, k), 0.0, 1.0, seed=41)
    b32 = synthetic.normal((b_, k, n), 0.0, 1.0, seed=42)
    a, b = O.to_storage(a32, dt), O.to_storage(b32, dt)
    got = O.from_storage(run(A, a, b, dt), dt).astype(np.float64)
    r = O.from_storage(ref(a, b, dt), dt).astype(np.float64)
    af = O.from_storage(a, dt).astype(np.float64)
    bf = O.from_storage(b, dt).astype(np.float64)
    scale = np.abs(af) @ np.abs(bf)
    if dt == O.F32:
        tol = 1e-4 * math.sqrt(k) * scale
    else:
        tol = 1e-2 * np.maximum(np.abs(r), scale / math.sqrt(k))
    assert np.all(np.abs(got - r) <= tol)


def test_matmul_errors(A):
    from phptensors._abi import InvalidArgumentException
    a = np.ones((2, 3), np.float32)
    with pytest.raises(InvalidArgumentException):
        run(A, a, a, O.F32)  # inner mismatch via shape check
    x = np.ones((3,), np.float32)
    with pytest.raises(InvalidArgumentException):
        A.matmul(A.to_device(x).ptr, A.to_device(x).ptr, A.DeviceBuffer(4).ptr, O.F32,
                 (3,), [1], (3,), [1], (1,))
    with pytest.raises(InvalidArgumentException):
        A.matmul(A.to_device(a).ptr, A.to_device(a).ptr, A.DeviceBuffer(64).ptr, O.F64,
                 (2, 3), [3, 1], (3, 2), [2, 1], (2, 2))


def test_matmul_empty(A):
    a = np.zeros((2, 0), np.float32)
    b = np.zeros((0, 3), np.float32)
    assert np.array_equal(run(A, a, b, O.F32), np.zeros((2, 3), np.float32))
    assert run(A, np.zeros((0, 2, 3), np.float32), np.ones((3, 2), np.float32), O.F32).shape == (0, 2, 2)


@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32], ids=["bf16", "f16", "f32"])
def test_config4_full_size_sampled(A, dt):
    """A,B [32,2048,2048] N(0,0.02): 512 sampled outputs against float64 dot
    products (tolerances above), plus exact RNE of the sampled fp32 sums."""
    from phptensors import synthetic
    shape = (32, 2048, 2048)
    a32 = synthetic.normal(shape, 0.0, 0.02, seed=4)
    b32 = synthetic.normal(shape, 0.0, 0.02, seed=5)
    a, b = O.to_storage(a32, dt), O.to_storage(b32, dt)
    del a32, b32
    got = run(A, a, b, dt)
    af = O.from_storage(a, dt)
    bf = O.from_storage(b, dt)
    rng = np.random.default_rng(6)
    idx = rng.integers(0, [32, 2048, 2048], size=(512, 3))
    k = 2048
    for bb, i, j in idx:
        row = af[bb, i, :].astype(np.float64)
        col = bf[bb, :, j].astype(np.float64)
        exact = float(row @ col)
        scale = float(np.abs(row) @ np.abs(col))
        g = float(O.from_storage(np.array([got[bb, i, j]]), dt)[0])
        if dt == O.F32:
            assert abs(g - exact) <= 1e-4 * math.sqrt(k) * scale
        else:
            assert abs(g - exact) <= 1e-2 * max(abs(exact), scale / math.sqrt(k))


@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32], ids=["bf16", "f16", "f32"])
def test_config4_full_size_every_output(A, dt):
    """Every one of the 134 M outputs of config 4 (A,B [32,2048,2048]
    N(0,0.02), seeds 4/5), so that every 256x256 tile, batch and XCD-remapped
    workgroup is checked, against an fp32 product of the same rounded operands
    on the host (numpy matmul, i.e. the BLAS sgemm; this library and torch do
    not share a process).  The reference's own error is at most
    K * 2^-24 = 1.2e-4 of |A|.|B| in the worst case, 3 % of the fp32 tolerance
    and about half of the 16-bit floor, and a random walk of
    sqrt(K) * 2^-24 = 2.7e-6 of it in practice.  Tolerances: fp32
    1e-4 * sqrt(K) * (|A|.|B|), bf16 / fp16 1e-2 relative with the floor
    (|A|.|B|) / sqrt(K) of the sampled test above.  A transposed operand, a
    wrong tile origin or a skipped K step moves outputs by O(|C|) and fails."""
    from phptensors import synthetic
    shape, k = (32, 2048, 2048), 2048
    a = O.to_storage(synthetic.normal(shape, 0.0, 0.02, seed=4), dt)
    b = O.to_storage(synthetic.normal(shape, 0.0, 0.02, seed=5), dt)
    got = O.from_storage(run(A, a, b, dt), dt).astype(np.float32)
    af = O.from_storage(a, dt).astype(np.float32)
    bf = O.from_storage(b, dt).astype(np.float32)
    del a, b
    ref32 = np.matmul(af, bf)
    scale = np.matmul(np.abs(af), np.abs(bf))
    del af, bf
    if dt == O.F32:
        bound = np.float32(1e-4 * math.sqrt(k)) * scale
    else:
        bound = np.float32(1e-2) * np.maximum(np.abs(ref32), scale / np.float32(math.sqrt(k)))
    del scale
    err = np.abs(got - ref32)
    bad = int(np.count_nonzero(err > bound))
    worst = float(np.max(err / bound))
    assert np.isfinite(got).all()
    assert bad == 0, f"{bad} outputs outside tolerance (worst {worst:.3g} of the bound)"


@pytest.mark.parametrize("dt", [O.BF16, O.F16], ids=["bf16", "f16"])
def test_ring_gemm_nan_and_inf_outputs(A, dt):
    """The 16-bit ring kernel's epilogue on non-finite sums: a NaN planted in
    a row of A and a column of B, and infinities of both signs beside them,
    give NaN exactly where the float64 product of the same operands is NaN,
    infinities of the same sign where it is infinite, and the fp32 /
    16-bit bar everywhere else (the packed conversion's NaN pairs take the
    scalar payload rule; every pair of a NaN row holds one)."""
    from phptensors import synthetic
    m = n = 4096
    k = 64
    a = O.from_storage(O.to_storage(synthetic.normal((1, m, k), 0.0, 1.0, seed=41), dt), dt).astype(np.float64)
    b = O.from_storage(O.to_storage(synthetic.normal((1, k, n), 0.0, 1.0, seed=42), dt), dt).astype(np.float64)
    a[0, 5, 3] = np.nan
    a[0, 100, 7] = np.inf
    a[0, 101, 7] = -np.inf
    b[0, 9, 200] = np.nan
    b[0, 10, 300] = -np.inf
    b[0, 11, 301] = np.inf
    a_s, b_s = O.to_storage(a, dt), O.to_storage(b, dt)
    got = O.from_storage(run(A, a_s, b_s, dt), dt).astype(np.float64)
    assert A.backend_info().last_matmul.decode().startswith("mfma-lds")
    with np.errstate(invalid="ignore"):
        exact = a @ b
        scale = np.abs(a) @ np.abs(b)
    nan = np.isnan(exact)
    assert nan[0, 5].all() and nan[0, :, 200].all() and not nan.all()
    np.testing.assert_array_equal(np.isnan(got), nan)
    inf = np.isinf(exact)
    assert inf.any()
    np.testing.assert_array_equal(got[inf], exact[inf])
    fin = ~(nan | inf)
    assert np.all(np.abs(got[fin] - exact[fin]) <= 1e-2 * np.maximum(np.abs(exact[fin]), scale[fin] / math.sqrt(k)))


def test_config1_on_the_gpu(A):
    """Config 1 (A[256,512] @ B[512,256] fp32 U(-1,1) from seed S1 = 1, the
    HostArray product of contiguous_array_ce.c:1295-1343) through the HIP
    fp32 GEMM, element-wise against the oracle's sequential-fmaf product
    within the north-star GEMM bar 1e-4 * sqrt(K) * (|A||B|)_ij, and within
    gamma_K of the float64 product."""
    a, b = O.config1_operands()
    got = run(A, a, b, O.F32).astype(np.float64)
    expect = ref(a, b, O.F32).astype(np.float64)
    scale = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    assert got.shape == (256, 256)
    assert np.all(np.abs(got - expect) <= 1e-4 * math.sqrt(512) * scale)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.all(np.abs(got - exact) <= 512 * 2.0 ** -24 * scale)
    assert A.backend_info().last_matmul.decode().startswith("mfma-fp32")


# ------------------------------------------------ precision policy and tuning
def test_matmul_precision_reference():
    """matmul_precision.phpt:14-57 on a device without TF32: strict fp32 is the
    default, an unknown mode is refused without changing it, and a TF32
    request raises RuntimeException (gfx950 has no xf32 MFMA)."""
    from phptensors import backend as B
    from phptensors import InvalidArgumentException, RuntimeException
    assert B.cuda_get_backend_info()["precision"] == "fp32-strict"
    with pytest.raises(InvalidArgumentException):
        B.cuda_set_matmul_precision("unknown")
    assert B.cuda_get_backend_info()["precision"] == "fp32-strict"
    with pytest.raises(RuntimeException):
        B.cuda_set_matmul_precision("tf32")
    assert B.cuda_get_backend_info()["precision"] == "fp32-strict"
    B.cuda_set_matmul_precision("fp32-strict")


def test_matmul_tuning_reference():
    """matmul_tuning.phpt:12-46: tuning a 256x256 product measures candidates,
    selects exactly one, later products of that shape use it and stay exact,
    and a 32x32 product is not eligible."""
    from phptensors import backend as B
    from phptensors import CudaArray, InvalidArgumentException
    left, right = CudaArray.ones([256, 256]), CudaArray.ones([256, 256])
    tuning = B.cuda_tune_matmul(left, right)
    assert tuning["precision"] == "fp32-strict"
    assert tuning["candidateCount"] > 0
    assert 0 <= tuning["selectedCandidate"] < tuning["candidateCount"]
    selected = 0
    for i, cand in enumerate(tuning["candidates"]):
        assert cand["workspaceBytes"] == 0
        assert np.isfinite(cand["medianMs"]) and cand["medianMs"] > 0
        if cand["selected"]:
            assert i == tuning["selectedCandidate"]
            selected += 1
    assert selected == 1
    assert np.all(tuning["product"].toNumpy() == 256.0)
    product = left.matmul(right).toNumpy()
    assert product.shape == (256, 256) and np.all(product == 256.0)
    assert B.cuda_get_backend_info()["lastMatmul"].endswith("-tuned")
    with pytest.raises(InvalidArgumentException):
        B.cuda_tune_matmul(CudaArray.ones([32, 32]), CudaArray.ones([32, 32]))
    # a tuned choice applies to its own shape only
    other = CudaArray.ones([256, 128]).matmul(CudaArray.ones([128, 256]))
    assert np.all(other.toNumpy() == 128.0)
    assert not B.cuda_get_backend_info()["lastMatmul"].endswith("-tuned")


def test_matmul_large_dispatch_reference():
    """matmul_large_dispatch.phpt: a 4096x4096 fp32 product of ones is exact
    (4096 everywhere) and runs the large-problem strict-fp32 kernel, here the
    fp32 LDS-ring MFMA kernel."""
    from phptensors import backend as B
    from phptensors import CudaArray
    out = CudaArray.ones([4096, 4096]).matmul(CudaArray.ones([4096, 4096])).toNumpy()
    assert np.all(out == 4096.0)
    assert B.cuda_get_backend_info()["lastMatmul"] == "mfma-fp32-ring"
