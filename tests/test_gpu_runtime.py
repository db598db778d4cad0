"""GPU tests of the runtime part of the C-ABI: pool allocations, transfers,
byte fills, streams/events and graph capture + replay (every replay checked
against the eager result, with eager work and synchronizations between
replays)."""
import ctypes

import numpy as np
import pytest

from phptensors import _abi as A

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    lib = A.load()
    A.check(lib.pt_init(), "init")
    return lib


def test_device_info(lib):
    info = A.device_info()
    assert info.arch.decode().startswith("gfx950")
    assert info.warp_size == 64 and info.compute_units >= 1
    assert info.total_memory > (1 << 30)


@pytest.mark.parametrize("nbytes", [1, 3, 255, 4096, 1 << 20, (1 << 20) + 7])
def test_memset_and_copies(lib, nbytes):
    buf = A.DeviceBuffer(nbytes)
    A.check(lib.pt_memset(buf.ptr, 0xA5, nbytes, None), "memset")
    got = buf.download(np.uint8, (nbytes,))
    assert np.all(got == 0xA5)
    src = np.random.default_rng(nbytes).integers(0, 256, nbytes, dtype=np.uint8)
    buf.upload(src)
    dst = A.DeviceBuffer(nbytes)
    A.check(lib.pt_memcpy_d2d(dst.ptr, buf.ptr, nbytes, None), "d2d")
    assert np.array_equal(dst.download(np.uint8, (nbytes,)), src)


@pytest.mark.parametrize("nbytes", [(4 << 20) - 1, 4 << 20, (37 << 20) + 13, (70 << 20) + 5])
@pytest.mark.parametrize("offset", [0, 3])
def test_staged_transfers_round_trip(lib, nbytes, offset):
    """Pageable host buffers of 4 MiB and more move through the pinned
    staging ring (ragged last chunks, odd host and device offsets); smaller
    ones through one hipMemcpyAsync.  Both directions byte-exact."""
    rng = np.random.default_rng(nbytes + offset)
    host = np.empty(nbytes + offset, np.uint8)[offset:]
    host[:] = rng.integers(0, 256, nbytes, dtype=np.uint8)
    dev = A.DeviceBuffer(nbytes + offset)
    before = A.backend_info().staged_copies
    A.check(lib.pt_memcpy_h2d(dev.ptr + offset, host.ctypes.data, nbytes, None), "h2d")
    back = np.empty(nbytes + 5, np.uint8)[5:]
    A.check(lib.pt_memcpy_d2h(back.ctypes.data, dev.ptr + offset, nbytes, None), "d2h")
    assert np.array_equal(back, host)
    staged = A.backend_info().staged_copies - before
    assert staged == (2 if nbytes >= 4 << 20 else 0)
    # the device copy itself holds the bytes (checked without the staging path)
    probe = A.DeviceBuffer(nbytes)
    A.check(lib.pt_memcpy_d2d(probe.ptr, dev.ptr + offset, nbytes, None), "d2d")
    A.check(lib.pt_device_synchronize(), "sync")
    pinned = ctypes.c_void_p()
    A.check(lib.pt_host_alloc_pinned(ctypes.byref(pinned), nbytes), "pinned")
    try:
        view = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(pinned.value))
        view[:] = 0
        A.check(lib.pt_memcpy_d2h(pinned.value, probe.ptr, nbytes, None), "d2h pinned")
        assert np.array_equal(view, host)
        assert A.backend_info().staged_copies - before == staged  # pinned: copied directly
    finally:
        A.check(lib.pt_host_free_pinned(pinned.value), "free pinned")


def test_staged_transfers_from_several_threads(lib):
    """Four host threads move pageable buffers through the one staging ring
    at the same time (the foreign calls run without the interpreter lock):
    the transfers take turns and every byte arrives."""
    import threading
    nbytes = (9 << 20) + 123
    errors = []

    def worker(seed):
        try:
            rng = np.random.default_rng(seed)
            dev = A.DeviceBuffer(nbytes)
            for _ in range(3):
                host = rng.integers(0, 256, nbytes, dtype=np.uint8)
                A.check(lib.pt_memcpy_h2d(dev.ptr, host.ctypes.data, nbytes, None), "h2d")
                back = np.empty(nbytes, np.uint8)
                A.check(lib.pt_memcpy_d2h(back.ctypes.data, dev.ptr, nbytes, None), "d2h")
                if not np.array_equal(back, host):
                    errors.append(f"thread {seed}: bytes differ")
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(f"thread {seed}: {e}")

    before = A.backend_info().staged_copies
    threads = [threading.Thread(target=worker, args=(s,)) for s in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a transfer thread did not finish"
    assert not errors, errors
    assert A.backend_info().staged_copies - before == 4 * 3 * 2


def test_pool_reuse_and_info(lib):
    bufs = [A.DeviceBuffer(s) for s in (1 << 10, 1 << 20, 1 << 24, 3, 1 << 16)]
    for b in bufs:
        b.free()
    free, total, reserved = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    A.check(lib.pt_mem_info(ctypes.byref(free), ctypes.byref(total), ctypes.byref(reserved)), "mem info")
    assert total.value >= free.value > 0


def test_fill_dtypes(lib):
    for dt, npdt, val, raw in ((A.FLOAT32, np.float32, 2.5, 2.5), (A.INT32, np.int32, -7, -7),
                               (A.FLOAT64, np.float64, 1.25, 1.25), (A.UINT8, np.uint8, 200, 200)):
        buf = A.DeviceBuffer(1000 * np.dtype(npdt).itemsize)
        s = A.scalar(val, dt)
        A.check(lib.pt_fill(buf.ptr, dt, 1000, ctypes.byref(s), None), "fill")
        assert np.all(buf.download(npdt, (1000,)) == raw)


def test_graph_capture_replays_match_eager(lib):
    """A captured plan (fill -> scalar op -> row sum, plus a byte fill) is
    replayed 5 times; eager work and synchronizations run between replays and
    every replay is checked against the eager result."""
    rows, n = 64, 1000
    x = np.random.default_rng(5).standard_normal((rows, n)).astype(np.float32)
    dx = A.to_device(x)
    tmp = A.DeviceBuffer(x.nbytes)
    out = A.DeviceBuffer(rows * 4)
    flag = A.DeviceBuffer(256)
    shape, strides = A.ints([rows, n]), A.sizes([n, 1])
    two = A.scalar(2.0, A.FLOAT32)

    def launch(stream):
        A.check(lib.pt_memset(flag.ptr, 0, 256, stream), "memset")
        A.check(lib.pt_scalar(dx.ptr, A.FLOAT32, strides, 0, ctypes.byref(two), 0, tmp.ptr, A.FLOAT32,
                              A.OP["mul"], shape, 2, stream), "scalar")
        A.check(lib.pt_reduce(tmp.ptr, out.ptr, A.FLOAT32, A.OP["sum"], shape, strides, 2, 1, 0, stream),
                "reduce")

    launch(None)
    A.synchronize()
    eager = out.download(np.float32, (rows,))
    stream = ctypes.c_void_p()
    A.check(lib.pt_stream_create(ctypes.byref(stream)), "stream")
    A.check(lib.pt_graph_begin_capture(stream), "capture")
    launch(stream)
    g = ctypes.c_void_p()
    A.check(lib.pt_graph_end_capture(stream, ctypes.byref(g)), "end capture")
    nodes = ctypes.c_size_t()
    A.check(lib.pt_graph_node_count(g, ctypes.byref(nodes)), "nodes")
    assert nodes.value >= 3
    for i in range(5):
        # clobber the outputs eagerly, then replay
        A.check(lib.pt_memset(out.ptr, 0xFF, rows * 4, None), "memset")
        A.check(lib.pt_memset(flag.ptr, 0x11, 256, None), "memset")
        A.synchronize()
        A.check(lib.pt_graph_launch(g, stream), "launch")
        A.check(lib.pt_stream_synchronize(stream), "sync")
        assert np.array_equal(out.download(np.float32, (rows,)), eager), f"replay {i}"
        assert np.all(flag.download(np.uint8, (256,)) == 0), f"replay {i} fill"
    A.check(lib.pt_graph_destroy(g), "destroy")
    A.check(lib.pt_stream_destroy(stream), "stream destroy")


def test_events_time_a_kernel(lib):
    ev0, ev1 = ctypes.c_void_p(), ctypes.c_void_p()
    A.check(lib.pt_event_create(ctypes.byref(ev0)), "event")
    A.check(lib.pt_event_create(ctypes.byref(ev1)), "event")
    buf = A.DeviceBuffer(1 << 24)
    A.check(lib.pt_event_record(ev0, None), "record")
    A.check(lib.pt_memset(buf.ptr, 1, 1 << 24, None), "memset")
    A.check(lib.pt_event_record(ev1, None), "record")
    A.check(lib.pt_event_synchronize(ev1), "sync")
    done = ctypes.c_int()
    A.check(lib.pt_event_query(ev1, ctypes.byref(done)), "query")
    assert done.value == 1
    ms = ctypes.c_float()
    A.check(lib.pt_event_elapsed_ms(ev0, ev1, ctypes.byref(ms)), "elapsed")
    assert ms.value >= 0.0
    lib.pt_event_destroy(ev0)
    lib.pt_event_destroy(ev1)


def test_rtc_compile_error_is_reported(lib):
    mod = ctypes.c_void_p()
    log = ctypes.create_string_buffer(4096)
    st = lib.pt_rtc_compile(b"extern \"C\" __global__ void k(){ this is not c++ }", b"bad.hip",
                            ctypes.byref(mod), log, 4096)
    assert st == 5  # PT_ERR_COMPILE
    assert b"error" in log.value


def test_rtc_compile_and_launch(lib):
    src = (b"extern \"C\" __global__ void k(float* o, const float* a, unsigned n)"
           b"{unsigned i=blockIdx.x*blockDim.x+threadIdx.x; if(i<n) o[i]=a[i]*3.0f+1.0f;}")
    mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
    A.check(lib.pt_rtc_compile(src, b"k.hip", ctypes.byref(mod), None, 0), "compile")
    A.check(lib.pt_module_function(mod, b"k", ctypes.byref(fn)), "function")
    a = np.arange(1000, dtype=np.float32)
    da, do = A.to_device(a), A.DeviceBuffer(a.nbytes)
    po, pa, pn = ctypes.c_void_p(do.ptr), ctypes.c_void_p(da.ptr), ctypes.c_uint(1000)
    params = (ctypes.c_void_p * 3)(ctypes.addressof(po), ctypes.addressof(pa), ctypes.addressof(pn))
    A.check(lib.pt_launch(fn, 4, 256, params, None), "launch")
    A.synchronize()
    assert np.array_equal(do.download(np.float32, (1000,)), a * 3.0 + 1.0)
    A.check(lib.pt_module_unload(mod), "unload")
