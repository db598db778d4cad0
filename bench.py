#!/usr/bin/env python3
"""Benchmark of the php-gpu-tensors hot path on one MI355X.

Metric: GEMM TFLOP/s + reduce/fused-eltwise HBM GB/s as a
percentage of MI355X peak, 1 GPU.  Families measured:
  reduce : config 2 — X[8192,4096] fp32 N(0,1): sum, mean, max, argmax, var
           along the last axis, row softmax, layerNorm(eps=1e-5, gamma=1,
           beta=0)
  fused  : config 3 — Fusion plan tanh(x + y*z), x,z [16384,8192], y [8192],
           replayed through hipGraph
  gemm   : config 4 — batched A[32,2048,2048] @ B[32,2048,2048] in bf16
           (fp32 accumulate), fp16 and fp32
Inputs are resident in HBM before timing.  Kernels are captured into a HIP
graph (so host launch overhead does not stretch the timed region) and timed
with HIP events on the stream they run on.  Reduction inputs rotate over
enough replicas to exceed the 256 MB Infinity Cache so that every launch
streams from HBM.

Prints ONE JSON line.  `--gpus N` with N > 1 exits: this build runs on one
GPU.  Every workload here shards without exchange (batch of the GEMM, rows
of the reductions and of the fused plan); the MLP step would shard its batch
with one gradient all-reduce per step.
"""
import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "php-gpu-tensors_amd"))

import numpy as np  # noqa: E402

from phptensors import _abi as A  # noqa: E402
from phptensors import synthetic  # noqa: E402

HBM_PEAK_GBS = 8000.0

# HBM bytes per dispatch of each timed kernel: rocprofv3 --pmc FETCH_SIZE and
# --pmc WRITE_SIZE passes over this script (--no-cpu --copy-calibration
# --steps 2 --warmup 1 --only reduce,fused,gemm), each scaled by what the
# counter reads for a 128 MiB device copy (fetch x 2.0, write x 1.0).
# Re-measured when a kernel changes.
PMC_TRAFFIC_BYTES = {
    "reduce:sum": 134_491_134, "reduce:mean": 134_492_158, "reduce:max": 134_492_158,
    "reduce:argmax": 134_496_253, "reduce:var": 134_521_849, "reduce:softmax": 268_487_671,
    "reduce:layernorm": 269_103_243, "fused:tanh_x_plus_y_z": 1_610_491_925,
    "gemm:bf16": 1_073_920_169, "gemm:fp16": 1_088_352_095, "gemm:fp32": 3_757_844_716,
}
PEAK_TFLOPS = {"bf16": 2516.6, "fp16": 2516.6, "fp32": 157.3}
# pt_backend_info last_matmul path -> kernel symbol
GEMM_KERNELS = {"mfma-lds-wholeline": "k_gemm_wl", "mfma-lds-pingpong": "k_gemm_pp", "mfma-lds-ring": "k_gemm_ring",
                "mfma-direct-lds": "k_gemm_direct", "mfma-fp32": "k_gemm", "mfma-low-precision": "k_gemm",
                "mfma-fp32-ring": "k_gemm_f32r"}
MALL_BYTES = 256 << 20


# Untimed warm-up per timed kernel, in milliseconds of its own work.  The
# MI355X shader clock rises over the first tens of milliseconds of sustained
# load (three consecutive 40-launch windows of the bf16 config-4 GEMM ran at
# 564, 508 and 496 us per launch), so a fixed count of a few launches would
# time the ramp rather than the steady state.  The vendor legs use the same rule.
WARM_MS = 100.0


def warm_up(run, calls, launches_per_call=1):
    """Call run(calls) (which returns ms per launch) until WARM_MS of work has
    run, and at least once."""
    spent = 0.0
    while True:
        spent += run(calls) * calls * launches_per_call
        if spent >= WARM_MS:
            return


class GraphTimer:
    """Capture `launch()` `reps` times into a graph on a private stream and
    time replays with HIP events recorded on that stream."""

    def __init__(self, launch, reps):
        lib = A.load()
        self.lib = lib
        self.stream = ctypes.c_void_p()
        A.check(lib.pt_stream_create(ctypes.byref(self.stream)), "stream")
        self.reps = reps
        A.check(lib.pt_graph_begin_capture(self.stream), "capture")
        try:
            for r in range(reps):
                launch(self.stream, r)
        finally:
            g = ctypes.c_void_p()
            A.check(lib.pt_graph_end_capture(self.stream, ctypes.byref(g)), "end capture")
        self.graph = g
        self.ev0, self.ev1 = ctypes.c_void_p(), ctypes.c_void_p()
        A.check(lib.pt_event_create(ctypes.byref(self.ev0)), "event")
        A.check(lib.pt_event_create(ctypes.byref(self.ev1)), "event")

    def run(self, replays):
        lib = self.lib
        A.check(lib.pt_event_record(self.ev0, self.stream), "record")
        for _ in range(replays):
            A.check(lib.pt_graph_launch(self.graph, self.stream), "graph launch")
        A.check(lib.pt_event_record(self.ev1, self.stream), "record")
        A.check(lib.pt_event_synchronize(self.ev1), "sync")
        ms = ctypes.c_float()
        A.check(lib.pt_event_elapsed_ms(self.ev0, self.ev1, ctypes.byref(ms)), "elapsed")
        return ms.value / (replays * self.reps)  # ms per launch

    def close(self):
        self.lib.pt_graph_destroy(self.graph)
        self.lib.pt_event_destroy(self.ev0)
        self.lib.pt_event_destroy(self.ev1)
        self.lib.pt_stream_destroy(self.stream)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------- config 2
def reduce_family(steps, warmup):
    lib = A.load()
    rows, n = 8192, 4096
    x = synthetic.normal((rows, n), 0.0, 1.0, seed=2)
    nbytes = x.nbytes
    replicas = max(2, int(math.ceil(2 * MALL_BYTES / nbytes)))
    xs = [A.to_device(x) for _ in range(replicas)]
    shape, strides = A.ints([rows, n]), A.sizes([n, 1])
    out = A.DeviceBuffer(rows * 4)
    big = A.DeviceBuffer(rows * n * 4)
    gamma = A.to_device(np.ones(n, np.float32))
    beta = A.to_device(np.zeros(n, np.float32))
    red_bytes = nbytes + rows * 4
    row_bytes = 2 * nbytes

    def mk(kind):
        def launch(stream, r):
            p = xs[r % replicas].ptr
            if kind == "argmax":
                st = lib.pt_arg_reduce(p, out.ptr, A.FLOAT32, A.OP["argmax"], shape, strides, 2, 1, 0, stream)
            elif kind == "var":
                st = lib.pt_moments(p, out.ptr, A.FLOAT32, A.FLOAT32, shape, strides, 2, 1, 0, 0, stream)
            elif kind == "softmax":
                st = lib.pt_softmax(p, big.ptr, A.FLOAT32, A.FLOAT32, shape, strides, 2, 1, stream)
            elif kind == "layernorm":
                st = lib.pt_layernorm(p, big.ptr, A.FLOAT32, A.FLOAT32, rows, n, 1e-5,
                                      gamma.ptr, beta.ptr, stream)
            else:
                st = lib.pt_reduce(p, out.ptr, A.FLOAT32, A.OP[kind], shape, strides, 2, 1, 0, stream)
            A.check(st, kind)
        return launch

    results = {}
    for kind in ("sum", "mean", "max", "argmax", "var", "softmax", "layernorm"):
        t = GraphTimer(mk(kind), reps=2 * replicas)
        warm_up(t.run, max(1, warmup), t.reps)
        ms = t.run(max(1, steps))
        t.close()
        b = row_bytes if kind in ("softmax", "layernorm") else red_bytes
        gbs = b / (ms * 1e-3) / 1e9
        results[kind] = {"ms": ms, "bytes": b, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS,
                         "kernel": {"softmax": "k_row_softmax", "layernorm": "k_row_layernorm"}.get(
                             kind, "k_row_reduce")}
        log(f"reduce {kind}: {ms * 1e3:.1f} us  {gbs:.0f} GB/s  {100 * gbs / HBM_PEAK_GBS:.1f}% of HBM")
    total_ms = sum(r["ms"] for r in results.values())
    total_bytes = sum(r["bytes"] for r in results.values())
    # the HIP runtime's device-to-device copy of X (same bytes read and
    # written as softmax / layerNorm): the practical ceiling of a kernel
    # that streams one read and one write of equal size on this box
    def copy(stream, r):
        A.check(lib.pt_memcpy_d2d(big.ptr, xs[r % replicas].ptr, nbytes, stream), "copy")
    t = GraphTimer(copy, reps=2 * replicas)
    warm_up(t.run, max(1, warmup), t.reps)
    ms = t.run(max(1, steps))
    t.close()
    copy_gbs = row_bytes / (ms * 1e-3) / 1e9
    log(f"reduce copy reference (hipMemcpy D2D of X): {ms * 1e3:.1f} us  {copy_gbs:.0f} GB/s  "
        f"{100 * copy_gbs / HBM_PEAK_GBS:.1f}% of HBM")
    fam = {"workload": "config2: X[8192,4096] fp32 N(0,1) seed 2; sum/mean/max/argmax/var(-1), "
                       "softmax(-1), layerNorm([1],1e-5,1,0)",
           "ms_per_step": total_ms, "GB/s": total_bytes / (total_ms * 1e-3) / 1e9,
           "frac": total_bytes / (total_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "ops": results,
           "replicas": replicas,
           "copy_reference": {"op": "hipMemcpyAsync device-to-device of X (not timed in value)",
                              "ms": ms, "bytes": row_bytes, "GB/s": copy_gbs,
                              "frac": copy_gbs / HBM_PEAK_GBS}}
    return fam


# ---------------------------------------------------------------- config 3
def fused_family(steps, warmup, replays=100):
    """Fusion::compile of tanh(x + y*z), replayed through its HIP graph."""
    from phptensors import CudaArray, Fusion
    lib = A.load()
    rows, n = 16384, 8192
    x = CudaArray.fromNumpy(synthetic.uniform((rows, n), -2.0, 2.0, seed=3))
    z = CudaArray.fromNumpy(synthetic.uniform((rows, n), -2.0, 2.0, seed=31))
    y = CudaArray.fromNumpy(synthetic.uniform((n,), -2.0, 2.0, seed=32))
    graph = Fusion.compile(lambda a, b, c: (a + b * c).tanh(), [x, y, z], cudaGraph=True)
    plan = graph.getPlan()
    bytes_per = 3 * rows * n * 4 + n * 4
    ev0, ev1 = ctypes.c_void_p(), ctypes.c_void_p()
    A.check(lib.pt_event_create(ctypes.byref(ev0)), "event")
    A.check(lib.pt_event_create(ctypes.byref(ev1)), "event")

    def timed(count):
        # the plan runs on the runtime stream (NULL handle); events go there too
        A.check(lib.pt_event_record(ev0, None), "record")
        graph.replay(count, x, y, z)
        A.check(lib.pt_event_record(ev1, None), "record")
        A.check(lib.pt_event_synchronize(ev1), "sync")
        ms = ctypes.c_float()
        A.check(lib.pt_event_elapsed_ms(ev0, ev1, ctypes.byref(ms)), "elapsed")
        return ms.value / count

    warm_up(timed, max(1, warmup) * 10)
    samples = sorted(timed(replays) for _ in range(max(1, steps // 5)))
    ms = samples[len(samples) // 2]
    # FusionGraph::run as the reference calls it: bind, replay, synchronize per call
    t0 = time.perf_counter()
    for _ in range(10):
        graph.run(x, y, z)
    run_ms = (time.perf_counter() - t0) / 10 * 1e3
    stats = graph.getStats()
    lib.pt_event_destroy(ev0)
    lib.pt_event_destroy(ev1)
    gbs = bytes_per / (ms * 1e-3) / 1e9
    log(f"fused tanh(x+y*z): {ms * 1e3:.1f} us/replay  {gbs:.0f} GB/s  {100 * gbs / HBM_PEAK_GBS:.1f}% of HBM;"
        f" run() incl. bind+sync {run_ms * 1e3:.1f} us")
    res = {"ms": ms, "bytes": bytes_per, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS, "kernel": "fk0_v",
           "run_ms_with_sync": run_ms, "replays_per_sample": replays, "launches": replays}
    return {"workload": "config3: Fusion tanh(x + y*z), x,z [16384,8192] U(-2,2) seeds 3/31, "
                        "y [8192] seed 32; compiled once, replayed 100x via hipGraph",
            "ms_per_step": ms * replays, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS,
            "ops": {"tanh_x_plus_y_z": res}, "plan": plan,
            "stats": {k: stats[k] for k in ("fusedKernels", "graphLaunches", "executions", "cudaGraphCompatible")}}


def eager_family(steps, warmup):
    """Config 3 on the eager elementwise backend: m = y*z (row broadcast of
    y), s = x + m, t = tanh(s), three launches through the C-ABI
    (pt_broadcast, pt_broadcast, pt_unary), each timed against HBM."""
    lib = A.load()
    rows, n = 16384, 8192
    x = A.to_device(synthetic.uniform((rows, n), -2.0, 2.0, seed=3))
    z = A.to_device(synthetic.uniform((rows, n), -2.0, 2.0, seed=31))
    y = A.to_device(synthetic.uniform((n,), -2.0, 2.0, seed=32))
    m, s_, t = (A.DeviceBuffer(rows * n * 4) for _ in range(3))
    shape = A.ints([rows, n])
    dense, row_b = A.sizes([n, 1]), A.sizes([0, 1])
    big = rows * n * 4
    ops = {
        "mul_row_broadcast": (lambda st: lib.pt_broadcast(y.ptr, A.FLOAT32, row_b, 0, z.ptr, A.FLOAT32, dense, 0,
                                                          m.ptr, A.FLOAT32, A.OP["mul"], shape, 2, st),
                              2 * big + n * 4, "k_binary_f32_rows"),
        "add": (lambda st: lib.pt_broadcast(x.ptr, A.FLOAT32, dense, 0, m.ptr, A.FLOAT32, dense, 0,
                                            s_.ptr, A.FLOAT32, A.OP["add"], shape, 2, st),
                3 * big, "k_binary_f32_contig"),
        "tanh": (lambda st: lib.pt_unary(s_.ptr, A.FLOAT32, dense, 0, t.ptr, A.OP["tanh"], shape, 2, st),
                 2 * big, "k_unary_f32_contig"),
    }
    results = {}
    for name, (fn, nbytes, kernel) in ops.items():
        tm = GraphTimer(lambda stream, r, fn=fn: A.check(fn(stream), name), reps=4)
        warm_up(tm.run, max(1, warmup), tm.reps)
        ms = tm.run(max(1, steps))
        tm.close()
        gbs = nbytes / (ms * 1e-3) / 1e9
        results[name] = {"ms": ms, "bytes": nbytes, "GB/s": gbs, "frac": gbs / HBM_PEAK_GBS, "kernel": kernel}
        log(f"eager {name}: {ms * 1e3:.1f} us  {gbs:.0f} GB/s  {100 * gbs / HBM_PEAK_GBS:.1f}% of HBM")
    total_ms = sum(r["ms"] for r in results.values())
    total_b = sum(r["bytes"] for r in results.values())
    return {"workload": "config3 eager: m = y*z, s = x + m, t = tanh(s); x,z [16384,8192] U(-2,2), y [8192]",
            "ms_per_step": total_ms, "GB/s": total_b / (total_ms * 1e-3) / 1e9,
            "frac": total_b / (total_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "ops": results}


def fused_cpu_baseline(sample_rows=512):
    """Oracle tanh(x + y*z) (per-op rounding, libm tanhf, 1 thread) on a row sample."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    n = 8192
    x = synthetic.uniform((sample_rows, n), -2.0, 2.0, seed=3)
    z = synthetic.uniform((sample_rows, n), -2.0, 2.0, seed=31)
    y = synthetic.uniform((n,), -2.0, 2.0, seed=32)
    t0 = time.perf_counter()
    m = O.binary(y, O.F32, z, O.F32, "mul", O.F32)
    s = O.binary(x, O.F32, m, O.F32, "add", O.F32)
    O.unary(s, O.F32, "tanh")
    dt = time.perf_counter() - t0
    b = 3 * x.nbytes + y.nbytes
    return {"value": b / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{sample_rows} of 16384 rows of config 3 on one host core; {dt:.2f} s"}


def cpu_threads():
    """Host threads for the CPU baselines: the box's CPU share for one GPU
    (16), or fewer where the host has fewer."""
    return max(1, min(16, os.cpu_count() or 1))


def gemm_cpu_baseline():
    """Oracle matmul (the HostArray restatement: one sequential fmaf sum per
    output, contiguous_array_ce.c:1295-1343) on one whole batch of config 4,
    its outputs split over the host threads; the 32 batches take 32 times as
    long."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    m = k = n = 2048
    threads = cpu_threads()
    a = synthetic.normal((32, m, k), 0.0, 0.02, seed=4)[0]
    b = synthetic.normal((32, k, n), 0.0, 0.02, seed=5)[0]
    t0 = time.perf_counter()
    O.matmul(a, b, O.F32, threads=threads)
    dt = time.perf_counter() - t0
    return {"value": 2.0 * m * k * n / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "config_ms": 32 * dt * 1e3,
            "sample": f"fp32, batch 0 of 32 of config 4 (2048 x 2048 x 2048) on {threads} host threads; {dt:.2f} s; "
                      f"the 32 batches extrapolate to {32 * dt:.0f} s"}


# ---------------------------------------------------------------- config 4
def gemm_family(steps, warmup, dtypes=("bf16", "fp16", "fp32")):
    lib = A.load()
    bsz, m, n, k = 32, 2048, 2048, 2048
    flops = 2.0 * bsz * m * n * k
    a32 = synthetic.normal((bsz, m, k), 0.0, 0.02, seed=4)
    b32 = synthetic.normal((bsz, k, n), 0.0, 0.02, seed=5)
    results = {}
    code = {"bf16": A.BFLOAT16, "fp16": A.FLOAT16, "fp32": A.FLOAT32}
    for name in dtypes:
        dt = code[name]
        if dt == A.FLOAT32:
            ha, hb = a32, b32
        elif dt == A.FLOAT16:
            ha, hb = a32.astype(np.float16).view(np.uint16), b32.astype(np.float16).view(np.uint16)
        else:
            ha, hb = _to_bf16(a32), _to_bf16(b32)
        da, db = A.to_device(ha), A.to_device(hb)
        dc = A.DeviceBuffer(bsz * m * n * ha.itemsize)
        shp = A.ints([bsz, m, k])
        st = A.sizes([m * k, k, 1])

        def launch(stream, r, da=da, db=db, dc=dc, dt=dt):
            A.check(lib.pt_matmul(da.ptr, db.ptr, dc.ptr, dt, shp, st, 3, shp, st, 3, shp, 3,
                                  stream), "matmul")

        # four launches per graph, as the other families capture several: the
        # GPU leaves a few microseconds between two graph launches
        t = GraphTimer(launch, reps=4)
        warm_up(t.run, max(1, warmup), 4)
        ms = t.run(max(1, steps))
        t.close()
        path = A.backend_info().last_matmul.decode()
        tf = flops / (ms * 1e-3) / 1e12
        results[name] = {"ms": ms, "flop": flops, "TFLOP/s": tf, "peak": PEAK_TFLOPS[name],
                         "frac": tf / PEAK_TFLOPS[name], "kernel": GEMM_KERNELS.get(path, "k_gemm"),
                         "path": path}
        log(f"gemm {name}: {ms * 1e3:.1f} us  {tf:.1f} TFLOP/s  {100 * tf / PEAK_TFLOPS[name]:.1f}% of peak")
        del da, db, dc
    fam = {"workload": "config4: A,B [32,2048,2048] N(0,0.02) seeds 4/5; batched matmul "
                       + "/".join(dtypes),
           "ms_per_step": sum(r["ms"] for r in results.values()),
           "frac": results[dtypes[0]]["frac"], "ops": results}
    return fam


# torch.bmm on the config-4 operands (hipBLASLt / rocBLAS through PyTorch):
# a comparison point on the same box, run in a child process so that the
# library and torch never share one process.  Not the product path.
_VENDOR_GEMM = r"""
import json, time, torch
bsz, m, n, k = 32, 2048, 2048, 2048
g = torch.Generator(device="cuda").manual_seed(4)
out = {}
for name, dt in (("bf16", torch.bfloat16), ("fp16", torch.float16), ("fp32", torch.float32)):
    a = (torch.randn(bsz, m, k, device="cuda", generator=g) * 0.02).to(dt).contiguous()
    b = (torch.randn(bsz, k, n, device="cuda", generator=g) * 0.02).to(dt).contiguous()
    c = torch.empty(bsz, m, n, device="cuda", dtype=dt)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while True:  # warm-up: at least WARM_MS of work, as for this build's kernels
        for _ in range(STEPS // 2 + 1):
            torch.bmm(a, b, out=c)
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= WARM_MS_HERE:
            break
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(STEPS):
        torch.bmm(a, b, out=c)
    e1.record()
    e1.synchronize()
    out[name] = e0.elapsed_time(e1) / STEPS
    del a, b, c
print(json.dumps({"torch": torch.__version__, "ms": out,
                  "allow_tf32": torch.backends.cuda.matmul.allow_tf32}))
"""


def vendor_gemm(steps):
    """Time torch.bmm on the config-4 shapes in a child process."""
    import subprocess
    code = _VENDOR_GEMM.replace("STEPS", str(max(2, steps))).replace("WARM_MS_HERE", repr(WARM_MS))
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    if proc.returncode != 0:
        return {"error": proc.stderr.strip().splitlines()[-1] if proc.stderr.strip() else f"rc {proc.returncode}"}
    r = json.loads(proc.stdout.strip().splitlines()[-1])
    flops = 2.0 * 32 * 2048 * 2048 * 2048
    r["TFLOP/s"] = {k: flops / (v * 1e-3) / 1e12 for k, v in r["ms"].items()}
    log("torch.bmm: " + "  ".join(f"{k} {v * 1e3:.1f} us {r['TFLOP/s'][k]:.1f} TF/s" for k, v in r["ms"].items()))
    return r


# ---------------------------------------------------------------- config 5
def mlp_family(steps, warmup):
    """MLP training step (784->1024->1024->10, batch 4096, softmax-CE,
    backward, clip, AdamW) recorded once by Fusion.compile and replayed."""
    from phptensors import CudaArray, mlp
    from phptensors.optimizer import Optimizer
    lib = A.load()
    layers, rows = (784, 1024, 1024, 10), 4096
    params = mlp.init_parameters(layers, 5)
    x, y = mlp.synthetic_batch(rows, layers[0], layers[-1], 5)
    xt, yt = CudaArray.fromNumpy(x), CudaArray.fromNumpy(y)
    opt = Optimizer.adamW()
    state = opt.initState(params)
    rate = CudaArray.full([1], 1e-3)
    inputs = mlp.training_inputs(xt, yt, rate, params, state)
    graph = mlp.compile_training_plan(inputs, opt)
    ev0, ev1 = ctypes.c_void_p(), ctypes.c_void_p()
    A.check(lib.pt_event_create(ctypes.byref(ev0)), "event")
    A.check(lib.pt_event_create(ctypes.byref(ev1)), "event")

    def timed(count):
        A.check(lib.pt_event_record(ev0, None), "record")
        graph.replay(count, *inputs)
        A.check(lib.pt_event_record(ev1, None), "record")
        A.check(lib.pt_event_synchronize(ev1), "sync")
        ms = ctypes.c_float()
        A.check(lib.pt_event_elapsed_ms(ev0, ev1, ctypes.byref(ms)), "elapsed")
        return ms.value / count

    warm_up(timed, max(1, warmup))
    ms = timed(max(1, steps))
    # eager: the same step through the Python-level autograd, synchronized
    A.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        out = mlp.train_batch(xt, yt, params, opt, state, rate)
    out["loss"].item()
    eager_ms = (time.perf_counter() - t0) / 3 * 1e3
    lib.pt_event_destroy(ev0)
    lib.pt_event_destroy(ev1)
    flops = mlp.step_flops(rows, layers)
    tf = flops / (ms * 1e-3) / 1e12
    log(f"mlp step (compiled plan): {ms * 1e3:.1f} us  {tf:.1f} TFLOP/s  {100 * tf / PEAK_TFLOPS['fp32']:.1f}% of fp32;"
        f" eager {eager_ms * 1e3:.1f} us")
    kinds = [s["kind"] for s in graph.getPlan()]
    return {"workload": "config5: MLP 784-1024-1024-10 fp32, batch 4096, softmax-CE, backward, clip 5, AdamW 1e-3",
            "ms_per_step": ms, "TFLOP/s": tf, "frac": tf / PEAK_TFLOPS["fp32"], "flop_per_step": flops,
            "eager_ms_per_step": eager_ms, "plan_steps": len(kinds), "plan_native_steps": kinds.count("native"),
            "plan_kernels": kinds.count("fused"), "workspace_bytes": graph.getStats().get("workspaceBytes"),
            "row_chains": graph.getStats().get("rowChains"), "row_chain_steps": graph.getStats().get("rowChainSteps")}


# The step's products with the operand layouts the compiled plan hands to
# pt_matmul: name -> (A shape, A strides, B shape, B strides), row-major
# storage of x [4096, 784], h1 / dZ2 / dZ1 [4096, 1024], W1 [784, 1024],
# W2 [1024, 1024] (transposes are strided views, as in the plan).
_MLP_GEMMS = {
    "G1 x.W1": ((4096, 784), (784, 1), (784, 1024), (1024, 1)),
    "G2 h1.W2": ((4096, 1024), (1024, 1), (1024, 1024), (1024, 1)),
    "dH1 dZ2.W2T": ((4096, 1024), (1024, 1), (1024, 1024), (1, 1024)),
    "dW2 h1T.dZ2": ((1024, 4096), (1, 1024), (4096, 1024), (1024, 1)),
    "dW1 xT.dZ1": ((784, 4096), (1, 784), (4096, 1024), (1024, 1)),
}


def mlp_gemms(steps):
    """The five large fp32 products of the config-5 step, each timed alone
    (graph replays of pt_matmul on synthetic operands of the step's shapes
    and layouts).  Split-K scratch comes from a workspace sized by one
    measuring call and handed in with pt_workspace_begin, as the compiled
    plan hands it to its native steps, so the graph holds no allocation
    nodes."""
    lib = A.load()
    rng = np.random.default_rng(5)
    out = {}
    c = A.DeviceBuffer(4096 * 1024 * 4)
    for name, (ash, ast, bsh, bst) in _MLP_GEMMS.items():
        span_a = 1 + sum((d - 1) * st for d, st in zip(ash, ast))
        span_b = 1 + sum((d - 1) * st for d, st in zip(bsh, bst))
        da = A.to_device((rng.standard_normal(span_a, dtype=np.float32) * 0.05).astype(np.float32))
        db = A.to_device((rng.standard_normal(span_b, dtype=np.float32) * 0.05).astype(np.float32))
        m, k, n = ash[0], ash[1], bsh[1]
        sa, sta, sb, stb, sc = A.ints(list(ash)), A.sizes(list(ast)), A.ints(list(bsh)), A.sizes(list(bst)), A.ints([m, n])

        def matmul(stream, da=da, db=db, sa=sa, sta=sta, sb=sb, stb=stb, sc=sc):
            A.check(lib.pt_matmul(da.ptr, db.ptr, c.ptr, A.FLOAT32, sa, sta, 2, sb, stb, 2, sc, 2, stream), "matmul")
        A.check(lib.pt_workspace_begin(None, 0), "workspace")
        matmul(None)
        peak = ctypes.c_size_t()
        A.check(lib.pt_workspace_end(ctypes.byref(peak)), "workspace")
        ws_bytes = max(256, peak.value)
        ws = A.DeviceBuffer(ws_bytes)

        def launch(stream, r, matmul=matmul, ws=ws, ws_bytes=ws_bytes):
            A.check(lib.pt_workspace_begin(ws.ptr, ws_bytes), "workspace")
            try:
                matmul(stream)
            finally:
                A.check(lib.pt_workspace_end(None), "workspace")
        t = GraphTimer(launch, reps=4)
        warm_up(t.run, 2, t.reps)
        ms = t.run(max(2, steps))
        t.close()
        out[name] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1)}
    log("config-5 products: " + "  ".join(f"{k} {v['us']} us" for k, v in out.items()))
    return out


_VENDOR_MLP = r"""
import json, time, torch
torch.backends.cuda.matmul.allow_tf32 = False
g = torch.Generator(device="cuda").manual_seed(5)
SHAPES = SHAPES_HERE
out = {}
for name, (ash, ast, bsh, bst) in SHAPES.items():
    def operand(shape, strides):
        span = 1 + sum((d - 1) * s for d, s in zip(shape, strides))
        base = torch.randn(span, device="cuda", generator=g) * 0.05
        return torch.as_strided(base, shape, strides)
    a, b = operand(ash, ast), operand(bsh, bst)
    c = torch.empty(ash[0], bsh[1], device="cuda")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while True:  # warm-up: at least WARM_MS of work, as for this build's kernels
        for _ in range(STEPS // 2 + 1):
            torch.mm(a, b, out=c)
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= WARM_MS_HERE:
            break
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(STEPS):
        torch.mm(a, b, out=c)
    e1.record()
    e1.synchronize()
    out[name] = e0.elapsed_time(e1) / STEPS
print(json.dumps({"ms": out}))
"""


def vendor_mlp_gemms(steps):
    """torch.mm (hipBLASLt / rocBLAS) on the same five products, in a child
    process: a comparison point only."""
    import subprocess
    code = (_VENDOR_MLP.replace("STEPS", str(max(4, steps))).replace("SHAPES_HERE", repr(_MLP_GEMMS))
            .replace("WARM_MS_HERE", repr(WARM_MS)))
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=600)
    if proc.returncode != 0:
        return {"error": proc.stderr.strip().splitlines()[-1] if proc.stderr.strip() else f"rc {proc.returncode}"}
    r = json.loads(proc.stdout.strip().splitlines()[-1])
    out = {k: round(v * 1e3, 1) for k, v in r["ms"].items()}
    log("torch.mm on the config-5 products: " + "  ".join(f"{k} {v} us" for k, v in out.items()))
    return {"us": out}


def transfer_family(steps, nbytes=256 << 20):
    """Host <-> device transfers through pt_memcpy_h2d / pt_memcpy_d2h
    (tensor_transfer.c:45-65): a pageable numpy buffer (staged through the
    library's pinned ring) and a pinned one (pt_host_alloc_pinned, copied
    directly: the link's own rate), each timed on the host clock around the
    synchronous call, best of `steps`."""
    lib = A.load()
    dev = A.DeviceBuffer(nbytes)
    pageable = np.full(nbytes, 7, np.uint8)
    pinned = ctypes.c_void_p()
    A.check(lib.pt_host_alloc_pinned(ctypes.byref(pinned), nbytes), "pinned")
    out = {"bytes": nbytes}
    try:
        np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(pinned.value))[:] = 7
        for name, host in (("pageable", pageable.ctypes.data), ("pinned", pinned.value)):
            for way, fn in (("h2d", lambda: lib.pt_memcpy_h2d(dev.ptr, host, nbytes, None)),
                            ("d2h", lambda: lib.pt_memcpy_d2h(host, dev.ptr, nbytes, None))):
                best = None
                for _ in range(max(3, steps)):
                    t0 = time.perf_counter()
                    A.check(fn(), way)
                    dt = time.perf_counter() - t0
                    best = dt if best is None else min(best, dt)
                out[f"{way}_{name}_GB/s"] = round(nbytes / best / 1e9, 1)
    finally:
        A.check(lib.pt_host_free_pinned(pinned.value), "free pinned")
    log(f"transfers: {out}")
    return out


def mlp_cpu_baseline(sample_rows=4096):
    """The reference's CPU path for the config-5 step: its eight GEMMs at the
    config-5 shapes (the full batch of 4096 rows) through the oracle's
    HostArray matmul restatement (sequential fmaf, contiguous_array_ce.c:
    1295-1343), the outputs of each product split over the host threads.
    The elementwise, loss and AdamW work (under 0.1 % of the step's FLOPs)
    is left out."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    r = sample_rows
    threads = cpu_threads()
    # (M, K, N): forward x.W1, h1.W2, h2.W3; backward dZ3.W3^T, dZ2.W2^T,
    # h2^T.dZ3, h1^T.dZ2, x^T.dZ1
    shapes = [(r, 784, 1024), (r, 1024, 1024), (r, 1024, 10), (r, 10, 1024), (r, 1024, 1024),
              (1024, r, 10), (1024, r, 1024), (784, r, 1024)]
    ops = []
    for i, (m, k, n) in enumerate(shapes):
        ops.append((synthetic.normal((m, k), 0.0, 0.05, seed=50 + i),
                    synthetic.normal((k, n), 0.0, 0.05, seed=70 + i)))
    t0 = time.perf_counter()
    for a, b in ops:
        O.matmul(a, b, O.F32, threads=threads)
    dt = time.perf_counter() - t0
    flops = sum(2.0 * m * k * n for m, k, n in shapes)
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "step_ms_at_4096_rows": dt * 4096 / r * 1e3,
            "sample": f"the step's 8 GEMMs at {r} of 4096 rows through the oracle's HostArray matmul "
                      f"restatement (sequential fmaf) on {threads} host threads; {dt:.2f} s"}


def _to_bf16(x):
    """float32 -> bfloat16 bits, round to nearest even (NaN-free input)."""
    u = x.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def reduce_cpu_baseline(min_seconds=10.0):
    """The oracle (scalar C restatement, 1 thread) on the full config-2 input."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    rows, n = 8192, 4096
    x = synthetic.normal((rows, n), 0.0, 1.0, seed=2)
    ones, zeros = np.ones(n, np.float32), np.zeros(n, np.float32)
    # repeat the full step until about 10 s of single-core work have run
    steps = 0
    t0 = time.perf_counter()
    while True:
        O.reduce(x, O.F32, "sum", 1)
        O.reduce(x, O.F32, "mean", 1)
        O.reduce(x, O.F32, "max", 1)
        O.arg_reduce(x, O.F32, "argmax", 1)
        O.moments(x, O.F32, 1)
        O.softmax_lastaxis(x)
        O.layernorm_lastaxis(x, 1e-5, ones, zeros)
        steps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or steps >= 64:
            break
    total_bytes = steps * (5 * (x.nbytes + rows * 4) + 2 * 2 * x.nbytes)
    return {"value": total_bytes / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{steps} full config-2 steps (all 7 ops over X[8192,4096]) on one host core; "
                      f"{dt:.2f} s", "seconds": dt}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", default="reduce,fused,gemm,mlp,eager,transfer")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--vendor", action="store_true",
                    help="also time torch.bmm on the config-4 shapes (child process; comparison only)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 128 MiB device copy first (reference for PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU only: this build has no multi-GPU path "
              "(each workload would shard by batch or rows on one process per GPU).", file=sys.stderr)
        sys.exit(2)
    if os.environ.get("RANK", "0") != "0":
        return
    lib = A.load()
    A.check(lib.pt_init(), "init")
    info = A.device_info()
    log(f"device {info.name.decode()} {info.arch.decode()} CUs={info.compute_units}")
    if args.copy_calibration:
        src = A.DeviceBuffer(128 << 20)
        dst = A.DeviceBuffer(128 << 20)
        for _ in range(3):
            A.check(lib.pt_memcpy_d2d(dst.ptr, src.ptr, 128 << 20, None), "copy")
        A.synchronize()
        log("copy calibration: 3 x 128 MiB device-to-device copies")
    fams = {}
    t_wall = time.perf_counter()
    only = set(args.only.split(","))
    if "reduce" in only:
        fams["reduce"] = reduce_family(args.steps, args.warmup)
    if "fused" in only:
        fams["fused"] = fused_family(args.steps, args.warmup)
    if "gemm" in only:
        fams["gemm"] = gemm_family(args.steps, args.warmup)
        if args.vendor:
            fams["gemm"]["vendor_torch_bmm"] = vendor_gemm(args.steps)
    # config 5 is reported beside the metric (it is not one of its families)
    extra = {}
    if "mlp" in only:
        extra["mlp"] = mlp_family(max(1, args.steps // 2), args.warmup)
        extra["mlp"]["products"] = mlp_gemms(args.steps)
        if args.vendor:
            extra["mlp"]["vendor_torch_mm"] = vendor_mlp_gemms(args.steps)
    if "eager" in only:
        extra["eager"] = eager_family(args.steps, args.warmup)
    if "transfer" in only:
        extra["transfer"] = transfer_family(args.steps)
    wall = time.perf_counter() - t_wall

    # dominant kernel: the largest share of a step (time per launch x
    # launches per step: the fused plan replays 100 times per step)
    dom = None
    for fname, fam in fams.items():
        for k, r in fam.get("ops", {}).items():
            if dom is None or r["ms"] * r.get("launches", 1) > dom[2]["ms"] * dom[2].get("launches", 1):
                dom = (fname, k, r)
    roofline = None
    if dom is not None:
        r = dom[2]
        op = f"{dom[0]}:{dom[1]}"
        if "GB/s" in r:
            roofline = {"bound": "hbm", "kernel": r["kernel"], "op": op,
                        "achieved": round(r["GB/s"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(r["GB/s"] / HBM_PEAK_GBS, 4),
                        "traffic": PMC_TRAFFIC_BYTES.get(op)}
        else:
            roofline = {"bound": "mfma", "kernel": r["kernel"], "op": op,
                        "achieved": round(r["TFLOP/s"], 1), "peak": r["peak"], "unit": "TFLOP/s",
                        "frac": round(r["frac"], 4), "traffic": PMC_TRAFFIC_BYTES.get(op)}
        roofline["traffic_unit"] = "bytes per launch (HBM, PMC)"
        roofline["share_of_step"] = round(r["ms"] * r.get("launches", 1) / sum(
            f["ms_per_step"] for f in fams.values()), 4)
    # every timed kernel against its own roofline
    kernels = []
    for fname, fam in fams.items():
        for k, r in fam.get("ops", {}).items():
            op = f"{fname}:{k}"
            kernels.append({"op": op, "kernel": r["kernel"], "us": round(r["ms"] * 1e3, 2),
                            "achieved": round(r.get("GB/s", r.get("TFLOP/s", 0.0)), 1),
                            "unit": "GB/s" if "GB/s" in r else "TFLOP/s", "frac": round(r["frac"], 4),
                            "traffic": PMC_TRAFFIC_BYTES.get(op)})
    fracs = [f["frac"] for f in fams.values()]
    value = 100.0 * sum(fracs) / len(fracs) if fracs else 0.0
    cpu = None
    if not args.no_cpu and "reduce" in fams:
        cpu = reduce_cpu_baseline()
        cpu["cpu_model"] = _cpu_model()
        cpu["nproc"] = os.cpu_count()
        if "fused" in fams:
            fams["fused"]["cpu_baseline"] = fused_cpu_baseline()
        if "gemm" in fams:
            fams["gemm"]["cpu_baseline"] = gemm_cpu_baseline()
        if "mlp" in extra:
            extra["mlp"]["cpu_baseline"] = mlp_cpu_baseline()
    ms_step = sum(f["ms_per_step"] for f in fams.values())
    line = {
        "metric": "GEMM TFLOP/s + reduce/fused-eltwise HBM GB/s, % of MI355X peak, 1 GPU",
        "value": round(value, 2),
        "unit": "% of MI355X peak (mean over families)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        # the reduce and fused families compute in fp32, the GEMM headline in
        # bf16 with fp32 accumulation (fp16 and fp32 GEMMs reported beside it)
        "dtype": "fp32+bf16", "data": "synthetic (SplitMix64/Box-Muller, fixed seeds)",
        "config": {"workload": "configs 2-4: fp32 row reductions X[8192,4096]; Fusion tanh(x+y*z) [16384,8192] x100 "
                               "hipGraph replays; batched GEMM [32,2048,2048]^2 bf16 (fp16, fp32 beside)",
                   "families": sorted(fams),
                   "details": {f: fams[f]["workload"] for f in ("reduce", "fused", "gemm") if f in fams}},
        "families": {k: {kk: vv for kk, vv in v.items()} for k, v in fams.items()},
        "roofline": roofline,
        # the north-star kernel (bf16 batched GEMM) against the dense bf16 MFMA peak
        "gemm_bf16_roofline": ({"kernel": fams["gemm"]["ops"]["bf16"]["kernel"],
                                "achieved": round(fams["gemm"]["ops"]["bf16"]["TFLOP/s"], 1),
                                "peak": PEAK_TFLOPS["bf16"], "unit": "TFLOP/s",
                                "frac": round(fams["gemm"]["ops"]["bf16"]["frac"], 4),
                                "traffic": PMC_TRAFFIC_BYTES.get("gemm:bf16")}
                               if "gemm" in fams and "bf16" in fams["gemm"]["ops"] else None),
        "kernels": kernels,
        "config5_mlp": extra.get("mlp"),
        "config3_eager": extra.get("eager"),
        "transfers": extra.get("transfer"),
        "cpu_baseline": cpu,
        "wall_s": round(wall, 2),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
