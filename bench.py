#!/usr/bin/env python3
"""Benchmark of the tensor-op hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only N]

The headline line measures config 2, the fused elementwise/broadcast map chain
y = tanh(0.75 x - 0.25) * exp(-x^2) + bias[col] over x f32 [8192][8192]: one step is one
vdsl_op_map_chain call over the whole tensor, inputs resident in HBM before the timed region.
`value` is achieved HBM GB/s from algorithmic bytes (read x, write y, read bias) over the HIP-event
time of the K steps on the op's own queue.  The other configs are reported under `per_config`
with their own units and roofline fractions.  Prints exactly one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, GB/s
PEAK_FP32_TFLOPS = 157.3       # vector FP32 (packed FMA), TFLOP/s
PEAK_BF16_TFLOPS = 2516.6      # dense MFMA bf16
PEAK_INT8_TOPS = 5033.2        # dense MFMA int8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (profiles/traffic.json, written from the counter runs described in profiles/traffic_counters.md,
    each counter scaled by what it reads for a 512 MiB copy); None if not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)["kernels"][kernel]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def measured_valu_issue():
    """VALU-issue share of the escape-time kernel's cycles from the committed rocprofv3 counter pass
    (profiles/escape_time_valu.json: SQ_INSTS_VALU x 4 cycles / 1024 SIMDs over SQ_BUSY_CYCLES per
    shader engine, as profiles/escape_time_valu_counters.md derives it); None if not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "escape_time_valu.json")) as f:
            d = json.load(f)
        return {"valu_issue_frac": d["valu_issue_frac"], "effective_clock_ghz": d["effective_clock_ghz"],
                "source": d["source"]}
    except (OSError, KeyError, ValueError):
        return None


def time_launches(q, dev, fn, reps, warmup=30, warmup_ms=25.0):
    """Mean duration of one fn() call from HIP events on q's stream around `reps` back-to-back
    stream launches, after at least `warmup` untimed calls and at least `warmup_ms` of wall time
    spent in them (the clocks take milliseconds of GPU work to ramp up after host-side setup: a
    GEMM timed after 30 launches, ~2 ms, reads 7-10% low).  This is the per-kernel figure; graph
    replays (time_replays) add the graph's launch latency to the first node."""
    from vernondsl_amd.rhi import Event
    t0 = time.perf_counter()
    n = 0
    while n < warmup or (time.perf_counter() - t0) * 1e3 < warmup_ms:
        fn()
        n += 1
        if n % 8 == 0:
            q.sync()
    q.sync()
    e0, e1 = Event(dev), Event(dev)
    e0.record(q)
    for _ in range(reps):
        fn()
    e1.record(q)
    q.sync()
    ms = e0.elapsed_ms(e1) / reps
    e0.destroy()
    e1.destroy()
    return ms


def time_replays(q, dev, fn, steps, warmup, per_graph=1, warmup_ms=25.0):
    """Records `per_graph` consecutive calls of fn() into one hipGraph, replays it at least `warmup`
    times and for at least `warmup_ms` of wall time, then `steps` times; returns (ms per call from
    HIP events on q's stream, wall ms per call).  fn() runs once eagerly first: a map chain the
    library compiles at run time is compiled there (nothing is compiled while recording)."""
    from vernondsl_amd.rhi import Event
    fn()
    q.sync()
    with q.capture() as rec:
        for _ in range(per_graph):
            fn()
    g = rec.graph
    t0 = time.perf_counter()
    n = 0
    while n < warmup or (time.perf_counter() - t0) * 1e3 < warmup_ms:
        g.launch(q)
        n += 1
        if n % 4 == 0:
            q.sync()
    q.sync()
    e0, e1 = Event(dev), Event(dev)
    t0 = time.perf_counter()
    e0.record(q)
    for _ in range(steps):
        g.launch(q)
    e1.record(q)
    q.sync()
    wall = (time.perf_counter() - t0) * 1e3
    ms = e0.elapsed_ms(e1)
    g.destroy()
    e0.destroy()
    e1.destroy()
    n = steps * per_graph
    return ms / n, wall / n


def time_ops_in_step(q, dev, exe, reps, warmup_ms=25.0):
    """In-step duration of every op of an Executable's step: `reps` steps are issued op by op on q,
    back to back on their real buffers, with a HIP event recorded on q after each op; the mean over
    the steps of the time between consecutive events.  An untimed lead step ahead of them keeps the
    queue busy, so no event waits on a launch from the host (after at least `warmup_ms` of wall time
    in untimed steps).  Returns (per-op ms list, mean ms of the whole evented step)."""
    from vernondsl_amd.rhi import Event
    ops = exe.graph.ops
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warmup_ms:
        exe.run(q)
        q.sync()
    evs = [[Event(dev) for _ in range(len(ops) + 1)] for _ in range(reps)]
    exe.run(q)  # the lead step
    for r in range(reps):
        evs[r][0].record(q)
        exe.run(q, events=evs[r][1:])
    q.sync()
    tot = [0.0] * len(ops)
    whole = 0.0
    for ev in evs:
        for i in range(len(ops)):
            tot[i] += ev[i].elapsed_ms(ev[i + 1])
        whole += ev[0].elapsed_ms(ev[-1])
    for ev in evs:
        for e in ev:
            e.destroy()
    return [t / reps for t in tot], whole / reps


def in_step_report(exe, op_ms, peak, unit_scale=1e12):
    """Per-op in-step rows and the dominant GEMM op (the one with the most in-step time):
    (label, ms, flops, op kind)."""
    rows, dom = [], None
    for op, ms in zip(exe.graph.ops, op_ms):
        fl = exe.op_flops(op)
        row = {"op": exe.op_label(op), "ms": round(ms, 5)}
        if fl:
            rate = fl / (ms * 1e-3) / unit_scale
            row.update(rate=round(rate, 1), frac=round(rate / peak, 4))
            if dom is None or ms > dom[1]:
                dom = (row["op"], ms, fl, op.kind)
        rows.append(row)
    return rows, dom


NOT_CHECKED = "not checked (--no-cpu: the oracle runs only in the CPU-baseline leg)"


def time_cpu(fn, reps=5):
    """Median wall time of `reps` runs of fn() after one untimed run."""
    fn()  # warm-up
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(oracle, run, work, unit, sample, run_1=None, work_1=None, sample_1=None, reps=5):
    """The oracle module (the CPU restatement of the path: kind "port", imported by the caller's
    CPU-baseline leg) timed on the host's cores.  run() does
    `work` units of the workload (a bounded sample, described by `sample`), timed as the median of
    `reps` runs with every OpenMP thread, then run_1() (a smaller sample, default the same) with one
    thread.  value = work / seconds in `unit`."""
    threads = oracle.num_threads()
    t = time_cpu(run, reps)
    run_1, work_1, sample_1 = run_1 or run, work_1 or work, sample_1 or sample
    oracle.set_num_threads(1)
    try:
        t1 = time_cpu(run_1, reps)
    finally:
        oracle.set_num_threads(threads)
    return {"value": work / t, "unit": unit, "cores": threads, "kind": "port", "sample": sample,
            "seconds_median": t, "single_core_value": work_1 / t1, "single_core_sample": sample_1,
            "single_core_seconds_median": t1, "median_of": reps, "model": cpu_model()}


# ---- config 2 (headline) -------------------------------------------------------------------------
def bench_map_chain(dev, q, steps, warmup, do_cpu):
    from vernondsl_amd import kernels, mapchain as mc, spec
    from vernondsl_amd.rhi import Tensor
    rows = cols = 8192
    x, bias = spec.map_chain_inputs(rows, cols)
    prog = mc.compile(spec.map_chain_expr())
    tx, tb = Tensor.from_numpy(dev, q, x), Tensor.from_numpy(dev, q, bias)
    ty = Tensor(dev, (rows, cols), "f32")
    q.sync()
    # 10 launches per graph replay so inter-replay gaps do not count against the kernel
    per = 10
    ms, wall_ms = time_replays(q, dev, lambda: kernels.map_chain(q, prog, [tx, tb], ty), max(1, steps // per),
                               max(1, warmup // per), per_graph=per)
    nbytes = spec.map_chain_bytes(rows, cols)
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"ms": ms, "wall_ms": wall_ms, "gbs": gbs, "bytes": nbytes, "parity": NOT_CHECKED}
    if do_cpu:
        # CPU-baseline leg: the oracle is timed on the full workload and, as the checker, its output
        # on three rows is compared with the benchmarked GPU output.
        from oracle import oracle
        got = ty.numpy(q)
        res["parity"] = "ok"
        for r in (0, 4097, rows - 1):
            ref = oracle.map_chain(prog, [x, bias], rows, cols, row_range=(r, r + 1))[0]
            u = ((np.float32(spec.MAP_A) * x[r]) + np.float32(spec.MAP_B)).astype(np.float64)
            sc = np.abs(np.tanh(u) * np.exp(-(x[r].astype(np.float64) ** 2))) + np.abs(bias.astype(np.float64))
            if not np.all(np.abs(got[r].astype(np.float64) - ref) <= 1e-5 * sc):
                res["parity"] = f"FAIL row {r}"
        r1 = 1024
        res["cpu"] = cpu_baseline(oracle, lambda: oracle.map_chain(prog, [x, bias], rows, cols), nbytes / 1e9, "GB/s",
                                  f"the full workload ([{rows}][{cols}] f32), oracle orc_map_chain",
                                  lambda: oracle.map_chain(prog, [x, bias], rows, cols, row_range=(0, r1)),
                                  nbytes * r1 / rows / 1e9, f"first {r1} of {rows} rows")
    for t_ in (tx, tb, ty):
        t_.free()
    return res


def bench_map_chain_generic(dev, q, steps, warmup, do_cpu):
    """The map chain as an op class: config 2's chain in the generic interpreter (the headline runs
    it compiled at run time), and a second chain of another shape, sigmoid(x) * colvec[row] + x^2
    with a per-row operand, in both forms.  All on [8192][8192] f32, HBM GB/s from algorithmic
    bytes."""
    from vernondsl_amd import _lib, kernels, mapchain as mc, spec
    from vernondsl_amd.rhi import Tensor
    rows = cols = 8192
    x, bias = spec.map_chain_inputs(rows, cols)
    colv = np.ascontiguousarray(bias[:rows])
    tx, tb, tc = Tensor.from_numpy(dev, q, x), Tensor.from_numpy(dev, q, bias), Tensor.from_numpy(dev, q, colv)
    ty = Tensor(dev, (rows, cols), "f32")
    q.sync()
    out = []
    p1 = mc.compile(spec.map_chain_expr())
    p2 = mc.compile(mc.sigmoid(mc.Input(0)) * mc.Input(1, "col") + mc.Input(0) * mc.Input(0))
    b1, b2 = spec.map_chain_bytes(rows, cols), 8 * rows * cols + 4 * rows
    c2 = "sigmoid(x) * colvec[row] + x^2"
    cases = (("config-2 chain, generic interpreter", p1, [tx, tb], 1, b1),
             (c2 + ", generic interpreter", p2, [tx, tc], 1, b2),
             (c2 + ", compiled at run time", p2, [tx, tc], 0, b2))
    for name, prog, ins, mode, nbytes in cases:
        _lib.call("vdsl_debug_map_chain_mode", mode)
        per = 10
        try:
            ms, _ = time_replays(q, dev, lambda: kernels.map_chain(q, prog, ins, ty), max(1, steps // per),
                                 max(1, warmup // per), per_graph=per)
        finally:
            _lib.call("vdsl_debug_map_chain_mode", 0)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res = {"config": "2-generic", "workload": f"map chain {name}, [{rows}][{cols}] f32", "metric": "achieved HBM GB/s",
               "value": gbs, "unit": "GB/s", "ms_per_launch": ms, "parity": NOT_CHECKED,
               "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": gbs / PEAK_HBM_GBS, "bytes_per_launch": nbytes}}
        if do_cpu:
            from oracle import oracle
            hx = [x, bias] if prog is p1 else [x, colv]
            got = ty.numpy(q)
            r = 4097
            ref = oracle.map_chain(prog, hx, rows, cols, row_range=(r, r + 1))[0].astype(np.float64)
            ok = np.all(np.abs(got[r].astype(np.float64) - ref) <= 1e-5 * (np.abs(ref) + 1.0))
            res["parity"] = "ok (row 4097 against the oracle)" if ok else "FAIL"
            sample, s1 = 2048, 256
            res["cpu_baseline"] = cpu_baseline(
                oracle, lambda: oracle.map_chain(prog, hx, rows, cols, row_range=(0, sample)), nbytes * sample / rows / 1e9, "GB/s",
                f"first {sample} of {rows} rows, oracle orc_map_chain",
                lambda: oracle.map_chain(prog, hx, rows, cols, row_range=(0, s1)), nbytes * s1 / rows / 1e9,
                f"first {s1} of {rows} rows", reps=3)
        out.append(res)
    for t_ in (tx, tb, tc, ty):
        t_.free()
    return out


# ---- the vector vocabulary: MVP vertex transform and a swizzle (color.mlir, README.md:23-55) -------
def bench_vecmat(dev, q, steps, warmup, do_cpu):
    from vernondsl_amd import kernels, mapchain as mc
    from vernondsl_amd.rhi import Tensor
    out = []
    r = np.random.default_rng(0x5EED0008)
    # the vertex shader of color.mlir:10-39 over 2^24 vertices: vec3 in, 3 mat4 uniforms, vec4 out + varying
    n = 1 << 24
    pos = r.standard_normal((n, 3)).astype(np.float32)
    mats = r.standard_normal((3, 4, 4)).astype(np.float32)
    tp, tm = Tensor.from_numpy(dev, q, pos), Tensor.from_numpy(dev, q, mats)
    to, tv = Tensor(dev, (n, 4), "f32"), Tensor(dev, (n, 3), "f32")
    per = 10
    ms, _ = time_replays(q, dev, lambda: kernels.vec_transform(q, tp, tm, to, tv), max(1, steps // per),
                         max(1, warmup // per), per_graph=per)
    nbytes = n * (12 + 16 + 12)
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"config": "vec_transform", "workload": f"MVP vertex transform (color.mlir vertex_main) of {n} vec3 vertices, "
           "3 mat4 uniforms, vec4 gl_Position + vec3 varying out", "metric": "achieved HBM GB/s", "value": gbs,
           "unit": "GB/s", "ms_per_launch": ms, "parity": NOT_CHECKED,
           "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                        "bytes_per_launch": nbytes, "traffic": measured_traffic("vec_transform")}}
    if do_cpu:
        from oracle import oracle
        idx = np.array([0, 1, n // 2, n - 1])
        got = to.numpy(q)
        res["parity"] = "ok" if np.array_equal(got[idx], oracle.vec_transform(pos[idx], mats)) else "FAIL"
        s, s1 = 1 << 22, 1 << 19
        res["cpu_baseline"] = cpu_baseline(
            oracle, lambda: oracle.vec_transform(pos[:s], mats), s * 40 / 1e9, "GB/s",
            f"first {s} of {n} vertices, oracle orc_vec_transform", lambda: oracle.vec_transform(pos[:s1], mats),
            s1 * 40 / 1e9, f"first {s1} of {n} vertices", reps=3)
    out.append(res)
    for t_ in (tp, tm, to, tv):
        t_.free()
    # a swizzle: vec4 [4096][4096] -> .bgra
    rows = cols = 4096
    x = r.standard_normal((rows, cols, 4)).astype(np.float32)
    prog = mc.compile(mc.VecInput(0, 4).bgra)
    tx, ty = Tensor.from_numpy(dev, q, x), Tensor(dev, (rows, cols, 4), "f32")
    ms, _ = time_replays(q, dev, lambda: kernels.map_chain_v(q, prog, [tx], ty), max(1, steps // per),
                         max(1, warmup // per), per_graph=per)
    nbytes = 2 * rows * cols * 16
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"config": "swizzle", "workload": f"swizzle .bgra of vec4 [{rows}][{cols}] (vdsl_op_map_chain_v)",
           "metric": "achieved HBM GB/s", "value": gbs, "unit": "GB/s", "ms_per_launch": ms,
           "parity": "ok" if np.array_equal(ty.numpy(q)[::511], x[::511][..., [2, 1, 0, 3]]) else "FAIL",
           "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                        "bytes_per_launch": nbytes, "traffic": measured_traffic("swizzle")}}
    if do_cpu:
        from oracle import oracle
        s, s1 = 1024, 128
        res["cpu_baseline"] = cpu_baseline(
            oracle, lambda: oracle.map_chain_v(prog, [x], rows, cols, row_range=(0, s)), nbytes * s / rows / 1e9, "GB/s",
            f"first {s} of {rows} rows, oracle orc_map_chain_v_rows",
            lambda: oracle.map_chain_v(prog, [x], rows, cols, row_range=(0, s1)), nbytes * s1 / rows / 1e9,
            f"first {s1} of {rows} rows", reps=3)
    out.append(res)
    tx.free()
    ty.free()
    # a matrix operand per element: mat4 [4096][4096] times vec4 -> vec4 (linalg.matvec per element,
    # the mat4 records staged through LDS by the compiled kernel)
    v = r.standard_normal((rows, cols, 4)).astype(np.float32)
    m = r.standard_normal((rows, cols, 4, 4)).astype(np.float32)
    prog = mc.compile(mc.MatInput(1, 4, "full") @ mc.VecInput(0, 4))
    tv, tm, ty = Tensor.from_numpy(dev, q, v), Tensor.from_numpy(dev, q, m), Tensor(dev, (rows, cols, 4), "f32")
    ms, _ = time_replays(q, dev, lambda: kernels.map_chain_v(q, prog, [tv, tm], ty), max(1, steps // per),
                         max(1, warmup // per), per_graph=per)
    nbytes = rows * cols * (64 + 16 + 16)
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"config": "matvec", "workload": f"mat4 @ vec4 per element, [{rows}][{cols}] (vdsl_op_map_chain_v MATVEC)",
           "metric": "achieved HBM GB/s", "value": gbs, "unit": "GB/s", "ms_per_launch": ms, "parity": NOT_CHECKED,
           "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                        "bytes_per_launch": nbytes, "traffic": measured_traffic("matvec"), "kernel": "vdsl_map_jit32"}}
    if do_cpu:
        from oracle import oracle
        got = ty.numpy(q)
        rs = (0, 2049, rows - 1)
        ok = all(np.array_equal(got[i], oracle.map_chain_v(prog, [v, m], rows, cols, row_range=(i, i + 1))[0]) for i in rs)
        res["parity"] = "ok (3 rows bit-exact)" if ok else "FAIL"
        s, s1 = 512, 64
        res["cpu_baseline"] = cpu_baseline(
            oracle, lambda: oracle.map_chain_v(prog, [v, m], rows, cols, row_range=(0, s)), nbytes * s / rows / 1e9, "GB/s",
            f"first {s} of {rows} rows, oracle orc_map_chain_v_rows",
            lambda: oracle.map_chain_v(prog, [v, m], rows, cols, row_range=(0, s1)), nbytes * s1 / rows / 1e9,
            f"first {s1} of {rows} rows", reps=3)
    out.append(res)
    for t_ in (tv, tm, ty):
        t_.free()
    return out


# ---- config 1 ------------------------------------------------------------------------------------
def bench_fractal(dev, q, steps, warmup, do_cpu):
    from vernondsl_amd import kernels, spec
    from vernondsl_amd.rhi import Tensor
    params = spec.mandelbrot_params()
    p = kernels.escape_time_params(**params)
    out = Tensor(dev, (p.ni, p.nj), "i32")
    ms, wall_ms = time_replays(q, dev, lambda: kernels.escape_time(q, p, out), max(10, steps // 5), warmup, per_graph=20)
    got = out.numpy(q)
    total = int(got.sum(dtype=np.int64))
    parity = NOT_CHECKED
    if do_cpu:  # CPU-baseline leg (timed below); its output is the checker
        from oracle import oracle
        ref = oracle.escape_time(params)
        parity = "ok" if np.array_equal(got, ref) else f"FAIL {int((got != ref).sum())} px"
    gpix = total / (ms * 1e-3) / 1e9
    tflops = 8 * total / (ms * 1e-3) / 1e12
    res = {"config": 1, "workload": "Mandelbrot 1024x1024, max_iter 256, |z|^2>4, int32 counts (fma rounding form)",
           "metric": "Gpix-iter/s (fractal)", "value": gpix, "unit": "Gpix-iter/s", "ms_per_launch": ms,
           "pixel_iterations": total, "parity": parity,
           "roofline": {"bound": "valu", "achieved": tflops, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                        "frac": tflops / PEAK_FP32_TFLOPS, "flop_per_pixel_iteration": 8,
                        "valu_issue": measured_valu_issue(),
                        "note": "pixel-iterations counted as the program makes them (sum of counts); lanes whose "
                                "orbit becomes exactly periodic stop early, so about 17% fewer trips execute"}}
    if do_cpu:
        res["cpu_baseline"] = cpu_baseline(oracle, lambda: oracle.escape_time(params), total / 1e9, "Gpix-iter/s",
                                           "the full 1024x1024 grid")
    out.free()
    return res


def bench_pixel_program(dev, q, steps, warmup, do_cpu):
    """Struct-for bodies by the general path (vdsl_op_pixel_program: the lowered Taichi kernel,
    compiled at run time): Mandelbrot beside the hand-tuned escape-time kernel in the same
    rounding form (the cost of generality), and the Burning Ship, which only the general path
    runs (its update folds |x|, |y| and is not a complex polynomial)."""
    from vernondsl_amd import _lib, kernels, spec, taichi_compat as tc
    from vernondsl_amd.rhi import Tensor
    ex = os.path.join(ROOT, "vernondsl_amd", "examples")
    mandel = tc.lower_source_kernel(open(os.path.join(ex, "mandelbrot_counts.py")).read(), "render", {"limit": 256},
                                    general=True)
    ship = tc.lower_source_kernel(open(os.path.join(ex, "burning_ship.py")).read(), "ship", {"zoom": 3.2})
    esc = kernels.escape_time_params(**spec.mandelbrot_params(rounding=_lib.ESC_ROUND_SEPARATE))
    out = Tensor(dev, (1024, 1024), "i32")
    res = []
    esc_ms, _ = time_replays(q, dev, lambda: kernels.escape_time(q, esc, out), max(10, steps // 5), warmup, per_graph=20)
    for name, low, flop, desc in (
            ("mandelbrot", mandel, 8, "Mandelbrot 1024x1024, max_iter 256, separately rounded (examples/"
                                      "mandelbrot_counts.py by the general path)"),
            ("burning_ship", ship, 8, "Burning Ship 1024x1024, max_iter 256 (examples/burning_ship.py)")):
        prog = low.program
        ms, _ = time_replays(q, dev, lambda: kernels.pixel_program(q, prog, [], out), max(10, steps // 5), warmup,
                             per_graph=20)
        got = out.numpy(q)
        total = int(got.sum(dtype=np.int64))
        parity = NOT_CHECKED
        if do_cpu:  # CPU-baseline leg (timed below); its output is the checker
            from oracle import oracle
            ref = oracle.pixel_program(prog, 1024, 1024)
            parity = "ok" if np.array_equal(got, ref) else f"FAIL {int((got != ref).sum())} px"
        tflops = flop * total / (ms * 1e-3) / 1e12
        r = {"config": "1-general", "workload": desc + ", vdsl_op_pixel_program", "metric": "Gpix-iter/s (fractal)",
             "value": total / (ms * 1e-3) / 1e9, "unit": "Gpix-iter/s", "ms_per_launch": ms,
             "pixel_iterations": total, "parity": parity,
             "roofline": {"bound": "valu", "achieved": tflops, "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                          "frac": tflops / PEAK_FP32_TFLOPS, "flop_per_pixel_iteration": flop,
                          "note": "pixel-iterations counted as the program makes them (sum of counts); these "
                                  "programs store only the count, so lanes whose loop state recurs exactly stop "
                                  "early, as in the escape-time kernel; Burning Ship's two |.| per trip are not "
                                  "counted as flops"}}
        if name == "mandelbrot":
            r["escape_time_kernel_ms"] = esc_ms  # the same counts from the hand-tuned op
        if do_cpu:
            r["cpu_baseline"] = cpu_baseline(oracle, lambda: oracle.pixel_program(prog, 1024, 1024), total / 1e9,
                                             "Gpix-iter/s", "the full 1024x1024 grid")
        res.append(r)
    out.free()
    res.append(bench_pixel_stencil(dev, q, steps, warmup, do_cpu))
    return res


HEAT_N = 8192


def heat_program(n=HEAT_N):
    """examples/heat.py's diffuse kernel (a clamped five-point stencil, k = 0.2) lowered for an n x n
    plate: the example's W, H set to n."""
    from vernondsl_amd import taichi_compat as tc
    text = open(os.path.join(ROOT, "vernondsl_amd", "examples", "heat.py")).read()
    text = text.replace("W, H = 384, 256", f"W, H = {n}, {n}")
    return tc.lower_source_kernel(text, "diffuse", {"k": 0.2}).program


def bench_pixel_stencil(dev, q, steps, warmup, do_cpu):
    """A memory-bound struct-for body by the general path: examples/heat.py's diffusion step on an
    8192 x 8192 f32 plate (one field read through five clamped gathers, one written: 8 B per pixel
    reach HBM when the neighbours' rows are reused on chip)."""
    from vernondsl_amd import kernels, rng, spec
    from vernondsl_amd.rhi import Tensor
    n = HEAT_N
    prog = heat_program(n)
    u = rng.uniform(spec.SEEDS[2] + 7, n * n).reshape(n, n)
    tu, tv = Tensor.from_numpy(dev, q, u), Tensor(dev, (n, n), "f32")
    ms, _ = time_replays(q, dev, lambda: kernels.pixel_program(q, prog, [tu], tv), max(10, steps // 5), warmup,
                         per_graph=10)
    nbytes = 8 * n * n
    gbs = nbytes / (ms * 1e-3) / 1e9
    parity = NOT_CHECKED
    if do_cpu:  # CPU-baseline leg (timed below); its output is the checker, on the border and middle rows
        from oracle import oracle
        got = tv.numpy(q)
        bad = 0
        for r0 in (0, n // 2 - 1, n - 3):
            ref = oracle.pixel_program(prog, n, n, [u], rows=(r0, r0 + 3))
            bad += int((got[r0:r0 + 3].view(np.uint32) != ref.view(np.uint32)).sum())
        parity = "ok (rows 0-2, 4095-4097, 8189-8191 bit-exact)" if bad == 0 else f"FAIL {bad} px"
    r = {"config": "1-general-hbm", "workload": f"heat diffusion step {n}x{n} f32 (examples/heat.py's diffuse "
                                                "kernel, W = H = 8192), vdsl_op_pixel_program",
         "metric": "achieved HBM GB/s", "value": gbs, "unit": "GB/s", "ms_per_launch": ms, "parity": parity,
         "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                      "bytes_per_launch": nbytes, "traffic": measured_traffic("pixel_stencil")}}
    if do_cpu:
        n1 = 1024
        r["cpu_baseline"] = cpu_baseline(
            oracle, lambda: oracle.pixel_program(prog, n, n, [u]), nbytes / 1e9, "GB/s", f"the full {n}x{n} plate",
            lambda: oracle.pixel_program(prog, n, n, [u], rows=(0, n1)), 8 * n1 * n / 1e9, f"first {n1} of {n} rows")
    tu.free()
    tv.free()
    return r


# ---- config 3 ------------------------------------------------------------------------------------
def bench_softmax(dev, q, steps, warmup, do_cpu):
    from vernondsl_amd import kernels, rng, spec
    from vernondsl_amd.rhi import Tensor
    rows, cols = 16384, 4096
    x, orows, ocols = spec.softmax_inputs(rows, cols)
    out = []
    for name, dt in (("f32", "f32"), ("bf16", "bf16")):
        xh = x if dt == "f32" else rng.f32_to_bf16(x)
        tx = Tensor.from_numpy(dev, q, xh, dt)
        ts, tm, tsm = Tensor(dev, (rows,), "f32"), Tensor(dev, (rows,), "f32"), Tensor(dev, (rows, cols), dt)
        ms, _ = time_replays(q, dev, lambda: kernels.row_reduce_softmax(q, tx, ts, tm, tsm), max(1, steps // 10),
                             max(1, warmup // 10), per_graph=10)
        nbytes = spec.softmax_bytes(rows, cols, tx.dtype)
        gbs = nbytes / (ms * 1e-3) / 1e9
        gm = tm.numpy(q)
        xf = x if dt == "f32" else rng.bf16_to_f32(xh)
        ok = np.array_equal(gm, xf.max(axis=1))  # row max is exact
        if do_cpu:  # CPU-baseline leg (timed below): the oracle's softmax row as the checker
            from oracle import oracle
            r = 4097
            rs, rm, rsm = oracle.row_reduce_softmax(xh, row_range=(r, r + 1))
            got = tsm.numpy(q)[r]
            a = got.astype(np.float64) if dt == "f32" else rng.bf16_to_f32(got).astype(np.float64)
            b = rsm[0].astype(np.float64) if dt == "f32" else rng.bf16_to_f32(rsm[0]).astype(np.float64)
            ok = ok and np.all(np.abs(a - b) <= (1e-5 if dt == "f32" else 1e-2) * np.abs(b) + 1e-38)
        res = {"config": 3, "workload": f"row sum/max/softmax [{rows}][{cols}] {dt}", "metric": "achieved HBM GB/s",
               "value": gbs, "unit": "GB/s", "ms_per_launch": ms,
               "parity": ("ok" if ok else "FAIL") if do_cpu else ("row max exact; softmax " + NOT_CHECKED if ok else "FAIL"),
               "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": gbs / PEAK_HBM_GBS, "bytes_per_launch": nbytes,
                            "traffic": measured_traffic("softmax_" + dt)}}
        if do_cpu:
            n_rows, n1 = 4096, 512
            res["cpu_baseline"] = cpu_baseline(
                oracle, lambda: oracle.row_reduce_softmax(xh, row_range=(0, n_rows)), spec.softmax_bytes(n_rows, cols, tx.dtype) / 1e9,
                "GB/s", f"first {n_rows} of {rows} rows (rows are independent)",
                lambda: oracle.row_reduce_softmax(xh, row_range=(0, n1)), spec.softmax_bytes(n1, cols, tx.dtype) / 1e9,
                f"first {n1} of {rows} rows")
        out.append(res)
        for t_ in (tx, ts, tm, tsm):
            t_.free()
    return out


# ---- config 4 ------------------------------------------------------------------------------------
def bench_mlp(dev, q, steps, warmup, do_cpu):
    from vernondsl_amd import graph, spec
    B, D, Hd, O = 2048, 4096, 4096, 4096
    x, w1, w2, t = spec.mlp_inputs(B, D, Hd, O)
    g, _ = graph.mlp_train_graph(B, D, Hd, O)
    exe = g.compile(dev)
    for name, arr in (("X", x), ("W1", w1), ("W2", w2), ("T", t)):
        exe.write(q, name, arr)
    step = exe.capture(q)
    n = max(5, steps // 5)
    # graph replays, after the same >= 25 ms warm-up as every other timing
    ms = time_launches(q, dev, lambda: step.launch(q), n, warmup=max(1, warmup // 5))
    # the same step issued op by op on the stream (no graph), for comparison
    eager_ms = time_launches(q, dev, lambda: exe.run(q), n, warmup=2)
    # every op's in-step duration: events between the ops of eagerly issued steps
    op_ms, ev_step_ms = time_ops_in_step(q, dev, exe, n)
    rows, (dom_op, dom_ms, dom_flop, dom_kind) = in_step_report(exe, op_ms, PEAK_BF16_TFLOPS)
    flops = spec.mlp_flops(B, D, Hd, O)
    tflops = flops / (ms * 1e-3) / 1e12
    gemm_ms = sum(r["ms"] for r in rows if "rate" in r)
    loss = float(exe.read(q, "loss")[0])
    b = 64  # the rows the CPU leg runs; their forward outputs are checked against its oracle run
    y_rows, h_rows = exe.read(q, "Y")[:b], exe.read(q, "H")[:b]
    step.destroy()
    exe.free()
    gt = dom_flop / (dom_ms * 1e-3) / 1e12
    res = {"config": 4, "workload": "2-layer MLP 4096-4096-4096, GELU, MSE, batch 2048, bf16 MFMA, fwd+bwd as one hipGraph",
           "metric": "MFMA TFLOPS (GEMM)", "value": tflops, "unit": "TFLOP/s", "ms_per_step": ms,
           "eager_ms_per_step": eager_ms, "flop_per_step": flops, "loss": loss,
           "in_step": {"ops": rows, "gemm_ms": gemm_ms, "gemm_frac": flops / (gemm_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                       "evented_step_ms": ev_step_ms,
                       "method": "HIP events after every op of eagerly issued steps on the real buffers"},
           "roofline": {"bound": "mfma", "achieved": gt, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": gt / PEAK_BF16_TFLOPS, "kernel": f"dominant in-step op: {dom_op}",
                        "kernel_ms": dom_ms, "traffic": measured_traffic("c4:" + dom_kind)},
           "whole_graph_frac_of_peak": tflops / PEAK_BF16_TFLOPS, "parity": NOT_CHECKED}
    if do_cpu:  # CPU-baseline leg; its oracle run on the first rows is also the checker
        from oracle import oracle
        from vernondsl_amd import rng as vrng
        b1 = 8
        ref = oracle.mlp_train_step(x[:b], w1, w2, t[:b])

        def frob(got, want):
            got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
            return float(np.linalg.norm(got - want) / np.linalg.norm(want))
        ey, eh = frob(y_rows, ref["Y"]), frob(vrng.bf16_to_f32(h_rows), vrng.bf16_to_f32(ref["H"]))
        res["parity"] = (f"ok (Y, H of {b} rows: Frobenius-relative {ey:.1e}, {eh:.1e} <= 1e-2)" if max(ey, eh) <= 1e-2
                         else f"FAIL (Y {ey:.2e}, H {eh:.2e})")
        res["cpu_baseline"] = cpu_baseline(
            oracle, lambda: oracle.mlp_train_step(x[:b], w1, w2, t[:b]), spec.mlp_flops(b, D, Hd, O) / 1e12, "TFLOP/s",
            f"the same step at batch {b} of {B} (every GEMM keeps its 4096x4096 weight shape), f64-accumulating oracle",
            lambda: oracle.mlp_train_step(x[:b1], w1, w2, t[:b1]), spec.mlp_flops(b1, D, Hd, O) / 1e12,
            f"the same step at batch {b1} of {B}", reps=3)
    return res


# ---- config 5 ------------------------------------------------------------------------------------
def bench_w8a8(dev, q, steps, warmup, do_cpu):
    from vernondsl_amd import graph, spec
    B, widths = 512, spec.W8A8_WIDTHS
    x, layers = spec.w8a8_inputs(B, widths)
    g = graph.w8a8_infer_graph(B, widths)
    exe = g.compile(dev)
    exe.write(q, "X", x)
    for li, (w, sc) in enumerate(layers):
        exe.write(q, f"W{li}", w)
        exe.write(q, f"S{li}", sc)
    step = exe.capture(q)
    n = max(5, steps // 2)
    ms = time_launches(q, dev, lambda: step.launch(q), n, warmup=max(1, warmup // 5))
    eager_ms = time_launches(q, dev, lambda: exe.run(q), n, warmup=2)
    op_ms, ev_step_ms = time_ops_in_step(q, dev, exe, n)
    rows, _ = in_step_report(exe, op_ms, PEAK_INT8_TOPS)
    ops = spec.w8a8_ops(B, widths)
    tops = ops / (ms * 1e-3) / 1e12
    got = exe.read(q, "Y")
    parity = NOT_CHECKED
    if do_cpu:  # CPU-baseline leg (timed below): the oracle's forward of two rows as the checker
        from oracle import oracle
        rows_chk = np.array([0, 511])
        parity = "ok" if np.array_equal(got[rows_chk], oracle.w8a8_forward(x[rows_chk], layers)) else "FAIL"
    step.destroy()
    exe.free()
    # dominant kernel: the three 512x8192x8192 layer GEMMs, each timed inside the step (their
    # weights stream from HBM there: 192 MB rotate through the 256 MB last-level cache)
    big = [r for r in rows if r["op"].startswith("w8a8_packed") and r["op"].endswith("512x8192x8192")]
    kms = sum(r["ms"] for r in big) / len(big)
    gt = 2 * B * 8192 * 8192 / (kms * 1e-3) / 1e12
    gemm_ms = sum(r["ms"] for r in rows if "rate" in r)
    res = {"config": 5, "workload": "int8 W8A8 MLP 8192-8192-8192-8192-1024, batch 512, dequant+ReLU fused, one hipGraph",
           "metric": "MFMA TOPS (int8 GEMM)", "value": tops, "unit": "TOP/s", "ms_per_step": ms,
           "eager_ms_per_step": eager_ms, "ops_per_step": ops,
           "parity": parity,
           "in_step": {"ops": rows, "gemm_ms": gemm_ms, "gemm_frac": ops / (gemm_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS,
                       "evented_step_ms": ev_step_ms,
                       "method": "HIP events after every op of eagerly issued steps on the real buffers"},
           "roofline": {"bound": "mfma", "achieved": gt, "peak": PEAK_INT8_TOPS, "unit": "TOP/s",
                        "frac": gt / PEAK_INT8_TOPS,
                        "kernel": "gemm_w8a8_bpk 512x8192x8192 (dequant+ReLU), mean of the three layers as timed inside the step",
                        "kernel_ms": kms, "traffic": measured_traffic("c5:w8a8_packed")},
           "whole_graph_frac_of_peak": tops / PEAK_INT8_TOPS}
    if do_cpu:
        r, r1 = 16, 2
        res["cpu_baseline"] = cpu_baseline(
            oracle, lambda: oracle.w8a8_forward(x[:r], layers), spec.w8a8_ops(r, widths) / 1e12, "TOP/s",
            f"{r} of {B} rows through all 4 layers (rows are independent)",
            lambda: oracle.w8a8_forward(x[:r1], layers), spec.w8a8_ops(r1, widths) / 1e12,
            f"{r1} of {B} rows through all 4 layers", reps=3)
    return res


# ---- HBM traffic from counter passes ----------------------------------------------------------------
# traffic key -> (--kernel run it is measured in, substring of the profiled kernel's name, grid size
# in work-items or None, algorithmic bytes per launch).  The c4:/c5: keys are the GEMMs of the
# config-4 and config-5 steps as they run inside the step (one eager step per rep), keyed by the
# graph op kind whose in-step time bench.py reports.
_MB = 1 << 20
_C4_BPK = "gemm_bf16_bpk<vdsl::BpkConfig<vdsl::MfmaBf16, 4, 2, 4, 3>, "


def _traffic_kernels():
    from vernondsl_amd import _lib, spec
    return {
        "copy": ("copy", "copyBuffer", None, 2 * (512 << 20)),
        "map_chain": ("map_chain", "vdsl_map_jit", None, spec.map_chain_bytes(8192, 8192)),  # compiled at run time
        "softmax_f32": ("softmax_f32", "row_softmax_split<0", None, spec.softmax_bytes(16384, 4096, _lib.F32)),
        "softmax_bf16": ("softmax_bf16", "row_softmax_split<1", None, spec.softmax_bytes(16384, 4096, _lib.BF16)),
        # vec3 positions read, vec4 positions and vec3 varyings written (2^24 vertices)
        "vec_transform": ("vec_transform", "mat_transform_kernel", None, (1 << 24) * 40),
        # vec4 [4096][4096] read and written
        "swizzle": ("swizzle", "vdsl_map_jit", None, 2 * 4096 * 4096 * 16),  # the chain compiled at run time
        # mat4 and vec4 [4096][4096] read, vec4 written
        "matvec": ("matvec", "vdsl_map_jit", None, 4096 * 4096 * 96),
        # heat.py's stencil on 8192^2 f32: the field read once, the result written once
        "pixel_stencil": ("pixel_stencil", "vdsl_pix_jit", None, 8 * HEAT_N * HEAT_N),
        # config 4 (2048 x 4096 x 4096 and 4096 x 4096 x 2048 bf16): operands read once, outputs written once
        # X, W1 read; H (bf16) and GELU'(pre) (f32) written
        "c4:linear": ("c4_step", _C4_BPK + "0, true>", None, (16 + 32 + 16 + 32) * _MB),
        # H, W2, T read; Y (f32) and dL/dY (bf16) written (the weight gradient reads dL/dY as stored)
        "c4:linear_mse": ("c4_step", "gemm_bf16_bpk_mse", None, (16 + 32 + 32 + 32 + 16) * _MB),
        # dL/dY (or dL/dpre) and H (or X) read, both K-major; the f32 weight gradient written
        "c4:gemm": ("c4_step", "gemm_bf16_dma<vdsl::DmaConfig<vdsl::MfmaBf16, 256, 256, 2, 4, 3, 64>, false, true, true>",
                    None, (16 + 16 + 64) * _MB),
        # dL/dY, W2^T, GELU'(pre) read; dL/dpre written
        "c4:gemm_mul_bwd": ("c4_step", _C4_BPK + "2, false>", None, (16 + 32 + 32 + 16) * _MB),
        # config 5 layer 512 x 8192 x 8192 (256 blocks): int8 A, B and both scale vectors read; bf16 Y written
        "c5:w8a8_packed": ("c5_step", "gemm_w8a8_bpk<vdsl::BpkConfig<vdsl::MfmaI8, 4, 1, 4, 3>", 256 * 256,
                           512 * 8192 + 8192 * 8192 + 4 * (512 + 8192) + 2 * 512 * 8192),
    }


def traffic_summary(run_dir):
    """Builds profiles/traffic.json from the rocprofv3 counter runs in run_dir (one directory per
    kernel and counter, traffic_<kernel>_<FETCH_SIZE|WRITE_SIZE>/run_counter_collection.csv, as the
    commands in profiles/traffic_counters.md write them) and prints the summary table.  Each
    counter is scaled so that it reads the known traffic of the 512 MiB copy."""
    import csv
    def per_dispatch(run, counter, name_part, grid):
        path = os.path.join(run_dir, f"traffic_{run}_{counter}", "run_counter_collection.csv")
        vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(path))
                if name_part in r["Kernel_Name"] and r["Counter_Name"] == counter
                and (grid is None or int(r["Grid_Size"]) == grid)]
        if not vals:
            raise SystemExit(f"{path}: no dispatch of a kernel named *{name_part}*")
        return sum(vals) / len(vals)
    ks = _traffic_kernels()
    cf = per_dispatch("copy", "FETCH_SIZE", ks["copy"][1], None)
    cw = per_dispatch("copy", "WRITE_SIZE", ks["copy"][1], None)
    half = (512 << 20) / 1024  # KiB read and KiB written by the copy
    ff, wf = half / cf, half / cw
    out = {"fetch_factor": round(ff, 4), "write_factor": round(wf, 4), "kernels": {}}
    rows = []
    for k, (run, part, grid, alg) in ks.items():
        if k == "copy":
            continue
        f, w = per_dispatch(run, "FETCH_SIZE", part, grid), per_dispatch(run, "WRITE_SIZE", part, grid)
        t = (f * ff + w * wf) * 1024
        out["kernels"][k] = {"traffic_bytes": int(round(t)), "algorithmic_bytes": alg, "fetch_kib": f, "write_kib": w}
        rows.append(f"| {k} | {f:.0f} | {w:.0f} | {int(round(t)):,} | {alg:,} | {t / alg:.3f} |")
    with open(os.path.join(ROOT, "profiles", "traffic.json"), "w") as fh:
        json.dump(out, fh, indent=1)
    print(f"copy: FETCH_SIZE {cf:.0f} KiB, WRITE_SIZE {cw:.0f} KiB per dispatch -> factors {ff:.4f}, {wf:.4f}")
    print("| Kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | Traffic (scaled) B | Algorithmic B | Traffic / algorithmic |")
    print("|---|---|---|---|---|---|")
    print("\n".join(rows))


# ---- single-kernel mode (for rocprofv3 counter passes) ---------------------------------------------
def run_kernel_only(dev, q, name, reps):
    """Runs one kernel `reps` times on the config's shape and nothing else (no parity, no CPU):
    the program a `rocprofv3 --pmc` pass profiles.  `copy` is a 512 MiB device-to-device copy
    (known traffic: 512 MiB read + 512 MiB written) used to calibrate FETCH_SIZE / WRITE_SIZE."""
    from vernondsl_amd import _lib, kernels, mapchain as mc, spec
    from vernondsl_amd.rhi import Tensor
    ts = []
    if name == "map_chain":
        x, bias = spec.map_chain_inputs(8192, 8192)
        tx, tb, ty = Tensor.from_numpy(dev, q, x), Tensor.from_numpy(dev, q, bias), Tensor(dev, (8192, 8192), "f32")
        prog = mc.compile(spec.map_chain_expr())
        fn, ts = (lambda: kernels.map_chain(q, prog, [tx, tb], ty)), [tx, tb, ty]
    elif name in ("softmax_f32", "softmax_bf16"):
        dt = name.split("_")[1]
        tx = Tensor(dev, (16384, 4096), dt)
        tx.buffer.fill_u32(q, 0x3F803F80)
        outs = [Tensor(dev, (16384,), "f32"), Tensor(dev, (16384,), "f32"), Tensor(dev, (16384, 4096), dt)]
        fn, ts = (lambda: kernels.row_reduce_softmax(q, tx, *outs)), [tx] + outs
    elif name == "gemm_bf16":
        x, w1, _, _ = spec.mlp_inputs()
        A, B0 = Tensor.from_numpy(dev, q, x, "bf16"), Tensor.from_numpy(dev, q, w1, "bf16")
        B = Tensor(dev, (4096, 4096), "bf16")
        kernels.pack_bf16_weights(q, B0, B)
        H, P = Tensor(dev, (2048, 4096), "bf16"), Tensor(dev, (2048, 4096), "f32")
        fn, ts = (lambda: kernels.gemm_bf16_packed(q, A, B, H, _lib.EPI_GELU, P)), [A, B0, B, H, P]
    elif name == "gemm_w8a8":
        _, layers = spec.w8a8_inputs()
        A = Tensor.from_numpy(dev, q, np.ascontiguousarray(layers[1][0][:512]))
        B0 = Tensor.from_numpy(dev, q, layers[0][0])
        B = Tensor(dev, (8192, 8192), "i8")
        kernels.pack_w8a8_weights(q, B0, B)
        xs, ws, Y = Tensor(dev, (512,), "f32"), Tensor.from_numpy(dev, q, layers[0][1]), Tensor(dev, (512, 8192), "bf16")
        xs.buffer.fill_u32(q, 0x3F800000)
        wsb = kernels.gemm_w8a8_packed_workspace_bytes(512, 8192, 8192)
        W = Tensor(dev, (wsb,), "i8") if wsb else None
        if W is not None:
            W.buffer.fill_u32(q, 0)
        fn, ts = (lambda: kernels.gemm_w8a8_packed(q, A, xs, B, ws, Y, True, None, W)), [A, B0, B, xs, ws, Y] + ([W] if W else [])
    elif name == "c4_step":  # one eager config-4 training step per rep (every kernel of the step)
        from vernondsl_amd import graph
        x, w1, w2, t = spec.mlp_inputs()
        g, _ = graph.mlp_train_graph()
        exe = g.compile(dev)
        for nm, arr in (("X", x), ("W1", w1), ("W2", w2), ("T", t)):
            exe.write(q, nm, arr)
        fn, ts = (lambda: exe.run(q)), [exe]
    elif name == "c5_step":  # one eager config-5 forward per rep
        from vernondsl_amd import graph
        x, layers = spec.w8a8_inputs()
        g = graph.w8a8_infer_graph()
        exe = g.compile(dev)
        exe.write(q, "X", x)
        for li, (w, sc) in enumerate(layers):
            exe.write(q, f"W{li}", w)
            exe.write(q, f"S{li}", sc)
        fn, ts = (lambda: exe.run(q)), [exe]
    elif name == "vec_transform":
        n = 1 << 24
        tp, tm = Tensor(dev, (n, 3), "f32"), Tensor(dev, (3, 4, 4), "f32")
        tp.buffer.fill_u32(q, 0x3F800000)
        tm.buffer.fill_u32(q, 0x3F000000)
        to, tv = Tensor(dev, (n, 4), "f32"), Tensor(dev, (n, 3), "f32")
        fn, ts = (lambda: kernels.vec_transform(q, tp, tm, to, tv)), [tp, tm, to, tv]
    elif name == "swizzle":
        tx, ty = Tensor(dev, (4096, 4096, 4), "f32"), Tensor(dev, (4096, 4096, 4), "f32")
        tx.buffer.fill_u32(q, 0x3F800000)
        prog = mc.compile(mc.VecInput(0, 4).bgra)
        fn, ts = (lambda: kernels.map_chain_v(q, prog, [tx], ty)), [tx, ty]
    elif name == "matvec":
        tv, tm = Tensor(dev, (4096, 4096, 4), "f32"), Tensor(dev, (4096, 4096, 4, 4), "f32")
        tv.buffer.fill_u32(q, 0x3F800000)
        tm.buffer.fill_u32(q, 0x3F000000)
        ty = Tensor(dev, (4096, 4096, 4), "f32")
        prog = mc.compile(mc.MatInput(1, 4, "full") @ mc.VecInput(0, 4))
        fn, ts = (lambda: kernels.map_chain_v(q, prog, [tv, tm], ty)), [tv, tm, ty]
    elif name == "pixel_stencil":
        prog = heat_program()
        tu, tv = Tensor(dev, (HEAT_N, HEAT_N), "f32"), Tensor(dev, (HEAT_N, HEAT_N), "f32")
        tu.buffer.fill_u32(q, 0x3F000000)
        fn, ts = (lambda: kernels.pixel_program(q, prog, [tu], tv)), [tu, tv]
    elif name == "escape_time":
        p = kernels.escape_time_params(**spec.mandelbrot_params())
        out = Tensor(dev, (1024, 1024), "i32")
        fn, ts = (lambda: kernels.escape_time(q, p, out)), [out]
    elif name == "copy":
        n = 512 << 20
        a, b = Tensor(dev, (n,), "i8"), Tensor(dev, (n,), "i8")
        fn, ts = (lambda: _lib.call("vdsl_buffer_copy", q.handle, b.handle, 0, a.handle, 0, n)), [a, b]
    else:
        raise SystemExit(f"unknown kernel {name!r}")
    for _ in range(reps):
        fn()
    q.sync()
    for t_ in ts:
        t_.free()
    print(json.dumps({"kernel": name, "reps": reps}), flush=True)


def _round(x, sig=4):
    if isinstance(x, float):
        return float(f"{x:.{sig}g}")
    if isinstance(x, dict):
        return {k: _round(v, sig) for k, v in x.items()}
    if isinstance(x, list):
        return [_round(v, sig) for v in x]
    return x


# Fields the one-line summary leaves out (the full records go to stderr as each config finishes):
# the single-core and median details of a CPU baseline and explanatory notes.
_CPU_KEEP = ("value", "unit", "cores", "kind", "sample", "single_core_value")


def _compact(entry):
    """A per-config record as it appears in the printed line: values to 4 significant digits, the
    CPU baseline reduced to its value, unit, cores, kind, sample and single-core value, notes
    dropped, in-step op lists reduced to (op, ms, frac)."""
    e = {k: v for k, v in entry.items() if k not in ("note", "metric")}
    if isinstance(e.get("cpu_baseline"), dict):
        e["cpu_baseline"] = {k: v for k, v in e["cpu_baseline"].items() if k in _CPU_KEEP}
    if isinstance(e.get("roofline"), dict):
        rf = {k: v for k, v in e["roofline"].items() if k != "note"}
        if isinstance(rf.get("valu_issue"), dict):
            rf["valu_issue"] = rf["valu_issue"].get("valu_issue_frac")
        e["roofline"] = rf
    if isinstance(e.get("in_step"), dict) and isinstance(e["in_step"].get("ops"), list):
        e["in_step"] = dict(e["in_step"], ops=[{k: o[k] for k in ("op", "ms", "frac") if k in o} for o in e["in_step"]["ops"]])
    return _round(e)


def _summary_row(entry):
    """[config, value, unit, roofline frac, ms] of one per-config record, with the kernel or
    example named where several records share a config id."""
    cid = entry.get("config")
    wl = str(entry.get("workload", ""))
    tag = {"Burning": "ship", "heat": "heat", "bf16": "bf16", "generic interpreter": "interp",
           "compiled at run time": "jit", "sigmoid": "sigmoid"}
    names = [v for k, v in tag.items() if k in wl]
    label = str(cid) + ("/" + "/".join(names) if names else "")
    rf = entry.get("roofline") or {}
    ms = entry.get("ms_per_launch", entry.get("ms_per_step"))
    frac = rf.get("frac")
    return [label, _round(entry.get("value")), entry.get("unit"), round(frac, 4) if isinstance(frac, float) else frac,
            _round(ms)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # 100 untimed steps (~9 ms of GPU work for config 2): the clocks ramp up during the first
    # milliseconds after host-side setup, and a shorter warm-up reads the kernel up to 5% low
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline timings")
    ap.add_argument("--only", type=int, default=0, help="run only the headline and one extra config "
                    "(1, 3, 4, 5; 2: the generic map chains; 6: the vector ops; 7: the general per-pixel programs)")
    ap.add_argument("--skip", default="", metavar="IDS",
                    help="comma-separated config ids (as for --only) to leave out of the run")
    ap.add_argument("--kernel", default="", help="run one kernel --reps times and exit (for rocprofv3 --pmc): "
                    "map_chain, softmax_f32, softmax_bf16, gemm_bf16, gemm_w8a8, escape_time, pixel_stencil, vec_transform, "
                    "swizzle, matvec, copy, c4_step, c5_step")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--traffic-summary", default="", metavar="DIR",
                    help="write profiles/traffic.json from the counter runs in DIR and exit (no GPU needed)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.traffic_summary:
        traffic_summary(args.traffic_summary)
        return
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each config would shard rows or "
              "batch across GPUs with no exchange except config 4's gradient all-reduce; not built). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    from vernondsl_amd.rhi import Device, Queue
    dev = Device(0)
    q = Queue(dev)
    if args.kernel:
        run_kernel_only(dev, q, args.kernel, args.reps)
        q.destroy()
        dev.close()
        return
    info = dev.info()
    log("bench: device", info)
    do_cpu = not args.no_cpu

    head = bench_map_chain(dev, q, args.steps, args.warmup, do_cpu)
    log("bench: config 2", {k: v for k, v in head.items() if k != "cpu"})
    per_config = []
    skip = {int(c) for c in args.skip.split(",") if c.strip()}
    for fn, cid in ((bench_map_chain_generic, 2), (bench_fractal, 1), (bench_pixel_program, 7), (bench_softmax, 3),
                    (bench_mlp, 4),
                    (bench_w8a8, 5), (bench_vecmat, 6)):
        if (args.only and args.only != cid) or cid in skip:
            continue
        r = fn(dev, q, args.steps, args.warmup, do_cpu)
        log(f"bench: config {cid}", r)
        per_config.extend(r if isinstance(r, list) else [r])

    line = {
        "metric": "achieved HBM GB/s (fused map)",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (splitmix64 seeded, x ~ N(0,1), bias ~ U(-1,1))",
        "config": {"workload": "config 2: fused map chain y = tanh(0.75*x - 0.25) * exp(-x^2) + bias[col]",
                   "rows": 8192, "cols": 8192, "dtype": "f32", "bytes_per_step": head["bytes"]},
        "parity": head["parity"],
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / PEAK_HBM_GBS, 4), "traffic": measured_traffic("map_chain"),
                     "kernel": "vdsl_map_jit32 (the chain compiled at run time)"},
        "cpu_baseline": head.get("cpu"),
        "device": {"name": info["name"], "arch": info["arch"], "compute_units": info["compute_units"]},
        "per_config": [_compact(e) for e in per_config],
        # last, so that a reader keeping only the line's final ~2000 characters still sees every
        # config's figure: [config, value, unit, roofline fraction, ms per launch or step]
        "summary": [_summary_row(e) for e in per_config],
    }
    q.destroy()
    dev.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
