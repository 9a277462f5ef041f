"""Scatter-adds (VDSL_PIX_ATOMIC_ADD, Taichi's atomic `field[index] += v`) on the GPU against the
CPU oracle.  int32 targets are exact in any order, so they are compared bit for bit, on every path
of the device: one atomic per lane, one per wave where the indices are wave-uniform (the row
mapping) or constants (any mapping, after an escape loop too), grids that are not whole blocks
(lanes past the grid add nothing), indices outside the target (dropped).  f32 targets are summed
in no fixed order on the device: bit for bit where every partial sum is exact (small dyadic
values), else within the bound any summation order meets, 2 (n - 1) u sum|x| per element (n the
terms added into it, u = 2^-24).  Then the examples: the histogram (escape counts binned, a 0-D
total) bit for bit, the particle splat's kernels (grid mass within the bound, the kernels after
it bit for bit on the device's grid), and the host-side field operations they use."""
import contextlib
import ctypes
import io
import json
import os

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, pixprog as pp, run, taichi_compat as tc
from vernondsl_amd.rhi import Tensor
from test_taichi_general import lower_named, run_ops
from test_taichi_scatter import escape_counts, mpm88_p2g_terms

pytestmark = pytest.mark.gpu
EX = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vernondsl_amd", "examples")
f32 = np.float32
U = 2.0 ** -24


def run_scatter(dev, q, prog, inputs, ni, nj, out_shape=None):
    """Runs prog on the device; returns (its output or None, every input read back)."""
    ts = [Tensor.from_numpy(dev, q, np.ascontiguousarray(a, np.int32 if prog.in_dtypes[k] == pp.I32 else f32))
          for k, a in enumerate(inputs)]
    out = None
    if prog.out_kind != pp.OUT_NONE:
        int_out = prog.out_kind in (pp.OUT_COUNT, pp.OUT_I32)
        out = Tensor(dev, out_shape or (ni, nj), "i32" if int_out else "f32")
    kernels.pixel_program(q, prog, ts, out, grid=(ni, nj))
    got = out.numpy(q) if out is not None else None
    back = [t.numpy(q) for t in ts]
    for t in ts + ([out] if out is not None else []):
        t.free()
    return got, back


def bound_ok(got, want, n_terms, abs_sum):
    """|got - want| <= 2 (n - 1) u sum|x| element by element (float64 arithmetic)."""
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    return bool(np.all(err <= 2.0 * np.maximum(n_terms - 1, 0) * U * abs_sum))


def hist_program(bins, scale, dtype=pp.I32, value=1.0):
    """target[0][floor(x * scale)] += value for input 0's pixel (a data-dependent index: one
    atomic per lane)."""
    b = pp.Builder()
    x = b.load(0)
    e = b.scatter_add(1, 0.0, b.op("floor", b.op("mul", x, scale)), b.op("mul", x, value) if value != 1.0 else value)
    return pp.compile_program(b, out=None, effects=[e], in_dtypes=[pp.F32, dtype], in_extents=[None, (1, bins)])


@pytest.mark.parametrize("ni, nj, bins", [(37, 53, 16), (1, 1000, 16), (300, 1, 16), (256, 256, 16), (1, 1, 16),
                                          (256, 256, 8192), (256, 256, 8193), (97, 301, 5000), (97, 301, 20000)])
def test_histogram_bins_per_lane_bit_exact(dev, q, ni, nj, bins):
    """Up to 8192 bins each block adds into its own copy in LDS and then adds the copy's non-zero
    bins; above, every lane adds into memory."""
    rng = np.random.default_rng(ni * 1000 + nj + bins)
    x = rng.random((ni, nj)).astype(f32)
    prog = hist_program(bins, float(bins))
    h0 = rng.integers(-5, 5, (1, bins)).astype(np.int32)
    _, (_, got) = run_scatter(dev, q, prog, [x, h0], ni, nj)
    want = h0.copy()
    oracle.pixel_program(prog, ni, nj, [x, want])
    assert np.array_equal(got, want)
    assert int(got.sum() - h0.sum()) == ni * nj  # every pixel in the grid added once, no other lane


def test_row_uniform_and_constant_indices_add_once_per_wave(dev, q):
    """target[i % 5][0] += i + j (row-uniform in the row mapping) and total[0][0] += 1 (constant):
    int32, bit for bit; the ragged grid leaves lanes past it in the last waves."""
    ni, nj = 70, 333
    b = pp.Builder()
    i, j = b.index(0), b.index(1)
    row = b.op("sub", i, b.op("mul", b.op("floor", b.op("mul", i, 0.2)), 5.0))  # i % 5, exact for small i
    effects = [b.scatter_add(0, row, 0.0, b.op("add", i, j)), b.scatter_add(1, 0.0, 0.0, 1.0)]
    prog = pp.compile_program(b, out=None, effects=effects, in_dtypes=[pp.I32, pp.I32], in_extents=[(5, 1), (1, 1)])
    t0, t1 = np.zeros((5, 1), np.int32), np.zeros((1, 1), np.int32)
    _, (g0, g1) = run_scatter(dev, q, prog, [t0, t1], ni, nj)
    oracle.pixel_program(prog, ni, nj, [t0, t1])
    assert np.array_equal(g0, t0) and np.array_equal(g1, t1) and int(g1[0, 0]) == ni * nj


def test_constant_index_after_an_escape_loop(dev, q):
    """An escape-loop program (16x16 patches, no row mapping) that stores its count, bins it per
    lane and adds it to a constant-index total (one add per wave)."""
    ni, nj, MAX = 130, 97, 64
    b = pp.Builder()
    x0 = b.op("add", b.op("mul", b.index(0), 3.0 / 130), -2.0)
    y0 = b.op("add", b.op("mul", b.index(1), 2.4 / 97), -1.2)
    x, y = b.state("x"), b.state("y")
    r2 = b.op("add", b.op("mul", x, x), b.op("mul", y, y))
    effects = [b.scatter_add(0, 0.0, b.count(), 1.0), b.scatter_add(1, 0.0, 0.0, b.count())]
    prog = pp.compile_program(b, init={"x": 0.0, "y": 0.0}, test=("le", r2, 4.0),
                              body={"x": b.op("add", b.op("sub", b.op("mul", x, x), b.op("mul", y, y)), x0),
                                    "y": b.op("add", b.op("mul", b.op("mul", x, y), 2.0), y0)},
                              max_iter=MAX, out=pp.COUNT, effects=effects, in_dtypes=[pp.I32, pp.I32],
                              in_extents=[(1, MAX + 1), (1, 1)])
    h, t = np.zeros((1, MAX + 1), np.int32), np.zeros((1, 1), np.int32)
    counts, (gh, gt) = run_scatter(dev, q, prog, [h, t], ni, nj)
    want = oracle.pixel_program(prog, ni, nj, [h, t])
    assert np.array_equal(counts, want)
    assert np.array_equal(gh, h) and np.array_equal(gt, t)
    assert np.array_equal(gh[0], np.bincount(counts.ravel(), minlength=MAX + 1)) and int(gt[0, 0]) == int(counts.sum())


def test_indices_outside_the_target_are_dropped(dev, q):
    specials = np.array([-1.0, -0.5, -0.0, 0.0, 0.75, 2.0, 2.999, 3.0, 4.0, np.nan, np.inf, -np.inf, 1e30, 2.0**31],
                        f32)
    rows, cols = np.meshgrid(specials, specials, indexing="ij")
    b = pp.Builder()
    e = [b.scatter_add(1, b.load(0, 0), b.load(0, 1), 1.0), b.scatter_add(2, b.load(0, 0), b.load(0, 1), 2.0e9)]
    prog = pp.compile_program(b, out=None, effects=e, in_widths=[2, 1, 1], in_dtypes=[pp.F32, pp.I32, pp.I32],
                              in_extents=[None, (3, 3), (3, 3)])
    xy = np.stack([rows, cols], -1).astype(f32)
    c, w = np.zeros((3, 3), np.int32), np.zeros((3, 3), np.int32)
    n = specials.size
    _, (_, gc, gw) = run_scatter(dev, q, prog, [xy, c, w], n, n)
    oracle.pixel_program(prog, n, n, [xy, c, w])
    assert np.array_equal(gc, c) and np.array_equal(gw, w) and int(c.sum()) == 25  # 5 x 5 in-range pairs (-0.0 is one)


@pytest.mark.parametrize("uniform, bins", [(False, 8), (True, 1), (False, 9000)])
def test_f32_dyadic_sums_bit_exact(dev, q, uniform, bins):
    """Values k / 64 with |k| < 256 into 8 bins (per lane, into LDS copies), one element (summed
    per thread and block) or 9000 bins (per lane, into memory): every partial sum of at most 2^13
    of them is exact in f32, so any order gives the oracle's bits."""
    ni, nj = 48, 160
    rng = np.random.default_rng(31 + uniform + bins)
    v = (rng.integers(-255, 256, (ni, nj)) / 64.0).astype(f32)
    b = pp.Builder()
    if uniform:
        col = 0.0
    elif bins == 8:
        col = b.op("floor", b.op("mul", b.index(1), 0.05))  # j // 20: 8 bins
    else:
        col = b.op("floor", b.op("mul", b.load(0), 4.0))  # floor(4 v) in -16 .. 15, + 64: columns 48 .. 79
        col = b.op("add", col, 64.0)
    e = b.scatter_add(1, 0.0, col, b.load(0))
    prog = pp.compile_program(b, out=None, effects=[e], in_dtypes=[pp.F32, pp.F32], in_extents=[None, (1, bins)])
    t = np.zeros((1, bins), f32)
    _, (_, got) = run_scatter(dev, q, prog, [v, t], ni, nj)
    oracle.pixel_program(prog, ni, nj, [v, t])
    assert np.array_equal(got, t)


@pytest.mark.parametrize("uniform", [False, True])
def test_f32_sums_within_the_any_order_bound(dev, q, uniform):
    ni, nj = 200, 300
    rng = np.random.default_rng(41 + uniform)
    v = rng.standard_normal((ni, nj)).astype(f32)
    b = pp.Builder()
    col = 0.0 if uniform else b.op("floor", b.op("mul", b.index(1), 0.1))  # j // 10: 30 bins
    e = b.scatter_add(1, 0.0, col, b.load(0))
    nb = 1 if uniform else 30
    prog = pp.compile_program(b, out=None, effects=[e], in_dtypes=[pp.F32, pp.F32], in_extents=[None, (1, nb)])
    t0 = rng.standard_normal((1, nb)).astype(f32)
    _, (_, got) = run_scatter(dev, q, prog, [v, t0], ni, nj)
    want = t0.copy()
    oracle.pixel_program(prog, ni, nj, [v, want])
    jb = np.floor(np.arange(nj).astype(f32) * f32(0.1)).astype(np.int64)  # the program's floor(j * 0.1) in f32
    bins = np.zeros(v.shape, np.int64) if uniform else np.broadcast_to(jb, (ni, nj))
    n_terms = np.bincount(bins.ravel(), minlength=nb).astype(np.float64) + 1
    abs_sum = np.abs(t0[0]).astype(np.float64) + np.bincount(bins.ravel(), np.abs(v).ravel().astype(np.float64), nb)
    assert bound_ok(got[0], want[0], n_terms, abs_sum)
    assert not np.array_equal(got, t0)


def test_scatter_programs_refused(dev, q):
    b = pp.Builder()
    ok = pp.compile_program(b, out=b.load(0), effects=[b.scatter_add(1, 0.0, 0.0, 1.0)], in_extents=[None, (1, 1)])

    def call(p, ins, out):
        hs = (ctypes.c_void_p * len(ins))(*[t.handle for t in ins])
        with pytest.raises(_lib.VdslError) as ei:
            _lib.call("vdsl_op_pixel_program", q.handle, 8, 8, ctypes.byref(p), hs, len(ins), None if out is None else out.handle)
        return ei.value.message

    def mutate(p, pc=None, **kw):
        m = pp.PixelProgram()
        ctypes.memmove(ctypes.byref(m), ctypes.byref(p), ctypes.sizeof(m))
        for k, v in kw.items():
            if pc is None:
                setattr(m, k, v)
            else:
                setattr(m.code[pc], k, v)
        return m

    field, one = Tensor(dev, (8, 8), "f32"), Tensor(dev, (1, 1), "f32")
    out = Tensor(dev, (8, 8), "f32")
    ro = Tensor(dev, (1, 1), "f32", _lib.BIND_UNIFORM_CONSTANT)
    try:
        total = ok.n_post
        at = next(k for k in range(total) if ok.code[k].op == pp.OP["atomic_add"])
        assert "also reads" in call(mutate(ok, at, a=0), [field, one], out)  # into the input it loads
        assert "not there" in call(mutate(ok, at, imm=1.0), [field, one], out)  # component 1 of a scalar field
        assert "not there" in call(mutate(ok, at, a=2), [field, one], out)  # no input 2
        assert "also the output" in call(
            pp.compile_program(b, out=b.load(0), effects=[b.scatter_add(1, 0.0, 0.0, 1.0)]), [field, out], out)
        assert "read-only" in call(ok, [field, ro], out)  # a uniform_constant buffer takes no adds
        loop = pp.compile_program(b, init={"s": 0.0}, body={"s": b.op("add", b.state("s"), 1.0)}, max_iter=2, out=b.state("s"))
        loop_body = mutate(loop, loop.n_pre, op=pp.OP["atomic_add"], a=0, b=0, c=0, dst=0, imm=0.0)
        assert "loop's sections" in call(loop_body, [one], out)
        # a program that stores nothing takes no output buffer
        none = pp.compile_program(b, out=None, effects=[b.scatter_add(0, 0.0, 0.0, 2.0)], in_extents=[(1, 1)])
        hs = (ctypes.c_void_p * 1)(one.handle)
        one.buffer.fill_u32(q, 0)
        _lib.call("vdsl_op_pixel_program", q.handle, 8, 8, ctypes.byref(none), hs, 1, None)
        assert float(one.numpy(q)[0, 0]) == 128.0
    finally:
        for t in (field, one, out, ro):
            t.free()


# ---- examples -------------------------------------------------------------------------------------
def run_program(path, frames):
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        assert run.main([path, "--frames", str(frames)]) == 0
    return json.loads(buf.getvalue().strip().splitlines()[-1]), tc._state["last_gui"].last_image


def test_histogram_example_bit_exact(dev, q):
    """One frame: counts by the escape loop, their histogram by scatter-adds, the image shaded by
    the histogram's cumulative share (a gather at the count): equal to the numpy restatement."""
    res, img = run_program(os.path.join(EX, "histogram.py"), 1)
    assert res["frames"] == 1 and img.shape == (640, 480)
    counts = escape_counts(640, 480, 200, -0.745, 0.11, 0.004)
    h = np.bincount(counts.ravel(), minlength=201)
    cdf = (h.cumsum() / max(h.sum(), 1)).astype(f32)
    assert np.array_equal(img, cdf[counts])


def grid_array(a, shape):
    """A field's array as its program grid ([1][N], [R][C], [1][1]) plus components."""
    return np.ascontiguousarray(a.reshape(tc._grid_of(shape) + a.shape[len(shape):]))


def test_splat_kernels_on_the_device(dev, q):
    """p2g on the device against the oracle within the any-order bound (mass and momentum), the
    particles' weights summing to their count; grid_update and g2p on the device's grid bit for
    bit against the oracle run on that same grid."""
    text = open(os.path.join(EX, "splat.py")).read()
    N, G = 8192, 128
    rng = np.random.default_rng(77)
    x = (rng.random((N, 2)) * 0.9 + 0.05).astype(f32)
    v = rng.standard_normal((N, 2)).astype(f32)
    p2g, names = lower_named(text, "p2g", {})
    shapes = {"x": (N,), "v": (N,), "grid_m": (G, G), "grid_v": (G, G)}
    host = {"x": x, "v": v, "grid_m": np.zeros((G, G), f32), "grid_v": np.zeros((G, G, 2), f32)}
    ts = {k: Tensor.from_numpy(dev, q, grid_array(a, shapes[k])) for k, a in host.items()}
    try:
        op = p2g.ops()[0]
        kernels.pixel_program(q, op.program, [ts[names[id(f)]] for f in op.inputs], None, grid=op.grid)
        gm, gv = ts["grid_m"].numpy(q), ts["grid_v"].numpy(q)
        want = {k: grid_array(a.copy(), shapes[k]) for k, a in host.items()}
        oracle.pixel_program(op.program, op.grid[0], op.grid[1], [want[names[id(f)]] for f in op.inputs])
        # terms and |x| per node (each weight is at most 1), in f64
        base = np.trunc((x * f32(G)) - f32(0.5)).astype(np.int64)
        n_terms = np.ones((G, G))
        abs_m, abs_v = np.zeros((G, G)), np.zeros((G, G, 2))
        for i in range(3):
            for j in range(3):
                idx = (base[:, 0] + i, base[:, 1] + j)
                np.add.at(n_terms, idx, 1)
                np.add.at(abs_m, idx, 1.0)
                for c in range(2):
                    np.add.at(abs_v[:, :, c], idx, np.abs(v[:, c]).astype(np.float64))
        assert bound_ok(gm, want["grid_m"], n_terms, abs_m)
        for c in range(2):
            assert bound_ok(gv[:, :, c], want["grid_v"][:, :, c], n_terms, abs_v[:, :, c])
        assert abs(float(gm.sum(dtype=np.float64)) - N) < 1e-2
        # the kernels after it, on the device's grid, bit for bit
        upd, names_u = lower_named(text, "grid_update", {})
        op = upd.ops()[0]
        grid_in = {"grid_m": gm.copy(), "grid_v": gv.copy()}
        kernels.pixel_program(q, op.program, [ts[names_u[id(f)]] for f in op.inputs], ts[names_u[id(op.field)]], grid=op.grid)
        want_v = oracle.pixel_program(op.program, G, G, [grid_in[names_u[id(f)]] for f in op.inputs])
        gv2 = ts["grid_v"].numpy(q)
        assert np.array_equal(gv2, want_v)
        g2p, names_g = lower_named(text, "g2p", {})
        cur = {"x": grid_array(x, (N,)), "v": grid_array(v, (N,)), "grid_v": gv2}
        for op in g2p.ops():  # v first (it reads x before x's store), then x
            got_ins = [ts[names_g[id(f)]] for f in op.inputs]
            kernels.pixel_program(q, op.program, got_ins, ts[names_g[id(op.field)]], grid=op.grid)
            ref = oracle.pixel_program(op.program, op.grid[0], op.grid[1], [cur[names_g[id(f)]] for f in op.inputs])
            cur[names_g[id(op.field)]] = ref
            assert np.array_equal(ts[names_g[id(op.field)]].numpy(q), ref)
    finally:
        for t in ts.values():
            t.free()


def test_splat_example_runs(dev, q):
    res, pos = run_program(os.path.join(EX, "splat.py"), 2)
    assert res["frames"] == 2 and pos.shape == (8192, 2) and np.isfinite(pos).all()
    assert 0.2 < float(pos[:, 1].min()) and float(pos[:, 1].max()) < 0.75  # falling, not yet at the floor


def test_field_host_operations(dev, q):
    """fill, from_numpy, 0-D field[None] reads and writes, as the examples use them."""
    tc.init(arch=tc.gpu)
    s = tc.field(dtype=float, shape=())
    s[None] = 2.5
    assert float(s[None]) == 2.5 and s.to_numpy().shape == ()
    h = tc.field(dtype=int, shape=7)
    h.fill(3)
    assert np.array_equal(h.to_numpy(), np.full(7, 3, np.int32))
    vf = tc.Vector.field(2, dtype=float, shape=(3, 4))
    arr = np.arange(24, dtype=f32).reshape(3, 4, 2)
    vf.from_numpy(arr)
    assert np.array_equal(vf.to_numpy(), arr)
    vf.fill(-1.5)
    assert np.array_equal(vf.to_numpy(), np.full((3, 4, 2), -1.5, f32))
    with pytest.raises(ValueError):
        vf.from_numpy(np.zeros((4, 3, 2), f32))


def elem_shape(fld):
    return fld.mat or ((fld.width,) if fld.width > 1 else ())


def test_mpm88_substeps_on_the_device(dev, q):
    """Two substeps of the mpm88 example, each of its 12 programs run on the device beside the
    oracle from the same inputs: the particle-to-grid adds (f32, in no fixed order on the device)
    within the any-order bound per node (and the device's grid carried on), every other program
    (grid update, the grid-to-particle parts joined by hidden fields, the particle stores) bit for
    bit."""
    text = open(os.path.join(EX, "mpm88.py")).read()
    n, G = 8192, 128
    init, names_i = lower_named(text, "init", {})
    sub, names = lower_named(text, "substep", {})
    host = {"x": np.zeros((n, 2), f32), "v": np.zeros((n, 2), f32), "C": np.zeros((n, 2, 2), f32),
            "J": np.zeros(n, f32), "grid_v": np.zeros((G, G, 2), f32), "grid_m": np.zeros((G, G), f32)}
    run_ops(init, names_i, host)
    fields = {}
    for op in sub.ops():
        for f in op.inputs + ([op.field] if op.field is not None else []):
            fields.setdefault(id(f), f)
    ts = {}

    def tensor(f):
        nm = names[id(f)]
        if nm not in ts:
            a = host.get(nm)
            a = np.zeros(f.shape + elem_shape(f), f32) if a is None else a
            ts[nm] = Tensor.from_numpy(dev, q, np.ascontiguousarray(
                a.reshape(tc._grid_of(f.shape) + ((f.width,) if f.width > 1 else ())), f32))
        return ts[nm]

    def read(f):
        return ts[names[id(f)]].numpy(q).reshape(f.shape + elem_shape(f))

    try:
        for step in range(2):
            for k, op in enumerate(sub.ops()):
                before = {nm: host[nm].copy() for nm in ("x", "v", "C", "J")}
                run_ops(op, names, host)  # the oracle (names the hidden fields it makes)
                ins = [tensor(f) for f in op.inputs]
                out = tensor(op.field) if op.field is not None else None
                if out is not None and op.field not in op.inputs:
                    out.buffer.fill_u32(q, 0x7FC00000)  # NaN: every element must be written
                kernels.pixel_program(q, op.program, ins, out, grid=op.grid)
                if op.field is not None:
                    assert np.array_equal(read(op.field), host[names[id(op.field)]]), (step, k, names[id(op.field)])
                    continue
                # the particle-to-grid adds: within the bound, then the device's grid is the state
                idx, terms = mpm88_p2g_terms(before["x"], before["v"], before["C"], before["J"])
                n_terms = np.ones((G, G))
                np.add.at(n_terms, idx, 1)
                gv_d = read(fields[next(i for i, nm in names.items() if nm == "grid_v")])
                gm_d = read(fields[next(i for i, nm in names.items() if nm == "grid_m")])
                for got, want, t in ((gv_d[:, :, 0], host["grid_v"][:, :, 0], terms[0]),
                                     (gv_d[:, :, 1], host["grid_v"][:, :, 1], terms[1]), (gm_d, host["grid_m"], terms[2])):
                    abs_sum = np.zeros((G, G))
                    np.add.at(abs_sum, idx, np.abs(t).astype(np.float64))
                    assert bound_ok(got, want, n_terms, abs_sum), (step, k)
                host["grid_v"], host["grid_m"] = gv_d.copy(), gm_d.copy()
        assert abs(float(host["grid_m"].sum(dtype=np.float64)) - n * (1.0 / 256) ** 2) < 1e-6
    finally:
        for t in ts.values():
            t.free()


def test_mpm88_example_runs(dev, q):
    res, pos = run_program(os.path.join(EX, "mpm88.py"), 2)
    assert res["frames"] == 2 and pos.shape == (8192, 2) and np.isfinite(pos).all()
    assert 0.0 < float(pos.min()) and float(pos.max()) < 1.0
    assert float(pos[:, 1].mean()) < 0.4  # the block has fallen (it starts at 0.2 - 0.6)


@pytest.mark.parametrize("where", ["lane", "row", "const", "escape"])
def test_scatter_max_min_bit_exact(dev, q, where):
    """ti.atomic_max / atomic_min on every device path (one per lane into memory, row-uniform
    per wave, constant per block, constant after an escape loop in 16 x 16 patches), f32 with NaN,
    signed zeros and infinities among the values, and int32: equal to the oracle (fmaxf / fminf
    give one value in any order; a zero result may differ in sign only)."""
    ni, nj = 70, 333
    rng = np.random.default_rng(50 + len(where))
    v = rng.standard_normal((ni, nj)).astype(f32)
    v.ravel()[rng.choice(v.size, 300, replace=False)] = rng.choice(np.array([np.nan, 0.0, -0.0, np.inf, -np.inf], f32), 300)
    b = pp.Builder()
    x = b.load(0)
    if where == "lane":
        row, col, R, C = 0.0, b.op("floor", b.op("mul", b.op("abs", x), 3.0)), 1, 12
    elif where == "row":
        row, col, R, C = b.op("sub", b.index(0), b.op("mul", b.op("floor", b.op("mul", b.index(0), 0.125)), 8.0)), 0.0, 8, 1
    else:
        row, col, R, C = 0.0, 0.0, 1, 1
    eff = [b.scatter_add(1, row, col, x, op="max"), b.scatter_add(2, row, col, x, op="min"),
           b.scatter_add(3, row, col, b.op("mul", x, 100.0), op="max")]
    kw = dict(out=None)
    if where == "escape":  # a test loop first: the patch mapping
        s = b.state("s")
        kw = dict(init={"s": 0.0}, test=("lt", s, b.op("abs", x)), body={"s": b.op("add", s, 0.5)}, max_iter=9, out=pp.COUNT)
    prog = pp.compile_program(b, effects=eff, in_dtypes=[pp.F32, pp.F32, pp.F32, pp.I32],
                              in_extents=[None, (R, C), (R, C), (R, C)], **kw)
    t = [np.full((R, C), -7.0, f32), np.full((R, C), 7.0, f32), np.full((R, C), -5, np.int32)]
    got_out, back = run_scatter(dev, q, prog, [v] + [a.copy() for a in t], ni, nj)
    want_out = oracle.pixel_program(prog, ni, nj, [v] + t)
    if where == "escape":
        assert np.array_equal(got_out, want_out)
    assert np.array_equal(back[1], t[0], equal_nan=True) and np.array_equal(back[2], t[1], equal_nan=True)
    assert np.array_equal(back[3], t[2])
    assert np.isinf(t[0]).any() or where == "lane"  # the infinities reached the maxima


def test_stores_at_computed_indices_on_the_device(dev, q):
    """The interior stencil, boundary and transposed-store kernels of the front-end test, each
    program run on the device beside the oracle from the same fields: bit for bit (no two pixels
    store to one element)."""
    from test_taichi_scatter import STORES
    rng = np.random.default_rng(22)
    host = {"u": rng.random((40, 30)).astype(f32), "v": rng.random((40, 30)).astype(f32),
            "code": rng.integers(-9, 9, (40, 30)).astype(np.int32)}
    ts = {k: Tensor.from_numpy(dev, q, a) for k, a in host.items()}
    try:
        for kern in ("interior", "boundary", "transpose_into"):
            low, names = lower_named(STORES, kern, {})
            for op in low.ops():
                kernels.pixel_program(q, op.program, [ts[names[id(f)]] for f in op.inputs], None, grid=op.grid)
                run_ops(op, names, host)
            for k in ("v", "code"):
                assert np.array_equal(ts[k].numpy(q), host[k]), (kern, k)
    finally:
        for t in ts.values():
            t.free()


_RX = tc.field(dtype=float, shape=(64, 48))
_RV = tc.Vector.field(2, dtype=float, shape=1000)


@tc.kernel
def _energy() -> float:
    e = 0.0
    for i in _RV:
        e += 0.5 * _RV[i].norm_sqr()
    for i, j in _RX:
        e -= _RX[i, j]
    return e


@tc.kernel
def _count(t: float) -> int:
    n = 0
    for i, j in _RX:
        if _RX[i, j] > t:
            n += 1
    return n


def test_kernel_scope_reductions_return_values(dev, q):
    """A kernel returning a kernel-scope sum: the device's value within the any-order bound of
    the f32 sum, an int32 count exactly; called again (the graph-replayed form from the second
    call) the accumulators start from their initial values each time."""
    tc.init(arch=tc.gpu)
    rng = np.random.default_rng(23)
    X = rng.random((64, 48)).astype(f32)
    V = rng.standard_normal((1000, 2)).astype(f32)
    _RX.from_numpy(X)
    _RV.from_numpy(V)
    terms = np.concatenate([(f32(0.5) * (V[:, 0] * V[:, 0] + V[:, 1] * V[:, 1])).astype(np.float64), -X.ravel().astype(np.float64)])
    exact = float(terms.sum())
    for _ in range(4):
        e = _energy()
        assert isinstance(e, float) and abs(e - exact) <= 2 * terms.size * U * float(np.abs(terms).sum())
        n = _count(0.25)
        assert n == int((X > f32(0.25)).sum())
    assert _energy.lower().graph and _count.lower(0.25).graph


_RP = tc.Vector.field(2, dtype=float, shape=4096)


@tc.kernel
def _scatter_points():
    for i in _RP:
        _RP[i] = [ti_random_pair() * 2.0, tc.random()]


@tc.func
def ti_random_pair():
    return tc.random()


def test_random_numbers_on_the_device(dev, q):
    """ti.random on the device equals the oracle's numbers for the same generator state, bit for
    bit; every call (eager, then graph replays) advances the state, so the numbers change."""
    from test_taichi_scatter import RANDOM
    low, names = lower_named(RANDOM, "seed", {})
    prog = low.program
    state = np.array([[123]], np.int32)
    got, _ = run_scatter(dev, q, prog, [state], 1, 5000, out_shape=(1, 5000, 2))
    assert np.array_equal(got.reshape(5000, 2), oracle.pixel_program(prog, 1, 5000, [state]).reshape(5000, 2))
    tc.init(arch=tc.gpu)
    seen = []
    for _ in range(4):
        _scatter_points()
        a = _RP.to_numpy()
        assert 0.0 <= a[:, 1].min() and a[:, 1].max() < 1.0 and 0.0 <= a[:, 0].min() and a[:, 0].max() < 2.0
        assert all(not np.array_equal(a, b) for b in seen)
        seen.append(a)
    assert _scatter_points.lower().graph
