"""Scatter-adds (Taichi's `field[index] += v` at an index other than the loop's, an atomic add)
on the CPU: the oracle's VDSL_PIX_ATOMIC_ADD is pinned by numpy's `np.add.at` (unbuffered adds
in index order, the order the oracle runs pixels in) and by the drop rule written out per index;
the front end's lowering of scatter-adds (histograms, 0-D totals, vector indices base + offset,
adds in if branches, 3-D targets, bodies that also store) is pinned by numpy restatements run in
the same order, so bit for bit."""
import os
import re

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import pixprog as pp, taichi_compat as tc
from test_taichi_general import lower_named, run_ops

EX = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vernondsl_amd", "examples")
f32 = np.float32


def scatter_program(b, effects, dtypes, widths, extents, out=None):
    return pp.compile_program(b, out=out, effects=effects, in_dtypes=dtypes, in_widths=widths, in_extents=extents)


# ---- the oracle's scatter-add ---------------------------------------------------------------------
def test_oracle_scatter_add_equals_numpy_add_at():
    """f32 (a vector field's component 1) and int32 targets of their own extents, indices from an
    input field: the oracle adds in row-major pixel order, as np.add.at does over raveled
    indices, so the f32 sums agree bit for bit."""
    ni, nj, R, C = 23, 31, 5, 7
    rng = np.random.default_rng(5)
    rows = rng.integers(0, R, (ni, nj)).astype(f32)
    cols = rng.integers(0, C, (ni, nj)).astype(f32)
    val = rng.standard_normal((ni, nj)).astype(f32)
    b = pp.Builder()
    r, c, v = b.load(0, 0), b.load(0, 1), b.load(0, 2)  # one input of three components
    effects = [b.scatter_add(1, r, c, v, 1), b.scatter_add(2, r, c, b.op("mul", v, 100.0))]
    prog = scatter_program(b, effects, [pp.F32, pp.F32, pp.I32], [3, 2, 1], [None, (R, C), (R, C)])
    assert prog.out_kind == pp.OUT_NONE
    t_f = rng.standard_normal((R, C, 2)).astype(f32)
    t_i = rng.integers(-50, 50, (R, C)).astype(np.int32)
    want_f, want_i = t_f.copy(), t_i.astype(np.int64)
    assert oracle.pixel_program(prog, ni, nj, [np.stack([rows, cols, val], -1), t_f, t_i]) is None
    idx = (rows.astype(int).ravel(), cols.astype(int).ravel())
    np.add.at(want_f[:, :, 1], idx, val.ravel())
    np.add.at(want_i, idx, np.trunc(val * f32(100.0)).astype(np.int64).ravel())
    assert np.array_equal(t_f, want_f)  # component 0 untouched, component 1 summed in order
    assert np.array_equal(t_i, want_i.astype(np.int32))


def test_oracle_scatter_add_drops_indices_outside_the_target():
    """An add happens only where 0 <= row < R and 0 <= col < C (NaN, negative and too large
    indices are dropped, not clamped); fractional indices truncate; int32 adds wrap."""
    specials = np.array([-1.0, -0.5, 0.0, 0.75, 2.0, 2.999, 3.0, 4.0, np.nan, np.inf, -np.inf, 1e30], f32)
    n = specials.size
    rows, cols = np.meshgrid(specials, specials, indexing="ij")
    b = pp.Builder()
    effects = [b.scatter_add(2, b.load(0), b.load(1), 1.0), b.scatter_add(3, b.load(0), b.load(1), 2.0e9)]
    prog = scatter_program(b, effects, [pp.F32, pp.F32, pp.F32, pp.I32], [1] * 4, [None, None, (3, 3), (3, 3)])
    cnt = np.zeros((3, 3), f32)
    wrap = np.zeros((3, 3), np.int32)
    oracle.pixel_program(prog, n, n, [rows.astype(f32), cols.astype(f32), cnt, wrap])
    want = np.zeros((3, 3), np.int64)
    for x in specials:
        for y in specials:
            if 0 <= x < 3 and 0 <= y < 3:  # False for NaN
                want[int(x), int(y)] += 1
    assert np.array_equal(cnt, want.astype(f32))
    assert np.array_equal(wrap, ((want * 2_000_000_000 + 2**31) % 2**32 - 2**31).astype(np.int32))


def test_oracle_scatter_add_skips_nothing_it_should_run():
    """A program that stores and scatter-adds: the store is the plain program's, and the adds
    follow the loop (here the escape count of each pixel, binned)."""
    b = pp.Builder()
    x0 = b.op("mul", b.index(0), 0.25)
    x = b.state("x")
    count_bin = b.scatter_add(0, 0.0, b.count(), 1.0)
    prog = pp.compile_program(b, init={"x": x0}, test=("lt", x, 3.0), body={"x": b.op("add", b.op("mul", x, x), 0.5)},
                              max_iter=9, out=pp.COUNT, effects=[count_bin], in_dtypes=[pp.I32], in_extents=[(1, 10)])
    hist = np.zeros((1, 10), np.int32)
    counts = oracle.pixel_program(prog, 12, 3, [hist])
    assert np.array_equal(hist[0], np.bincount(counts.ravel(), minlength=10))


# ---- the front end ----------------------------------------------------------------------------------
def escape_counts(W, H, MAX, cx, cy, scale):
    """The histogram example's escape loop in numpy f32 (the same operations in the same order)."""
    i, j = np.meshgrid(np.arange(W), np.arange(H), indexing="ij")
    x0 = f32(cx) + (i.astype(f32) - f32(W / 2)) * f32(scale)
    y0 = f32(cy) + (j.astype(f32) - f32(H / 2)) * f32(scale)
    x = np.zeros((W, H), f32)
    y = np.zeros((W, H), f32)
    k = np.zeros((W, H), np.int32)
    live = np.ones((W, H), bool)
    for _ in range(MAX):
        live &= (x * x + y * y) <= f32(4.0)
        if not live.any():
            break
        nx, ny = x * x - y * y + x0, f32(2.0) * x * y + y0
        x, y = np.where(live, nx, x), np.where(live, ny, y)
        k += live
    return k


def test_histogram_example_lowers_to_one_program_with_its_adds():
    text = open(os.path.join(EX, "histogram.py")).read()
    args = {"cx": -0.745, "cy": 0.11, "scale": 0.004}
    low, names = lower_named(text, "escape", args)
    assert low.kind == "pixel_program" and names[id(low.field)] == "counts"
    assert low.program.out_kind == pp.OUT_COUNT and [names[id(f)] for f in low.inputs] == ["hist", "total"]
    arrays = {"counts": None, "hist": np.zeros(201, np.int32), "total": np.zeros((), np.int32)}
    run_ops(low, names, arrays)
    counts = arrays["counts"]
    assert np.array_equal(counts, escape_counts(640, 480, 200, *args.values()))
    assert np.array_equal(arrays["hist"], np.bincount(counts.ravel(), minlength=201))
    assert int(arrays["total"]) == int(counts.sum())
    shade, names2 = lower_named(text, "shade", {})
    k = [names2[id(f)] for f in shade.inputs].index("cdf")  # cdf[counts[i, j]]: a gather in cdf's own grid
    assert shade.program.in_rows[k] == 1 and shade.program.in_cols[k] == 201


def weights(fx):
    """The quadratic B-spline weights of the splat example, per axis (f32, its operation order)."""
    return [f32(0.5) * ((f32(1.5) - fx) * (f32(1.5) - fx)), f32(0.75) - (fx - f32(1.0)) * (fx - f32(1.0)),
            f32(0.5) * ((fx - f32(0.5)) * (fx - f32(0.5)))]


def splat_nodes(x, G):
    """Per particle and node (i, j) of ti.ndrange(3, 3): row, column and weight, [N][3][3]."""
    xs = x * f32(G)
    base = np.trunc(xs - f32(0.5))
    w = weights(xs - base)
    i, j = np.meshgrid(np.arange(3), np.arange(3), indexing="ij")
    rows = base[:, 0, None, None].astype(np.int64) + i
    cols = base[:, 1, None, None].astype(np.int64) + j
    wt = np.stack([np.stack([w[a][:, 0] * w[b][:, 1] for b in range(3)], -1) for a in range(3)], -2)
    return rows, cols, wt


def test_splat_p2g_equals_sequential_numpy_adds():
    """The splat example's particle-to-grid kernel (quadratic B-spline weights, base + offset
    vector indices, a scalar and a vector target) against its numpy restatement, adding in the
    oracle's order: particle by particle, the nine nodes in ti.ndrange order (np.add.at over the
    [N][3][3] arrays raveled in C order adds in that order)."""
    text = open(os.path.join(EX, "splat.py")).read()
    low, names = lower_named(text, "p2g", {})
    assert low.kind == "pixel_program" and low.field is None and low.program.out_kind == pp.OUT_NONE
    N, G = 8192, 128
    rng = np.random.default_rng(9)
    x = (rng.random((N, 2)) * 0.9 + 0.05).astype(f32)  # every node inside the grid
    v = rng.standard_normal((N, 2)).astype(f32)
    arrays = {"x": x, "v": v, "grid_m": np.zeros((G, G), f32), "grid_v": np.zeros((G, G, 2), f32)}
    run_ops(low, names, arrays)
    rows, cols, wt = splat_nodes(x, G)
    gm, gv = np.zeros((G, G), f32), np.zeros((G, G, 2), f32)
    idx = (rows.ravel(), cols.ravel())
    np.add.at(gm, idx, wt.ravel())
    for c in range(2):
        np.add.at(gv[:, :, c], idx, (wt * v[:, c, None, None]).ravel())
    assert np.array_equal(arrays["grid_m"], gm) and np.array_equal(arrays["grid_v"], gv)
    assert abs(float(gm.sum(dtype=np.float64)) - N) < 1e-2  # the weights of a particle sum to 1


def test_splat_g2p_gathers_at_vector_indices():
    text = open(os.path.join(EX, "splat.py")).read()
    low, names = lower_named(text, "g2p", {})
    assert [names[id(o.field)] for o in low.ops()] == ["v", "x"]
    N, G = 8192, 128
    rng = np.random.default_rng(10)
    x = (rng.random((N, 2)) * 0.9 + 0.05).astype(f32)  # every node inside the grid
    gv = rng.standard_normal((G, G, 2)).astype(f32)
    arrays = {"x": x.copy(), "v": np.zeros((N, 2), f32), "grid_v": gv}
    run_ops(low, names, arrays)
    rows, cols, wt = splat_nodes(x, G)
    want = np.zeros((N, 2), f32)
    for i in range(3):
        for j in range(3):  # new_v += w * grid_v[...], node by node
            want = want + wt[:, i, j, None] * gv[rows[:, i, j], cols[:, i, j]]
    assert np.array_equal(arrays["v"], want)
    assert np.array_equal(arrays["x"], x + f32(2e-4) * want)


KERNELS = """import taichi as ti
a = ti.field(dtype=float, shape=(16, 12))
cnt = ti.field(dtype=int, shape=(4, 3))
acc = ti.field(dtype=float, shape=8)
vol = ti.field(dtype=int, shape=(3, 4, 5))
s = ti.field(dtype=float, shape=())
out = ti.field(dtype=float, shape=(16, 12))

@ti.kernel
def branchy():
    for i, j in a:
        if a[i, j] > 0.5:
            cnt[i % 4, j % 3] += 1
        else:
            ti.atomic_sub(acc[i % 8], a[i, j])
        ti.atomic_add(s[None], 1.0)

@ti.kernel
def three_d():
    for i, j in a:
        vol[i - 2, j - 3, (i + j) % 7] += 1

@ti.kernel
def store_and_add():
    for i, j in a:
        out[i, j] = a[i, j] * 2.0
        a[i, j] = a[i, j] + 1.0
        acc[j % 8] += out[i, j]

@ti.kernel
def read_total():
    for i, j in out:
        out[i, j] = s[None] + i
"""


def test_adds_in_branches_happen_where_the_branch_runs():
    low, names = lower_named(KERNELS, "branchy", {})
    rng = np.random.default_rng(11)
    a = rng.random((16, 12)).astype(f32)
    arrays = {"a": a, "cnt": np.zeros((4, 3), np.int32), "acc": np.zeros(8, f32), "s": np.zeros((), f32)}
    run_ops(low, names, arrays)
    i, j = np.meshgrid(np.arange(16), np.arange(12), indexing="ij")
    hi = a > f32(0.5)
    want_cnt = np.zeros((4, 3), np.int64)
    np.add.at(want_cnt, ((i % 4)[hi], (j % 3)[hi]), 1)
    want_acc = np.zeros(8, f32)
    np.add.at(want_acc, (i % 8)[~hi], -a[~hi])  # row-major order, as the oracle adds
    assert np.array_equal(arrays["cnt"], want_cnt.astype(np.int32))
    assert np.array_equal(arrays["acc"], want_acc)
    assert float(arrays["s"]) == 16 * 12


def test_three_d_target_drops_each_axis_on_its_own():
    """vol[i - 2, j - 3, (i + j) % 7] of a [3][4][5] field: an index past one axis is dropped,
    not carried into the next (as flattening [A B][C] alone would do)."""
    low, names = lower_named(KERNELS, "three_d", {})
    arrays = {"a": np.zeros((16, 12), f32), "vol": np.zeros((3, 4, 5), np.int32)}
    run_ops(low, names, arrays)
    want = np.zeros((3, 4, 5), np.int64)
    for i in range(16):
        for j in range(12):
            a_, b_, c_ = i - 2, j - 3, (i + j) % 7
            if 0 <= a_ < 3 and 0 <= b_ < 4 and 0 <= c_ < 5:
                want[a_, b_, c_] += 1
    assert np.array_equal(arrays["vol"], want.astype(np.int32))


def test_a_body_that_stores_two_fields_runs_its_adds_once():
    low, names = lower_named(KERNELS, "store_and_add", {})
    ops = low.ops()
    assert sum(o.field is None for o in ops) == 1  # one program of the adds, beside the stores
    rng = np.random.default_rng(12)
    a0 = rng.random((16, 12)).astype(f32)
    arrays = {"a": a0.copy(), "out": np.zeros((16, 12), f32), "acc": np.zeros(8, f32)}
    run_ops(low, names, arrays)
    assert np.array_equal(arrays["out"], a0 * f32(2.0)) and np.array_equal(arrays["a"], a0 + f32(1.0))
    want = np.zeros(8, f32)
    j = np.broadcast_to(np.arange(12), (16, 12))
    np.add.at(want, (j % 8).ravel(), (a0 * f32(2.0)).ravel())  # the adds read a before its store
    assert np.array_equal(arrays["acc"], want)


def test_zero_d_field_read_in_a_kernel():
    low, names = lower_named(KERNELS, "read_total", {})
    assert low.program.in_rows[0] == 1 and low.program.in_cols[0] == 1
    arrays = {"out": np.zeros((16, 12), f32), "s": np.array(2.5, f32)}
    run_ops(low, names, arrays)
    assert np.array_equal(arrays["out"], f32(2.5) + np.arange(16, dtype=f32)[:, None] + np.zeros((1, 12), f32))


@pytest.mark.parametrize("body, msg", [
    ("        cnt[i % 4, j % 3] += 1\n        a[i, j] = cnt[0, 0] * 1.0", "also read"),
    ("        a[i, j] = 1.0\n        a[i + 1, j] += 1.0", "both stored"),
    ("        k = 0\n        while k < 3:\n            acc[k] += 1.0\n            k += 1", "inside a runtime loop"),
    ("        acc[i % 8] *= 2.0", "only += and -="),
    ("        x = ti.atomic_add(acc[0], 1.0)", "as a statement"),
])
def test_scatter_forms_refused(body, msg):
    text = KERNELS.split("@ti.kernel")[0] + "@ti.kernel\ndef bad():\n    for i, j in a:\n" + body + "\n"
    with pytest.raises(tc.TaichiLoweringError, match=re.escape(msg)):
        lower_named(text, "bad", {})


# ---- MPM88: matrices, matrix fields, field-element components, splits between static iterations
def mpm88_constants(G=128):
    dx = f32(1.0 / G)
    dt, E = f32(2e-4), f32(400.0)
    p_vol = f32((1.0 / G * 0.5) ** 2)
    p_mass = f32(p_vol * 1.0)
    return dx, dt, dx * dx, ((-dt * f32(4.0)) * E) * p_vol, p_mass


def bspline(Xp):
    base = np.trunc(Xp - f32(0.5))
    fx = Xp - base
    w = [f32(0.5) * ((f32(1.5) - fx) * (f32(1.5) - fx)), f32(0.75) - (fx - f32(1.0)) * (fx - f32(1.0)),
         f32(0.5) * ((fx - f32(0.5)) * (fx - f32(0.5)))]
    return base, fx, w


def mpm88_p2g_terms(x, v, C, J, G=128):
    """The particle-to-grid adds of the mpm88 example: (rows, columns) and the momentum (two
    components) and mass terms, particle by particle and node by node (np.add.at's order)."""
    dx, dt, inv_dx2, k_stress, p_mass = mpm88_constants(G)
    base, fx, w = bspline(x / dx)
    stress = (k_stress * (J - f32(1.0))) / inv_dx2
    a00 = stress + p_mass * C[:, 0, 0]
    a01 = f32(0.0) + p_mass * C[:, 0, 1]
    a10 = f32(0.0) + p_mass * C[:, 1, 0]
    a11 = stress + p_mass * C[:, 1, 1]
    rows, cols, vals_v0, vals_v1, vals_m = [], [], [], [], []
    for i in range(3):
        for j in range(3):
            d0 = (f32(i) - fx[:, 0]) * dx
            d1 = (f32(j) - fx[:, 1]) * dx
            wt = w[i][:, 0] * w[j][:, 1]
            m0 = p_mass * v[:, 0] + (a00 * d0 + a01 * d1)
            m1 = p_mass * v[:, 1] + (a10 * d0 + a11 * d1)
            rows.append(base[:, 0].astype(np.int64) + i)
            cols.append(base[:, 1].astype(np.int64) + j)
            vals_v0.append(wt * m0)
            vals_v1.append(wt * m1)
            vals_m.append(wt * p_mass)
    order = lambda lst: np.stack(lst, 1).ravel()  # particle by particle, node by node
    return (order(rows), order(cols)), (order(vals_v0), order(vals_v1), order(vals_m))


def mpm88_numpy_substep(x, v, C, J, G=128):
    """One substep of the mpm88 example in numpy f32, the same operations in the same order
    (constants folded in f32 as the front end folds them); the particle-to-grid adds in the
    oracle's order (particle by particle, node by node)."""
    n = x.shape[0]
    dx, dt, inv_dx2, k_stress, p_mass = mpm88_constants(G)  # dx ** 2 and the stress constant folded in f32
    gravity = f32(9.8)
    gv = np.zeros((G, G, 2), f32)
    gm = np.zeros((G, G), f32)
    idx, terms = mpm88_p2g_terms(x, v, C, J, G)
    np.add.at(gv[:, :, 0], idx, terms[0])
    np.add.at(gv[:, :, 1], idx, terms[1])
    np.add.at(gm, idx, terms[2])
    Xp = x / dx
    base, fx, w = bspline(Xp)
    # grid update
    i, j = np.meshgrid(np.arange(G), np.arange(G), indexing="ij")
    has = gm > f32(0.0)
    with np.errstate(all="ignore"):
        vx = np.where(has, gv[:, :, 0] / gm, gv[:, :, 0])
        vy = np.where(has, gv[:, :, 1] / gm, gv[:, :, 1])
    vy = vy - dt * gravity
    vx = np.where((i < 3) & (vx < 0), f32(0.0), vx)
    vx = np.where((i > G - 3) & (vx > 0), f32(0.0), vx)
    vy = np.where((j < 3) & (vy < 0), f32(0.0), vy)
    vy = np.where((j > G - 3) & (vy > 0), f32(0.0), vy)
    gv = np.stack([vx, vy], -1).astype(f32)
    # grid to particles
    nv = [np.zeros(n, f32), np.zeros(n, f32)]
    nC = [[np.zeros(n, f32), np.zeros(n, f32)], [np.zeros(n, f32), np.zeros(n, f32)]]
    for a in range(3):
        for c in range(3):
            d = [(f32(a) - fx[:, 0]) * dx, (f32(c) - fx[:, 1]) * dx]
            wt = w[a][:, 0] * w[c][:, 1]
            g = gv[base[:, 0].astype(np.int64) + a, base[:, 1].astype(np.int64) + c]
            for k in range(2):
                nv[k] = nv[k] + wt * g[:, k]
            s = f32(4.0) * wt
            for r in range(2):
                for q in range(2):
                    nC[r][q] = nC[r][q] + (s * (g[:, r] * d[q])) / inv_dx2
    v2 = np.stack(nv, -1)
    x2 = x + dt * v2
    J2 = J * (f32(1.0) + dt * (nC[0][0] + nC[1][1]))
    C2 = np.stack([np.stack(nC[0], -1), np.stack(nC[1], -1)], -2)
    return x2, v2, C2, J2, gv, gm


def test_mpm88_substeps_on_the_oracle_equal_numpy():
    """The example's init and two substeps (12 programs each: the grid-to-particle loop runs as
    parts joined by hidden fields, split between static iterations) against the numpy
    restatement, bit for bit: matrices (ti.Matrix, @, outer_product, trace, matrix fields), the
    grid-velocity component updates and the scatter-adds."""
    text = open(os.path.join(EX, "mpm88.py")).read()
    init, names_i = lower_named(text, "init", {})
    sub, names = lower_named(text, "substep", {})
    n, G = 8192, 128
    arrays = {"x": np.zeros((n, 2), f32), "v": np.zeros((n, 2), f32), "C": np.zeros((n, 2, 2), f32),
              "J": np.zeros(n, f32), "grid_v": np.zeros((G, G, 2), f32), "grid_m": np.zeros((G, G), f32)}
    run_ops(init, names_i, arrays)
    p = np.arange(n)
    x0 = np.stack([((p * 37 % 1009).astype(f32) / f32(1009.0)) * f32(0.4) + f32(0.2),
                   ((p * 59 % 997).astype(f32) / f32(997.0)) * f32(0.4) + f32(0.2)], -1)
    assert np.array_equal(arrays["x"], x0) and np.all(arrays["J"] == 1.0)
    ref = (arrays["x"].copy(), arrays["v"].copy(), arrays["C"].copy(), arrays["J"].copy())
    for _ in range(2):
        run_ops(sub, names, arrays)
        x2, v2, C2, J2, gv, gm = mpm88_numpy_substep(*ref)
        assert np.array_equal(arrays["grid_m"], gm)
        assert np.array_equal(arrays["grid_v"], gv)
        for k, want in (("v", v2), ("x", x2), ("C", C2), ("J", J2)):
            assert np.array_equal(arrays[k], want), k
        ref = (x2, v2, C2, J2)
    assert abs(float(arrays["grid_m"].sum(dtype=np.float64)) - n * (1.0 / 256) ** 2) < 1e-6  # mass is conserved


# ---- scatter max / min (ti.atomic_max / atomic_min) -------------------------------------------------
def test_oracle_scatter_max_min_equal_numpy():
    """f32 max / min as fmaxf / fminf (np.fmax.at / np.fmin.at: a NaN value is ignored), int32
    exactly (np.maximum.at / np.minimum.at), over NaN, signed zeros and infinities."""
    ni, nj, bins = 19, 23, 6
    rng = np.random.default_rng(15)
    v = rng.standard_normal((ni, nj)).astype(f32)
    v.ravel()[rng.choice(v.size, 40, replace=False)] = rng.choice(np.array([np.nan, 0.0, -0.0, np.inf, -np.inf], f32), 40)
    col = rng.integers(0, bins, (ni, nj)).astype(f32)
    b = pp.Builder()
    x, c = b.load(0, 0), b.load(0, 1)
    eff = [b.scatter_add(1, 0.0, c, x, op="max"), b.scatter_add(2, 0.0, c, x, op="min"),
           b.scatter_add(3, 0.0, c, b.op("mul", x, 1000.0), op="max"), b.scatter_add(3, 0.0, c, 1.0, op="add")]
    prog = pp.compile_program(b, out=None, effects=eff, in_widths=[2, 1, 1, 1], in_dtypes=[pp.F32, pp.F32, pp.F32, pp.I32],
                              in_extents=[None, (1, bins), (1, bins), (1, bins)])
    mx = np.full((1, bins), -5.0, f32)
    mn = np.full((1, bins), np.nan, f32)  # a NaN element takes the first value
    im = np.zeros((1, bins), np.int32)
    oracle.pixel_program(prog, ni, nj, [np.stack([v, col], -1), mx, mn, im])
    idx = (np.zeros(v.size, np.int64), col.astype(np.int64).ravel())
    want_mx, want_mn = np.full((1, bins), -5.0, f32), np.full((1, bins), np.nan, f32)
    np.fmax.at(want_mx, idx, v.ravel())
    np.fmin.at(want_mn, idx, v.ravel())
    assert np.array_equal(mx, want_mx, equal_nan=True) and np.array_equal(mn, want_mn, equal_nan=True)
    # the int32 target takes max(trunc(1000 v)) (NaN -> 0, infinities saturate) and then + 1 per
    # pixel (wrapping), in program order pixel by pixel
    want_i = np.zeros(bins, np.int64)
    for val, k in zip(v.ravel(), col.astype(np.int64).ravel()):
        t = 0 if np.isnan(val) else int(np.clip(np.trunc(np.float64(np.float32(val * np.float32(1000.0)))), -2**31, 2**31 - 1))
        want_i[k] = (max(want_i[k], t) + 1 + 2**31) % 2**32 - 2**31  # the add wraps in int32
    assert np.array_equal(im[0], want_i.astype(np.int32))


ATOMIC_EXT = """import taichi as ti
x = ti.field(dtype=float, shape=(30, 20))
mx = ti.field(dtype=float, shape=())
mn = ti.field(dtype=float, shape=4)
peak = ti.field(dtype=float, shape=(30, 20))

@ti.kernel
def k():
    for i, j in x:
        ti.atomic_max(mx[None], x[i, j])
        ti.atomic_min(mn[j % 4], x[i, j] * 2.0)
        ti.atomic_max(peak[i, j], x[i, j] - 0.5)
"""


def test_front_end_atomic_max_min():
    low, names = lower_named(ATOMIC_EXT, "k", {})
    rng = np.random.default_rng(16)
    x = rng.standard_normal((30, 20)).astype(f32)
    p0 = rng.standard_normal((30, 20)).astype(f32)
    arr = {"x": x, "mx": np.array(-100.0, f32), "mn": np.full(4, 100.0, f32), "peak": p0.copy()}
    run_ops(low, names, arr)
    assert float(arr["mx"]) == float(x.max())
    j = np.broadcast_to(np.arange(20), (30, 20))
    assert np.array_equal(arr["mn"], np.array([(x * f32(2.0))[j % 4 == k].min() for k in range(4)], f32))
    assert np.array_equal(arr["peak"], np.maximum(p0, x - f32(0.5)))  # the pixel's own element: a plain max


# ---- stores at computed indices (VDSL_PIX_STORE_AT) --------------------------------------------------
STORES = """import taichi as ti
W, H = 40, 30
u = ti.field(dtype=float, shape=(W, H))
v = ti.field(dtype=float, shape=(W, H))
code = ti.field(dtype=int, shape=(W, H))
@ti.kernel
def interior():
    for i, j in ti.ndrange((1, W - 1), (1, H - 1)):
        v[i, j] = 0.25 * (u[i - 1, j] + u[i + 1, j] + u[i, j - 1] + u[i, j + 1])
@ti.kernel
def boundary():
    for i in range(W):
        v[i, 0] = 1.0
        v[i, H - 1] = -1.0
        code[i, (i * 7) % H] = i * 2.5
@ti.kernel
def transpose_into():
    for i, j in ti.ndrange(30, 40):
        v[j, i] = u[j, i] * 2.0
        if u[j, i] > 0.5:
            code[j, i] = -3
"""


def test_stores_at_computed_indices():
    """An interior ti.ndrange((1, W - 1), ...) stencil, boundary rows written from a 1-D loop (an
    int field storing a truncated float), and a transposed loop with a store inside an if: every
    store lands where numpy's assignment puts it, nothing else changes."""
    rng = np.random.default_rng(21)
    u = rng.random((40, 30)).astype(f32)
    v0 = rng.random((40, 30)).astype(f32)
    c0 = rng.integers(-9, 9, (40, 30)).astype(np.int32)
    arr = {"u": u, "v": v0.copy(), "code": c0.copy()}
    want_v, want_c = v0.copy(), c0.copy()
    low, names = lower_named(STORES, "interior", {})
    assert low.field is None and low.grid == (38, 28)
    run_ops(low, names, arr)
    want_v[1:-1, 1:-1] = f32(0.25) * (((u[:-2, 1:-1] + u[2:, 1:-1]) + u[1:-1, :-2]) + u[1:-1, 2:])
    assert np.array_equal(arr["v"], want_v)
    low, names = lower_named(STORES, "boundary", {})
    run_ops(low, names, arr)
    i = np.arange(40)
    want_v[:, 0], want_v[:, -1] = 1.0, -1.0
    want_c[i, (i * 7) % 30] = np.trunc(i * 2.5).astype(np.int32)
    assert np.array_equal(arr["v"], want_v) and np.array_equal(arr["code"], want_c)
    low, names = lower_named(STORES, "transpose_into", {})
    run_ops(low, names, arr)
    want_v = u * f32(2.0)
    want_c = np.where(u > f32(0.5), np.int32(-3), want_c)
    assert np.array_equal(arr["v"], want_v) and np.array_equal(arr["code"], want_c)


def test_oracle_store_at_drops_outside_and_keeps_the_rest():
    b = pp.Builder()
    e = b.scatter_add(1, b.load(0, 0), b.load(0, 1), b.load(0, 2), op="store")
    prog = pp.compile_program(b, out=None, effects=[e], in_widths=[3, 1], in_extents=[None, (4, 5)])
    pts = np.array([[[0, 0, 1.5], [3, 4, 2.5], [4, 0, 9.0], [-1, 2, 9.0], [2, np.nan, 9.0], [1.7, 2.2, 3.5]]], f32)
    t = np.full((4, 5), -1.0, f32)
    oracle.pixel_program(prog, 1, 6, [pts, t])
    want = np.full((4, 5), -1.0, f32)
    want[0, 0], want[3, 4], want[1, 2] = 1.5, 2.5, 3.5
    assert np.array_equal(t, want)


# ---- kernel-scope reductions: `e = 0.0; for ...: e += ...; return e` --------------------------------
REDUCE = """import taichi as ti
x = ti.field(dtype=float, shape=(50, 40))
v = ti.Vector.field(2, dtype=float, shape=300)
@ti.kernel
def energy() -> float:
    e = 0.0
    n = 0
    for i in v:
        e += 0.5 * v[i].norm_sqr()
    for i, j in x:
        if x[i, j] > 0.5:
            n += 1
        e -= x[i, j]
    return e
"""


def test_kernel_scope_reductions_on_the_oracle():
    """Each kernel-scope scalar is a hidden 0-D field: its initial value stored, the loops' += / -=
    added at a constant index, the returned one named by Lowered.ret; the oracle's sums (pixel by
    pixel) equal numpy's sequential f32 sums."""
    low, names = lower_named(REDUCE, "energy", {})
    assert low.ret is not None and low.ret.shape == () and low.ret.dtype == tc.f32
    rng = np.random.default_rng(2)
    X = rng.random((50, 40)).astype(f32)
    V = rng.standard_normal((300, 2)).astype(f32)
    arrays = {"x": X, "v": V}
    for op in low.ops():
        for f in op.inputs + ([op.field] if op.field is not None else []):
            if id(f) not in names:  # the hidden accumulators
                names[id(f)] = f"acc{len(names)}"
                arrays[names[id(f)]] = np.zeros((), np.int32 if f.dtype == tc.i32 else f32)
    run_ops(low, names, arrays)
    e = f32(0.0)
    for a, c in V:
        e = e + f32(0.5) * (a * a + c * c)
    for xv in X.ravel():
        e = e + (-xv)
    got = {a.dtype.kind: a for k, a in arrays.items() if k.startswith("acc")}
    assert float(got["f"]) == float(e) and int(got["i"]) == int((X > f32(0.5)).sum())


def test_kernel_scope_forms_refused():
    for body, msg in (("    e = 0.0\n    for i in v:\n        e += 1.0\n    e = e * 2.0\n    return e", "kernel body"),
                      ("    e = x[0, 0]\n    for i in v:\n        e += 1.0\n    return e", "constant")):
        text = REDUCE.split("@ti.kernel")[0] + "@ti.kernel\ndef bad() -> float:\n" + body + "\n"
        with pytest.raises(tc.TaichiLoweringError, match=msg):
            lower_named(text, "bad", {})


# ---- ti.random ----------------------------------------------------------------------------------
def lowbias32(x):
    """Chris Wellons' lowbias32 integer hash, in numpy uint32 arithmetic."""
    x = np.atleast_1d(np.asarray(x, np.uint32))
    with np.errstate(over="ignore"):  # the multiplies wrap modulo 2^32, as the hash means them to
        x = x ^ (x >> np.uint32(16))
        x = x * np.uint32(0x7feb352d)
        x = x ^ (x >> np.uint32(15))
        x = x * np.uint32(0x846ca68b)
        x = x ^ (x >> np.uint32(16))
    return x


RANDOM = """import taichi as ti
p = ti.Vector.field(2, dtype=float, shape=5000)
@ti.kernel
def seed():
    for i in p:
        p[i] = [ti.random() * 0.4 + 0.2, ti.random(float)]
"""


def test_random_numbers_on_the_oracle():
    """Each ti.random() call site is a draw of its own: the oracle's numbers equal the hash
    restated in numpy (seed, draw, pixel), lie in [0, 1), and look uniform and independent."""
    low, names = lower_named(RANDOM, "seed", {})
    prog = low.program
    draws = [int(prog.code[k].imm) for k in range(prog.n_pre + prog.n_post) if prog.code[k].op == pp.OP["random"]]
    assert len(draws) == 2 and draws[0] != draws[1]
    names[id(tc._rng_state())] = "rng"
    for seed in (0, 7):
        arr = {"p": np.zeros((5000, 2), f32), "rng": np.array(seed, np.int32)}
        run_ops(low, names, arr)
        pix = np.arange(5000, dtype=np.uint32)
        u = [(lowbias32(lowbias32(lowbias32(seed) ^ np.uint32(d)) ^ pix) >> np.uint32(8)).astype(f32) * f32(2.0 ** -24)
             for d in draws]
        assert np.array_equal(arr["p"][:, 0], u[0] * f32(0.4) + f32(0.2)) and np.array_equal(arr["p"][:, 1], u[1])
        assert 0.0 <= u[1].min() and u[1].max() < 1.0 and abs(float(u[1].mean()) - 0.5) < 0.02
        assert abs(float(np.corrcoef(u[0], u[1])[0, 1])) < 0.05
