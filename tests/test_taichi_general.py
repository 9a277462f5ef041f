"""The general path of the Taichi-subset front end on the CPU: struct-for bodies that are not of
the escape-time form lower to per-pixel register programs (vernondsl_amd.pixprog), which the CPU
oracle runs (oracle.pixel_program).  The oracle's interpreter is pinned here by independent numpy
restatements of whole programs (same f32 operations in the same order, so bit for bit where the
program has only exactly rounded operations) and by agreement with the escape-time oracle on the
programs both express."""
import os

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, pixprog as pp, spec, taichi_compat as tc

EX = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vernondsl_amd", "examples")
REF = "/root/reference/fractal.py"
f32 = np.float32


def ex(name):
    return open(os.path.join(EX, name)).read()


def general(text, kernel, args):
    """Lowers by the general path even where the escape-time form also applies."""
    return tc.lower_source_kernel(text, kernel, args, general=True)


def test_mandelbrot_by_the_general_path_equals_the_escape_time_oracle():
    low = general(ex("mandelbrot_counts.py"), "render", {"limit": 256})
    assert low.kind == "pixel_program" and low.program.out_kind == pp.OUT_COUNT and low.program.max_iter == 256
    got = oracle.pixel_program(low.program, 1024, 1024)
    assert int(got.sum()) == 49_860_131  # the separately-rounded grid's known sum
    assert np.array_equal(got, oracle.escape_time(spec.mandelbrot_params(rounding=_lib.ESC_ROUND_SEPARATE)))


def test_julia_by_the_general_path_equals_the_escape_time_oracle():
    text = ex("rabbit_drift.py")
    low = general(text, "draw", {"angle": 0.3})
    _, p = tc.lower_source(text, "draw", {"angle": 0.3})
    assert np.array_equal(oracle.pixel_program(low.program, 512, 512), oracle.escape_time(p))


@pytest.mark.skipif(not os.path.exists(REF), reason="the reference tree is only mounted in the build container")
def test_reference_fractal_py_keeps_the_escape_time_op():
    low = tc.lower_source_kernel(open(REF).read(), "paint", {"t": 0.03})
    assert low.kind == "escape_time"


def burning_ship_numpy(n, limit, zoom):
    i = np.arange(n, dtype=np.float32)[:, None] * np.ones((1, n), np.float32)
    j = np.ones((n, 1), np.float32) * np.arange(n, dtype=np.float32)[None, :]
    cx = ((i / f32(n)) + f32(-0.5)) * f32(zoom) + f32(-0.45)
    cy = ((j / f32(n)) + f32(-0.5)) * f32(zoom) + f32(-0.5)
    x = np.zeros_like(cx)
    y = np.zeros_like(cx)
    cnt = np.zeros(cx.shape, np.int32)
    live = np.ones(cx.shape, bool)
    for _ in range(limit):
        live &= (x * x + y * y) <= f32(4.0)
        if not live.any():
            break
        ax, ay = np.abs(x), np.abs(y)
        nx = (ax * ax - ay * ay) + cx
        ny = (f32(2.0) * ax) * ay + cy
        x = np.where(live, nx, x)
        y = np.where(live, ny, y)
        cnt += live
    return cnt


def test_burning_ship_program_against_numpy():
    low = tc.lower_source_kernel(ex("burning_ship.py"), "ship", {"zoom": 3.2})
    assert low.kind == "pixel_program" and low.field.dtype == "i32"
    got = oracle.pixel_program(low.program, 1024, 1024, rows=(0, 256))
    ref = burning_ship_numpy(1024, 256, 3.2)[:256]
    assert np.array_equal(got, ref)
    assert got.max() == 256 and got.min() >= 1


def test_interference_programs_against_numpy():
    text = ex("interference.py")
    mask_low = tc.lower_source_kernel(text, "make_mask", {})
    assert mask_low.kind == "pixel_program" and not mask_low.program.loop and mask_low.inputs == []
    n = 768
    mask = oracle.pixel_program(mask_low.program, n, n)
    i = np.arange(n, dtype=np.float64)[:, None]
    j = np.arange(n, dtype=np.float64)[None, :]
    mref = np.exp(-((i - 384.0) ** 2 + (j - 384.0) ** 2) * 1e-5)
    assert np.all(np.abs(mask - mref) <= 2e-6 * mref)
    low = tc.lower_source_kernel(text, "waves", {"phase": 0.5})
    assert [f.shape for f in low.inputs] == [(n, n)]
    got = oracle.pixel_program(low.program, n, n, [mask]).astype(np.float64)
    d1 = np.sqrt((i - 200.0) ** 2 + (j - 300.0) ** 2)
    d2 = np.sqrt((i - 560.0) ** 2 + (j - 420.0) ** 2)
    ref = 0.5 + 0.25 * (np.sin(d1 * 0.08 - 0.5) + np.sin(d2 * 0.08 - 0.5)) * mask
    assert np.all(np.abs(got - ref) <= 2e-5)


LOGISTIC = '''
import taichi as ti
n = 96
f = ti.field(dtype=float, shape=(n, n))
g = ti.field(dtype=float, shape=(n, n))

@ti.kernel
def k():
    for i, j in f:
        r = 2.5 + i / n * 1.5
        x = 0.25 + g[i, j] * 0.5
        for _ in range(STEPS):
            x = r * x * (1.0 - x)
        f[i, j] = x
'''


@pytest.mark.parametrize("steps", [0, 1, 37])
def test_fixed_trip_loop_against_numpy(steps):
    low = tc.lower_source_kernel(LOGISTIC.replace("STEPS", str(steps)), "k", {})
    p = low.program
    assert p.loop == 1 and p.test == 0 and p.max_iter == steps
    g = np.random.default_rng(5).random((96, 96), dtype=np.float32)
    got = oracle.pixel_program(p, 96, 96, [g])
    i = np.arange(96, dtype=np.float32)[:, None] * np.ones((1, 96), np.float32)
    r = f32(2.5) + (i / f32(96)) * f32(1.5)
    x = f32(0.25) + g * f32(0.5)
    for _ in range(steps):
        x = (r * x) * (f32(1.0) - x)
    assert np.array_equal(got, x)


def test_count_stored_into_f32_and_parallel_swap():
    text = '''
import taichi as ti
f = ti.field(dtype=float, shape=(16, 24))

@ti.kernel
def k():
    for i, j in f:
        a = i * 1.0
        b = j * 1.0
        m = 0
        while a < b and m < 50:
            a, b = b, a + 1.0
            m += 1
        f[i, j] = m * 0.5 + a - b
'''
    low = tc.lower_source_kernel(text, "k", {})
    got = oracle.pixel_program(low.program, 16, 24)
    ref = np.zeros((16, 24), np.float32)
    for i in range(16):
        for j in range(24):
            a, b, m = f32(i), f32(j), 0
            while a < b and m < 50:
                a, b = b, a + f32(1.0)
                m += 1
            ref[i, j] = (f32(m) * f32(0.5) + a) - b
    assert np.array_equal(got, ref)


def test_while_body_reads_its_counter():
    """x = 0 + 1 + ... + 9 in a while loop whose body reads the counter (the trip)."""
    text = ("import taichi as ti\nf = ti.field(dtype=float, shape=(8, 8))\n@ti.kernel\ndef k():\n    for i, j in f:\n"
            "        x = 0.0\n        k = 0\n        while k < 10 and x < i * 4.0:\n            x = x + k\n            k += 1\n"
            "        f[i, j] = x + k * 0.01\n")
    low = tc.lower_source_kernel(text, "k", {})
    got = oracle.pixel_program(low.program, 8, 8)
    ref = np.zeros((8, 8), np.float32)
    for i in range(8):
        x, k = f32(0), 0
        while k < 10 and x < f32(i) * f32(4.0):
            x, k = x + f32(k), k + 1
        ref[i, :] = x + f32(k) * f32(0.01)
    assert np.array_equal(got, ref) and len(np.unique(ref)) > 4


@pytest.mark.parametrize("body,msg", [
    ("        k = 0\n        while k < 10:\n            k += 1\n            k += 1\n        f[i, j] = k", "counter|loop"),
    ("        f[i, j] = 1.0\n        for _ in range(3):\n            x = 2.0", "after the loop"),
    ("        x = 0.0\n        for _ in range(3):\n            y = 1.0\n            for _ in range(2):\n                x = x + y\n        f[i, j] = x", "statement"),
    ("        x = 0.0\n        for _ in range(3):\n            f[i, j] = x", "store inside the loop"),
    ("        f[i, j] = i << j", "known when"),
    ("        if i > j:\n            y = 1.0\n        f[i, j] = y", "one branch"),
    ("        x = 1.0", "must store"),
])
def test_rejected_general_bodies(body, msg):
    text = "import taichi as ti\nf = ti.field(dtype=float, shape=(8, 8))\n@ti.kernel\ndef k():\n    for i, j in f:\n" + body + "\n"
    with pytest.raises(tc.TaichiLoweringError, match=msg):
        tc.lower_source_kernel(text, "k", {})


def test_register_pressure_is_reported():
    b = pp.Builder()
    vals = [b.op("sin", b.op("mul", b.index(0), float(k + 1))) for k in range(80)]
    acc = vals[0]
    for v in vals[1:]:
        acc = b.op("add", acc, v)
    pp.compile_program(b, out=acc)  # a chain: few registers live at once
    wide = b.op("add", vals[0], vals[1])
    for k in range(2, 80):
        wide = b.op("add", wide, b.op("mul", vals[k], vals[(k + 37) % 80]))
    with pytest.raises(pp.ProgramError, match="registers|instructions"):
        pp.compile_program(b, out=wide)


def grid(ni, nj):
    i = np.arange(ni, dtype=np.float32)[:, None] * np.ones((1, nj), np.float32)
    j = np.ones((ni, 1), np.float32) * np.arange(nj, dtype=np.float32)[None, :]
    return i, j


def body_kernel(body, shape=(40, 56), extra=""):
    return ("import taichi as ti\nn = 40\nf = ti.field(dtype=float, shape=" + repr(shape) + ")\n" + extra +
            "@ti.kernel\ndef k():\n    for i, j in f:\n" + body + "\n")


def test_if_else_store_with_floor_division_and_mod():
    body = ("        if (i // 8 + j // 8) % 2 == 0:\n            f[i, j] = 1.0\n"
            "        else:\n            f[i, j] = 0.25")
    low = tc.lower_source_kernel(body_kernel(body), "k", {})
    got = oracle.pixel_program(low.program, 40, 56)
    i, j = grid(40, 56)
    ref = np.where(((np.floor(i / f32(8)) + np.floor(j / f32(8))) % 2) == 0, f32(1.0), f32(0.25))
    assert np.array_equal(got, ref) and set(np.unique(got)) == {0.25, 1.0}


def test_store_in_one_branch_keeps_the_field():
    body = "        if i < j:\n            f[i, j] = f[i, j] * 2.0 + 1.0"
    low = tc.lower_source_kernel(body_kernel(body), "k", {})
    assert [fl.shape for fl in low.inputs] == [(40, 56)] and low.inputs[0] is low.field
    g = np.random.default_rng(2).standard_normal((40, 56)).astype(np.float32)
    got = oracle.pixel_program(low.program, 40, 56, [g])
    i, j = grid(40, 56)
    assert np.array_equal(got, np.where(i < j, g * f32(2.0) + f32(1.0), g))


def test_conditions_select_and_reading_back_a_store():
    body = ("        v = i * 0.1 - j * 0.05\n"
            "        w = ti.select(v > 0.0 and not (i % 3 == 0), v, -v * 0.5)\n"
            "        f[i, j] = w if (w < 1.5 or j > 40) else 1.5\n"
            "        f[i, j] = f[i, j] + (1.0 if i == j else 0.0)")
    low = tc.lower_source_kernel(body_kernel(body), "k", {})
    assert low.inputs == []
    got = oracle.pixel_program(low.program, 40, 56)
    i, j = grid(40, 56)
    v = i * f32(0.1) - j * f32(0.05)
    w = np.where((v > 0) & ~((i - np.floor(i / f32(3)) * f32(3)) == 0), v, (-v) * f32(0.5))
    st = np.where((w < f32(1.5)) | (j > 40), w, f32(1.5))
    assert np.array_equal(got, st + np.where(i == j, f32(1.0), f32(0.0)))


BOUNCE = '''
        x = i / n
        y = j / n
        k = 0
        while k < 100 and x * x + y * y < 4.0 and abs(x - y) < 1.5:
            if x > y:
                x = x * x - y + 0.1
            else:
                x, y = y * 0.9, x * 1.1 - 0.3
            k += 1
        f[i, j] = k + x'''


def test_compound_loop_test_and_if_inside_the_loop():
    low = tc.lower_source_kernel(body_kernel(BOUNCE), "k", {})
    p = low.program
    assert p.loop and p.test == pp.TESTS["gt"] and p.max_iter == 100
    got = oracle.pixel_program(p, 40, 56)
    i, j = grid(40, 56)
    x, y = i / f32(40), j / f32(40)
    cnt = np.zeros_like(x)
    live = np.ones(x.shape, bool)
    for _ in range(100):
        live &= ((x * x + y * y) < f32(4.0)) & (np.abs(x - y) < f32(1.5))
        nx = np.where(x > y, (x * x - y) + f32(0.1), y * f32(0.9))
        ny = np.where(x > y, y, x * f32(1.1) - f32(0.3))
        x, y = np.where(live, nx, x), np.where(live, ny, y)
        cnt += live
    assert np.array_equal(got, cnt.astype(np.float32) + x)
    assert 0 < cnt.min() < cnt.max() <= 100


SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 2.5, -2.5, 1e-40, -1e-40, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan,
                     7.0, -7.25, 123456.75, -0.1], np.float32)


def test_compare_select_floor_opcodes_against_numpy():
    """The new opcodes on every pair of special values (signed zeros, subnormals, infinities,
    NaN): comparisons as IEEE predicates, select on `!= 0` (NaN true, -0 false), floor as
    np.floor, trunc as np.trunc (toward zero; -0.5 -> -0)."""
    n = len(SPECIALS)
    a = np.repeat(SPECIALS[:, None], n, axis=1)
    c = np.repeat(SPECIALS[None, :], n, axis=0)
    b = pp.Builder()
    la, lc = b.load(0), b.load(1)
    cases = {"lt": a < c, "le": a <= c, "eq": a == c, "ne": a != c}
    for kind, want in cases.items():
        prog = pp.compile_program(b, out=b.op(kind, la, lc))
        assert np.array_equal(oracle.pixel_program(prog, n, n, [a, c]), want.astype(np.float32)), kind
    prog = pp.compile_program(b, out=b.op("select", la, lc, b.op("neg", lc)))
    sel = oracle.pixel_program(prog, n, n, [a, c])
    want = np.where(a != 0, c, -c)
    assert np.array_equal(sel.view(np.uint32), want.view(np.uint32))
    prog = pp.compile_program(b, out=b.op("floor", la))
    fl = oracle.pixel_program(prog, n, n, [a, c])
    assert np.array_equal(fl.view(np.uint32), np.floor(a).view(np.uint32))
    prog = pp.compile_program(b, out=b.op("trunc", la))
    tr = oracle.pixel_program(prog, n, n, [a, c])
    assert np.array_equal(tr.view(np.uint32), np.trunc(a).view(np.uint32))


def ulp_distance(got, want):
    """Distance in units in the last place between two f32 arrays (the gap in the ordered bit
    patterns), 0 where both are NaN, a huge value where only one is."""
    def ordered(x):
        i = np.asarray(x, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    d = np.abs(ordered(g) - ordered(w))
    both = np.isnan(g) & np.isnan(w)
    one = np.isnan(g) ^ np.isnan(w)
    return np.where(both, 0, np.where(one, 1 << 40, d))


MATH_DOMAIN = np.concatenate([np.linspace(-1.2, 1.2, 301), np.linspace(-40, 40, 257), np.geomspace(1e-6, 1e6, 97),
                              -np.geomspace(1e-6, 1e6, 97), [0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan]]).astype(np.float32)
MATH_UNARY = {"asin": np.arcsin, "acos": np.arccos, "atan": np.arctan, "tan": np.tan}


def test_inverse_trig_tan_atan2_pow_opcodes_against_numpy():
    """asin, acos, atan, tan, atan2 and powf take the C library's float functions in the oracle:
    within 2 ulp of numpy's double-precision result rounded to f32 on a domain crossing every
    branch (|x| > 1 gives NaN for asin/acos; signed zeros, infinities, NaN), and the IEEE special
    cases of atan2 (quadrants, signed zeros) and pow (x^0 = 1, 1^y = 1, negative base with a
    fractional exponent = NaN, 0^-1 = inf) exactly."""
    x = MATH_DOMAIN
    n = len(x)
    b = pp.Builder()
    la, lc = b.load(0), b.load(1)
    for name, fn in MATH_UNARY.items():
        got = oracle.pixel_program(pp.compile_program(b, out=b.op(name, la)), 1, n, [x[None], x[None]])[0]
        with np.errstate(all="ignore"):
            want = fn(x.astype(np.float64)).astype(np.float32)
        assert ulp_distance(got, want).max() <= 2, name
    y = MATH_DOMAIN[::7]
    a = np.repeat(y[:, None], len(y), axis=1)
    c = np.repeat(y[None, :], len(y), axis=0)
    for name, fn in (("atan2", np.arctan2), ("powf", np.power)):
        got = oracle.pixel_program(pp.compile_program(b, out=b.op(name, la, lc)), len(y), len(y), [a, c])
        with np.errstate(all="ignore"):
            want = fn(a.astype(np.float64), c.astype(np.float64)).astype(np.float32)
        assert ulp_distance(got, want).max() <= 2, name
    sp = np.array([[0.0, 0.0], [-0.0, 0.0], [0.0, -0.0], [-0.0, -0.0], [0.0, -1.0], [-0.0, -1.0], [1.0, 0.0], [-1.0, -0.0], [1.0, 1.0],
                   [-1.0, 1.0]], np.float32)
    got = oracle.pixel_program(pp.compile_program(b, out=b.op("atan2", la, lc)), 1, len(sp), [sp[None, :, 0], sp[None, :, 1]])[0]
    pi = np.float32(np.pi)
    want = np.array([0.0, -0.0, pi, -pi, pi, -pi, pi / 2, -pi / 2, pi / 4, -pi / 4], np.float32)
    assert np.array_equal(np.signbit(got), np.signbit(want)) and ulp_distance(got, want).max() <= 1
    pw = np.array([[5.0, 0.0], [np.nan, 0.0], [1.0, np.nan], [-8.0, 1.0 / 3.0], [0.0, -1.0], [-2.0, 3.0], [4.0, 0.5]],
                  np.float32)
    got = oracle.pixel_program(pp.compile_program(b, out=b.op("powf", la, lc)), 1, len(pw), [pw[None, :, 0], pw[None, :, 1]])[0]
    assert np.array_equal(got, np.array([1.0, 1.0, 1.0, np.nan, np.inf, -8.0, 2.0], np.float32), equal_nan=True)


MATH_KERNELS = """
import taichi as ti
import taichi.math as tm
ti.init(arch=ti.gpu)
u = ti.field(dtype=float, shape=(16, 32))
out = ti.Vector.field(4, dtype=float, shape=(16, 32))

@ti.kernel
def polar():
    for i, j in out:
        x = u[i, j]
        r = ti.sqrt(x * x + 1.0) ** 1.5
        out[i, j] = [ti.atan2(x, i - 7.5), ti.asin(ti.min(ti.max(x, -1.0), 1.0)) + ti.acos(0.25), ti.atan(x) * ti.tan(0.1 * j), r]
"""


def test_taichi_atan2_asin_pow_lower_to_math_opcodes():
    """ti.atan2 / ti.asin / ti.acos / ti.atan / ti.tan and x ** y with a fractional exponent lower
    to the math opcodes (a constant argument folds in f32 on the host): the oracle's result is
    within a few f32 ulp of numpy's double-precision restatement of the kernel."""
    low = tc.lower_source_kernel(MATH_KERNELS, "polar", {})
    names = {v: k for k, v in pp.OP.items()}
    prog = low.program
    count = prog.n_pre + prog.n_test + prog.n_body + prog.n_post
    ops = {names.get(prog.code[k].op) for k in range(count)}
    u = np.random.default_rng(5).uniform(-2, 2, (16, 32)).astype(np.float32)
    got = oracle.pixel_program(low.program, 16, 32, [u])
    i = np.arange(16, dtype=np.float64)[:, None] * np.ones((1, 32))
    j = np.ones((16, 1)) * np.arange(32, dtype=np.float64)[None, :]
    x = u.astype(np.float64)
    want = np.stack([np.arctan2(x, i - 7.5), np.arcsin(np.clip(x, -1, 1)) + np.arccos(0.25),
                     np.arctan(x) * np.tan(np.float32(0.1) * j.astype(np.float32)),
                     np.sqrt(x * x + 1.0) ** 1.5], axis=-1).astype(np.float32)
    # the kernel's f32 roundings (x * x + 1, the sum asin + acos near its zero) against double
    # precision: within a few f32 ulp of the terms' magnitude (|terms| < 3)
    assert np.allclose(got, want, rtol=2e-6, atol=1e-6)
    assert {"atan2", "asin", "atan", "tan", "powf"} <= ops

def palette_numpy(shift, W=800, H=600, limit=120):
    x, y = grid(W, H)
    c0 = (x / f32(W)) * f32(3.0) + f32(-1.5)
    c1 = (y / f32(H)) * f32(2.4) + f32(-1.2)
    z0 = np.zeros_like(c0)
    z1 = np.zeros_like(c0)
    n = np.zeros(c0.shape, np.int32)
    live = np.ones(c0.shape, bool)
    for _ in range(limit):
        live &= (z0 * z0 + z1 * z1) < f32(16.0)
        re2 = z0 * z0 - z1 * z1
        im2 = (f32(2.0) * z0) * z1
        n0 = (z0 * re2 - z1 * im2) + c0
        n1 = (z0 * im2 + z1 * re2) + c1
        z0, z1 = np.where(live, n0, z0), np.where(live, n1, z1)
        n += live
    t = n.astype(np.float32) / f32(limit) + f32(shift)
    col = np.stack([f32(0.5) + f32(0.5) * np.cos(f32(6.2831) * (t + f32(o)), dtype=np.float32)
                    for o in (0.0, 0.33, 0.67)], axis=-1)
    col[:, :, 0] = f32(0.5) + f32(0.5) * np.cos(f32(6.2831) * t, dtype=np.float32)
    return np.where((n == limit)[:, :, None], f32(0.0), col), n


def test_vector_fields_palette_example_against_numpy():
    text = ex("palette.py")
    low = tc.lower_source_kernel(text, "render", {"shift": 0.05})
    assert low.kind == "pixel_program" and low.field.width == 3 and low.program.out_width == 3
    img = oracle.pixel_program(low.program, 800, 600, rows=(300, 500))
    ref, n = palette_numpy(0.05)
    ref = ref[300:500]
    assert img.shape == (200, 600, 3)
    inside = n[300:500] == 120
    assert inside.any() and (~inside).any()
    assert np.array_equal(img[inside], ref[inside])                # exact zeros inside the set
    assert np.max(np.abs(img - ref)) <= 2e-6                       # cosf against numpy's cos
    vig = tc.lower_source_kernel(text, "vignette", {})
    assert [f.width for f in vig.inputs] == [3] and list(vig.program.in_widths)[:1] == [3]
    full = oracle.pixel_program(low.program, 800, 600)
    sh = oracle.pixel_program(vig.program, 800, 600, [full])
    x, y = grid(800, 600)
    d0, d1 = x / f32(800) + f32(-0.5), y / f32(600) + f32(-0.5)
    k = f32(1.0) - f32(1.2) * (d0 * d0 + d1 * d1)
    want = np.stack([full[:, :, 0] * k, full[:, :, 1] * k, np.minimum(full[:, :, 2] * k + f32(0.05), f32(1.0))], -1)
    assert np.array_equal(sh, want)


def test_vector_field_stores_and_errors():
    text = ('import taichi as ti\nv = ti.Vector.field(2, dtype=float, shape=(8, 8))\n'
            'w = ti.Vector.field(4, dtype=float, shape=(8, 8))\n'
            '@ti.kernel\ndef fill():\n    for i, j in v:\n        v[i, j] = i * 0.5\n'
            '@ti.kernel\ndef swap():\n    for i, j in w:\n        a = v[i, j]\n        w[i, j] = [a.y, a.x, a[0] + a[1], 1.0]\n'
            '@ti.kernel\ndef bad():\n    for i, j in v:\n        v[i, j] = ti.Vector([1.0, 2.0, 3.0])\n')
    low = tc.lower_source_kernel(text, "fill", {})
    vv = oracle.pixel_program(low.program, 8, 8)
    i, _ = grid(8, 8)
    assert vv.shape == (8, 8, 2) and np.array_equal(vv, np.stack([i * f32(0.5)] * 2, -1))
    low = tc.lower_source_kernel(text, "swap", {})
    g = np.random.default_rng(4).standard_normal((8, 8, 2)).astype(np.float32)
    ww = oracle.pixel_program(low.program, 8, 8, [g])
    assert np.array_equal(ww, np.stack([g[..., 1], g[..., 0], g[..., 0] + g[..., 1], np.ones((8, 8), np.float32)], -1))
    with pytest.raises(tc.TaichiLoweringError, match="2-vectors stores 2"):
        tc.lower_source_kernel(text, "bad", {})


def shading_numpy(t, m, W=480, H=400):
    """examples/shading.py's draw(t) restated in numpy f32 (Taichi's definitions of the
    taichi.math functions: normalized = v * (1 / |v|), mix = x (1 - a) + y a, ...)."""
    x, y = grid(W, H)
    p0 = (x / f32(W) + f32(-0.5)) * f32(2.0)
    p1 = (y / f32(H) + f32(-0.5)) * f32(2.0)

    def norm3(a, b, c):
        inv = f32(1.0) / np.sqrt((a * a + b * b) + c * c)
        return a * inv, b * inv, c * inv

    l0, l1, l2 = norm3(f32(0.3), f32(0.5), f32(1.0))
    n0, n1, n2 = norm3(p0, p1, np.ones_like(p0))
    sh = np.minimum(np.maximum((n0 * l0 + n1 * l1) + n2 * l2, f32(0.0)), f32(1.0))
    fx = p0 * f32(3.0) + f32(t)
    length = np.sqrt(p0 * p0 + p1 * p1)
    tt = np.minimum(np.maximum((length - f32(0.2)) / (f32(0.8) - f32(0.2)), f32(0.0)), f32(1.0))
    base = [fx - np.floor(fx), (tt * tt) * (f32(3.0) - f32(2.0) * tt), np.where(p1 < f32(0.0), f32(0.0), f32(1.0))]
    sign = np.where(f32(0.0) < p0, f32(1.0), np.where(p0 < f32(0.0), f32(-1.0), f32(0.0)))
    acc = [base[k] * sh + (sign * f32(0.1)) * f32(k) for k in range(3)]
    cz = [acc[1] * f32(1.0) - acc[2] * f32(0.0), acc[2] * f32(0.0) - acc[0] * f32(1.0), acc[0] * f32(0.0) - acc[1] * f32(0.0)]
    return np.stack([(acc[k] * (f32(1.0) - f32(0.25)) + cz[k] * f32(0.25)) * m for k in range(3)], -1)


def test_math_functions_ndrange_and_static_loops():
    text = ex("shading.py")
    low = tc.lower_source_kernel(text, "draw", {"t": 0.25})
    assert low.kind == "pixel_program" and low.field.width == 3 and [f.width for f in low.inputs] == [1]
    m = np.random.default_rng(3).random((480, 400), dtype=np.float32)
    got = oracle.pixel_program(low.program, 480, 400, [m])
    assert np.array_equal(got, shading_numpy(0.25, m))
    mk = oracle.pixel_program(tc.lower_source_kernel(text, "make_mask", {}).program, 480, 400)
    assert set(np.unique(mk)) == {0.5, 1.0}


def life_numpy(a):
    c = sum(np.roll(np.roll(a, -di, 0), -dj, 1) for di in (-1, 0, 1) for dj in (-1, 0, 1) if (di, dj) != (0, 0))
    return ((c == 3) | ((a == 1) & (c == 2))).astype(np.int32)


def test_life_example_int_fields_and_neighbour_reads():
    text = ex("life.py")
    seed = tc.lower_source_kernel(text, "seed", {})
    assert seed.kind == "pixel_program" and seed.program.out_kind == pp.OUT_I32
    st = oracle.pixel_program(seed.program, 320, 320)
    i, j = np.meshgrid(np.arange(320), np.arange(320), indexing="ij")
    assert np.array_equal(st, ((i * 37 + j * 91 + i * j) % 7 < 2).astype(np.int32))
    step = tc.lower_source_kernel(text, "step", {})
    assert [(f.dtype, f.width) for f in step.inputs] == [("i32", 1)]
    for _ in range(3):
        nx = oracle.pixel_program(step.program, 320, 320, [st])
        assert np.array_equal(nx, life_numpy(st))
        st = nx
    back = tc.lower_source_kernel(text, "copy_back", {})
    assert np.array_equal(oracle.pixel_program(back.program, 320, 320, [st]), st)


def test_heat_example_clamped_stencil():
    text = ex("heat.py")
    u = oracle.pixel_program(tc.lower_source_kernel(text, "init", {}).program, 384, 256)
    prog = tc.lower_source_kernel(text, "diffuse", {"k": 0.2}).program
    for _ in range(3):
        v = oracle.pixel_program(prog, 384, 256, [u])
        up = np.concatenate([u[:1], u[:-1]], 0)
        dn = np.concatenate([u[1:], u[-1:]], 0)
        lf = np.concatenate([u[:, :1], u[:, :-1]], 1)
        rt = np.concatenate([u[:, 1:], u[:, -1:]], 1)
        assert np.array_equal(v, u + f32(0.2) * ((((up + dn) + lf) + rt) - f32(4.0) * u))
        u = v


def test_gather_clamps_and_int_store_truncates():
    """LOAD_AT clamps its indices to the field (NaN and negatives to 0, past the end to the last
    row / column); an int32 field store truncates toward zero, NaN gives 0, large values
    saturate."""
    b = pp.Builder()
    vals = b.load(0)
    rowi = b.op("sub", b.op("mul", b.index(0), 3.0), 5.0)  # 3i - 5: below 0 and past the end
    colv = b.load(1)                                       # arbitrary per-pixel values
    prog = pp.compile_program(b, out=b.load_at(0, rowi, colv), in_widths=[1, 1])
    rng = np.random.default_rng(6)
    src = rng.standard_normal((9, 7)).astype(np.float32)
    cols = np.array(rng.choice([-3.0, 0.0, 2.5, 6.9, 7.0, 100.0, np.nan, 1e30], size=(9, 7)), np.float32)
    got = oracle.pixel_program(prog, 9, 7, [src, cols])

    def index(x, n):
        return 0 if not x >= 0 else min(int(min(x, 2.0 ** 30)), n - 1)

    want = np.array([[src[index(3 * i - 5.0, 9), index(cols[i, j], 7)] for j in range(7)] for i in range(9)], np.float32)
    assert np.array_equal(got, want)
    b = pp.Builder()
    prog = pp.compile_program(b, out=b.load(0), out_i32=True)
    x = np.array([[2.7, -2.7, 0.5, -0.5, np.nan, 3e9, -3e9, 2147483520.0, -2147483648.0]], np.float32)
    got = oracle.pixel_program(prog, 1, 9, [x])
    assert got.dtype == np.int32
    assert got.tolist() == [[2, -2, 0, 0, 0, 2147483647, -2147483648, 2147483520, -2147483648]]


def test_integer_index_arithmetic_within_2_24_is_exact():
    """(i * j) % 7, (i * 3 - j) // 5 and -(i + j) % 4 on a 1021 x 1023 grid: every intermediate stays
    below 2^24 in magnitude, so the f32 program gives Taichi's int32 values exactly (numpy int64)."""
    body = "        f[i, j] = (i * j) % 7 + ((i * 3 - j) // 5) * 10.0 + (-(i + j) % 4) * 1000.0"
    low = tc.lower_source_kernel(body_kernel(body, shape=(1021, 1023)), "k", {})
    got = oracle.pixel_program(low.program, 1021, 1023)
    i = np.arange(1021, dtype=np.int64)[:, None]
    j = np.arange(1023, dtype=np.int64)[None, :]
    ref = ((i * j) % 7 + ((i * 3 - j) // 5) * 10 + (-(i + j) % 4) * 1000).astype(np.float32)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("body", ["        f[i, j] = (i * j) % 7",
                                  "        f[i, j] = (i * j * 3) // 11 + 0.5",
                                  "        k = i * j\n        f[i, j] = k * 2.0"])
def test_integer_index_arithmetic_beyond_2_24_is_refused(body):
    """On an 8192 x 8192 grid i * j reaches 67,092,481 > 2^24: f32 registers cannot hold it exactly
    while Taichi computes it in int32, so lowering refuses instead of giving other values.  The
    check is on every integer intermediate, so it also refuses a product that is only used as a
    float afterwards (k * 2.0, where the two would round alike)."""
    with pytest.raises(tc.TaichiLoweringError, match="2\\^24"):
        tc.lower_source_kernel(body_kernel(body, shape=(8192, 8192)), "k", {})


def lower_named(text, kernel, args):
    """(the lowered kernel, {id(field): its module-level name})."""
    kern, funcs, env = tc._parse_source(text, kernel, args)
    low = tc.lower_kernel(kern, tc._FuncResolver(env, funcs), env)
    return low, {id(v): k for k, v in env.items() if isinstance(v, tc.Field)}


def run_ops(low, names, arrays):
    """Runs a lowered kernel's programs in order on the oracle over {field name: array}, as the
    device runs them (each program reads the fields as the programs before it left them; a
    snapshot copy is named after its field with a trailing ', a field the lowering made between
    the parts of a body is named hidden<n>).  1-D fields run as one row.  A field scatter-added
    into is updated in its array (which must be float32 / int32 and C-contiguous)."""
    for op in low.ops():
        if op.kind == "copy":
            names[id(op.field)] = names[id(op.inputs[0])] + "'"
            arrays[names[id(op.field)]] = arrays[names[id(op.inputs[0])]].copy()
            continue
        ni, nj = op.grid

        def as_input(k, f):  # an input of the loop's shape in the grid, one of its own in its own grid
            a = arrays[names[id(f)]]
            p = op.program
            r, c = (p.in_rows[k], p.in_cols[k]) if p.in_rows[k] else (ni, nj)
            return a.reshape((r, c) + ((f.width,) if f.width > 1 else ()))  # a matrix field: its components flat
        out = oracle.pixel_program(op.program, ni, nj, [as_input(k, f) for k, f in enumerate(op.inputs)])
        if op.field is None:  # scatter-adds only
            continue
        shape = op.field.shape
        names.setdefault(id(op.field), f"hidden{len(names)}")  # a field the lowering made (between parts)
        if op.field.mat:
            out = out.reshape(out.shape[:2] + op.field.mat)
        arrays[names[id(op.field)]] = out.reshape(tuple(shape) + out.shape[2:])
    return arrays


def two_fields(body, extra_fields=("c",)):
    decl = "".join(f"{nm} = ti.field(dtype=float, shape=(24, 40))\n" for nm in ("a", "b") + tuple(extra_fields))
    return "import taichi as ti\n" + decl + "@ti.kernel\ndef k():\n    for i, j in a:\n" + body + "\n"


def test_two_stored_fields_and_reading_one_back_at_the_pixel():
    low, names = lower_named(two_fields("        a[i, j] = i * 0.5 - j\n        b[i, j] = a[i, j] * a[i, j] + 1.0"), "k", {})
    assert low.kind == "sequence" and [names[id(o.field)] for o in low.ops()] == ["a", "b"]
    assert all(o.reads == [] for o in low.ops())  # b's part recomputes a's value, it does not load it
    out = run_ops(low, names, {"a": None, "b": None})
    i, j = grid(24, 40)
    a = i * f32(0.5) - j
    assert np.array_equal(out["a"], a) and np.array_equal(out["b"], a * a + f32(1.0))


def test_a_field_loaded_before_its_store_is_read_by_the_other_part_first():
    """b reads a's value from before the loop, so b's program must run before a's; c is only read."""
    body = ("        b[i, j] = a[i, j] * 2.0 + c[(i + 1) % 24, j]\n"
            "        a[i, j] = a[i, j] + 1.0")
    low, names = lower_named(two_fields(body), "k", {})
    assert [names[id(o.field)] for o in low.ops()] == ["b", "a"]
    rng = np.random.default_rng(12)
    a0, c = (rng.standard_normal((24, 40)).astype(np.float32) for _ in range(2))
    out = run_ops(low, names, {"a": a0.copy(), "b": np.zeros((24, 40), np.float32), "c": c})
    assert np.array_equal(out["b"], a0 * f32(2.0) + np.roll(c, -1, 0))
    assert np.array_equal(out["a"], a0 + f32(1.0))


def test_in_place_updates_of_two_fields_need_no_order():
    """Each part evaluates the whole body; a load only dead code reads is no dependency."""
    body = ("        p = a[i, j]\n        q = b[i, j]\n"
            "        a[i, j] = p * 2.0\n        b[i, j] = q * 3.0 + p")
    low, names = lower_named(two_fields(body, ()), "k", {})
    assert [names[id(o.field)] for o in low.ops()] == ["b", "a"]  # b reads a: b first
    assert [[names[id(f)] for f in o.reads] for o in low.ops()] == [["a", "b"], ["a"]]
    rng = np.random.default_rng(13)
    a0, b0 = (rng.standard_normal((24, 40)).astype(np.float32) for _ in range(2))
    out = run_ops(low, names, {"a": a0.copy(), "b": b0.copy()})
    assert np.array_equal(out["a"], a0 * f32(2.0)) and np.array_equal(out["b"], b0 * f32(3.0) + a0)


def test_fields_that_load_each_other_are_read_from_a_snapshot():
    """a, b = b, a through a temporary: each program loads the field the other stores, so one of
    them is first copied to a snapshot, which the other program loads."""
    body = "        t = a[i, j]\n        a[i, j] = b[i, j]\n        b[i, j] = t"
    low, names = lower_named(two_fields(body, ()), "k", {})
    kinds = [op.kind for op in low.ops()]
    assert kinds == ["copy", "pixel_program", "pixel_program"]
    rng_ = np.random.default_rng(14)
    a0, b0 = (rng_.standard_normal((24, 40)).astype(np.float32) for _ in range(2))
    out = run_ops(low, names, {"a": a0.copy(), "b": b0.copy()})
    assert np.array_equal(out["a"], b0) and np.array_equal(out["b"], a0)


def gray_scott_numpy(u, v, dt, Du=0.16, Dv=0.08, feed=0.035, kill=0.065):
    """examples/reaction.py's step(dt) restated in numpy f32, operations in the program's order."""
    def lap(x):
        return (((np.roll(x, -1, 0) + np.roll(x, 1, 0)) + np.roll(x, -1, 1)) + np.roll(x, 1, 1)) - f32(4.0) * x
    r = (u * v) * v
    nu = u + f32(dt) * ((f32(Du) * lap(u) - r) + f32(feed) * (f32(1.0) - u))
    nv = v + f32(dt) * ((f32(Dv) * lap(v) + r) - (f32(feed) + f32(kill)) * v)
    return nu, nv


def test_reaction_example_two_struct_fors_and_two_stores_per_loop():
    text = ex("reaction.py")
    seed, names = lower_named(text, "seed", {})
    assert seed.kind == "sequence" and len(seed.ops()) == 2
    f = run_ops(seed, names, {})
    i, j = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    inside = (np.abs(i - 128) < 12) & (np.abs(j - 128) < 12)
    assert np.array_equal(f["u"], np.where(inside, f32(0.5), f32(1.0)))
    assert np.array_equal(f["v"], np.where(inside, f32(0.25) + f32(0.01) * ((i * 7 + j * 3) % 5).astype(np.float32), f32(0)))
    step, names = lower_named(text, "step", {"dt": 1.0})
    assert [p.kind for p in step.parts] == ["sequence", "sequence"]
    assert [names[id(o.field)] for o in step.ops()] == ["nu", "nv", "u", "v"]
    f = {nm: f[nm] if nm in f else np.zeros((256, 256), np.float32) for nm in ("u", "v", "nu", "nv")}
    u, v = f["u"], f["v"]
    for _ in range(3):
        f = run_ops(step, names, f)
        u, v = gray_scott_numpy(u, v, 1.0)
        assert np.array_equal(f["u"], u) and np.array_equal(f["v"], v)
        assert np.array_equal(f["nu"], u) and np.array_equal(f["nv"], v)


ONE_D = '''import taichi as ti
N = 1000
x = ti.field(dtype=float, shape=N)
y = ti.field(dtype=float, shape=N)
p = ti.Vector.field(2, dtype=float, shape=N)

@ti.kernel
def fill():
    for i in x:
        x[i] = i * 0.5 - 7.0

@ti.kernel
def smooth():
    for i in y:
        y[i] = (x[(i + 1) % N] + x[(i + N - 1) % N]) * 0.5 + x[ti.min(i + 3, N - 1)]

@ti.kernel
def pairs():
    for k in range(N):
        p[k] = [k * 0.25, x[k] * x[k]]

@ti.kernel
def bump():
    for i in ti.ndrange(N):
        x[i] += 1.5
        x[i] *= 2.0
'''


def test_one_d_struct_fors_gathers_range_and_augmented_stores():
    low, names = lower_named(ONE_D, "fill", {})
    f = run_ops(low, names, {})
    i = np.arange(1000, dtype=np.float32)
    x = i * f32(0.5) - f32(7.0)
    assert np.array_equal(f["x"], x)
    low, names = lower_named(ONE_D, "smooth", {})
    assert [fl.shape for fl in low.inputs] == [(1000,)]
    f = run_ops(low, names, {"x": x})
    assert np.array_equal(f["y"], (np.roll(x, -1) + np.roll(x, 1)) * f32(0.5) + x[np.minimum(np.arange(1000) + 3, 999)])
    low, names = lower_named(ONE_D, "pairs", {})
    f = run_ops(low, names, {"x": x})
    assert f["p"].shape == (1000, 2) and np.array_equal(f["p"], np.stack([i * f32(0.25), x * x], -1))
    low, names = lower_named(ONE_D, "bump", {})
    f = run_ops(low, names, {"x": x})
    assert np.array_equal(f["x"], (x + f32(1.5)) * f32(2.0))


@pytest.mark.parametrize("kernel,msg", [
    ("    for i in x:\n        x[i, 0] = 1.0", "indexed with 2 indices"),
    ("    for i, j in ti.ndrange(N):\n        x[i] = 1.0", "2 integer extent"),
    ("    for i in range(N, 2, 1):\n        x[i] = 1.0", "extent"),
    ("    for i in x:\n        x[i + 1] = 1.0\n        x[i] = 2.0", "both stored"),
])
def test_one_d_errors(kernel, msg):
    text = "import taichi as ti\nN = 8\nx = ti.field(dtype=float, shape=N)\n@ti.kernel\ndef k():\n" + kernel + "\n"
    with pytest.raises(tc.TaichiLoweringError, match=msg):
        tc.lower_source_kernel(text, "k", {})


def particles_numpy(x, v, age, steps, g=-9.8, dt=0.002, damping=0.8):
    """examples/particles.py's step() restated in numpy f32, operations in the program's order."""
    x, v, age = x.copy(), v.copy(), age.copy()
    gdt = f32(g) * f32(dt)
    for _ in range(steps):
        vel = v.copy()
        vel[:, 1] = vel[:, 1] + gdt
        pos = x + vel * f32(dt)
        lo = pos[:, 1] < 0
        pos[lo, 1] = -pos[lo, 1]
        vel[lo, 1] = (-vel[lo, 1]) * f32(damping)
        side = (pos[:, 0] < 0) | (pos[:, 0] > 1)
        pos[side, 0] = np.minimum(np.maximum(pos[side, 0], f32(0)), f32(1))
        vel[side, 0] = (-vel[side, 0]) * f32(damping)
        x, v = pos, vel
        age = age + f32(dt)
    return x, v, age


def particles_seed(n=16384):
    i = np.arange(n)
    x = np.stack([((i * 37 % 1009).astype(np.float32) / f32(1009.0)),
                  f32(0.5) + (i * 59 % 997).astype(np.float32) / f32(1994.0)], -1)
    v = np.stack([((i * 13 % 17) - 8).astype(np.float32) * f32(0.25), np.zeros(n, np.float32)], -1)
    return x, v


def test_particles_example_one_d_vector_fields_and_snapshot():
    text = ex("particles.py")
    seed, names = lower_named(text, "seed", {})
    f = run_ops(seed, names, {})
    x0, v0 = particles_seed()
    assert np.array_equal(f["x"], x0) and np.array_equal(f["v"], v0)
    step, names = lower_named(text, "step", {})
    assert [op.kind for op in step.ops()] == ["copy", "pixel_program", "pixel_program", "pixel_program"]
    f["age"] = np.zeros(16384, np.float32)
    for _ in range(30):
        f = run_ops(step, names, f)
    x, v, age = particles_numpy(x0, v0, np.zeros(16384, np.float32), 30)
    assert np.array_equal(f["x"], x) and np.array_equal(f["v"], v) and np.array_equal(f["age"], age)
    assert (v0[:, 1] != v[:, 1]).all()


ROW_LOOPS = '''import taichi as ti
W, H = 37, 300
u = ti.field(dtype=float, shape=(W, H))
s = ti.field(dtype=float, shape=(W, H))
c = ti.field(dtype=ti.i32, shape=(W, H))

@ti.kernel
def prefix():
    for i, j in s:
        acc = 0.0
        for k in range(H):
            acc += ti.select(k <= j, u[i, k], 0.0)
        s[i, j] = acc

@ti.kernel
def window(r: int):
    for i, j in s:
        acc = 0.0
        for k in range(-40, 41):
            acc += u[i, ti.min(ti.max(j + k, 0), H - 1)] * (1.0 if abs(k) <= r else 0.0)
        s[i, j] = acc

@ti.kernel
def search():
    for i, j in c:
        k = 0
        while k < H and u[i, (j + k) % H] < 0.97:
            k += 1
        c[i, j] = k
'''


def test_loop_index_read_in_the_body_and_the_test():
    """The variable of a runtime `for k in range(...)` and the counter of a while loop are the
    loop's trip: prefix sums by a 300-trip loop, a window by range(-40, 41), a search whose test
    reads the counter (check-then-update: the count is the first k that fails)."""
    g = np.random.default_rng(15).random((37, 300)).astype(np.float32)
    low, names = lower_named(ROW_LOOPS, "prefix", {})
    assert low.program.loop and low.program.max_iter == 300
    f = run_ops(low, names, {"u": g})
    ref = np.zeros_like(g)
    acc = np.zeros(37, np.float32)
    for j in range(300):  # the same f32 additions in the same order: acc_j = u[:, 0] + ... + u[:, j]
        acc = acc + g[:, j]
        ref[:, j] = acc
    # each pixel adds u[i, k] for k <= j, then zeros: its sum is the running sum to j, plus +0s
    assert np.array_equal(f["s"], ref)
    low, names = lower_named(ROW_LOOPS, "window", {"r": 5})
    f = run_ops(low, names, {"u": g})
    ref = np.zeros_like(g)
    for k in range(-40, 41):
        ref = ref + g[:, np.clip(np.arange(300) + k, 0, 299)] * (f32(1.0) if abs(k) <= 5 else f32(0.0))
    assert np.array_equal(f["s"], ref)
    low, names = lower_named(ROW_LOOPS, "search", {})
    f = run_ops(low, names, {"u": g})
    ref = np.full((37, 300), 300, np.int32)
    for i in range(37):
        for j in range(300):
            for k in range(300):
                if not g[i, (j + k) % 300] < f32(0.97):
                    ref[i, j] = k
                    break
    assert np.array_equal(f["c"], ref) and ref.min() == 0 and 0 < np.median(ref) < 300


def test_trip_is_refused_after_the_loop_and_in_initial_values():
    b = pp.Builder()
    with pytest.raises(pp.ProgramError, match="trip"):
        pp.compile_program(b, body={"x": b.op("add", b.state("x"), b.trip())}, init={"x": 0.0}, max_iter=4,
                           out=b.op("add", b.trip(), 1.0), loop=True)
    with pytest.raises(pp.ProgramError, match="trip"):
        pp.compile_program(b, init={"x": b.trip()}, body={"x": b.state("x")}, max_iter=4, out=b.state("x"), loop=True)


def nbody_forces_numpy(x, n, soft=0.001):
    """examples/nbody.py's forces() in numpy f32, the program's operations in its order:
    acc += d / (r2 sqrt(r2)), r2 = (d0 d0 + d1 d1) + soft, over j in order, then acc / N."""
    acc = np.zeros_like(x)
    for j in range(n):
        d = x[j] - x
        r2 = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + f32(soft)
        den = r2 * np.sqrt(r2)
        acc = acc + d / den[:, None]
    return acc / f32(n)


def test_nbody_example_loop_over_all_particles():
    text = ex("nbody.py").replace("N = 4096", "N = 512")
    seed, names = lower_named(text, "seed", {})
    f = run_ops(seed, names, {})
    forces, fn = lower_named(text, "forces", {})
    p = forces.program
    assert p.loop and p.max_iter == 512 and p.test == pp.TESTS["none"]
    advance, an = lower_named(text, "advance", {})
    x, v = f["x"], f["v"]
    for _ in range(3):
        f = run_ops(forces, fn, {"x": x})
        a = nbody_forces_numpy(x, 512)
        assert np.array_equal(f["a"], a)
        g = run_ops(advance, an, {"x": x, "v": v, "a": a})
        v = v + a * f32(0.0005)
        x = x + v * f32(0.0005)
        assert np.array_equal(g["v"], v) and np.array_equal(g["x"], x)


NESTS = '''import taichi as ti
W, H, R = 40, 56, 20
u = ti.field(dtype=float, shape=(W, H))
s = ti.field(dtype=float, shape=(W, H))

@ti.kernel
def count3():
    for i, j in s:
        x = 0.0
        for _ in range(3):
            for _ in range(2):
                x = x + 1.0
        s[i, j] = x

@ti.kernel
def window():
    for i, j in s:
        acc = 0.0
        for di in range(-R, R + 1):
            for dj in range(-R, R + 1):
                w = 1.0 / (1.0 + di * di + dj * dj)
                acc += w * u[ti.min(ti.max(i + di, 0), W - 1), ti.min(ti.max(j + dj, 0), H - 1)]
        s[i, j] = acc

@ti.kernel
def triple():
    for i, j in s:
        acc = 0.0
        for a in range(2, 5):
            for b in range(7):
                for c in range(-3, 2):
                    acc += a * 100.0 + b * 10.0 + c + u[i, j] * 0.0
        s[i, j] = acc
'''


def test_perfect_nests_of_range_loops_run_as_one_loop():
    """Nested range loops become one loop over the product of their extents, each variable
    recovered from the trip (innermost fastest, exact integer // and %): the counting nest, a
    41 x 41 window (too large to unroll) against numpy in the same order, a triple nest."""
    g = np.random.default_rng(18).random((40, 56)).astype(np.float32)
    low, names = lower_named(NESTS, "count3", {})
    assert low.program.max_iter == 6
    assert np.array_equal(run_ops(low, names, {"u": g})["s"], np.full((40, 56), 6.0, np.float32))
    low, names = lower_named(NESTS, "window", {})
    assert low.program.max_iter == 41 * 41
    got = run_ops(low, names, {"u": g})["s"]
    ref = np.zeros_like(g)
    ii, jj = np.meshgrid(np.arange(40), np.arange(56), indexing="ij")
    for di in range(-20, 21):
        for dj in range(-20, 21):
            w = f32(1.0) / ((f32(1.0) + f32(di * di)) + f32(dj * dj))
            ref = ref + w * g[np.clip(ii + di, 0, 39), np.clip(jj + dj, 0, 55)]
    assert np.array_equal(got, ref)
    low, names = lower_named(NESTS, "triple", {})
    got = run_ops(low, names, {"u": g})["s"]
    acc = f32(0)
    for a in range(2, 5):
        for b in range(7):
            for c in range(-3, 2):
                acc = acc + (((f32(a) * f32(100.0)) + f32(b) * f32(10.0)) + f32(c) + f32(0.0))
    assert np.array_equal(got, np.full((40, 56), acc, np.float32))


CACHED_F = tc.field(dtype=float, shape=(8, 8))
CACHED_SCALE = 2.0


@tc.kernel
def _cached_kernel(a: float):
    for i, j in CACHED_F:
        CACHED_F[i, j] = i * a + CACHED_SCALE


def test_kernel_lowerings_are_cached_per_argument_values():
    """A kernel is lowered once per argument tuple (the last 64 kept); module-level values are
    taken at that first lowering, as Taichi takes Python globals as compile-time constants."""
    global CACHED_SCALE
    k = _cached_kernel
    first = k.lower(1.5)
    assert k.lower(1.5) is first and k.lower(2.5) is not first
    assert k.lower(1) is k.lower(1.0)  # an int argument to a float parameter is coerced first
    CACHED_SCALE = 5.0
    try:
        assert k.lower(1.5) is first
        fresh = k.lower(3.5)
        got = oracle.pixel_program(fresh.program, 8, 8)
        i, _ = grid(8, 8)
        assert np.array_equal(got, i * f32(3.5) + f32(5.0))
    finally:
        CACHED_SCALE = 2.0
    for v in range(70):
        k.lower(float(v) + 0.25)
    assert len(k._cache) == tc.Kernel.CACHE_SIZE and k.lower(1.5) is not first


TWO_LOOPS = '''import taichi as ti
W, H = 48, 40
u = ti.field(dtype=float, shape=(W, H))
f = ti.field(dtype=float, shape=(W, H))
g = ti.Vector.field(2, dtype=float, shape=(W, H))

@ti.kernel
def march():
    for i, j in f:
        t = 0.0
        k = 0
        while k < 60 and t < i * 0.5 + u[i, j]:
            t += 0.75
            k += 1
        p = ti.Vector([t, k * 1.0])
        s = 0.0
        for m in range(j % 7 + 20):
            s += p[0] * 0.125 + m
        shade = 1.0
        n = 0
        while n < 30 and shade > 0.2 + u[i, j] * 0.1:
            shade *= 0.9
            n += 1
        f[i, j] = s + shade + k + n * 0.01
        g[i, j] = [p[1], s]
'''


def test_struct_for_with_three_runtime_loops():
    """Three runtime loops in one body run as three parts, each passing the values the next one
    reads (t, k, p, s) through hidden per-pixel fields; the stores at the end read all of them."""
    u = np.random.default_rng(20).random((48, 40)).astype(np.float32)
    low, names = lower_named(TWO_LOOPS, "march", {})
    assert low.kind == "sequence"
    f = run_ops(low, names, {"u": u})
    ref_f = np.zeros((48, 40), np.float32)
    ref_g = np.zeros((48, 40, 2), np.float32)
    for i in range(48):
        for j in range(40):
            t, k = f32(0), 0
            while k < 60 and t < f32(i) * f32(0.5) + u[i, j]:
                t, k = t + f32(0.75), k + 1
            p = (t, f32(k) * f32(1.0))
            s = f32(0)
            for m in range(j % 7 + 20):
                s = s + (p[0] * f32(0.125) + f32(m))
            shade, n = f32(1), 0
            while n < 30 and shade > f32(0.2) + u[i, j] * f32(0.1):
                shade, n = shade * f32(0.9), n + 1
            ref_f[i, j] = ((s + shade) + f32(k)) + f32(n) * f32(0.01)
            ref_g[i, j] = (p[1], s)
    assert np.array_equal(f["f"], ref_f) and np.array_equal(f["g"], ref_g)


def test_range_of_a_per_pixel_integer_and_its_errors():
    """range(N) with N an integer expression of the indices runs as a loop of at most N's bound
    trips with the test k < N; a float N is refused."""
    text = ("import taichi as ti\nf = ti.field(dtype=float, shape=(12, 9))\n@ti.kernel\ndef k():\n    for i, j in f:\n"
            "        s = 0.0\n        for m in range(i * 2 - j):\n            s += m * 0.5 + 1.0\n        f[i, j] = s\n"
            "@ti.kernel\ndef bad():\n    for i, j in f:\n        s = 0.0\n        for m in range(i * 0.5):\n"
            "            s += 1.0\n        f[i, j] = s\n")
    low = tc.lower_source_kernel(text, "k", {})
    assert low.program.max_iter == 11 * 2 + 8 and low.program.test == pp.TESTS["lt"]
    ref = np.zeros((12, 9), np.float32)
    for i in range(12):
        for j in range(9):
            s = f32(0)
            for m in range(i * 2 - j):
                s = s + (f32(m) * f32(0.5) + f32(1.0))
            ref[i, j] = s
    assert np.array_equal(oracle.pixel_program(low.program, 12, 9), ref)
    with pytest.raises(tc.TaichiLoweringError, match="range"):
        tc.lower_source_kernel(text, "bad", {})


BIG_BODY = ("import taichi as ti\nf = ti.field(dtype=float, shape=(20, 30))\n@ti.kernel\ndef k():\n    for i, j in f:\n"
            "        a = i * 0.5\n        b = j * 0.25\n" +
            "".join(f"        a = a * {1 + (k % 7) * 0.001:.3f} + b * {0.01 * (k % 5 + 1):.2f}\n"
                    f"        b = b - a * 0.0625\n" for k in range(60)) + "        f[i, j] = a + b\n")


def test_bodies_too_large_for_one_program_are_split():
    """A straight-line body of 120 dependent statements (about 240 instructions, beyond the 128 of
    one program) runs as several programs passing their state through hidden fields: the same
    values as one pass in numpy, operation for operation."""
    low, names = lower_named(BIG_BODY, "k", {})
    assert low.kind == "sequence" and len(low.ops()) >= 2
    got = run_ops(low, names, {})["f"]
    i, j = grid(20, 30)
    a, b = i * f32(0.5), j * f32(0.25)
    for k in range(60):
        a = a * f32(float(f"{1 + (k % 7) * 0.001:.3f}")) + b * f32(float(f"{0.01 * (k % 5 + 1):.2f}"))
        b = b - a * f32(0.0625)
    assert np.array_equal(got, a + b)


VOLUME = '''import taichi as ti
A, B, C = 12, 10, 36
u = ti.field(dtype=float, shape=(A, B, C))
v = ti.field(dtype=float, shape=(A, B, C))
g = ti.Vector.field(3, dtype=float, shape=(A, B, C))

@ti.kernel
def init():
    for i, j, k in u:
        u[i, j, k] = ((i * 7 + j * 3 + k) % 11) * 0.125

@ti.kernel
def diffuse(c: float):
    for i, j, k in v:
        s = (u[ti.max(i - 1, 0), j, k] + u[ti.min(i + 1, A - 1), j, k] + u[i, ti.max(j - 1, 0), k]
             + u[i, ti.min(j + 1, B - 1), k] + u[i, j, ti.max(k - 1, 0)] + u[i, j, ti.min(k + 1, C - 1)])
        v[i, j, k] = u[i, j, k] + c * (s - 6.0 * u[i, j, k])

@ti.kernel
def grad():
    for i, j, k in ti.ndrange(A, B, C):
        g[i, j, k] = [u[i + 1, j, k] - u[i, j, k], u[i, j + 1, k] - u[i, j, k], u[i, j, k + 1] - u[i, j, k]]
'''


def test_three_d_fields_stencils_and_gathers_past_an_axis():
    """3-D fields run as [A B][C] grids with i, j from the row by exact integer // and %: an init
    from the indices, a clamped seven-point stencil, and gathers one past the last index of each
    axis (clamped to that axis, not run into the next row)."""
    low, names = lower_named(VOLUME, "init", {})
    f = run_ops(low, names, {})
    i, j, k = np.meshgrid(np.arange(12), np.arange(10), np.arange(36), indexing="ij")
    u = (((i * 7 + j * 3 + k) % 11).astype(np.float32) * f32(0.125))
    assert f["u"].shape == (12, 10, 36) and np.array_equal(f["u"], u)
    low, names = lower_named(VOLUME, "diffuse", {"c": 0.1})
    f = run_ops(low, names, {"u": u})
    def sh(a, ax, d):
        idx = np.clip(np.arange(a.shape[ax]) + d, 0, a.shape[ax] - 1)
        return np.take(a, idx, axis=ax)
    s = ((((sh(u, 0, -1) + sh(u, 0, 1)) + sh(u, 1, -1)) + sh(u, 1, 1)) + sh(u, 2, -1)) + sh(u, 2, 1)
    assert np.array_equal(f["v"], u + f32(0.1) * (s - f32(6.0) * u))
    low, names = lower_named(VOLUME, "grad", {})
    f = run_ops(low, names, {"u": u})
    ref = np.stack([sh(u, 0, 1) - u, sh(u, 1, 1) - u, sh(u, 2, 1) - u], -1)
    assert f["g"].shape == (12, 10, 36, 3) and np.array_equal(f["g"], ref)


OTHER_SHAPES = '''import taichi as ti
W, H, N = 40, 30, 24
img = ti.field(dtype=float, shape=(W, H))
small = ti.field(dtype=float, shape=(W // 2, H // 3))
pos = ti.Vector.field(2, dtype=float, shape=N)
vol = ti.field(dtype=float, shape=(W, H, 5))

@ti.kernel
def blobs():
    for i, j in img:
        s = 0.0
        for k in range(N):
            d = pos[k] - ti.Vector([i * 1.0, j * 1.0])
            s += 20.0 / (d.dot(d) + 1.0)
        img[i, j] = ti.min(s, 1.0)

@ti.kernel
def upsample():
    for i, j in img:
        img[i, j] = small[i // 2, j // 3] + small[i // 2 + 1, j // 3] * 0.5

@ti.kernel
def project():
    for i, j in img:
        s = 0.0
        for k in range(5):
            s += vol[i, j, k] * (k + 1.0)
        img[i, j] = s + vol[i, j, 9]
'''


def test_fields_of_other_shapes_are_gathered_in_their_own_extents():
    """A 2-D struct-for reads a 1-D field of 2-vectors at the loop's trip, a smaller 2-D field
    (indices clamped to its own extents: i // 2 + 1 runs past its last row) and a 3-D field (its
    last index 9 clamped to 4): equal to numpy."""
    rng_ = np.random.default_rng(22)
    P = (rng_.random((24, 2)) * np.array([40, 30])).astype(np.float32)
    low, names = lower_named(OTHER_SHAPES, "blobs", {})
    assert [(low.program.in_rows[0], low.program.in_cols[0])] == [(1, 24)]
    got = run_ops(low, names, {"pos": P})["img"]
    i, j = grid(40, 30)
    s = np.zeros((40, 30), np.float32)
    for k in range(24):
        dx, dy = P[k, 0] - i * f32(1.0), P[k, 1] - j * f32(1.0)
        s = s + f32(20.0) / ((dx * dx + dy * dy) + f32(1.0))
    assert np.array_equal(got, np.minimum(s, f32(1.0)))
    sm = rng_.random((20, 10)).astype(np.float32)
    low, names = lower_named(OTHER_SHAPES, "upsample", {})
    got = run_ops(low, names, {"small": sm})["img"]
    ii, jj = np.meshgrid(np.arange(40), np.arange(30), indexing="ij")
    assert np.array_equal(got, sm[ii // 2, jj // 3] + sm[np.minimum(ii // 2 + 1, 19), jj // 3] * f32(0.5))
    v = rng_.random((40, 30, 5)).astype(np.float32)
    low, names = lower_named(OTHER_SHAPES, "project", {})
    got = run_ops(low, names, {"vol": v})["img"]
    ref = np.zeros((40, 30), np.float32)
    for k in range(5):
        ref = ref + v[:, :, k] * f32(k + 1.0)
    assert np.array_equal(got, ref + v[:, :, 4])


GROUPED = """import taichi as ti
a = ti.field(dtype=float, shape=(12, 9))
b = ti.Vector.field(2, dtype=float, shape=(12, 9))
c = ti.field(dtype=float, shape=20)
@ti.kernel
def k():
    for I in ti.grouped(a):
        a[I] = I[0] * 2.0 + I[1] + b[I].x
        b[I] = ti.Vector([I.x, a[I]])
    for I in ti.grouped(c):
        c[I] = I[0] * 0.5
"""


def test_grouped_struct_fors():
    """`for I in ti.grouped(F)`: I is the index vector, F[I] this pixel's element (a load at the
    pixel, not a gather), for 2-D and 1-D fields."""
    low, names = lower_named(GROUPED, "k", {})
    assert [names[id(o.field)] for o in low.ops()] == ["a", "b", "c"]
    assert all(ins.op != pp.OP["load_at"] for o in low.ops() for ins in o.program.code[:o.program.n_post])
    b0 = np.random.default_rng(1).random((12, 9, 2)).astype(np.float32)
    arr = {"a": np.zeros((12, 9), np.float32), "b": b0.copy(), "c": np.zeros(20, np.float32)}
    run_ops(low, names, arr)
    i, j = grid(12, 9)
    a = (i * f32(2.0) + j) + b0[:, :, 0]
    assert np.array_equal(arr["a"], a) and np.array_equal(arr["b"][:, :, 1], a) and np.array_equal(arr["b"][:, :, 0], i)
    assert np.array_equal(arr["c"], np.arange(20, dtype=np.float32) * f32(0.5))


JUMPS = """
import taichi as ti
ti.init(arch=ti.gpu)
u = ti.field(dtype=float, shape=(12, 20))
k = ti.field(dtype=ti.i32, shape=(12, 20))
out = ti.field(dtype=float, shape=(12, 20))
cnt = ti.field(dtype=ti.i32, shape=(12, 20))

@ti.kernel
def first_over():
    for i, j in out:
        s = 0.0
        for t in range(40):
            if s > u[i, j]:
                break
            s += 0.1
        out[i, j] = s

@ti.kernel
def skip_parity():
    for i, j in out:
        s = 0.0
        for t in range(9):
            if t % 2 == i % 2:
                continue
            s += t * u[i, j]
        out[i, j] = s

@ti.kernel
def escape_break():
    for i, j in cnt:
        x = u[i, j]
        n = 0
        while n < 30:
            x = x * x - 1.5
            if ti.abs(x) > 4.0:
                break
            n += 1
        cnt[i, j] = n

@ti.kernel
def own_trips():
    for i, j in out:
        s = 0.0
        for t in range((i * 7 + j) % 12):
            if t * 0.25 > u[i, j]:
                break
            elif t == 3:
                continue
            else:
                s += 1.0
            s *= 1.5
        out[i, j] = s
"""


def _jump_reference(kernel, u, kk):
    """The kernels above as plain Python loops, every value an f32 rounded where Taichi's is."""
    out = np.zeros(u.shape, np.float32)
    cnt = np.zeros(u.shape, np.int32)
    for i in range(u.shape[0]):
        for j in range(u.shape[1]):
            uv = u[i, j]
            s = f32(0.0)
            if kernel == "first_over":
                for _ in range(40):
                    if s > uv:
                        break
                    s = f32(s + f32(0.1))
            elif kernel == "skip_parity":
                for t in range(9):
                    if t % 2 == i % 2:
                        continue
                    s = f32(s + f32(f32(t) * uv))
            elif kernel == "escape_break":
                x, n = uv, 0
                while n < 30:
                    x = f32(f32(x * x) - f32(1.5))
                    if abs(x) > 4.0:
                        break
                    n += 1
                cnt[i, j] = n
            else:
                for t in range((i * 7 + j) % 12):
                    if f32(t) * f32(0.25) > uv:
                        break
                    elif t == 3:
                        continue
                    else:
                        s = f32(s + f32(1.0))
                    s = f32(s * f32(1.5))
            out[i, j] = s
    return cnt if kernel == "escape_break" else out


@pytest.mark.parametrize("kernel", ["first_over", "skip_parity", "escape_break", "own_trips"])
def test_break_and_continue_bit_exact(kernel):
    """break and continue in runtime loops (range loops, a while loop whose counter is read after
    it, a loop of a per-pixel trip count, break / continue in if / elif / else with statements
    after them): a break sets a flag the loop's test reads before the next trip, statements
    after a possible jump run only where none happened, and the while counter misses the
    increment of the trip that broke out.  Bit for bit against plain Python loops."""
    r = np.random.default_rng(3)
    u = r.uniform(-0.5, 2.5, (12, 20)).astype(np.float32)
    kk = r.integers(0, 12, (12, 20)).astype(np.int32)
    low, names = lower_named(JUMPS, kernel, {})
    arrays = {"u": u, "k": kk, "out": np.zeros((12, 20), np.float32), "cnt": np.zeros((12, 20), np.int32)}
    run_ops(low, names, arrays)
    got = arrays["cnt" if kernel == "escape_break" else "out"]
    want = _jump_reference(kernel, u, kk)
    assert np.array_equal(got, want), kernel
    assert len(np.unique(want)) > 3  # the jumps happen at different trips on different pixels


def test_continue_in_a_while_loop_is_refused():
    text = JUMPS.replace("            if ti.abs(x) > 4.0:\n                break", "            if ti.abs(x) > 4.0:\n                continue")
    with pytest.raises(tc.TaichiLoweringError, match="continue in a while loop"):
        tc.lower_source_kernel(text, "escape_break", {})


SMALL_MATH = """
import taichi as ti
import taichi.math as tm
ti.init(arch=ti.gpu)
u = ti.field(dtype=float, shape=(8, 16))
out = ti.Vector.field(3, dtype=float, shape=(8, 16))

@ti.kernel
def misc():
    for i, j in out:
        x = u[i, j]
        out[i, j] = [ti.rsqrt(x * x + 1.0), tm.mod(x, 0.3), 0.0]
        if ti.static(True):
            out[i, j].z = 2.0 * x
        if ti.static(False):
            out[i, j].z = 5.0
"""


def test_rsqrt_mod_and_static_conditions():
    """ti.rsqrt as 1 / sqrt (each exactly rounded), taichi.math.mod as x - y floor(x / y) (GLSL's
    mod: the sign of y), and `if ti.static(c)` decided when the kernel is lowered: bit for bit
    against numpy's f32 restatement."""
    low, names = lower_named(SMALL_MATH, "misc", {})
    u = np.random.default_rng(8).uniform(-2, 2, (8, 16)).astype(np.float32)
    arrays = {"u": u, "out": np.zeros((8, 16, 3), np.float32)}
    run_ops(low, names, arrays)
    got = arrays["out"]
    assert np.array_equal(got[..., 0], f32(1.0) / np.sqrt(u * u + f32(1.0)))
    y = f32(0.3)
    assert np.array_equal(got[..., 1], u - y * np.floor(u / y))
    assert np.array_equal(got[..., 2], f32(2.0) * u)
    assert (got[..., 1] >= 0).all()  # GLSL's mod takes the sign of the divisor


def test_bit_opcodes_against_numpy_int32():
    """band / bor / bxor / shl / shr: the registers converted to int32 as an int32 store converts
    them (toward zero, NaN -> 0, saturating), numpy's int32 operation (shift counts taken mod
    32, >> arithmetic), the result back to f32."""
    vals = np.array([0, 1, -1, 5, -6, 255, 256, -256, 1 << 23, -(1 << 23), 7.9, -7.9, np.nan, 3e9, -3e9, 31, 32, 33],
                    np.float32)
    n = len(vals)
    a = np.repeat(vals[:, None], n, axis=1)
    c = np.repeat(vals[None, :], n, axis=0)

    def to_i32(x):
        with np.errstate(invalid="ignore"):
            return np.where(np.isnan(x), 0, np.clip(np.trunc(x.astype(np.float64)), -2**31, 2**31 - 1)).astype(np.int32)
    ia, ic = to_i32(a), to_i32(c)
    sh = (ic & 31).astype(np.uint32)
    want = {"band": ia & ic, "bor": ia | ic, "bxor": ia ^ ic,
            "shl": (ia.astype(np.uint32) << sh).astype(np.int32), "shr": ia >> sh.astype(np.int32)}
    b = pp.Builder()
    la, lc = b.load(0), b.load(1)
    for name, w in want.items():
        got = oracle.pixel_program(pp.compile_program(b, out=b.op(name, la, lc)), n, n, [a, c])
        assert np.array_equal(got, w.astype(np.float32)), name


BITS = """
import taichi as ti
ti.init(arch=ti.gpu)
u = ti.field(dtype=float, shape=(24, 40))
out = ti.field(dtype=float, shape=(24, 40))

@ti.kernel
def bits():
    for i, j in out:
        h = (i * 40 + j) ^ ((i << 3) | (j >> 2))
        out[i, j] = float((i & 3) + (j | 1) + (i ^ j) + (i << 1) + (j >> 1) + ((i - 12) >> 1) + (h & 255))

@ti.kernel
def float_bits():
    for i, j in out:
        out[i, j] = float(int(u[i, j]) & 1)

@ti.kernel
def var_shift():
    for i, j in out:
        out[i, j] = float(1 << j)

@ti.kernel
def wide_shift():
    for i, j in out:
        out[i, j] = float((i * j) << 20)
"""


def test_taichi_bit_operators():
    """&, |, ^, << and >> of indices and integer arithmetic of them lower to the bit opcodes (>>
    arithmetic on negatives): equal to numpy's int32 restatement.  Operands of no known integer
    bound (a value from a float field), shifts by a per-pixel count, and results that may pass
    2^24 are refused."""
    low, names = lower_named(BITS, "bits", {})
    arrays = {"u": np.zeros((24, 40), np.float32), "out": np.zeros((24, 40), np.float32)}
    run_ops(low, names, arrays)
    i, j = np.meshgrid(np.arange(24, dtype=np.int32), np.arange(40, dtype=np.int32), indexing="ij")
    h = (i * 40 + j) ^ ((i << 3) | (j >> 2))
    want = (i & 3) + (j | 1) + (i ^ j) + (i << 1) + (j >> 1) + ((i - 12) >> 1) + (h & 255)
    assert np.array_equal(arrays["out"], want.astype(np.float32))
    for kern, msg in (("float_bits", "known bound"), ("var_shift", "known when"), ("wide_shift", "beyond 2\\^24")):
        with pytest.raises(tc.TaichiLoweringError, match=msg):
            tc.lower_source_kernel(BITS, kern, {})


SURFACE = """
import taichi as ti
import taichi.math as tm
ti.init(arch=ti.gpu)
vec3 = ti.types.vector(3, float)
u = ti.field(dtype=float, shape=(10, 14))
v3 = ti.Vector.field(3, dtype=float, shape=(10, 14))
out = ti.Vector.field(4, dtype=float, shape=(10, 14))

@ti.func
def bent(x):
    a = x + 1.0
    if a > 0.5:
        a = a * 2.0
    else:
        a -= 3.0
    return a

@ti.kernel
def surface():
    for i, j in out:
        p = vec3(u[i, j], 1.0, 2.0)
        q = v3[i, j]
        r = tm.reflect(q, tm.normalize(p))
        a = b = q.zy.norm_sqr() + q.bgr.x
        nan = 1.0 if tm.isnan(u[i, j] / u[i, j]) else 0.0
        out[i, j] = [bent(u[i, j]) + q.sum() + q.max() - q.min(), r.y + ti.f32(q.n),
                     a + b + float(ti.i32(u[i, j] * 4.0)), nan + float(~i)]
"""


def test_taichi_surface_additions_bit_exact():
    """@ti.func bodies with ifs before their final return, ti.types.vector constructors, swizzles
    of 2-3 components (xyzw and rgba) and .n, vector sum / max / min, taichi.math.reflect and
    isnan, ti.f32 / ti.i32 casts, chained assignment and ~ of an index: bit for bit against
    numpy's f32 restatement."""
    low, names = lower_named(SURFACE, "surface", {})
    r = np.random.default_rng(12)
    u = r.uniform(-2, 2, (10, 14)).astype(np.float32)
    u[2, 3] = 0.0  # 0 / 0: NaN
    v3 = r.uniform(-1, 1, (10, 14, 3)).astype(np.float32)
    arrays = {"u": u, "v3": v3, "out": np.zeros((10, 14, 4), np.float32)}
    run_ops(low, names, arrays)
    got = arrays["out"]
    i = np.arange(10)[:, None] * np.ones((1, 14), np.int64)
    qx, qy, qz = v3[..., 0], v3[..., 1], v3[..., 2]
    a1 = u + f32(1.0)
    bent = np.where(a1 > f32(0.5), a1 * f32(2.0), a1 - f32(3.0))
    s = (qx + qy) + qz
    mx, mn = np.maximum(np.maximum(qx, qy), qz), np.minimum(np.minimum(qx, qy), qz)
    want0 = ((bent + s) + mx) - mn
    # the reflection through normalize(p): within f32 rounding of x - 2 dot(n, x) n
    pl = np.sqrt((u * u + f32(1.0)) + f32(4.0))
    px, py, pz = u / pl, f32(1.0) / pl, f32(2.0) / pl
    assert np.allclose(got[..., 1], (qy - f32(2.0) * ((px * qx + py * qy) + pz * qz) * py) + f32(3.0), atol=1e-6)
    ab = (qz * qz + qy * qy) + qz
    with np.errstate(invalid="ignore"):
        nan = np.isnan(u / u).astype(np.float32)
    want2 = (ab + ab) + np.trunc(u * f32(4.0))
    assert np.array_equal(got[..., 0], want0)
    assert np.array_equal(got[..., 2], want2)
    assert np.array_equal(got[..., 3], nan + (-i - 1).astype(np.float32))
    assert got[2, 3, 3] == 1.0 - 3.0


ROUND_VALUES = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, -0.49999997, 8388609.0, 4194304.5, -0.3, -0.0,
                         0.0, 3.7, -3.7, 1e-40, np.inf, -np.inf, np.nan, 3.4e38], np.float32)


def round_half_away(x):
    """Nearest integer, halfway cases away from zero, computed in f64 (|x| + 0.5 is exact there)."""
    with np.errstate(invalid="ignore"):
        return np.copysign(np.floor(np.abs(x.astype(np.float64)) + 0.5), x).astype(np.float32)


def test_round_opcode_and_ti_round():
    """VDSL_PIX_ROUND (C's roundf: halfway cases away from zero, signed zeros kept) against an f64
    restatement on halfway cases, the largest float below 0.5, values past 2^23, infinities and
    NaN; ti.round lowers to it (Taichi's own rounding of halfway cases is parity unpinned: Taichi
    is not importable here)."""
    x = ROUND_VALUES[None]
    b = pp.Builder()
    got = oracle.pixel_program(pp.compile_program(b, out=b.op("round", b.load(0))), 1, x.shape[1], [x])
    want = round_half_away(x)
    assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
    assert np.array_equal(np.isnan(got), np.isnan(want))
    text = SMALL_MATH.replace("out[i, j] = [ti.rsqrt(x * x + 1.0), tm.mod(x, 0.3), 0.0]",
                              "out[i, j] = [ti.round(x * 2.0), tm.round(x), 0.0]")
    low, names = lower_named(text, "misc", {})
    u = np.random.default_rng(8).uniform(-2, 2, (8, 16)).astype(np.float32)
    arrays = {"u": u, "out": np.zeros((8, 16, 3), np.float32)}
    run_ops(low, names, arrays)
    assert np.array_equal(arrays["out"][..., 0], round_half_away(u * f32(2.0)))
    assert np.array_equal(arrays["out"][..., 1], round_half_away(u))
