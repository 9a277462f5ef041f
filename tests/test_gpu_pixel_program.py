"""vdsl_op_pixel_program on the GPU against the CPU oracle (oracle.pixel_program): bit for bit for
programs of exactly rounded operations (+ - * / abs min max sqrt, moves, indices, loads, the
loop count), within stated bounds for the transcendentals (the device's sin/cos/log against the
C library's, exp and tanh from the map chains' own approximations).  Edge cases: grids that are
not whole 16x16 blocks, empty grids, loops of zero trips, loops without a test, four input
fields, the count read after the loop, invalid programs, graph recording."""
import contextlib
import io
import json
import os

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, pixprog as pp, run, taichi_compat as tc
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
REL = 1e-5  # the map chains' bound for their exp / tanh / sigmoid / log
EX = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vernondsl_amd", "examples")


def run_prog(dev, q, prog, inputs, ni, nj):
    ts = [Tensor.from_numpy(dev, q, np.ascontiguousarray(a, np.int32 if prog.in_dtypes[k] == pp.I32 else np.float32))
          for k, a in enumerate(inputs)]
    int_out = prog.out_kind in (pp.OUT_COUNT, pp.OUT_I32)
    w = 1 if int_out else prog.out_width
    out = Tensor(dev, (ni, nj) if w == 1 else (ni, nj, w), "i32" if int_out else "f32")
    if ni and nj:
        out.buffer.fill_u32(q, 0x7FC00000)  # NaN / a large count: every element must be written
    kernels.pixel_program(q, prog, ts, out)
    got = out.numpy(q)
    for t in ts + [out]:
        t.free()
    return got


def escape_program(c_re=-0.8, c_im=0.156, limit=200, scale=3.0, test="lt"):
    """Julia set as a plain program: z0 from the pixel, z <- z^2 + c while |z|^2 < 4."""
    b = pp.Builder()
    x0 = b.op("add", b.op("mul", b.op("div", b.index(0), 37.0), scale), -1.5)
    y0 = b.op("add", b.op("mul", b.op("div", b.index(1), 53.0), scale), -1.5)
    x, y = b.state("x"), b.state("y")
    r2 = b.op("add", b.op("mul", x, x), b.op("mul", y, y))
    return pp.compile_program(
        b, init={"x": x0, "y": y0}, test=(test, r2, 4.0),
        body={"x": b.op("add", b.op("sub", b.op("mul", x, x), b.op("mul", y, y)), c_re),
              "y": b.op("add", b.op("mul", b.op("mul", x, y), 2.0), c_im)},
        max_iter=limit, out=pp.COUNT)


@pytest.mark.parametrize("ni,nj", [(37, 53), (1, 1), (16, 16), (17, 15), (300, 129), (1024, 1024)])
def test_escape_program_counts_bit_exact(dev, q, ni, nj):
    prog = escape_program()
    got = run_prog(dev, q, prog, [], ni, nj)
    ref = oracle.pixel_program(prog, ni, nj)
    assert np.array_equal(got, ref)


def state_program(limit):
    """Mandelbrot whose stored value reads the loop state after the loop (|z|^2 + count / 1000):
    lanes keep the state of the trip they left the loop at."""
    b = pp.Builder()
    cx = b.op("add", b.op("mul", b.op("div", b.index(0), 300.0), 3.0), -2.0)
    cy = b.op("add", b.op("mul", b.op("div", b.index(1), 129.0), 3.0), -1.5)
    x, y = b.state("x"), b.state("y")
    r2 = b.op("add", b.op("mul", x, x), b.op("mul", y, y))
    return pp.compile_program(
        b, init={"x": 0.0, "y": 0.0}, test=("le", r2, 4.0),
        body={"x": b.op("add", b.op("sub", b.op("mul", x, x), b.op("mul", y, y)), cx),
              "y": b.op("add", b.op("mul", b.op("mul", x, y), 2.0), cy)},
        max_iter=limit, out=b.op("add", r2, b.op("mul", b.count(), 0.001)))


@pytest.mark.parametrize("limit", [0, 5, 16, 77, 256])
def test_state_read_after_the_loop_bit_exact(dev, q, limit):
    prog = state_program(limit)
    got = run_prog(dev, q, prog, [], 300, 129)
    assert np.array_equal(got, oracle.pixel_program(prog, 300, 129))


@pytest.mark.parametrize("limit", [3, 40, 256])
def test_test_section_value_read_after_the_loop(dev, q, limit):
    """A program (built by hand: the compiler recomputes instead) that stores a register the test
    section writes (and the body reuses as a temporary): a lane whose test failed stores the
    value of that test, one that made max_iter trips what its last body trip left there."""
    prog = escape_program(limit=limit)
    ts = prog.n_pre
    assert prog.n_test == 3 and prog.code[ts + 2].dst == prog.test_a
    prog.n_post, prog.out_kind, prog.out_width, prog.out_regs[0] = 0, pp.OUT_REG, 1, prog.test_a
    got = run_prog(dev, q, prog, [], 300, 129)
    ref = oracle.pixel_program(prog, 300, 129)
    assert np.array_equal(got, ref)
    assert np.any(ref > 4.0) and np.any(ref < 4.0)


def test_empty_grid_writes_nothing(dev, q):
    prog = escape_program()
    for ni, nj in [(0, 5), (5, 0), (0, 0)]:
        out = Tensor(dev, (max(ni, 1), max(nj, 1)), "i32")
        out.buffer.fill_u32(q, 7)
        _lib.call("vdsl_op_pixel_program", q.handle, ni, nj, __import__("ctypes").byref(prog), None, 0, out.handle)
        q.sync()
        assert np.all(out.numpy(q) == 7)
        out.free()


def logistic_program(steps, with_count_in_post):
    """A loop without a test (fixed trip count) over a state read from an input field; the post
    section reads the count."""
    b = pp.Builder()
    r = b.op("add", b.op("mul", b.op("div", b.index(0), 64.0), 1.5), 2.5)
    x = b.state("x")
    out = x if not with_count_in_post else b.op("add", x, b.op("mul", b.count(), 0.25))
    return pp.compile_program(b, init={"x": b.op("add", b.op("mul", b.load(0), 0.5), 0.25)},
                              body={"x": b.op("mul", b.op("mul", r, x), b.op("sub", 1.0, x))},
                              max_iter=steps, out=out, loop=True)


@pytest.mark.parametrize("steps", [0, 1, 7, 300])
@pytest.mark.parametrize("post", [False, True])
def test_fixed_trip_loops_bit_exact(dev, q, steps, post):
    g = np.random.default_rng(steps).random((64, 200), dtype=np.float32)
    prog = logistic_program(steps, post)
    assert np.array_equal(run_prog(dev, q, prog, [g], 64, 200), oracle.pixel_program(prog, 64, 200, [g]))


def test_four_inputs_no_loop_bit_exact(dev, q):
    rng = np.random.default_rng(11)
    ins = [rng.standard_normal((77, 91)).astype(np.float32) for _ in range(4)]
    ins[3] = np.abs(ins[3]) + 0.5
    b = pp.Builder()
    l0, l1, l2, l3 = (b.load(k) for k in range(4))
    v = b.op("add", b.op("mul", l0, l1), b.op("div", l2, l3))
    v = b.op("max", b.op("min", v, b.op("sqrt", b.op("add", b.op("abs", l0), b.index(1)))), b.op("neg", b.index(0)))
    v = b.op("fma", v, l3, b.op("sub", l2, b.op("square", l1)))
    prog = pp.compile_program(b, out=v)
    assert not prog.loop
    assert np.array_equal(run_prog(dev, q, prog, ins, 77, 91), oracle.pixel_program(prog, 77, 91, ins))


def test_transcendentals_within_bounds(dev, q):
    ni, nj = 96, 160
    b = pp.Builder()
    t = b.op("add", b.op("mul", b.index(0), 0.37), b.op("mul", b.index(1), -0.21))  # about [-34, 35]
    progs = {
        "sin": b.op("sin", t), "cos": b.op("cos", t), "exp": b.op("exp", b.op("mul", t, 0.5)),
        "log": b.op("log", b.op("add", b.op("abs", t), 1e-3)), "tanh": b.op("tanh", b.op("mul", t, 0.1)),
        "sigmoid": b.op("sigmoid", t),
    }
    for name, node in progs.items():
        prog = pp.compile_program(b, out=node)
        got = run_prog(dev, q, prog, [], ni, nj).astype(np.float64)
        ref = oracle.pixel_program(prog, ni, nj).astype(np.float64)
        if name in ("sin", "cos"):  # values in [-1, 1]: absolute bound
            assert np.max(np.abs(got - ref)) <= 4e-7, name
        else:
            assert np.all(np.abs(got - ref) <= REL * np.abs(ref) + 1e-37), name


def test_inverse_trig_tan_atan2_pow_within_ulp_of_oracle(dev, q):
    """asin, acos, atan, tan, atan2 and powf from the device math library against the C library's
    (the oracle) over a domain crossing every branch (|x| > 1, signed zeros, infinities, NaN,
    tiny and huge values): within 4 ulp, NaN exactly where the oracle has NaN; and the kernel
    using them through the Taichi front end within a few f32 ulp of the oracle."""
    from test_taichi_general import MATH_DOMAIN, MATH_KERNELS, ulp_distance
    x = MATH_DOMAIN[None]
    b = pp.Builder()
    la, lc = b.load(0), b.load(1)
    worst = {}
    for name in ("asin", "acos", "atan", "tan"):
        prog = pp.compile_program(b, out=b.op(name, la))
        got = run_prog(dev, q, prog, [x, x], 1, x.shape[1])
        worst[name] = int(ulp_distance(got, oracle.pixel_program(prog, 1, x.shape[1], [x, x])).max())
    y = MATH_DOMAIN[::7]
    a = np.repeat(y[:, None], len(y), axis=1)
    c = np.repeat(y[None, :], len(y), axis=0)
    for name in ("atan2", "powf"):
        prog = pp.compile_program(b, out=b.op(name, la, lc))
        got = run_prog(dev, q, prog, [a, c], len(y), len(y))
        worst[name] = int(ulp_distance(got, oracle.pixel_program(prog, len(y), len(y), [a, c])).max())
    print("ulp against the oracle:", worst)
    assert max(worst.values()) <= 4, worst
    low = tc.lower_source_kernel(MATH_KERNELS, "polar", {})
    u = np.random.default_rng(5).uniform(-2, 2, (16, 32)).astype(np.float32)
    got = run_prog(dev, q, low.program, [u], 16, 32)
    assert np.allclose(got, oracle.pixel_program(low.program, 16, 32, [u]), rtol=2e-6, atol=1e-6)

def test_invalid_programs_rejected(dev, q):
    import ctypes
    out = Tensor(dev, (8, 8), "f32")
    good = logistic_program(3, False)

    def call(p, n_inputs=1, ins=None):
        ins = ins or [Tensor(dev, (8, 8), "f32") for _ in range(n_inputs)]
        hs = (ctypes.c_void_p * max(1, len(ins)))(*[t.handle for t in ins])
        try:
            with pytest.raises(_lib.VdslError) as ei:
                _lib.call("vdsl_op_pixel_program", q.handle, 8, 8, ctypes.byref(p), hs, n_inputs, out.handle)
        finally:
            for t in ins:
                t.free()
        return ei.value.message

    def mutate(**kw):
        p = pp.PixelProgram()
        ctypes.memmove(ctypes.byref(p), ctypes.byref(good), ctypes.sizeof(p))
        for k, v in kw.items():
            setattr(p, k, v)
        return p

    assert "LOAD" in call(good, n_inputs=0, ins=[])
    assert "at most 256" in call(mutate(n_post=252))
    assert "unknown test" in call(mutate(test=9))
    p = mutate()
    p.code[0].dst = 32  # registers are 0..31
    assert "register out of range" in call(p)
    p = mutate()
    p.code[0].op = 99
    assert "unknown opcode" in call(p)
    assert "count needs a loop" in call(mutate(loop=0, n_body=0, out_kind=1))
    assert "n_inputs" in call(good, n_inputs=9, ins=[Tensor(dev, (8, 8), "f32") for _ in range(9)])
    small = Tensor(dev, (4, 8), "f32")
    hs = (ctypes.c_void_p * 1)(small.handle)
    with pytest.raises(_lib.VdslError):
        _lib.call("vdsl_op_pixel_program", q.handle, 8, 8, ctypes.byref(good), hs, 1, out.handle)
    small.free()
    out.free()


def test_recording_needs_a_compiled_program(dev, q):
    """A program first seen while a graph records is refused (nothing is compiled during
    recording); one run eagerly before records, and its replays equal the eager run.  Programs
    differing only in immediates and max_iter share one compiled kernel (those stay arguments)."""
    ni, nj = 130, 70
    fresh = escape_program(test="le")  # a test no earlier program used: a new kernel
    out = Tensor(dev, (ni, nj), "i32")
    with pytest.raises(_lib.VdslError) as ei:
        with q.capture():
            kernels.pixel_program(q, fresh, [], out)
    assert ei.value.status == -6  # VDSL_ERR_CAPTURE
    kernels.pixel_program(q, fresh, [], out)
    eager = out.numpy(q)
    assert np.array_equal(eager, oracle.pixel_program(fresh, ni, nj))
    same_kernel = escape_program(c_re=-0.4, c_im=0.6, limit=77, test="le")
    with q.capture() as rec:
        kernels.pixel_program(q, fresh, [], out)
    with q.capture() as rec2:
        kernels.pixel_program(q, same_kernel, [], out)
    other = oracle.pixel_program(same_kernel, ni, nj)
    assert not np.array_equal(other, eager)
    for _ in range(3):
        out.buffer.fill_u32(q, 0xFFFFFFFF)
        rec.graph.launch(q)
        q.sync()
        assert np.array_equal(out.numpy(q), eager)
        out.buffer.fill_u32(q, 0xFFFFFFFF)
        rec2.graph.launch(q)
        q.sync()
        assert np.array_equal(out.numpy(q), other)
    rec.graph.destroy()
    rec2.graph.destroy()
    out.free()


def run_program(path, frames):
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        assert run.main([path, "--frames", str(frames)]) == 0
    return json.loads(buf.getvalue().strip().splitlines()[-1]), tc._state["last_gui"].last_image


def test_burning_ship_example_bit_exact(dev, q):
    path = os.path.join(EX, "burning_ship.py")
    res, img = run_program(path, 1)
    assert res["frames"] == 1 and img.shape == (1024, 1024) and img.dtype == np.int32
    low = tc.lower_source_kernel(open(path).read(), "ship", {"zoom": 3.2})
    assert low.kind == "pixel_program"
    assert np.array_equal(img, oracle.pixel_program(low.program, 1024, 1024))
    assert int(img.sum()) == 51_201_175


def test_interference_example_frames(dev, q):
    path = os.path.join(EX, "interference.py")
    res, img = run_program(path, 3)
    assert res["frames"] == 3 and img.shape == (768, 768) and img.dtype == np.float32
    text = open(path).read()
    mask = oracle.pixel_program(tc.lower_source_kernel(text, "make_mask", {}).program, 768, 768)
    low = tc.lower_source_kernel(text, "waves", {"phase": 1.0})  # the third frame: 0.0 + 0.5 + 0.5
    ref = oracle.pixel_program(low.program, 768, 768, [mask]).astype(np.float64)
    # the mask's exp (relative REL) and the two sines (4e-7 each), scaled by 0.25 * |amp| <= 0.5
    assert np.max(np.abs(img.astype(np.float64) - ref)) <= 0.5 * REL + 2e-7 + 1e-7


SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 2.5, -2.5, 1e-40, -1e-40, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan,
                     7.0, -7.25, 123456.75, -0.1], np.float32)


def test_compare_select_floor_opcodes_bit_exact(dev, q):
    n = len(SPECIALS)
    a = np.ascontiguousarray(np.repeat(SPECIALS[:, None], n, axis=1))
    c = np.ascontiguousarray(np.repeat(SPECIALS[None, :], n, axis=0))
    b = pp.Builder()
    la, lc = b.load(0), b.load(1)
    for node in (b.op("lt", la, lc), b.op("le", la, lc), b.op("eq", la, lc), b.op("ne", la, lc),
                 b.op("select", la, lc, b.op("neg", lc)), b.op("floor", la), b.op("trunc", la),
                 b.op("select", b.op("lt", la, lc), b.op("floor", lc), b.op("max", la, lc))):
        prog = pp.compile_program(b, out=node)
        got = run_prog(dev, q, prog, [a, c], n, n)
        ref = oracle.pixel_program(prog, n, n, [a, c])
        if "max" in pp.describe(prog):  # max / min: equal values (the sign of a zero result may differ)
            assert np.array_equal(got, ref, equal_nan=True), pp.describe(prog)
        else:
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), pp.describe(prog)


BOUNCE = '''
import taichi as ti
n = 40
f = ti.field(dtype=float, shape=(300, 129))

@ti.kernel
def k():
    for i, j in f:
        x = i / n
        y = j / n
        k = 0
        while k < 100 and x * x + y * y < 4.0 and abs(x - y) < 1.5:
            if x > y:
                x = x * x - y + 0.1
            else:
                x, y = y * 0.9, x * 1.1 - 0.3
            k += 1
        f[i, j] = k + x
'''


def test_compound_test_and_if_in_the_loop_bit_exact(dev, q):
    low = tc.lower_source_kernel(BOUNCE, "k", {})
    got = run_prog(dev, q, low.program, [], 300, 129)
    assert np.array_equal(got, oracle.pixel_program(low.program, 300, 129))


def test_tiles_example_frames_bit_exact(dev, q):
    path = os.path.join(EX, "tiles.py")
    res, img = run_program(path, 4)
    assert res["frames"] == 4 and img.shape == (640, 640) and img.dtype == np.float32
    text = open(path).read()
    fade = tc.lower_source_kernel(text, "fade", {}).program
    trail = np.zeros((640, 640), np.float32)  # fields start zeroed
    t = 0.0
    for _ in range(4):
        canvas = oracle.pixel_program(tc.lower_source_kernel(text, "paint", {"t": t}).program, 640, 640)
        trail = oracle.pixel_program(fade, 640, 640, [canvas, trail])
        t += 0.25
    assert np.array_equal(img, trail)
    assert len(np.unique(img)) > 4


def test_vector_inputs_and_outputs_bit_exact(dev, q):
    """Inputs of 2 and 3 components read by component, a vec4 output in chosen component order."""
    rng = np.random.default_rng(8)
    a = rng.standard_normal((45, 70, 2)).astype(np.float32)
    c3 = rng.standard_normal((45, 70, 3)).astype(np.float32)
    b = pp.Builder()
    x, y = b.load(0, 0), b.load(0, 1)
    r, g, bl = b.load(1, 0), b.load(1, 1), b.load(1, 2)
    outs = [b.op("add", y, bl), x, b.op("mul", r, g), b.op("select", b.op("lt", x, y), r, bl)]
    prog = pp.compile_program(b, out=outs, in_widths=[2, 3])
    assert prog.out_width == 4
    got = run_prog(dev, q, prog, [a, c3], 45, 70)
    assert got.shape == (45, 70, 4)
    ref = oracle.pixel_program(prog, 45, 70, [a, c3])
    assert np.array_equal(got, ref)
    assert np.array_equal(ref[..., 1], a[..., 0]) and np.array_equal(ref[..., 2], c3[..., 0] * c3[..., 1])


def test_palette_example_vector_fields(dev, q):
    path = os.path.join(EX, "palette.py")
    res, img = run_program(path, 2)
    assert res["frames"] == 2 and img.shape == (800, 600, 3) and img.dtype == np.float32
    text = open(path).read()
    rgb = oracle.pixel_program(tc.lower_source_kernel(text, "render", {"shift": 0.05}).program, 800, 600)
    ref = oracle.pixel_program(tc.lower_source_kernel(text, "vignette", {}).program, 800, 600, [rgb])
    # cosf on the device against the C library's: at most a few ulp of values in [0, 1]
    assert np.max(np.abs(img.astype(np.float64) - ref)) <= 5e-7
    assert np.array_equal(img == 0, ref == 0)  # the same pixels reach the limit (black)


def test_shading_example_taichi_math_bit_exact(dev, q):
    """ti.ndrange, taichi.math (normalize, cross, clamp, mix, smoothstep, fract, step, sign), a
    ti.static loop setting vector components, a mask field: exactly rounded operations only, so
    every frame equals the oracle bit for bit."""
    path = os.path.join(EX, "shading.py")
    res, img = run_program(path, 3)
    assert res["frames"] == 3 and img.shape == (480, 400, 3)
    text = open(path).read()
    mask = oracle.pixel_program(tc.lower_source_kernel(text, "make_mask", {}).program, 480, 400)
    ref = oracle.pixel_program(tc.lower_source_kernel(text, "draw", {"t": 0.5}).program, 480, 400, [mask])
    assert np.array_equal(img, ref)


def life_numpy(a):
    c = sum(np.roll(np.roll(a, -di, 0), -dj, 1) for di in (-1, 0, 1) for dj in (-1, 0, 1) if (di, dj) != (0, 0))
    return ((c == 3) | ((a == 1) & (c == 2))).astype(np.int32)


def test_life_example_against_numpy(dev, q):
    """int32 fields, neighbour reads at wrapped offsets: eight generations on the device equal
    numpy's game of life (np.roll) and the oracle, cell for cell."""
    path = os.path.join(EX, "life.py")
    res, img = run_program(path, 8)
    assert res["frames"] == 8 and img.shape == (320, 320) and img.dtype == np.int32
    i, j = np.meshgrid(np.arange(320), np.arange(320), indexing="ij")
    st = ((i * 37 + j * 91 + i * j) % 7 < 2).astype(np.int32)
    for _ in range(8):
        st = life_numpy(st)
    assert np.array_equal(img, st) and 0 < st.sum() < st.size


_GRAPH_F = tc.field(dtype=float, shape=(64, 48))


@tc.kernel
def _graph_step(k: float):
    for i, j in _GRAPH_F:
        _GRAPH_F[i, j] = _GRAPH_F[i, j] * 0.5 + i * k - j


def test_repeated_kernel_calls_replay_a_graph(dev, q):
    """From its second call with the same arguments a kernel's launches are recorded as one
    hipGraph and replayed: every call still advances the field once, bit for bit as the oracle."""
    tc.init(arch=tc.gpu)
    prog = _graph_step.lower(0.25).program
    want = np.zeros((64, 48), np.float32)
    for n in range(1, 7):
        _graph_step(0.25)
        want = oracle.pixel_program(prog, 64, 48, [want])
        assert np.array_equal(_GRAPH_F.to_numpy(), want), n
    assert _graph_step.lower(0.25).graph  # recorded after the second call, replayed since
    _graph_step(0.5)  # other arguments: a lowering of their own, eager at first
    assert not getattr(_graph_step.lower(0.5), "graph", None)


def test_heat_example_bit_exact(dev, q):
    path = os.path.join(EX, "heat.py")
    res, img = run_program(path, 2)
    text = open(path).read()
    u0 = oracle.pixel_program(tc.lower_source_kernel(text, "init", {}).program, 384, 256)
    prog = tc.lower_source_kernel(text, "diffuse", {"k": 0.2}).program
    u = u0
    for _ in range(20):  # two frames of ten diffuse + swap each
        u = oracle.pixel_program(prog, 384, 256, [u])
    assert np.array_equal(img, u)
    assert (img > 0).sum() > (u0 > 0).sum() and img.max() <= 1.0  # the heat has spread


def test_gather_and_int32_store_bit_exact(dev, q):
    b = pp.Builder()
    rowi = b.op("sub", b.op("mul", b.index(0), 3.0), 5.0)
    prog = pp.compile_program(b, out=b.load_at(0, rowi, b.load(1)), in_widths=[1, 1])
    rng = np.random.default_rng(6)
    src = rng.standard_normal((90, 70)).astype(np.float32)
    cols = np.array(rng.choice([-3.0, 0.0, 2.5, 6.9, 69.0, 100.0, np.nan, 1e30, -np.inf], size=(90, 70)), np.float32)
    assert np.array_equal(run_prog(dev, q, prog, [src, cols], 90, 70), oracle.pixel_program(prog, 90, 70, [src, cols]))
    b = pp.Builder()
    prog = pp.compile_program(b, out=b.op("add", b.load(0), b.load(1)), in_dtypes=[pp.I32, pp.F32], out_i32=True)
    ints = rng.integers(-1000, 1000, size=(33, 65)).astype(np.int32)
    fl = np.array(rng.choice([0.25, -0.75, 2.5, np.nan, 3e9, -3e9, 1e-3], size=(33, 65)), np.float32)
    got = run_prog(dev, q, prog, [ints, fl], 33, 65)
    assert got.dtype == np.int32 and np.array_equal(got, oracle.pixel_program(prog, 33, 65, [ints, fl]))


def test_gathers_with_rows_that_vary_across_a_wave_bit_exact(dev, q):
    """A wave of the row mapping covers 64 pixels of one row, and a gather whose row operand the
    library finds wave-uniform (computed from i and constants only) forms its row offset once per
    wave.  These gathers' rows are not wave-uniform, and each must keep its own row: the
    transpose u[j, i], a row read from data u[v[i, j], j], a row from a fixed-trip loop's state
    that starts at j, and a row that is uniform before the loop and mixed with j inside it."""
    rng = np.random.default_rng(41)
    n = 300
    u = rng.standard_normal((n, n)).astype(np.float32)
    v = rng.integers(-5, n + 5, (n, n)).astype(np.float32)
    progs = []
    b = pp.Builder()                                        # transpose: row = j
    progs.append(pp.compile_program(b, out=b.load_at(0, b.index(1), b.index(0)), in_widths=[1, 1]))
    b = pp.Builder()                                        # row from data
    progs.append(pp.compile_program(b, out=b.op("add", b.load_at(0, b.load(1), b.index(1)), b.load_at(0, b.index(0), b.load(1))),
                                    in_widths=[1, 1]))
    b = pp.Builder()                                        # loop state from j used as a row
    x = b.state("x")
    progs.append(pp.compile_program(b, init={"x": b.op("add", b.index(1), 1.0)},
                                    body={"x": b.op("add", b.op("mul", x, 0.5), b.index(0))},
                                    max_iter=3, out=b.load_at(0, x, b.index(1)), loop=True, in_widths=[1, 1]))
    b = pp.Builder()                                        # uniform at entry, mixed with j by the loop
    y = b.state("y")
    progs.append(pp.compile_program(b, init={"y": b.op("add", b.index(0), 2.0)},
                                    body={"y": b.op("add", b.op("mul", y, 0.0), b.index(1))},
                                    max_iter=2, out=b.op("add", b.load_at(0, y, b.index(0)), b.load_at(0, b.index(0), y)),
                                    loop=True, in_widths=[1, 1]))
    for prog in progs:
        assert np.array_equal(run_prog(dev, q, prog, [u, v], n, n), oracle.pixel_program(prog, n, n, [u, v]))


def test_reaction_example_sequences_bit_exact(dev, q):
    """A kernel of two struct-fors, each storing two fields (four programs per step, run in
    order on one queue): two frames of eight steps equal the oracle run of the same programs and
    numpy's Gray-Scott update, element for element."""
    path = os.path.join(EX, "reaction.py")
    res, img = run_program(path, 2)
    assert res["frames"] == 2 and img.shape == (256, 256) and img.dtype == np.float32
    text = open(path).read()
    kern, funcs, env = tc._parse_source(text, "step", {"dt": 1.0})
    step = tc.lower_kernel(kern, tc._FuncResolver(env, funcs), env)
    names = {id(v): k for k, v in env.items() if isinstance(v, tc.Field)}
    i, j = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    inside = (np.abs(i - 128) < 12) & (np.abs(j - 128) < 12)
    f = {"u": np.where(inside, np.float32(0.5), np.float32(1.0)).astype(np.float32),
         "v": np.where(inside, np.float32(0.25) + np.float32(0.01) * ((i * 7 + j * 3) % 5).astype(np.float32),
                       np.float32(0)).astype(np.float32),
         "nu": np.zeros((256, 256), np.float32), "nv": np.zeros((256, 256), np.float32)}
    for _ in range(16):
        for op in step.ops():
            f[names[id(op.field)]] = oracle.pixel_program(op.program, 256, 256, [f[names[id(g)]] for g in op.inputs])
    assert np.array_equal(img, f["v"])
    assert float(img.max()) > 0.25 and (img > 0.01).sum() > 24 * 24  # the spot has reacted and spread


def test_particles_example_one_d_fields_bit_exact(dev, q):
    """1-D struct-fors over fields of 2-vectors, one program per stored field with a snapshot copy
    (x and v load each other), an augmented store: 30 frames of 10 steps on the device equal
    numpy's restatement of the update, particle for particle, bounces included."""
    from test_taichi_general import particles_numpy, particles_seed
    res, img = run_program(os.path.join(EX, "particles.py"), 30)
    assert res["frames"] == 30 and img.shape == (16384, 2) and img.dtype == np.float32
    x0, v0 = particles_seed()
    x, v, _ = particles_numpy(x0, v0, np.zeros(16384, np.float32), 300)
    assert np.array_equal(img, x)
    assert (v[:, 1] > 0).any() and (x[:, 1] >= 0).all()  # some have bounced off the floor


def test_loops_reading_their_trip_bit_exact(dev, q):
    """Runtime loops whose variable is read (the trip, the same on every live lane): prefix sums
    over 300 trips, a window over range(-40, 41), a while loop whose test reads its counter, and
    gathers at the trip, on grids of rows and of 16x16 patches (the search loop has a test)."""
    from test_taichi_general import ROW_LOOPS
    rng_ = np.random.default_rng(16)
    u = rng_.random((37, 300)).astype(np.float32)
    for kernel, args in (("prefix", {}), ("window", {"r": 5}), ("search", {})):
        low = tc.lower_source_kernel(ROW_LOOPS, kernel, args)
        got = run_prog(dev, q, low.program, [u], 37, 300)
        ref = oracle.pixel_program(low.program, 37, 300, [u])
        assert np.array_equal(got, ref), kernel


def test_nbody_example_bit_exact(dev, q):
    """O(N^2) forces by a 4096-trip loop gathering x[j] at the trip, then the kick-drift update
    (x's program first: it loads v before v's program stores it): two steps on the device from a
    random state equal the oracle's from the same state, program by program; the example runs."""
    from test_taichi_general import lower_named
    text = open(os.path.join(EX, "nbody.py")).read()
    rng_ = np.random.default_rng(17)
    f = {"x": (rng_.random((4096, 2)) * 2 - 1).astype(np.float32), "v": (rng_.random((4096, 2)) - 0.5).astype(np.float32)}
    for _ in range(2):
        for kernel in ("forces", "advance"):
            low, names = lower_named(text, kernel, {})
            for op in low.ops():
                src = [f[names[id(g)]].reshape(1, 4096, 2) for g in op.inputs]
                got = run_prog(dev, q, op.program, src, 1, 4096).reshape(4096, 2)
                assert np.array_equal(got, oracle.pixel_program(op.program, 1, 4096, src).reshape(4096, 2)), kernel
                f[names[id(op.field)]] = got
    assert np.isfinite(f["x"]).all() and not np.array_equal(f["a"], np.zeros_like(f["a"]))
    res, img = run_program(os.path.join(EX, "nbody.py"), 2)
    assert res["frames"] == 2 and img.shape == (4096, 2) and np.isfinite(img).all()


def test_nested_range_loops_bit_exact(dev, q):
    """Perfect nests of range loops run as one loop over their trips (a 41 x 41 window of clamped
    gathers, a triple nest), with the variables recovered from the trip: bit for bit."""
    from test_taichi_general import NESTS
    u = np.random.default_rng(19).random((40, 56)).astype(np.float32)
    for kernel in ("count3", "window", "triple"):
        low = tc.lower_source_kernel(NESTS, kernel, {})
        got = run_prog(dev, q, low.program, [u][:len(low.inputs)], 40, 56)
        assert np.array_equal(got, oracle.pixel_program(low.program, 40, 56, [u][:len(low.inputs)])), kernel


# ---- seeded random programs against the oracle -----------------------------------------------------
EXACT_UNARY = ("neg", "abs", "sqrt", "floor", "square", "trunc")
EXACT_BINARY = ("add", "sub", "mul", "div", "max", "min", "lt", "le", "eq", "ne")


def random_program(seed, binary=EXACT_BINARY):
    """A random program of exactly rounded operations (binary: the two-operand opcodes drawn
    from): pixel indices, constants, loads and clamped
    gathers of one or two inputs of 1-2 components, selects; half of them with a loop (with or
    without a test) over two states that reads the trip and gathers at state-derived indices,
    the output reading the states and the count."""
    r = np.random.default_rng(seed)
    b = pp.Builder()
    widths = [int(r.integers(1, 3)) for _ in range(int(r.integers(1, 3)))]
    pool = [b.index(0), b.index(1), b.const(float(np.float32(r.uniform(-3, 3))))]
    pool += [b.load(k, int(r.integers(0, w))) for k, w in enumerate(widths)]

    def grow(pool, n, extra=()):
        vals = list(pool) + list(extra)
        for _ in range(n):
            pick = lambda: vals[int(r.integers(len(vals)))]
            u = r.random()
            if u < 0.25:
                v = b.op(EXACT_UNARY[int(r.integers(len(EXACT_UNARY)))], pick())
            elif u < 0.8:
                v = b.op(binary[int(r.integers(len(binary)))], pick(), pick())
            elif u < 0.9:
                v = b.op("select", pick(), pick(), pick())
            else:
                k = int(r.integers(len(widths)))
                v = b.load_at(k, b.op("mul", pick(), 3.0), pick(), int(r.integers(0, widths[k])))
            vals.append(v)
        return vals

    vals = grow(pool, int(r.integers(3, 9)))
    if r.random() < 0.5:
        return pp.compile_program(b, out=vals[-1], in_widths=widths), widths
    x, y = b.state("x"), b.state("y")
    body = grow([x, y, b.trip()], int(r.integers(3, 8)), extra=vals[:4])
    test = None
    if r.random() < 0.6:
        test = (("lt", "le", "gt", "ge")[int(r.integers(4))], body[int(r.integers(3, len(body)))], 4.0)
    out = b.op("add", b.op("mul", x, 0.5), b.op("sub", y, b.op("mul", b.count(), 0.125)))
    prog = pp.compile_program(b, init={"x": vals[-1], "y": vals[int(r.integers(len(vals)))]}, test=test,
                              body={"x": body[-1], "y": body[int(r.integers(2, len(body)))]},
                              max_iter=int(r.integers(0, 40)), out=out, loop=True, in_widths=widths)
    return prog, widths


def same_values(a, b):
    """The same bits wherever the oracle has a number (signed zeros included), NaN where it has NaN."""
    nan = np.isnan(b)
    return bool(np.array_equal(np.isnan(a), nan) and np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan]))


@pytest.mark.parametrize("seed", range(24))
def test_random_programs_bit_exact(dev, q, seed):
    """Seeded random programs (every exactly rounded opcode, gathers, loops with and without a
    test, the trip, the count) on a grid of 16x16 patches and on row grids, against the oracle:
    the same bits (NaN where the oracle has NaN)."""
    try:
        prog, widths = random_program(seed)
    except pp.ProgramError:
        pytest.skip("the random program does not fit the device form")
    rng_ = np.random.default_rng(1000 + seed)
    for ni, nj in ((37, 53), (1, 300), (9, 260)):
        ins = [np.where(rng_.random((ni, nj, w)) < 0.05, np.float32(np.nan),
                        rng_.standard_normal((ni, nj, w)) * 4).astype(np.float32).reshape((ni, nj) if w == 1 else (ni, nj, w))
               for w in widths]
        got = run_prog(dev, q, prog, ins, ni, nj)
        ref = oracle.pixel_program(prog, ni, nj, ins)
        assert same_values(got, ref), (seed, ni, nj, pp.describe(prog))


@pytest.mark.parametrize("seed", range(100, 112))
def test_random_programs_with_bit_operations_bit_exact(dev, q, seed):
    """Seeded random programs that also draw the bit opcodes (int32 conversions of arbitrary
    values: fractions, NaN, values past int32, results past 2^24 rounded back to f32): the same
    bits as the oracle."""
    try:
        prog, widths = random_program(seed, EXACT_BINARY + ("band", "bor", "bxor", "shl", "shr"))
    except pp.ProgramError:
        pytest.skip("the random program does not fit the device form")
    rng_ = np.random.default_rng(1000 + seed)
    for ni, nj in ((37, 53), (1, 300)):
        ins = [np.where(rng_.random((ni, nj, w)) < 0.05, np.float32(np.nan),
                        rng_.standard_normal((ni, nj, w)) * 300).astype(np.float32).reshape((ni, nj) if w == 1 else (ni, nj, w))
               for w in widths]
        got = run_prog(dev, q, prog, ins, ni, nj)
        ref = oracle.pixel_program(prog, ni, nj, ins)
        assert same_values(got, ref), (seed, ni, nj, pp.describe(prog))


def test_body_with_three_loops_split_into_parts_bit_exact(dev, q):
    """A body of three runtime loops (a while loop, a range loop of a per-pixel trip count, another
    while loop) runs as parts passing values through hidden fields: every program of the sequence
    on the device equals the oracle's on the same inputs, and the stored fields equal the oracle's
    run of the whole sequence."""
    from test_taichi_general import TWO_LOOPS, lower_named
    u = np.random.default_rng(21).random((48, 40)).astype(np.float32)
    low, names = lower_named(TWO_LOOPS, "march", {})
    dev_f, ref_f = {"u": u}, {"u": u}
    for op in low.ops():
        names.setdefault(id(op.field), f"hidden{len(names)}")
        got = run_prog(dev, q, op.program, [dev_f[names[id(g)]] for g in op.inputs], 48, 40)
        ref = oracle.pixel_program(op.program, 48, 40, [ref_f[names[id(g)]] for g in op.inputs])
        assert np.array_equal(got, ref), names[id(op.field)]
        dev_f[names[id(op.field)]], ref_f[names[id(op.field)]] = got, ref
    assert len(low.ops()) >= 4 and np.array_equal(dev_f["f"], ref_f["f"]) and np.array_equal(dev_f["g"], ref_f["g"])


def test_body_too_large_for_one_program_bit_exact(dev, q):
    """A body beyond one program's 128 instructions runs as several programs joined by hidden
    fields; each program on the device equals the oracle's on the same inputs."""
    from test_taichi_general import BIG_BODY, lower_named
    low, names = lower_named(BIG_BODY, "k", {})
    dev_f, ref_f = {}, {}
    for op in low.ops():
        names.setdefault(id(op.field), f"hidden{len(names)}")
        got = run_prog(dev, q, op.program, [dev_f[names[id(g)]] for g in op.inputs], 20, 30)
        ref = oracle.pixel_program(op.program, 20, 30, [ref_f[names[id(g)]] for g in op.inputs])
        assert np.array_equal(got, ref), names[id(op.field)]
        dev_f[names[id(op.field)]], ref_f[names[id(op.field)]] = got, ref
    assert len(low.ops()) >= 2 and np.array_equal(dev_f["f"], ref_f["f"])


def test_three_d_fields_bit_exact(dev, q):
    """3-D fields as [A B][C] grids: init, a clamped seven-point stencil and gathers one past each
    axis on the device equal the oracle; the volume example's frames equal the oracle's run of
    the same kernels (the middle slice)."""
    from test_taichi_general import VOLUME, lower_named
    f_dev, f_ref = {}, {}
    for kernel, args in (("init", {}), ("diffuse", {"c": 0.1}), ("grad", {})):
        low, names = lower_named(VOLUME, kernel, args)
        for op in low.ops():
            src = [f_dev[names[id(g)]].reshape((120, 36) + ((g.width,) if g.width > 1 else ())) for g in op.inputs]
            got = run_prog(dev, q, op.program, src, 120, 36)
            ref = oracle.pixel_program(op.program, 120, 36, src)
            assert np.array_equal(got, ref), kernel
            f_dev[names[id(op.field)]] = got.reshape((12, 10, 36) + got.shape[2:])
    path = os.path.join(EX, "volume.py")
    res, img = run_program(path, 2)
    assert res["frames"] == 2 and img.shape == (96, 96)
    text = open(path).read()
    shape = (96 * 96, 96)
    u0 = oracle.pixel_program(tc.lower_source_kernel(text, "init", {}).program, *shape)
    diff = tc.lower_source_kernel(text, "diffuse", {"c": 0.15}).program
    u = u0
    for _ in range(10):
        u = oracle.pixel_program(diff, *shape, [u])
    assert np.array_equal(img, u.reshape(96, 96, 96)[:, :, 48])
    assert (img > 0).sum() > (u0.reshape(96, 96, 96)[:, :, 48] > 0).sum()  # the heat has spread


def test_fields_of_other_shapes_bit_exact(dev, q):
    """Gathers from fields of other shapes than the loop's (a 1-D field at the trip, a smaller 2-D
    field past its last row, a 3-D field past its last k), each clamped to its own extents: the
    device equals the oracle; the metaballs example runs and equals the oracle's frames."""
    from test_taichi_general import OTHER_SHAPES, lower_named
    rng_ = np.random.default_rng(23)
    data = {"pos": (rng_.random((1, 24, 2)) * np.array([40, 30])).astype(np.float32),
            "small": rng_.random((20, 10)).astype(np.float32), "vol": rng_.random((1200, 5)).astype(np.float32)}
    for kernel in ("blobs", "upsample", "project"):
        low, names = lower_named(OTHER_SHAPES, kernel, {})
        for op in low.ops():
            src = [data[names[id(g)]] for g in op.inputs]
            got = run_prog(dev, q, op.program, src, 40, 30)
            assert np.array_equal(got, oracle.pixel_program(op.program, 40, 30, src)), kernel
    path = os.path.join(EX, "metaballs.py")
    res, img = run_program(path, 3)
    assert res["frames"] == 3 and img.shape == (640, 480) and 0.0 < img.mean() < 1.0
    low, names = lower_named(open(path).read(), "render", {})
    p = np.zeros((1, 48, 2), np.float32)
    k = np.arange(48)
    p[0, :, 0], p[0, :, 1] = (k * 97 % 613) + 10.0, (k * 53 % 457) + 10.0
    assert low.program.in_rows[0] == 1 and low.program.in_cols[0] == 48
    got = run_prog(dev, q, low.program, [p], 640, 480)
    assert np.array_equal(got, oracle.pixel_program(low.program, 640, 480, [p]))


@pytest.mark.parametrize("kernel", ["first_over", "skip_parity", "escape_break", "own_trips", "misc"])
def test_break_continue_and_small_math_bit_exact(dev, q, kernel):
    """Loops with break / continue (flags read by the loop's test and guarding the statements
    after a jump), a while counter read after a break, rsqrt, taichi.math.mod and static
    conditions: every program of the kernel on the device equals the oracle bit for bit."""
    from test_taichi_general import JUMPS, SMALL_MATH, lower_named
    text = SMALL_MATH if kernel == "misc" else JUMPS
    low, names = lower_named(text, kernel, {})
    r = np.random.default_rng(3)
    fields = {"u": r.uniform(-0.5, 2.5, (12, 20)).astype(np.float32) if kernel != "misc"
              else r.uniform(-2, 2, (8, 16)).astype(np.float32)}
    for op in low.ops():
        ni, nj = op.grid
        src = [fields[names[id(f)]] for f in op.inputs]
        got = run_prog(dev, q, op.program, src, ni, nj)
        assert np.array_equal(got, oracle.pixel_program(op.program, ni, nj, src)), kernel


def test_bit_opcodes_and_operators_bit_exact(dev, q):
    """The bit opcodes on every pair of a set of values (negatives, fractions, NaN, values past
    int32, shift counts past 31) and the Taichi kernel using &, |, ^, <<, >> of indices: the
    device equals the oracle bit for bit."""
    from test_taichi_general import BITS, lower_named
    vals = np.array([0, 1, -1, 5, -6, 255, 256, -256, 1 << 23, -(1 << 23), 7.9, -7.9, np.nan, 3e9, -3e9, 31, 32, 33],
                    np.float32)
    n = len(vals)
    a = np.repeat(vals[:, None], n, axis=1)
    c = np.repeat(vals[None, :], n, axis=0)
    b = pp.Builder()
    la, lc = b.load(0), b.load(1)
    for name in ("band", "bor", "bxor", "shl", "shr"):
        prog = pp.compile_program(b, out=b.op(name, la, lc))
        assert np.array_equal(run_prog(dev, q, prog, [a, c], n, n), oracle.pixel_program(prog, n, n, [a, c])), name
    low, names = lower_named(BITS, "bits", {})
    for op in low.ops():
        ni, nj = op.grid
        assert not op.inputs
        assert np.array_equal(run_prog(dev, q, op.program, [], ni, nj), oracle.pixel_program(op.program, ni, nj, []))


def test_taichi_surface_additions_on_the_device(dev, q):
    """The kernel of @ti.func ifs, ti.types.vector, swizzles, vector reductions, reflect, isnan,
    casts and ~: every program on the device equals the oracle bit for bit."""
    from test_taichi_general import SURFACE, lower_named
    low, names = lower_named(SURFACE, "surface", {})
    r = np.random.default_rng(12)
    fields = {"u": r.uniform(-2, 2, (10, 14)).astype(np.float32), "v3": r.uniform(-1, 1, (10, 14, 3)).astype(np.float32)}
    fields["u"][2, 3] = 0.0
    for op in low.ops():
        ni, nj = op.grid
        src = [fields[names[id(f)]] for f in op.inputs]
        assert np.array_equal(run_prog(dev, q, op.program, src, ni, nj), oracle.pixel_program(op.program, ni, nj, src))


def test_round_opcode_bit_exact(dev, q):
    """VDSL_PIX_ROUND on halfway cases, signed zeros, values past 2^23, infinities and NaN: the
    device's roundf equals the oracle's bit for bit."""
    from test_taichi_general import ROUND_VALUES
    x = np.tile(ROUND_VALUES, 7)[None]
    b = pp.Builder()
    prog = pp.compile_program(b, out=b.op("round", b.load(0)))
    assert same_values(run_prog(dev, q, prog, [x], 1, x.shape[1]), oracle.pixel_program(prog, 1, x.shape[1], [x]))
