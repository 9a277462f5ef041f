"""Taichi-subset front end (vernondsl_amd.taichi_compat) on the CPU: lowering kernels to
escape-time op parameters from their AST, without running the programs."""
import os

import numpy as np
import pytest

from vernondsl_amd import _lib, spec, taichi_compat as tc

REF = "/root/reference/fractal.py"
EX = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vernondsl_amd", "examples")


def same_f32(p, ref):
    for k, v in ref.items():
        a, b = p[k], v
        if isinstance(b, float):
            assert np.float32(a) == np.float32(b), (k, a, b)
        else:
            assert a == b, (k, a, b)


@pytest.mark.skipif(not os.path.exists(REF), reason="the reference tree is only mounted in the build container")
@pytest.mark.parametrize("frame", [0, 1, 7, 999, 54321])
def test_reference_fractal_py_lowers_to_paint_params(frame):
    """fractal.py's `paint(t)` (fractal.py:16-25), read as text, lowers to the same op parameters as
    spec.julia_paint_params(t), for the frame times its loop passes (fractal.py:30-31)."""
    text = open(REF).read()
    fld, p = tc.lower_source(text, "paint", {"t": frame * 0.03})
    assert fld.shape == (640, 320) and fld.dtype == "f32"
    same_f32(p, spec.julia_paint_params(frame * 0.03))


def test_mandelbrot_example_lowers_to_config1_separate_form():
    fld, p = tc.lower_source(open(os.path.join(EX, "mandelbrot_counts.py")).read(), "render", {"limit": 256})
    assert fld.shape == (1024, 1024) and fld.dtype == "i32"
    same_f32(p, spec.mandelbrot_params(rounding=_lib.ESC_ROUND_SEPARATE))


def test_julia_example_lowering():
    fld, p = tc.lower_source(open(os.path.join(EX, "rabbit_drift.py")).read(), "draw", {"angle": 0.5})
    assert fld.shape == (512, 512) and fld.dtype == "f32"
    assert p["family"] == _lib.ESC_JULIA and p["escape_test"] == _lib.ESC_MAG2_GT and p["bound"] == 16.0
    assert p["max_iter"] == 128 and p["out_kind"] == _lib.ESC_OUT_F32_AFFINE
    a = np.float32(0.5)
    assert np.float32(p["c_re"]) == np.float32(-0.1226) + np.float32(0.05) * np.cos(a, dtype=np.float32)
    assert np.float32(p["c_im"]) == np.float32(0.7449) + np.float32(0.05) * np.sin(a, dtype=np.float32)
    for ax in ("re", "im"):
        assert p[f"{ax}_den"] == 512.0 and p[f"{ax}_off"] == 0.0
        assert np.float32(p[f"{ax}_scale"]) == np.float32(3.2) and np.float32(p[f"{ax}_post"]) == -np.float32(1.6)
    assert p["out_base"] == 1.0 and p["out_scale"] == -1.0 / 128


PROG = '''
import taichi as ti
n = 64
f = ti.field(dtype=float, shape=(n, n))

@ti.func
def sq(z):
    return ti.Vector([z[0] * z[0] - z[1] * z[1], {IM}])

@ti.kernel
def k(t: float):
    for i, j in f:
        c = ti.Vector([-0.5, 0.25])
        z = ti.Vector([i / n - 0.5, j / n - 0.5]) * 2
        it = 0
        while {COND}:
            z = sq(z) + c
            it += 1
        f[i, j] = {STORE}
'''


def prog(im="z[1] * z[0] * 2", cond="z.norm() < 4 and it < 20", store="1 - it * 0.05"):
    return PROG.replace("{IM}", im).replace("{COND}", cond).replace("{STORE}", store)


@pytest.mark.parametrize("im", ["z[1] * z[0] * 2", "z[0] * z[1] * 2", "2 * (z[0] * z[1])", "z[0] * z[1] + z[0] * z[1]"])
def test_accepted_square_forms(im):
    _, p = tc.lower_source(prog(im=im), "k", {"t": 0.0})
    assert p["rounding"] == _lib.ESC_ROUND_SEPARATE


@pytest.mark.parametrize("kw,msg", [
    (dict(im="2 * z[0] * z[1]"), "imaginary part"),           # (2*zr)*zi rounds differently when subnormal
    (dict(im="z[0] * z[1]"), "imaginary part"),
    (dict(cond="z.norm() <= 4 and it < 20"), "supported tests"),
    (dict(cond="it < 20"), "while condition"),
    (dict(store="it * it"), "a \\+ k \\* b"),
])
def test_rejected_bodies_raise(kw, msg):
    with pytest.raises(tc.TaichiLoweringError, match=msg):
        tc.lower_source(prog(**kw), "k", {"t": 0.0})


def test_non_escape_kernel_is_rejected():
    text = "import taichi as ti\nf = ti.field(dtype=float, shape=(4, 4))\n@ti.kernel\ndef k():\n    for i, j in f:\n        f[i, j] = i + j\n"
    with pytest.raises(tc.TaichiLoweringError):
        tc.lower_source(text, "k", {})
