"""Pins the CPU oracle's escape-time map (oracle/vdsl_oracle.c: orc_escape_time, following
fractal.py:11-25) with checks that do not reuse its code:

- an independent numpy evaluation, exactly rounded (numpy f32 ops are IEEE; fma is emulated
  exactly by round-to-odd in f64), equal bit for bit;
- the known answers of the 1024^2 Mandelbrot grid in the separately-rounded form
  (sum 49,860,131; 177,509 pixels at 256; sha256 prefix 747b980a873b342e; corner values);
- closed forms: main cardioid and period-2 bulb reach max_iter, |c|^2 > 4 stops at once;
- conjugate symmetry counts[i][j] == counts[i][n - j];
- f64 brute force away from the set boundary.
"""
import hashlib

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, spec


def fma32(a, b, c):
    """Correctly rounded f32 fma(a, b, c): the f64 product is exact, the f64 sum is made
    round-to-odd with TwoSum, and round-to-odd at 53 bits then nearest-even at 24 bits is exact."""
    a64, b64, c64 = (np.asarray(v, np.float32).astype(np.float64) for v in (a, b, c))
    p = a64 * b64
    s = p + c64
    bb = s - p
    err = (p - (s - bb)) + (c64 - bb)
    even = (s.view(np.int64) & 1) == 0
    bump = (err != 0) & even
    s = np.where(bump, np.nextafter(s, np.where(err > 0, np.inf, -np.inf)), s)
    return s.astype(np.float32)


def numpy_escape(params):
    """Vectorised f32 restatement of the check-then-update loop (fractal.py:22-24)."""
    p = dict(params)
    f = np.float32
    i = np.arange(p["ni"], dtype=np.float32)
    j = np.arange(p["nj"], dtype=np.float32)
    re = (((i / f(p["re_den"])) + f(p["re_off"])) * f(p["re_scale"])) + f(p["re_post"])
    im = (((j / f(p["im_den"])) + f(p["im_off"])) * f(p["im_scale"])) + f(p["im_post"])
    RE, IM = np.meshgrid(re, im, indexing="ij")
    if p["family"] == _lib.ESC_MANDELBROT:
        zr = np.zeros_like(RE); zi = np.zeros_like(RE); cr, ci = RE, IM
    else:
        zr, zi = RE.copy(), IM.copy()
        cr = np.full_like(RE, f(p["c_re"])); ci = np.full_like(RE, f(p["c_im"]))
    it = np.zeros(RE.shape, np.int32)
    live = np.ones(RE.shape, bool)
    bound = f(p["bound"])
    for _ in range(p["max_iter"]):
        if p["rounding"] == _lib.ESC_ROUND_SEPARATE:
            zr2 = zr * zr; zi2 = zi * zi
            mag = zr2 + zi2
            nzr = (zr2 - zi2) + cr
            nzi = ((zi * zr) * f(2.0)) + ci
        else:
            qq = zi * zi
            mag = fma32(zr, zr, qq)
            nzr = fma32(zr, zr, -qq) + cr
            nzi = fma32(zr + zr, zi, ci)
        go = ~(mag > bound) if p["escape_test"] == _lib.ESC_MAG2_GT else (np.sqrt(mag) < bound)
        live &= go
        if not live.any():
            break
        zr = np.where(live, nzr, zr); zi = np.where(live, nzi, zi)
        it += live
    if p["out_kind"] == _lib.ESC_OUT_I32_COUNT:
        return it
    return f(p["out_base"]) + it.astype(np.float32) * f(p["out_scale"])


@pytest.fixture(scope="module")
def grid_sep():
    return oracle.escape_time(spec.mandelbrot_params(rounding=_lib.ESC_ROUND_SEPARATE))


@pytest.fixture(scope="module")
def grid_fma():
    return oracle.escape_time(spec.mandelbrot_params(rounding=_lib.ESC_ROUND_FMA))


def test_fma32_emulation_is_exact():
    # Cases where a*b+c in f64 lies exactly halfway after one rounding: double rounding would fail.
    a = np.float32(1 + 2 ** -12); b = np.float32(1 + 2 ** -12)
    # a*b = 1 + 2^-11 + 2^-24 exactly; + c with c = -2^-24 * 0.5 ...
    for c in (np.float32(0), np.float32(2 ** -25), np.float32(-(2 ** -25)), np.float32(3 * 2 ** -26)):
        exact = (1 + 2 ** -12) ** 2 + float(c)  # exact as a Python float (fits 53 bits)
        from fractions import Fraction
        ex = Fraction(1 + 2 ** -12) ** 2 + Fraction(float(c))
        got = fma32(a, b, c)
        # the correctly rounded f32 is the f32 nearest to ex (ties to even)
        cand = np.float32(exact)
        lo, hi = np.nextafter(cand, np.float32(-1)), np.nextafter(cand, np.float32(2))
        best = min((lo, cand, hi), key=lambda v: (abs(Fraction(float(v)) - ex), int(np.float32(v).view(np.int32)) & 1))
        assert got == best


def test_known_answers_separate_rounding(grid_sep):
    c = grid_sep
    assert c.shape == (1024, 1024) and c.dtype == np.int32
    assert int(c.sum()) == 49_860_131
    assert int((c == 256).sum()) == 177_509
    assert c.min() == 1 and c.max() == 256
    assert c[0, 512] == 256  # c = -2 + 0i: 0 -> -2 -> 2 -> 2 ..., |z|^2 = 4 is never > 4
    assert c[0, 0] == 1 and c[1023, 1023] == 2
    assert hashlib.sha256(np.ascontiguousarray(c, "<i4").tobytes()).hexdigest().startswith("747b980a873b342e")


def test_numpy_restatement_bit_exact_separate(grid_sep):
    assert np.array_equal(numpy_escape(spec.mandelbrot_params(rounding=_lib.ESC_ROUND_SEPARATE)), grid_sep)


def test_numpy_restatement_bit_exact_fma(grid_fma):
    assert np.array_equal(numpy_escape(spec.mandelbrot_params(rounding=_lib.ESC_ROUND_FMA)), grid_fma)


def test_forms_differ_only_near_boundary(grid_sep, grid_fma):
    diff = grid_sep != grid_fma
    assert 0 < diff.sum() < 5000  # the two rounding forms are different programs
    # neither form touches the interior closed forms below


@pytest.mark.parametrize("rounding", [_lib.ESC_ROUND_SEPARATE, _lib.ESC_ROUND_FMA])
def test_closed_forms_and_symmetry(rounding, grid_sep, grid_fma):
    c = grid_sep if rounding == _lib.ESC_ROUND_SEPARATE else grid_fma
    n = 1024
    x = (np.arange(n) / n) * 3 - 2.0
    y = (np.arange(n) / n) * 3 - 1.5
    X, Y = np.meshgrid(x, y, indexing="ij")
    qq = (X - 0.25) ** 2 + Y ** 2
    cardioid = qq * (qq + (X - 0.25)) < 0.25 * Y ** 2 * 0.98  # strictly inside (margin)
    bulb = (X + 1) ** 2 + Y ** 2 < (1 / 16) * 0.95
    assert cardioid.sum() > 100_000 and bulb.sum() > 10_000
    assert (c[cardioid] == 256).all()
    assert (c[bulb] == 256).all()
    outside = X ** 2 + Y ** 2 > 4
    assert (c[outside] == 1).all()
    # conjugate symmetry about im = 0 (j = 512)
    assert np.array_equal(c[:, 1:512], c[:, 1024 - 1:512:-1])


def test_f64_brute_force_far_from_boundary(grid_fma):
    n = 1024
    rng = np.random.default_rng(7)
    ii = rng.integers(0, n, 400); jj = rng.integers(0, n, 400)
    checked = 0
    for i, j in zip(ii, jj):
        cr = -2 + 3 * i / n; ci = -1.5 + 3 * j / n
        zr = zi = 0.0; it = 0
        while it < 256 and zr * zr + zi * zi <= 4:
            zr, zi = zr * zr - zi * zi + cr, 2 * zr * zi + ci
            it += 1
        if it < 40:  # quickly escaping points are insensitive to rounding
            assert grid_fma[i, j] == it
            checked += 1
    assert checked > 100


def test_julia_program_of_fractal_py():
    """The exact program of fractal.py:7-25 (frame t = 0.03*k) against the numpy restatement."""
    for frame in (0, 17):
        p = spec.julia_paint_params(frame * 0.03)
        got = oracle.escape_time(p)
        assert got.shape == (640, 320) and got.dtype == np.float32
        assert np.array_equal(got, numpy_escape(p))
        vals = np.unique(got)
        assert vals.min() >= np.float32(1 - 50 * 0.02) - 1e-6 and vals.max() <= 1.0


def test_zero_iterations_and_empty():
    p = spec.mandelbrot_params(n=16, max_iter=0)
    assert (oracle.escape_time(p) == 0).all()
