"""GPU parity of the escape-time op (vdsl_op_escape_time) against the CPU oracle: bit-exact."""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, spec
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu


def run_gpu(dev, q, params):
    p = kernels.escape_time_params(**params)
    dt = "i32" if p.out_kind == _lib.ESC_OUT_I32_COUNT else "f32"
    out = Tensor(dev, (p.ni, p.nj), dt)
    out.buffer.fill_u32(q, 0xDEADBEEF)  # stale values must not survive
    kernels.escape_time(q, p, out)
    got = out.numpy(q)
    out.free()
    return got


@pytest.mark.parametrize("rounding", [_lib.ESC_ROUND_FMA, _lib.ESC_ROUND_SEPARATE])
def test_config1_mandelbrot_1024_bit_exact(dev, q, rounding):
    params = spec.mandelbrot_params(rounding=rounding)
    got = run_gpu(dev, q, params)
    ref = oracle.escape_time(params)
    assert np.array_equal(got, ref), f"{int((got != ref).sum())} pixels differ"
    if rounding == _lib.ESC_ROUND_SEPARATE:
        assert int(got.sum()) == 49_860_131


def test_fractal_py_julia_frames_bit_exact(dev, q):
    for frame in (0, 1, 50, 999):
        params = spec.julia_paint_params(frame * 0.03)
        got = run_gpu(dev, q, params)
        assert got.dtype == np.float32 and got.shape == (640, 320)
        assert np.array_equal(got, oracle.escape_time(params)), f"frame {frame}"


@pytest.mark.parametrize("ni,nj", [(1, 1), (37, 53), (16, 15), (100, 1), (1, 300)])
def test_ragged_grids(dev, q, ni, nj):
    params = spec.mandelbrot_params(n=64)
    params.update(ni=ni, nj=nj)
    got = run_gpu(dev, q, params)
    assert np.array_equal(got, oracle.escape_time(params))


def test_empty_and_zero_iterations(dev, q):
    params = spec.mandelbrot_params(n=32, max_iter=0)
    assert (run_gpu(dev, q, params) == 0).all()
    p = kernels.escape_time_params(**spec.mandelbrot_params(n=8))
    p.ni = 0  # an empty grid launches nothing and succeeds
    out = Tensor(dev, (1,), "i32")
    _lib.call("vdsl_op_escape_time", q.handle, ctypes.byref(p), out.handle)
    out.free()


def test_deterministic_repeat(dev, q):
    params = spec.mandelbrot_params(n=256, max_iter=1000)
    a = run_gpu(dev, q, params)
    b = run_gpu(dev, q, params)
    assert np.array_equal(a, b)
    assert np.array_equal(a, oracle.escape_time(params))


def test_bad_params_rejected(dev, q):
    p = kernels.escape_time_params(**spec.mandelbrot_params(n=8))
    p.family = 7
    out = Tensor(dev, (8, 8), "i32")
    with pytest.raises(_lib.VdslError) as ei:
        kernels.escape_time(q, p, out)
    assert ei.value.status == -1
    p = kernels.escape_time_params(**spec.mandelbrot_params(n=16))
    with pytest.raises((ValueError, _lib.VdslError)):
        kernels.escape_time(q, p, out)  # output too small
    out.free()


def _window(n, re0, re1, im0, im1, max_iter, rounding, family=_lib.ESC_MANDELBROT, c=(0.0, 0.0),
            test=_lib.ESC_MAG2_GT, bound=4.0, out_kind=_lib.ESC_OUT_I32_COUNT):
    """An n x n grid over [re0, re1) x [im0, im1): coordinate = (idx / n) * width + start."""
    return dict(ni=n, nj=n, family=family, escape_test=test, rounding=rounding, out_kind=out_kind,
                max_iter=max_iter, bound=bound, re_den=float(n), re_off=0.0, re_scale=re1 - re0, re_post=re0,
                im_den=float(n), im_off=0.0, im_scale=im1 - im0, im_post=im0, c_re=c[0], c_im=c[1],
                out_base=1.0, out_scale=-0.001)


@pytest.mark.parametrize("rounding", [_lib.ESC_ROUND_FMA, _lib.ESC_ROUND_SEPARATE])
@pytest.mark.parametrize("max_iter", [37, 256, 1000])
def test_periodic_orbits_exact(dev, q, rounding, max_iter):
    """Windows dominated by points whose f32 orbits become exactly periodic (the main cardioid,
    the period-2 and period-3 bulbs, c = 0 itself, which a 128-point grid over [-1, 1) holds):
    the kernel ends a lane at the first recurrence of its state it sees and counts max_iter,
    which must equal the oracle's plain iteration count, bit for bit, also when max_iter is not
    a whole number of 16-trip blocks."""
    for win in ((-1.0, 1.0, -1.0, 1.0), (-1.25, -0.75, -0.25, 0.25), (-0.2, 0.0, 0.65, 0.85)):
        params = _window(128, *win, max_iter=max_iter, rounding=rounding)
        got = run_gpu(dev, q, params)
        ref = oracle.escape_time(params)
        assert np.array_equal(got, ref), (win, int((got != ref).sum()))
        assert (ref == max_iter).sum() > 1000  # the window is mostly set interior


def test_periodic_julia_interior_exact(dev, q):
    """Filled Julia sets of c in the main cardioid and in the period-2 bulb (interior orbits
    converge to the attracting cycle), with the norm test and the f32 affine store of
    fractal.py:22-25."""
    for c in ((-0.12, 0.1), (-1.0, 0.05)):
        params = _window(192, -1.6, 1.6, -1.2, 1.2, max_iter=300, rounding=_lib.ESC_ROUND_SEPARATE,
                         family=_lib.ESC_JULIA, c=c, test=_lib.ESC_NORM_GE, bound=2.0,
                         out_kind=_lib.ESC_OUT_F32_AFFINE)
        got = run_gpu(dev, q, params)
        ref = oracle.escape_time(params)
        assert np.array_equal(got.view(np.int32), ref.view(np.int32)), c
        assert (ref == np.float32(1.0 - 0.001 * 300)).sum() > 1000
