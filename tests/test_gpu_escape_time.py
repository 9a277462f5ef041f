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
