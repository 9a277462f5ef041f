"""Taichi-style programs run unchanged on the HIP device through vernondsl_amd.run."""
import io
import json
import os
import contextlib

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, run, spec, taichi_compat as tc

pytestmark = pytest.mark.gpu
EX = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "vernondsl_amd", "examples")


def run_program(path, frames):
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        assert run.main([path, "--frames", str(frames)]) == 0
    return json.loads(buf.getvalue().strip().splitlines()[-1]), tc._state["last_gui"].last_image


def test_mandelbrot_program_equals_known_answers(dev, q):
    res, img = run_program(os.path.join(EX, "mandelbrot_counts.py"), 1)
    assert res["frames"] == 1 and img.shape == (1024, 1024) and img.dtype == np.int32
    assert int(img.sum()) == 49_860_131  # the separately-rounded grid's known sum
    assert np.array_equal(img, oracle.escape_time(spec.mandelbrot_params(rounding=_lib.ESC_ROUND_SEPARATE)))


def test_julia_program_frames_match_oracle(dev, q):
    res, img = run_program(os.path.join(EX, "rabbit_drift.py"), 3)
    assert res["frames"] == 3 and img.shape == (512, 512) and img.dtype == np.float32
    angle = 0.0
    for _ in range(2):  # the program's own accumulation: the third frame is drawn at 0.0 + 0.1 + 0.1
        angle += 0.1
    _, p = tc.lower_source(open(os.path.join(EX, "rabbit_drift.py")).read(), "draw", {"angle": angle})
    assert np.array_equal(img, oracle.escape_time(p))
    # every shade is 1 - k/128 for a count k in [0, 128]
    k = (1.0 - img.astype(np.float64)) * 128
    assert np.array_equal(k, np.round(k)) and k.min() >= 1 and k.max() == 128


def test_bindings_allocate_device_buffers(dev, q):
    import ctypes

    from vernondsl_amd import bindings, kernels, mapchain as mc
    from vernondsl_amd.rhi import Tensor
    text = ('func.func @k(%a: tensor<16x4xf32> {vernon.semantic = "input"}, '
            '%c: tensor<4xf32> {vernon.semantic = "uniform_constant"}) -> (tensor<16x4xf32> {vernon.semantic = "output"})')
    ts = bindings.allocate(dev, bindings.read_bindings(text, "k"))
    assert ts["%a"].shape == (16, 4) and ts["result0"].buffer.nbytes == 256
    b = ctypes.c_int()
    _lib.call("vdsl_buffer_binding", ts["%c"].handle, ctypes.byref(b))
    assert b.value == _lib.BIND_UNIFORM_CONSTANT
    # ops write "output" buffers; a uniform_constant buffer is device read-only and is refused
    prog = mc.compile(mc.Input(0) * 2.0)
    kernels.map_chain(q, prog, [ts["%a"]], ts["result0"])
    ro = Tensor(dev, (16, 4), "f32", binding="uniform_constant")
    with pytest.raises(_lib.VdslError) as ei:
        kernels.map_chain(q, prog, [ts["%a"]], ro)
    assert ei.value.status == -1 and "read-only" in ei.value.message
    for t in list(ts.values()) + [ro]:
        t.free()
