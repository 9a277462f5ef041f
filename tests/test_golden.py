"""The oracle reproduces every committed golden fixture (tests/golden/, written and cross-checked
by tests/golden/make_golden.py) and the known answers of the 1024^2 Mandelbrot grids."""
import hashlib
import json
import os

import numpy as np

from oracle import oracle
from vernondsl_amd import _lib, mapchain as mc, spec

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


def test_escape_fixtures():
    for tag, rnd in (("separate", _lib.ESC_ROUND_SEPARATE), ("fma", _lib.ESC_ROUND_FMA)):
        assert np.array_equal(oracle.escape_time(spec.mandelbrot_params(n=64, rounding=rnd)),
                              load(f"mandelbrot_64_{tag}.npz")["counts"])
    assert np.array_equal(oracle.escape_time(spec.julia_paint_params(0.0, n=40)), load("julia_paint_n40_t0.npz")["pixels"])


def test_known_answers_fma_grid():
    ka = json.load(open(os.path.join(G, "known_answers.json")))
    full = oracle.escape_time(spec.mandelbrot_params(rounding=_lib.ESC_ROUND_FMA))
    k = ka["mandelbrot_1024_fma"]
    assert int(full.sum()) == k["sum"] and int((full == 256).sum()) == k["pixels_at_max_iter"]
    assert hashlib.sha256(np.ascontiguousarray(full, "<i4").tobytes()).hexdigest() == k["sha256_int32_le"]
    assert ka["mandelbrot_1024_separate"]["sum"] == 49_860_131


def test_float_fixtures():
    f = load("map_chain_32x64.npz")
    assert np.array_equal(oracle.map_chain(mc.compile(spec.map_chain_expr()), [f["x"], f["bias"]], 32, 64), f["y"])
    for tag in ("f32", "bf16"):
        f = load(f"softmax_16x256_{tag}.npz")
        s, m, sm = oracle.row_reduce_softmax(f["x"])
        assert np.array_equal(s, f["row_sum"]) and np.array_equal(m, f["row_max"]) and np.array_equal(sm, f["softmax"])
    f = load("gemm_bf16_48x40x64_gelu.npz")
    c, pre = oracle.gemm_bf16(f["A"], f["B"], False, True, c_dtype=1, epilogue=1, want_pre=True)
    assert np.array_equal(pre, f["pre"]) and np.array_equal(c, f["C"])


def test_int8_fixture():
    f = load("w8a8_16_128_96_64.npz")
    y = oracle.w8a8_forward(f["x"], [(f["w0"], f["s0"]), (f["w1"], f["s1"])])
    assert np.array_equal(y, f["y"])
