"""The HIP device against the committed golden fixtures (tests/golden/): bit-exact for integer
outputs and the int8 network, within the op tolerances for floating point."""
import os

import numpy as np
import pytest

from vernondsl_amd import _lib, graph, kernels, mapchain as mc, rng, spec
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(G, name), allow_pickle=False)


def test_escape_fixtures(dev, q):
    cases = [(spec.mandelbrot_params(n=64, rounding=_lib.ESC_ROUND_SEPARATE), "mandelbrot_64_separate.npz", "counts"),
             (spec.mandelbrot_params(n=64, rounding=_lib.ESC_ROUND_FMA), "mandelbrot_64_fma.npz", "counts"),
             (spec.julia_paint_params(0.0, n=40), "julia_paint_n40_t0.npz", "pixels")]
    for params, fname, key in cases:
        p = kernels.escape_time_params(**params)
        out = Tensor(dev, (p.ni, p.nj), "i32" if p.out_kind == 0 else "f32")
        kernels.escape_time(q, p, out)
        assert np.array_equal(out.numpy(q), load(fname)[key]), fname
        out.free()


def test_map_chain_and_softmax_fixtures(dev, q):
    f = load("map_chain_32x64.npz")
    tx, tb = Tensor.from_numpy(dev, q, f["x"]), Tensor.from_numpy(dev, q, f["bias"])
    ty = Tensor(dev, (32, 64), "f32")
    kernels.map_chain(q, mc.compile(spec.map_chain_expr()), [tx, tb], ty)
    x64 = f["x"].astype(np.float64)
    u = ((np.float32(spec.MAP_A) * f["x"]) + np.float32(spec.MAP_B)).astype(np.float64)
    scale = np.abs(np.tanh(u) * np.exp(-x64 * x64)) + np.abs(f["bias"].astype(np.float64))
    assert np.all(np.abs(ty.numpy(q) - f["y"].astype(np.float64)) <= 1e-5 * scale)
    for t in (tx, tb, ty):
        t.free()
    for tag in ("f32", "bf16"):
        f = load(f"softmax_16x256_{tag}.npz")
        x = Tensor.from_numpy(dev, q, f["x"], tag)
        s, m, sm = Tensor(dev, (16,), "f32"), Tensor(dev, (16,), "f32"), Tensor(dev, (16, 256), tag)
        kernels.row_reduce_softmax(q, x, s, m, sm)
        assert np.array_equal(m.numpy(q), f["row_max"])
        xf = rng.bf16_to_f32(f["x"]) if tag == "bf16" else f["x"]
        assert np.all(np.abs(s.numpy(q) - f["row_sum"]) <= 1e-5 * np.abs(xf).sum(1))
        a = rng.bf16_to_f32(sm.numpy(q)) if tag == "bf16" else sm.numpy(q)
        b = rng.bf16_to_f32(f["softmax"]) if tag == "bf16" else f["softmax"]
        assert np.all(np.abs(a - b) <= (1e-2 if tag == "bf16" else 1e-5) * b)
        for t in (x, s, m, sm):
            t.free()


def test_gemm_and_int8_fixtures(dev, q):
    f = load("gemm_bf16_48x40x64_gelu.npz")
    tA, tB = Tensor.from_numpy(dev, q, f["A"], "bf16"), Tensor.from_numpy(dev, q, f["B"], "bf16")
    tC, tP = Tensor(dev, (48, 40), "bf16"), Tensor(dev, (48, 40), "f32")
    kernels.gemm_bf16(q, tA, tB, tC, False, True, _lib.EPI_GELU, tP)
    mag = np.abs(rng.bf16_to_f32(f["A"]).astype(np.float64)) @ np.abs(rng.bf16_to_f32(f["B"]).astype(np.float64)).T
    assert np.all(np.abs(tP.numpy(q) - f["pre"]) <= 1e-2 * mag)
    for t in (tA, tB, tC, tP):
        t.free()
    f = load("w8a8_16_128_96_64.npz")
    g = graph.w8a8_infer_graph(16, (128, 96, 64))
    exe = g.compile(dev)
    for k, v in (("X", f["x"]), ("W0", f["w0"]), ("S0", f["s0"]), ("W1", f["w1"]), ("S1", f["s1"])):
        exe.write(q, k, v)
    exe.run(q)
    assert np.array_equal(exe.read(q, "Y"), f["y"])
    exe.free()
