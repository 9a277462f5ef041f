"""GPU parity of the fused map chain (vdsl_op_map_chain) against the CPU oracle.

Tolerance (f32 elementwise, 1e-5 relative): |gpu - oracle| <= 1e-5 * S, where S is the sum of the
magnitudes of the terms of the final addition (|tanh(.) exp(.)| + |bias| for the config-2
chain), so that cancellation in the last add cannot turn a few-ulp error into an unbounded
relative one."""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, mapchain as mc, spec
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
REL = 1e-5


def config2_scale(x, bias):
    x64 = x.astype(np.float64)
    u = ((np.float32(spec.MAP_A) * x) + np.float32(spec.MAP_B)).astype(np.float64)
    return np.abs(np.tanh(u) * np.exp(-(x64 * x64))) + np.abs(bias.astype(np.float64))[None, :]


def run_chain(dev, q, prog, inputs, rows, cols):
    ts = [Tensor.from_numpy(dev, q, np.ascontiguousarray(a, np.float32)) for a in inputs]
    out = Tensor(dev, (rows, cols), "f32")
    out.buffer.fill_u32(q, 0x7FC00000)
    kernels.map_chain(q, prog, ts, out)
    got = out.numpy(q)
    for t in ts + [out]:
        t.free()
    return got


@pytest.mark.parametrize("rows,cols", [(512, 1024), (3, 4096), (130, 1028)])
def test_config2_chain_small(dev, q, rows, cols):
    x, bias = spec.map_chain_inputs(rows, cols)
    prog = mc.compile(spec.map_chain_expr())
    got = run_chain(dev, q, prog, [x, bias], rows, cols)
    ref = oracle.map_chain(prog, [x, bias], rows, cols)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= REL * config2_scale(x, bias)), float(np.max(err / config2_scale(x, bias)))


def test_config2_full_size_sampled(dev, q):
    rows = cols = 8192
    x, bias = spec.map_chain_inputs(rows, cols)
    prog = mc.compile(spec.map_chain_expr())
    got = run_chain(dev, q, prog, [x, bias], rows, cols)
    assert np.isfinite(got).all()
    # oracle on a seeded sample of rows, including the first and last
    rr = sorted({0, rows - 1, *np.random.default_rng(11).integers(0, rows, 62).tolist()})
    for r in rr:
        ref = oracle.map_chain(prog, [x, bias], rows, cols, row_range=(r, r + 1))[0]
        sc = config2_scale(x[r:r + 1], bias)[0]
        assert np.all(np.abs(got[r].astype(np.float64) - ref) <= REL * sc), f"row {r}"
    # size-independent property: where exp(-x^2) underflows (|x| > ~10) y == bias exactly;
    # elsewhere y - bias stays within tanh's range
    d = got.astype(np.float64) - bias[None, :]
    assert np.all(np.abs(d) <= 1.0 + 1e-6)


def test_generic_program_and_broadcasts(dev, q):
    rng = np.random.default_rng(5)
    rows, cols = 67, 1000
    a = rng.standard_normal((rows, cols)).astype(np.float32)
    colv = rng.uniform(0.5, 2, rows).astype(np.float32)
    rowv = rng.uniform(0.5, 2, cols).astype(np.float32)
    sc = np.array([1.5], np.float32)
    A, Cv, Rv, S = mc.Input(0), mc.Input(1, "col"), mc.Input(2, "row"), mc.Input(3, "scalar")
    e = mc.sigmoid(A) * Cv - mc.relu(A) / Rv + mc.maximum(mc.abs(A), S) + mc.fma(A, Rv, Cv) + mc.sqrt(mc.abs(A) + 1.0)
    prog = mc.compile(e)
    got = run_chain(dev, q, prog, [a, colv, rowv, sc], rows, cols)
    ref = oracle.map_chain(prog, [a, colv, rowv, sc], rows, cols)
    np.testing.assert_allclose(got, ref, rtol=REL, atol=REL * np.abs(ref).max())


def test_odd_columns_scalar_path(dev, q):
    rng = np.random.default_rng(9)
    rows, cols = 19, 1001
    a = rng.standard_normal((rows, cols)).astype(np.float32)
    bias = rng.uniform(-1, 1, cols).astype(np.float32)
    prog = mc.compile(spec.map_chain_expr())
    got = run_chain(dev, q, prog, [a, bias], rows, cols)
    ref = oracle.map_chain(prog, [a, bias], rows, cols)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= REL * config2_scale(a, bias))


def test_every_opcode(dev, q):
    rng = np.random.default_rng(2)
    rows, cols = 8, 256
    a = rng.uniform(0.1, 3, (rows, cols)).astype(np.float32)
    b = rng.uniform(-2, 2, (rows, cols)).astype(np.float32)
    A, B = mc.Input(0), mc.Input(1)
    exprs = [-A, mc.abs(B), A * A, mc.exp(B), mc.log(A), mc.tanh(B), mc.sigmoid(B), mc.relu(B), mc.sqrt(A),
             mc.recip(A), A + B, A - B, A * B, B / A, mc.maximum(A, B), mc.minimum(A, B), mc.fma(A, B, A),
             A * 0.3, B + 0.7, mc.const(2.5) + A * 0]
    for e in exprs:
        prog = mc.compile(e)
        got = run_chain(dev, q, prog, [a, b][:prog.n_inputs], rows, cols)
        ref = oracle.map_chain(prog, [a, b][:prog.n_inputs], rows, cols)
        np.testing.assert_allclose(got, ref, rtol=REL, atol=1e-30, err_msg=str(prog.code))


@pytest.mark.parametrize("cols_pad", [0, 1])
def test_transcendentals_ranges_and_specials(dev, q, cols_pad):
    """exp / tanh / sigmoid over their whole f32 range, across the tanh series-to-exponential switch
    at |u| = 0.4, and at +-inf, NaN, +-0 and results in the subnormal range; cols_pad = 1 makes the
    row width odd (the one-element path)."""
    vals = np.concatenate([np.linspace(-110, 95, 4096), np.linspace(-1, 1, 4097), np.linspace(0.39, 0.41, 512),
                           -np.linspace(0.39, 0.41, 512), np.logspace(-38, 1, 1024), -np.logspace(-38, 1, 1024),
                           [np.inf, -np.inf, np.nan, 0.0, -0.0, 88.7, 88.8, 89.0, -87.3, -103.0, -104.0]])
    cols = len(vals) + (len(vals) + cols_pad) % 2  # even or odd row width
    a = np.zeros((2, cols), np.float32)
    a[0, :len(vals)] = vals
    a[1, :len(vals)] = vals[::-1]
    A = mc.Input(0)
    for e in (mc.exp(A), mc.tanh(A), mc.sigmoid(A)):
        prog = mc.compile(e)
        got = run_chain(dev, q, prog, [a], 2, cols).astype(np.float64)
        ref = oracle.map_chain(prog, [a], 2, cols).astype(np.float64)
        assert np.array_equal(np.isnan(got), np.isnan(ref)), str(prog.code)
        inf = np.isinf(ref)
        assert np.array_equal(got[inf], ref[inf]), str(prog.code)
        fin = np.isfinite(ref)
        # results below the smallest normal f32 may be flushed by the hardware exp2
        assert np.all(np.abs(got[fin] - ref[fin]) <= REL * np.abs(ref[fin]) + 1.2e-38), str(prog.code)


def test_invalid_program_rejected(dev, q):
    prog = mc.compile(spec.map_chain_expr())
    prog.code[1] = ("mul_imm", 9, 0, 0, 0, 1.0)  # register 9 does not exist
    x = Tensor(dev, (4, 4), "f32")
    bias = Tensor(dev, (4,), "f32")
    out = Tensor(dev, (4, 4), "f32")
    with pytest.raises(_lib.VdslError) as ei:
        kernels.map_chain(q, prog, [x, bias], out)
    assert ei.value.status == -1
    for t in (x, bias, out):
        t.free()
