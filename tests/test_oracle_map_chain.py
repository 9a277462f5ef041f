"""Pins the CPU oracle's map chain (orc_map_chain) against f64 numpy evaluation of the same
expression, special values, and the map-chain compiler's register programs."""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, mapchain as mc, spec


def chain_tolerance_ok(got, x, bias, rel=1e-6):
    """|got - y64| <= rel * (|tanh(.) exp(.)| + |bias|): the error allowed is relative to the
    magnitudes of the two summands, so cancellation in the final add does not inflate it."""
    x64 = x.astype(np.float64)
    u = np.float32(spec.MAP_A) * x  # the f32 rounding of a*x+b is part of the spec
    u = (u + np.float32(spec.MAP_B)).astype(np.float64)
    te = np.tanh(u) * np.exp(-(x64 * x64))
    y = te + bias.astype(np.float64)[None, :]
    scale = np.abs(te) + np.abs(bias.astype(np.float64))[None, :]
    return np.all(np.abs(got.astype(np.float64) - y) <= rel * scale + 1e-37)


def test_compiler_program_for_config2():
    prog = mc.compile(spec.map_chain_expr())
    ops = [c[0] for c in prog.code]
    assert ops == ["load", "mul_imm", "add_imm", "tanh", "square", "neg", "exp", "mul", "load", "add"]
    assert prog.bcast == {0: _lib.BCAST_FULL, 1: _lib.BCAST_ROW}
    assert prog.out_reg == 0


def test_config2_chain_vs_f64():
    x, bias = spec.map_chain_inputs(rows=256, cols=512)
    prog = mc.compile(spec.map_chain_expr())
    got = oracle.map_chain(prog, [x, bias], 256, 512)
    assert chain_tolerance_ok(got, x, bias, rel=1e-6)


def test_special_values():
    prog = mc.compile(spec.map_chain_expr())
    x = np.zeros((4, 8), np.float32)
    x[1] = 50.0  # exp(-2500) underflows to 0: y == bias exactly
    x[2] = -50.0
    bias = np.linspace(-1, 1, 8, dtype=np.float32)
    got = oracle.map_chain(prog, [x, bias], 4, 8)
    assert np.array_equal(got[1], bias) and np.array_equal(got[2], bias)
    np.testing.assert_allclose(got[0], np.tanh(np.float64(spec.MAP_B)) + bias, rtol=1e-6)


def test_generic_ops_and_broadcasts():
    rng = np.random.default_rng(3)
    rows, cols = 33, 47
    a = rng.standard_normal((rows, cols)).astype(np.float32)
    colv = rng.uniform(0.5, 2, rows).astype(np.float32)
    rowv = rng.uniform(0.5, 2, cols).astype(np.float32)
    sc = np.array([1.5], np.float32)
    A, Cv, Rv, S = mc.Input(0), mc.Input(1, "col"), mc.Input(2, "row"), mc.Input(3, "scalar")
    e = mc.sigmoid(A) * Cv - mc.relu(A) / Rv + mc.maximum(mc.abs(A), S) + mc.fma(A, Rv, Cv) + mc.sqrt(mc.abs(A) + 1.0)
    prog = mc.compile(e)
    got = oracle.map_chain(prog, [a, colv, rowv, sc], rows, cols)
    a64 = a.astype(np.float64)
    ref = (1 / (1 + np.exp(-a64))) * colv[:, None] - np.maximum(a64, 0) / rowv[None, :] \
        + np.maximum(np.abs(a64), 1.5) + (a64 * rowv[None, :] + colv[:, None]) + np.sqrt(np.abs(a64) + 1)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)


def test_row_range_matches_full():
    x, bias = spec.map_chain_inputs(rows=64, cols=64)
    prog = mc.compile(spec.map_chain_expr())
    full = oracle.map_chain(prog, [x, bias], 64, 64)
    part = oracle.map_chain(prog, [x, bias], 64, 64, row_range=(10, 20))
    assert np.array_equal(full[10:20], part)


def test_compiler_limits():
    x = mc.Input(0)
    # right-deep sum: v1 + (v2 + (... + v9)) keeps all nine products and x live at once
    vals = [x * float(k) for k in range(1, 10)]
    e = vals[-1]
    for v in reversed(vals[:-1]):
        e = v + e
    with pytest.raises(ValueError, match="live registers"):
        mc.compile(e)
    # left-deep sum of 20 exp terms: 60 instructions
    e = mc.exp(x * 1.0)
    for k in range(2, 21):
        e = e + mc.exp(x * float(k))
    with pytest.raises(ValueError, match="instructions"):
        mc.compile(e)
    # a left-deep chain of 8 terms fits in both limits
    e = mc.exp(x * 1.0)
    for k in range(2, 9):
        e = e + mc.exp(x * float(k))
    assert len(mc.compile(e).code) <= 32
