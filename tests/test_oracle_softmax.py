"""Pins the CPU oracle's row reductions + softmax (orc_row_reduce_softmax, orc_col_reduce)
against f64 numpy and the mathematical invariants of softmax."""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import rng, spec


@pytest.fixture(scope="module")
def small():
    x, orows, ocols = spec.softmax_inputs(rows=400, cols=512)
    return x, orows, ocols


def test_sums_and_max_vs_f64(small):
    x = small[0]
    s, m, sm = oracle.row_reduce_softmax(x)
    x64 = x.astype(np.float64)
    assert np.array_equal(m, x.max(axis=1))
    np.testing.assert_allclose(s, x64.sum(axis=1), rtol=0, atol=1e-7 * np.abs(x64).sum(axis=1).max())
    ref = np.exp(x64 - x64.max(axis=1, keepdims=True))
    ref /= ref.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(sm, ref, rtol=1e-6, atol=1e-12)


def test_softmax_invariants(small):
    x, orows, ocols = small
    _, _, sm = oracle.row_reduce_softmax(x)
    np.testing.assert_allclose(sm.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)
    assert np.array_equal(np.argmax(sm[orows], axis=1), ocols)  # injected +20 outliers dominate
    assert len(orows) == 4  # 1% of 400 rows
    # shift invariance: softmax(x + 3) == softmax(x) up to rounding
    _, _, sm2 = oracle.row_reduce_softmax((x + np.float32(3.0)).astype(np.float32))
    np.testing.assert_allclose(sm2, sm, rtol=1e-5, atol=1e-12)


def test_constant_row_and_one_column():
    x = np.full((3, 4096), 0.7, np.float32)
    s, m, sm = oracle.row_reduce_softmax(x)
    assert (sm == np.float32(1.0 / 4096)).all()
    assert (m == np.float32(0.7)).all()
    x1 = np.array([[5.0], [-3.0]], np.float32)
    s, m, sm = oracle.row_reduce_softmax(x1)
    assert (sm == 1.0).all() and np.array_equal(s, x1[:, 0]) and np.array_equal(m, x1[:, 0])


def test_bf16_rows():
    x, _, _ = spec.softmax_inputs(rows=64, cols=512)
    xb = rng.f32_to_bf16(x)
    s, m, sm = oracle.row_reduce_softmax(xb)
    xf = rng.bf16_to_f32(xb).astype(np.float64)
    np.testing.assert_allclose(s, xf.sum(axis=1), atol=1e-6 * np.abs(xf).sum(axis=1).max())
    assert np.array_equal(m, rng.bf16_to_f32(xb).max(axis=1))
    ref = np.exp(xf - xf.max(axis=1, keepdims=True))
    ref /= ref.sum(axis=1, keepdims=True)
    got = rng.bf16_to_f32(sm).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2 ** -8 * np.abs(ref) + 1e-30)  # within half a bf16 ulp + f32 error


def test_col_reduce():
    x, _, _ = spec.softmax_inputs(rows=300, cols=200)
    cs, cm = oracle.col_reduce(x)
    np.testing.assert_allclose(cs, x.astype(np.float64).sum(axis=0), atol=1e-5)
    assert np.array_equal(cm, x.max(axis=0))


def test_outlier_placement_full_config():
    # the config-3 generator at full size: 164 outlier rows, sorted, columns in range
    _, orows, ocols = spec.softmax_inputs(rows=16384, cols=64)
    assert len(orows) == 164 and np.all(np.diff(orows) > 0) and ocols.max() < 64
