"""GPU parity of row reductions + softmax (vdsl_op_row_reduce_softmax) and column reductions.

Tolerances: row max exact; row sum |gpu - oracle| <= 1e-5 * sum|x|; f32 softmax 1e-5 relative;
bf16 softmax within 1e-2 relative (the bf16 outputs may differ by one bf16 ulp where the f32
values straddle a rounding boundary)."""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import kernels, rng, spec
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu


def run(dev, q, xh, dtype):
    rows, cols = xh.shape
    x = Tensor.from_numpy(dev, q, xh, dtype)
    s, m, sm = Tensor(dev, (rows,), "f32"), Tensor(dev, (rows,), "f32"), Tensor(dev, (rows, cols), dtype)
    for t in (s, m, sm):
        t.buffer.fill_u32(q, 0x7FC00000)
    kernels.row_reduce_softmax(q, x, s, m, sm)
    out = s.numpy(q), m.numpy(q), sm.numpy(q)
    for t in (x, s, m, sm):
        t.free()
    return out


def check(xh, got, ref, bf16):
    gs, gm, gsm = got
    rs, rm, rsm = ref
    xf = rng.bf16_to_f32(xh) if bf16 else xh
    assert np.array_equal(gm, rm)
    l1 = np.abs(xf.astype(np.float64)).sum(axis=1)
    assert np.all(np.abs(gs.astype(np.float64) - rs) <= 1e-5 * l1 + 1e-30)
    if bf16:
        a, b = rng.bf16_to_f32(gsm).astype(np.float64), rng.bf16_to_f32(rsm).astype(np.float64)
        assert np.all(np.abs(a - b) <= 1e-2 * np.abs(b) + 1e-38)
    else:
        np.testing.assert_allclose(gsm, rsm, rtol=1e-5, atol=1e-38)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("cols", [4096, 256, 512, 1000, 2048, 8192, 16384, 3])
@pytest.mark.parametrize("rows", [130, 160])
def test_softmax_shapes(dev, q, cols, bf16, rows):
    """Row counts that fill the last 4-row block partially (130) and exactly (160); widths that take
    the one-wave-per-row kernel (256, 512), the one-block-per-row kernel with 1, 2 and 4 vectors per
    lane (2048 f32, 4096, 8192, 16384 bf16) and the streaming kernel (1000, 3)."""
    x, _, _ = spec.softmax_inputs(rows=rows, cols=cols)
    xh = rng.f32_to_bf16(x) if bf16 else x
    got = run(dev, q, xh, "bf16" if bf16 else "f32")
    check(xh, got, oracle.row_reduce_softmax(xh), bf16)


@pytest.mark.parametrize("bf16", [False, True])
def test_config3_full_size(dev, q, bf16):
    x, orows, ocols = spec.softmax_inputs()
    xh = rng.f32_to_bf16(x) if bf16 else x
    got = run(dev, q, xh, "bf16" if bf16 else "f32")
    gs, gm, gsm = got
    # every row and element against the oracle (the whole [16384][4096] workload)
    check(xh, got, oracle.row_reduce_softmax(xh), bf16)
    # size-independent properties on every row
    smf = rng.bf16_to_f32(gsm) if bf16 else gsm
    tol = 3e-2 if bf16 else 1e-4
    assert np.all(np.abs(smf.astype(np.float64).sum(axis=1) - 1.0) <= tol)
    assert np.array_equal(np.argmax(smf[orows], axis=1), ocols)
    xf = rng.bf16_to_f32(xh) if bf16 else xh
    assert np.array_equal(gm, xf.max(axis=1))


@pytest.mark.parametrize("nrows", [8, 16])
def test_only_some_outputs_and_empty(dev, q, nrows):
    x = np.random.default_rng(4).standard_normal((nrows, 4096)).astype(np.float32)
    tx = Tensor.from_numpy(dev, q, x)
    m = Tensor(dev, (nrows,), "f32")
    kernels.row_reduce_softmax(q, tx, row_max=m)
    assert np.array_equal(m.numpy(q), x.max(axis=1))
    e = Tensor(dev, (0, 16), "f32")
    kernels.row_reduce_softmax(q, e)  # zero rows: nothing to do
    for t in (tx, m, e):
        t.free()


@pytest.mark.parametrize("bf16", [False, True])
def test_col_reduce(dev, q, bf16):
    x, _, _ = spec.softmax_inputs(rows=1000, cols=333)
    xh = rng.f32_to_bf16(x) if bf16 else x
    tx = Tensor.from_numpy(dev, q, xh, "bf16" if bf16 else "f32")
    cs, cm = Tensor(dev, (333,), "f32"), Tensor(dev, (333,), "f32")
    kernels.col_reduce(q, tx, cs, cm)
    rs, rm = oracle.col_reduce(xh)
    xf = rng.bf16_to_f32(xh) if bf16 else xh
    assert np.array_equal(cm.numpy(q), rm)
    assert np.all(np.abs(cs.numpy(q).astype(np.float64) - rs) <= 1e-5 * np.abs(xf.astype(np.float64)).sum(axis=0))
    for t in (tx, cs, cm):
        t.free()
