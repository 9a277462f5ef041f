"""GPU parity of the MFMA GEMMs, layout ops and autodiff blocks against the CPU oracle.

Tolerances: bf16 GEMM (f32 accumulate) - Frobenius-relative error <= 1e-2 and elementwise
|gpu - oracle| <= 1e-2 * (|A| |B|)[m][n] (the magnitude the sum was formed from); bf16 outputs
are compared after converting both sides to f32 with a one-bf16-ulp allowance.  int8: the int32
accumulators and the dequantised outputs are bit-exact.  Layout ops: bit-exact.
"""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, rng
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
F32, BF16 = 0, 1


def bf16_rand(shape, seed, lo=-1.0, hi=1.0):
    return rng.f32_to_bf16(rng.uniform(seed, int(np.prod(shape)), lo, hi)).reshape(shape)


def gemm_gpu(dev, q, A, B, ta, tb, c_dtype="f32", epi=_lib.EPI_NONE, want_pre=False):
    K, M = A.shape if ta else A.shape[::-1]
    N = B.shape[0] if tb else B.shape[1]
    tA, tB = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16")
    tC = Tensor(dev, (M, N), c_dtype)
    tC.buffer.fill_u32(q, 0x7FC07FC0)
    pre = Tensor(dev, (M, N), "f32") if want_pre else None
    wsb = kernels.gemm_bf16_workspace_bytes(ta, tb, M, N, K)
    ws = Tensor(dev, (max(1, wsb),), "i8") if wsb else None
    kernels.gemm_bf16(q, tA, tB, tC, ta, tb, epi, pre, ws)
    out = tC.numpy(q)
    p = pre.numpy(q) if want_pre else None
    for t in (tA, tB, tC, pre, ws):
        if t is not None:
            t.free()
    return (out, p) if want_pre else out


def magnitude(A, B, ta, tb):
    Af = np.abs(rng.bf16_to_f32(A).astype(np.float64))
    Bf = np.abs(rng.bf16_to_f32(B).astype(np.float64))
    return (Af.T if ta else Af) @ (Bf.T if tb else Bf)


def assert_gemm_close(got, ref, mag):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    fro = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert fro <= 1e-2, fro
    assert np.all(np.abs(got - ref) <= 1e-2 * mag + 1e-30), float(np.max(np.abs(got - ref) / (mag + 1e-30)))


def test_mfma_single_tile_layout(dev, q):
    # one 32x32x16 MFMA worth of work: checks the operand/accumulator lane layout exactly
    r = np.random.default_rng(0)
    A = rng.f32_to_bf16(r.integers(-4, 5, (32, 16)).astype(np.float32))
    B = rng.f32_to_bf16(r.integers(-4, 5, (32, 16)).astype(np.float32))
    got = gemm_gpu(dev, q, A, B, 0, 1)
    ref = rng.bf16_to_f32(A).astype(np.int64) @ rng.bf16_to_f32(B).astype(np.int64).T
    assert np.array_equal(got, ref.astype(np.float32))


def test_exact_small_integers_large_tile(dev, q):
    r = np.random.default_rng(1)
    A = rng.f32_to_bf16(r.integers(-8, 9, (256, 512)).astype(np.float32))
    B = rng.f32_to_bf16(r.integers(-8, 9, (384, 512)).astype(np.float32))
    got = gemm_gpu(dev, q, A, B, 0, 1)
    ref = rng.bf16_to_f32(A).astype(np.int64) @ rng.bf16_to_f32(B).astype(np.int64).T
    assert np.array_equal(got, ref.astype(np.float32))  # |sums| < 2^24: exact in f32


@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(256, 384, 192), (130, 70, 72), (1, 1, 8), (300, 129, 1000), (64, 64, 13)])
def test_layouts_and_edges(dev, q, ta, tb, M, N, K):
    A = bf16_rand((K, M) if ta else (M, K), M * 7 + K)
    B = bf16_rand((N, K) if tb else (K, N), N * 3 + K)
    got = gemm_gpu(dev, q, A, B, ta, tb)
    ref = oracle.gemm_bf16(A, B, ta, tb)
    assert_gemm_close(got, ref, magnitude(A, B, ta, tb))


@pytest.mark.parametrize("shape", [(256, 128, 256), (200, 100, 96), (64, 48, 40)])
@pytest.mark.parametrize("epi", [_lib.EPI_GELU, _lib.EPI_RELU])
def test_epilogues_bf16_out_and_pre(dev, q, epi, shape):
    """Whole tiles (the fixed-variant epilogue), ragged tiles on the direct-to-LDS loop and a K that
    takes the register-staged loop (both through the per-element epilogue)."""
    M, N, K = shape
    A, B = bf16_rand((M, K), 11, -2, 2), bf16_rand((N, K), 12, -2, 2)
    out, pre = gemm_gpu(dev, q, A, B, 0, 1, "bf16", epi, want_pre=True)
    rout, rpre = oracle.gemm_bf16(A, B, 0, 1, c_dtype=BF16, epilogue=epi, want_pre=True)
    mag = magnitude(A, B, 0, 1)
    assert_gemm_close(pre, rpre, mag)
    a, b = rng.bf16_to_f32(out).astype(np.float64), rng.bf16_to_f32(rout).astype(np.float64)
    assert np.all(np.abs(a - b) <= 1e-2 * np.maximum(np.abs(b), mag * 1e-2) + 1e-30)


def test_config4_shape_gemm(dev, q):
    """One forward GEMM of config 4 at full size, checked on sampled rows."""
    from vernondsl_amd import spec
    x, w1, _, _ = spec.mlp_inputs()
    out, pre = gemm_gpu(dev, q, x, w1, 0, 1, "bf16", _lib.EPI_GELU, want_pre=True)
    for r in (0, 1000, 2047):
        rout, rpre = oracle.gemm_bf16(x, w1, 0, 1, c_dtype=BF16, epilogue=_lib.EPI_GELU, want_pre=True,
                                      row_range=(r, r + 1))
        mag = magnitude(x[r:r + 1], w1, 0, 1)
        assert_gemm_close(pre[r:r + 1], rpre, mag)


@pytest.mark.parametrize("xdt,ydt", [("f32", "f32"), ("f32", "bf16"), ("bf16", "f32"), ("bf16", "bf16")])
def test_gelu_fwd(dev, q, xdt, ydt):
    x = np.concatenate([np.random.default_rng(7).normal(0, 3, 10000), np.linspace(-12, 12, 2001),
                        [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30, 30.0, -30.0]]).astype(np.float32)
    xh = rng.f32_to_bf16(x) if xdt == "bf16" else x
    tx = Tensor.from_numpy(dev, q, xh, xdt)
    ty = Tensor(dev, x.shape, ydt)
    kernels.gelu_fwd(q, tx, ty)
    got = ty.numpy(q)
    ref = oracle.gelu_fwd(xh, y_bf16=(ydt == "bf16"))
    g = (rng.bf16_to_f32(got) if ydt == "bf16" else got).astype(np.float64)
    r = (rng.bf16_to_f32(ref) if ydt == "bf16" else ref).astype(np.float64)
    assert np.array_equal(np.isnan(g), np.isnan(r))
    fin = ~np.isnan(r)
    tol = 1e-2 if ydt == "bf16" else 1e-5
    bad = np.abs(g[fin] - r[fin]) > tol * np.abs(r[fin]) + 1e-37
    xf = (rng.bf16_to_f32(xh) if xdt == "bf16" else xh)[fin]
    assert not bad.any(), list(zip(xf[bad][:5].tolist(), g[fin][bad][:5].tolist(), r[fin][bad][:5].tolist()))
    if xdt == ydt:  # in place
        kernels.gelu_fwd(q, tx, tx)
        assert np.array_equal(tx.numpy(q), got, equal_nan=True) if ydt == "f32" else np.array_equal(tx.numpy(q), got)
    tx.free()
    ty.free()


def test_transpose_and_cast(dev, q):
    # odd extents take the element-wise kernel; even bf16 extents the 2x2-pair kernel (one partial
    # 128x128 tile in each direction for (130, 258), (256, 2050)); bf16 extents that are multiples
    # of 8 the 16-byte kernel (partial 64x64 tiles for (72, 200), a single 8x8 corner for (8, 8))
    for shape in ((64, 64), (37, 1000), (1, 5), (513, 129), (2, 2), (130, 258), (256, 2050), (72, 200), (8, 8),
                  (2048, 4096)):
        x = rng.normal(3, int(np.prod(shape))).reshape(shape)
        for dt, h in (("f32", x), ("bf16", rng.f32_to_bf16(x))):
            ts = Tensor.from_numpy(dev, q, h, dt)
            td = Tensor(dev, shape[::-1], dt)
            kernels.transpose(q, ts, td)
            assert np.array_equal(td.numpy(q), h.T)
            ts.free()
            td.free()
    x = rng.normal(4, 10001)
    tx = Tensor.from_numpy(dev, q, x)
    tb = Tensor(dev, (10001,), "bf16")
    tf = Tensor(dev, (10001,), "f32")
    kernels.cast(q, tx, tb)
    kernels.cast(q, tb, tf)
    assert np.array_equal(tb.numpy(q), rng.f32_to_bf16(x))
    assert np.array_equal(tf.numpy(q), rng.bf16_to_f32(rng.f32_to_bf16(x)))
    for t in (tx, tb, tf):
        t.free()


# (70, 33): the element-wise kernel; the others the 16-byte kernel (rows % 8 == 0, cols % 4 == 0),
# (72, 100) and (8, 4) with partial tiles
@pytest.mark.parametrize("rows,cols", [(128, 192), (70, 33), (72, 100), (8, 4), (2048, 4096)])
def test_gelu_bwd(dev, q, rows, cols):
    dh = rng.normal(21, rows * cols).reshape(rows, cols) * np.float32(1e-3)
    pre = rng.normal(22, rows * cols, 0, 2).reshape(rows, cols)
    tdh, tpre = Tensor.from_numpy(dev, q, dh), Tensor.from_numpy(dev, q, pre)
    tda, tdat = Tensor(dev, (rows, cols), "bf16"), Tensor(dev, (cols, rows), "bf16")
    kernels.gelu_bwd(q, tdh, tpre, tda, tdat)
    da, dat = tda.numpy(q), tdat.numpy(q)
    rda, _ = oracle.gelu_bwd(dh, pre)
    a, b = rng.bf16_to_f32(da).astype(np.float64), rng.bf16_to_f32(rda).astype(np.float64)
    # 1e-2 relative, with a floor of |dh| * 2^-20: GELU' is O(1) and its f32 evaluation carries an
    # absolute error of a few 2^-24, which dominates where GELU'(pre) itself underflows (pre << 0)
    assert np.all(np.abs(a - b) <= 1e-2 * np.abs(b) + np.abs(dh.astype(np.float64)) * 2.0 ** -20)
    assert np.array_equal(dat, da.T)
    for t in (tdh, tpre, tda, tdat):
        t.free()


@pytest.mark.parametrize("rows,cols", [(128, 192), (70, 33), (72, 100), (2048, 4096)])
def test_relu_bwd_bit_exact(dev, q, rows, cols):
    """A select and one RNE: bit for bit, including pre = +-0, NaN and denormal, infinite dh."""
    dh = rng.normal(23, rows * cols).reshape(rows, cols)
    pre = rng.normal(24, rows * cols).reshape(rows, cols)
    pre[0, :4] = [0.0, -0.0, np.nan, 1e-45]
    dh[1, :2] = [np.inf, -np.inf]
    tdh, tpre = Tensor.from_numpy(dev, q, dh), Tensor.from_numpy(dev, q, pre)
    tda, tdat = Tensor(dev, (rows, cols), "bf16"), Tensor(dev, (cols, rows), "bf16")
    kernels.gelu_bwd(q, tdh, tpre, tda, tdat, act="relu")
    rda, rdat = oracle.relu_bwd(dh, pre)
    assert np.array_equal(tda.numpy(q), rda) and np.array_equal(tdat.numpy(q), rdat)
    for t in (tdh, tpre, tda, tdat):
        t.free()


# n % 4 == 0 takes the four-element kernel, the others the element-wise one
@pytest.mark.parametrize("n", [0, 1, 7, 4096, 100003, 2048 * 4096])
@pytest.mark.parametrize("dts", [("f32", "f32", "f32"), ("bf16", "bf16", "bf16"), ("bf16", "f32", "f32"),
                                 ("f32", "bf16", "bf16"), ("bf16", "bf16", "f32")])
def test_add_bit_exact(dev, q, n, dts):
    r = np.random.default_rng(n + 7)
    host = []
    for k, dt in enumerate(dts[:2]):
        x = r.standard_normal(n).astype(np.float32) * np.float32(10.0 ** -k)
        host.append(rng.f32_to_bf16(x) if dt == "bf16" else x)
    ta, tb = (Tensor.from_numpy(dev, q, h, dt) for h, dt in zip(host, dts[:2]))
    out = Tensor(dev, (n,), dts[2])
    if out.buffer.nbytes >= 4:  # NaN poison over whole words: every element must be written
        out.buffer.fill_u32(q, 0x7FC07FC0, 0, out.buffer.nbytes // 4 * 4)
    kernels.add(q, ta, tb, out)
    ref = oracle.add(host[0], host[1], oracle.BF16 if dts[2] == "bf16" else oracle.F32)
    assert np.array_equal(out.numpy(q).view(np.uint16 if dts[2] == "bf16" else np.uint32),
                          ref.view(np.uint16 if dts[2] == "bf16" else np.uint32))
    if n and dts[0] == dts[2]:  # in place: out is a
        kernels.add(q, ta, tb, ta)
        assert np.array_equal(ta.numpy(q).view(np.uint8), ref.view(np.uint8))
    for t in (ta, tb, out):
        t.free()


def test_add_rejects_mismatches(dev, q):
    a, b, short = Tensor(dev, (64,), "f32"), Tensor(dev, (64,), "bf16"), Tensor(dev, (32,), "f32")
    with pytest.raises(ValueError):
        kernels.add(q, a, short, a)
    # out is an operand read as another dtype: refused (a as a, then a as b, stored as bf16)
    with pytest.raises(_lib.VdslError, match="in-place"):
        _lib.call("vdsl_op_add", q.handle, 64, F32, a.handle, BF16, b.handle, BF16, a.handle)
    with pytest.raises(_lib.VdslError, match="in-place"):
        _lib.call("vdsl_op_add", q.handle, 64, BF16, b.handle, F32, a.handle, BF16, a.handle)
    with pytest.raises(_lib.VdslError, match="f32 and bf16"):
        _lib.call("vdsl_op_add", q.handle, 64, 2, a.handle, F32, a.handle, F32, a.handle)
    for t in (a, b, short):
        t.free()


@pytest.mark.parametrize("rows,cols", [(128, 192), (70, 33), (72, 100), (8, 4), (2048, 4096)])
def test_mse(dev, q, rows, cols):
    y = rng.normal(31, rows * cols).reshape(rows, cols)
    t = rng.normal(32, rows * cols).reshape(rows, cols)
    ty, tt = Tensor.from_numpy(dev, q, y), Tensor.from_numpy(dev, q, t)
    loss = Tensor(dev, (1,), "f32")
    dy, dyt = Tensor(dev, (rows, cols), "bf16"), Tensor(dev, (cols, rows), "bf16")
    part = Tensor(dev, (kernels.mse_partials_count(rows, cols),), "f32")
    kernels.mse_fwd_bwd(q, ty, tt, loss, dy, dyt, part)
    rl, rdy, _ = oracle.mse_fwd_bwd(y, t)
    assert abs(float(loss.numpy(q)[0]) - rl) <= 1e-6 * abs(rl)
    g = dy.numpy(q)
    assert np.array_equal(g, rdy)  # dy = (y - t) * 2^-k exactly, then RNE: bit-exact
    assert np.array_equal(dyt.numpy(q), g.T)
    for x in (ty, tt, loss, dy, dyt, part):
        x.free()


@pytest.mark.parametrize("rows,cols", [(72, 100), (70, 33)])
def test_optional_outputs_absent(dev, q, rows, cols):
    """gelu_bwd without da_t, MSE without dy or without dy_t: the outputs that are given match the
    full call, the loss is the same."""
    dh = rng.normal(51, rows * cols).reshape(rows, cols)
    pre = rng.normal(52, rows * cols).reshape(rows, cols)
    tdh, tpre = Tensor.from_numpy(dev, q, dh), Tensor.from_numpy(dev, q, pre)
    da1, da2, dat = Tensor(dev, (rows, cols), "bf16"), Tensor(dev, (rows, cols), "bf16"), Tensor(dev, (cols, rows), "bf16")
    kernels.gelu_bwd(q, tdh, tpre, da1, dat)
    kernels.gelu_bwd(q, tdh, tpre, da2, None)
    assert np.array_equal(da1.numpy(q), da2.numpy(q))
    part = Tensor(dev, (kernels.mse_partials_count(rows, cols),), "f32")
    l1, l2, l3 = (Tensor(dev, (1,), "f32") for _ in range(3))
    dy1, dyt1 = Tensor(dev, (rows, cols), "bf16"), Tensor(dev, (cols, rows), "bf16")
    dy2, dyt3 = Tensor(dev, (rows, cols), "bf16"), Tensor(dev, (cols, rows), "bf16")
    kernels.mse_fwd_bwd(q, tdh, tpre, l1, dy1, dyt1, part)
    kernels.mse_fwd_bwd(q, tdh, tpre, l2, dy2, None, part)
    call = _lib.call
    call("vdsl_op_mse_fwd_bwd", q.handle, rows, cols, tdh.handle, tpre.handle, l3.handle, None, dyt3.handle, part.handle)
    assert l1.numpy(q)[0] == l2.numpy(q)[0] == l3.numpy(q)[0]
    assert np.array_equal(dy1.numpy(q), dy2.numpy(q))
    assert np.array_equal(dyt1.numpy(q), dyt3.numpy(q))
    for t in (tdh, tpre, da1, da2, dat, part, l1, l2, l3, dy1, dyt1, dy2, dyt3):
        t.free()


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 4096), (300, 544, 256), (129, 96, 512)])
def test_gemm_bf16_packed_bit_identical(dev, q, M, N, K):
    """The packed-weight GEMM equals the row-major NT GEMM bit for bit (same k-steps, same order),
    with f32 output and with the GELU epilogue (bf16 out + f32 pre-activation), whole and ragged
    tiles; the packed weights hold the same bytes."""
    A = bf16_rand((M, K), 101)
    B = bf16_rand((N, K), 102)
    tA, tB = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16")
    tBp = Tensor(dev, (N, K), "bf16")
    kernels.pack_bf16_weights(q, tB, tBp)
    assert np.array_equal(np.sort(tBp.numpy(q).reshape(-1)), np.sort(B.reshape(-1)))
    outs = []
    for packed in (False, True):
        c32, h, pre = Tensor(dev, (M, N), "f32"), Tensor(dev, (M, N), "bf16"), Tensor(dev, (M, N), "f32")
        for t in (c32, h, pre):
            t.buffer.fill_u32(q, 0x7FC07FC0)
        if packed:
            kernels.gemm_bf16_packed(q, tA, tBp, c32)
            kernels.gemm_bf16_packed(q, tA, tBp, h, _lib.EPI_GELU, pre)
        else:
            kernels.gemm_bf16(q, tA, tB, c32, False, True)
            kernels.gemm_bf16(q, tA, tB, h, False, True, _lib.EPI_GELU, pre)
        outs.append([t.numpy(q) for t in (c32, h, pre)])
        for t in (c32, h, pre):
            t.free()
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    for t in (tA, tB, tBp):
        t.free()


@pytest.mark.parametrize("M,N,K", [(300, 544, 256), (256, 512, 512), (129, 96, 512)])
def test_gemm_gelu_bwd_packed_small(dev, q, M, N, K):
    """Packed fused GELU backward = plain GEMM + GELU backward, bit for bit, whole and ragged tiles
    (M % 8 != 0 takes the per-element transposed store)."""
    A, B = bf16_rand((M, K), 111), bf16_rand((N, K), 112)
    pre = (rng.normal(113, M * N) * 2.0).astype(np.float32).reshape(M, N)
    tA, tB, tpre = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16"), Tensor.from_numpy(dev, q, pre)
    tBp = Tensor(dev, (N, K), "bf16")
    kernels.pack_bf16_weights(q, tB, tBp)
    res = []
    for fused in (False, True):
        da, da_t = Tensor(dev, (M, N), "bf16"), Tensor(dev, (N, M), "bf16")
        for t in (da, da_t):
            t.buffer.fill_u32(q, 0x7FC07FC0)
        if fused:
            kernels.gemm_bf16_gelu_bwd(q, tA, tBp, tpre, da, da_t, packed=True)
        else:
            dh = Tensor(dev, (M, N), "f32")
            kernels.gemm_bf16(q, tA, tB, dh, False, True)
            kernels.gelu_bwd(q, dh, tpre, da, da_t)
            dh.free()
        res.append((da.numpy(q), da_t.numpy(q)))
        da.free()
        da_t.free()
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1])
    for t in (tA, tB, tBp, tpre):
        t.free()


def test_gemm_gelu_bwd_fused_config4(dev, q):
    """Config 4's dL/dpre at full size (2048x4096, K 4096): the fused op equals the plain GEMM +
    GELU backward bit for bit, and the values match the oracle's GELU backward of the oracle GEMM
    on sampled rows (bf16 tolerance)."""
    M, N, K = 2048, 4096, 4096
    A = bf16_rand((M, K), 91)
    B = bf16_rand((N, K), 92)
    pre = (rng.normal(93, M * N) * 2.0).astype(np.float32).reshape(M, N)
    tA, tB, tpre = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16"), Tensor.from_numpy(dev, q, pre)
    da, da_t, dh = Tensor(dev, (M, N), "bf16"), Tensor(dev, (N, M), "bf16"), Tensor(dev, (M, N), "f32")
    da2, da2_t = Tensor(dev, (M, N), "bf16"), Tensor(dev, (N, M), "bf16")
    kernels.gemm_bf16_gelu_bwd(q, tA, tB, tpre, da, da_t)
    kernels.gemm_bf16(q, tA, tB, dh, False, True, _lib.EPI_NONE)
    kernels.gelu_bwd(q, dh, tpre, da2, da2_t)
    g, gt = da.numpy(q), da_t.numpy(q)
    assert np.array_equal(g, da2.numpy(q))
    assert np.array_equal(gt, da2_t.numpy(q))
    assert np.array_equal(gt, g.T)
    tBp = Tensor(dev, (N, K), "bf16")  # the packed-weight form: same bits
    kernels.pack_bf16_weights(q, tB, tBp)
    for t in (da2, da2_t):
        t.buffer.fill_u32(q, 0x7FC07FC0)
    kernels.gemm_bf16_gelu_bwd(q, tA, tBp, tpre, da2, da2_t, packed=True)
    assert np.array_equal(g, da2.numpy(q))
    assert np.array_equal(gt, da2_t.numpy(q))
    tBp.free()
    rows = [0, 777, 2047]
    dh_ref = oracle.gemm_bf16(A[rows], B, False, True)
    ref, _ = oracle.gelu_bwd(dh_ref.astype(np.float32), pre[rows])
    got = rng.bf16_to_f32(g[rows]).astype(np.float64)
    mag = (np.abs(rng.bf16_to_f32(A[rows]).astype(np.float64)) @ np.abs(rng.bf16_to_f32(B).astype(np.float64)).T) * 1.2
    assert np.all(np.abs(got - rng.bf16_to_f32(ref).astype(np.float64)) <= 1e-2 * mag + 1e-30)
    for t in (tA, tB, tpre, da, da_t, dh, da2, da2_t):
        t.free()


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 4096), (256, 512, 512), (200, 544, 256)])
def test_gelu_deriv_forward_and_mul_backward(dev, q, M, N, K):
    """The stored-derivative pair: the forward GEMM with VDSL_EPI_GELU_DERIV gives the same H as
    VDSL_EPI_GELU bit for bit and GELU'(pre) (against the oracle's f64 GELU' of the same pre: the
    device GELU' is within 4e-7 relative plus 2e-7 absolute near its zero); the backward GEMM that
    multiplies by it (vdsl_op_gemm_bf16_mul_packed) equals the GELU-backward GEMM on pre bit for bit,
    da and da^T.  M = 200 leaves a ragged row tile (the per-element epilogues)."""
    X, W = bf16_rand((M, K), 101), bf16_rand((N, K), 102)
    G, W2 = bf16_rand((M, K), 103), bf16_rand((N, K), 104)  # the backward GEMM's dL/dy and W2^T
    tX, tW, tG, tW2 = (Tensor.from_numpy(dev, q, a, "bf16") for a in (X, W, G, W2))
    tWp, tW2p = Tensor(dev, (N, K), "bf16"), Tensor(dev, (N, K), "bf16")
    kernels.pack_bf16_weights(q, tW, tWp)
    kernels.pack_bf16_weights(q, tW2, tW2p)
    H1, H2 = Tensor(dev, (M, N), "bf16"), Tensor(dev, (M, N), "bf16")
    P, D = Tensor(dev, (M, N), "f32"), Tensor(dev, (M, N), "f32")
    kernels.gemm_bf16_packed(q, tX, tWp, H1, _lib.EPI_GELU, P)
    kernels.gemm_bf16_packed(q, tX, tWp, H2, _lib.EPI_GELU_DERIV, D)
    pre, dg = P.numpy(q), D.numpy(q)
    assert np.array_equal(H1.numpy(q), H2.numpy(q))
    ref = oracle.gelu_grad(pre).astype(np.float64)
    assert np.all(np.abs(dg.astype(np.float64) - ref) <= 4e-7 * np.abs(ref) + 2e-7)
    outs = []
    for mul in (False, True):
        da, da_t = Tensor(dev, (M, N), "bf16"), Tensor(dev, (N, M), "bf16")
        for t in (da, da_t):
            t.buffer.fill_u32(q, 0x7FC07FC0)
        if mul:
            kernels.gemm_bf16_mul_packed(q, tG, tW2p, D, da, da_t)
        else:
            kernels.gemm_bf16_gelu_bwd(q, tG, tW2p, P, da, da_t, packed=True)
        outs.append((da.numpy(q), da_t.numpy(q)))
        da.free()
        da_t.free()
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    assert np.array_equal(outs[1][1], outs[1][0].T)
    for t in (tX, tW, tG, tW2, tWp, tW2p, H1, H2, P, D):
        t.free()


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 4096), (128, 256, 256), (384, 768, 512)])
def test_gemm_mse_fused_equals_gemm_then_mse(dev, q, M, N, K):
    """vdsl_op_gemm_bf16_mse_packed against the packed GEMM (f32 out) followed by the MSE op on its
    output: y, dy and dy^T bit for bit, the loss (the same f64 sum in another order) to 1e-6; with
    y not requested the y buffer is left untouched; the loss also against the oracle's f64 MSE of
    the GPU's own y, and dy against the oracle's dy of it bit for bit."""
    A = bf16_rand((M, K), 95)
    B = bf16_rand((N, K), 96)
    T = rng.normal(97, M * N).reshape(M, N)
    tA, tB, tT = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16"), Tensor.from_numpy(dev, q, T)
    tBp = Tensor(dev, (N, K), "bf16")
    kernels.pack_bf16_weights(q, tB, tBp)
    part = Tensor(dev, (kernels.mse_partials_count(M, N),), "f32")
    y1, y2 = Tensor(dev, (M, N), "f32"), Tensor(dev, (M, N), "f32")
    l1, l2 = Tensor(dev, (1,), "f32"), Tensor(dev, (1,), "f32")
    d1, d2 = Tensor(dev, (M, N), "bf16"), Tensor(dev, (M, N), "bf16")
    t1, t2 = Tensor(dev, (N, M), "bf16"), Tensor(dev, (N, M), "bf16")
    for t in (y1, d1, t1, l1):
        t.buffer.fill_u32(q, 0x7FC07FC0)
    kernels.gemm_bf16_mse_packed(q, tA, tBp, tT, y1, l1, d1, t1, part)
    kernels.gemm_bf16_packed(q, tA, tBp, y2, _lib.EPI_NONE, None)
    kernels.mse_fwd_bwd(q, y2, tT, l2, d2, t2, part)
    y, d, dt_ = y1.numpy(q), d1.numpy(q), t1.numpy(q)
    assert np.array_equal(y, y2.numpy(q))
    assert np.array_equal(d, d2.numpy(q)) and np.array_equal(dt_, t2.numpy(q)) and np.array_equal(dt_, d.T)
    la, lb = float(l1.numpy(q)[0]), float(l2.numpy(q)[0])
    assert abs(la - lb) <= 1e-6 * abs(lb)
    rl, rdy, _ = oracle.mse_fwd_bwd(y, T)
    assert abs(la - rl) <= 1e-6 * abs(rl) and np.array_equal(d, rdy)
    # y not requested: same loss and gradients, y's buffer untouched
    y1.buffer.fill_u32(q, 0x7FC07FC1)
    kernels.gemm_bf16_mse_packed(q, tA, tBp, tT, None, l1, d1, None, part)
    assert float(l1.numpy(q)[0]) == la and np.array_equal(d1.numpy(q), d)
    assert np.all(y1.numpy(q).view(np.uint32) == 0x7FC07FC1)
    for t in (tA, tB, tT, tBp, part, y1, y2, l1, l2, d1, d2, t1, t2):
        t.free()


def test_gemm_mse_fused_shape_errors(dev, q):
    import ctypes
    tA, tBp, tT = Tensor(dev, (100, 256), "bf16"), Tensor(dev, (256, 256), "bf16"), Tensor(dev, (100, 256), "f32")
    loss, dy, part = Tensor(dev, (1,), "f32"), Tensor(dev, (100, 256), "bf16"), Tensor(dev, (4096,), "f32")
    st = _lib.lib.vdsl_op_gemm_bf16_mse_packed(q.handle, 100, 256, 256, tA.handle, tBp.handle, tT.handle, None,
                                               loss.handle, dy.handle, None, part.handle)
    assert st == -5 and b"M % 128" in _lib.lib.vdsl_last_error()
    for t in (tA, tBp, tT, loss, dy, part):
        t.free()


@pytest.mark.parametrize("rows,cols,dt", [(512, 8192, "bf16"), (37, 100, "f32"), (5, 16, "bf16"), (64, 8192, "f32"),
                                          (3, 16384, "bf16"), (7, 4096, "f32"), (9, 4104, "f32")])
def test_quantize_rows(dev, q, rows, cols, dt):
    x = rng.normal(41, rows * cols).reshape(rows, cols)
    if rows > 3:
        x[3] = 0
    xh = rng.f32_to_bf16(x) if dt == "bf16" else x
    tx = Tensor.from_numpy(dev, q, xh, dt)
    tq, ts = Tensor(dev, (rows, cols), "i8"), Tensor(dev, (rows,), "f32")
    kernels.quantize_rows_i8(q, tx, tq, ts)
    rq, rs = oracle.quantize_rows_i8(xh)
    assert np.array_equal(ts.numpy(q), rs)
    assert np.array_equal(tq.numpy(q), rq)
    for t in (tx, tq, ts):
        t.free()


@pytest.mark.parametrize("cols,dt", [(8192, "bf16"), (16384, "bf16"), (4096, "f32"), (8192, "f32")])
def test_quantize_rows_ties_and_scales(dev, q, cols, dt):
    """Rows that exercise the register-resident kernel's IEEE-division fallback: exact rounding ties
    (amax = 127/64, so s = 1/64 and x / s = 64 x hits k + 1/2), scales below 2^-120 and above 2^120,
    a zero row, and ordinary rows; bit for bit against the oracle's rintf(x / s)."""
    rows = 8
    x = rng.normal(43, rows * cols).reshape(rows, cols)
    k = np.arange(cols) % 127
    x[0] = ((2 * k + 1) / 128.0) * np.where(np.arange(cols) % 2, 1.0, -1.0)
    x[0, 5] = 127.0 / 64.0
    x[1] *= 2e-35
    x[2] *= 1e37
    x[2, 7] = 3e38
    x[3] = 0
    x = x.astype(np.float32)
    xh = rng.f32_to_bf16(x) if dt == "bf16" else x
    if dt == "bf16":
        assert rng.bf16_to_f32(xh[0, 5:6])[0] == np.float32(127.0 / 64.0)
    tx = Tensor.from_numpy(dev, q, xh, dt)
    tq, ts = Tensor(dev, (rows, cols), "i8"), Tensor(dev, (rows,), "f32")
    kernels.quantize_rows_i8(q, tx, tq, ts)
    rq, rs = oracle.quantize_rows_i8(xh)
    assert rs[0] == np.float32(1.0 / 64.0) and rs[1] < 2.0**-120 and rs[2] > 2.0**120
    assert np.array_equal(ts.numpy(q), rs)
    got = tq.numpy(q)
    bad = np.argwhere(got != rq)
    assert bad.size == 0, f"{len(bad)} differ, first at {bad[:4].tolist()}"
    for t in (tx, tq, ts):
        t.free()


@pytest.mark.parametrize("M,N,K,relu,dt", [(512, 8192, 8192, True, "bf16"), (512, 1024, 8192, False, "bf16"),
                                           (100, 70, 48, True, "f32"), (128, 128, 4096, False, "f32"),
                                           (33, 257, 272, True, "bf16")])
def test_w8a8_bit_exact(dev, q, M, N, K, relu, dt):
    r = np.random.default_rng(M + N + K)
    xq = r.integers(-127, 128, (M, K)).astype(np.int8)
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    xs = r.uniform(0.001, 0.01, M).astype(np.float32)
    ws = r.uniform(0.005, 0.02, N).astype(np.float32)
    txq, tw = Tensor.from_numpy(dev, q, xq), Tensor.from_numpy(dev, q, w)
    txs, tws = Tensor.from_numpy(dev, q, xs), Tensor.from_numpy(dev, q, ws)
    ty, tacc = Tensor(dev, (M, N), dt), Tensor(dev, (M, N), "i32")
    wsb = kernels.gemm_w8a8_workspace_bytes(M, N, K)
    twk = Tensor(dev, (max(1, wsb),), "i8")
    kernels.gemm_w8a8(q, txq, txs, tw, tws, ty, relu, tacc, twk if wsb else None)
    acc = tacc.numpy(q)
    y = ty.numpy(q)
    sample = slice(None) if M * N <= 1 << 20 else slice(0, 16)
    ry, racc = oracle.gemm_w8a8(xq[sample], xs[sample], w, ws, out_dtype=BF16 if dt == "bf16" else F32, relu=relu,
                                want_acc=True)
    assert np.array_equal(acc[sample], racc)
    assert np.array_equal(y[sample], ry)
    if M * N > 1 << 20:  # every row's accumulators against an exact int64 product of a column slice
        cols = slice(0, 64)
        ref = xq.astype(np.int64) @ w[cols].astype(np.int64).T
        assert np.array_equal(acc[:, cols], ref.astype(np.int32))
    for t in (txq, tw, txs, tws, ty, tacc, twk):
        t.free()
