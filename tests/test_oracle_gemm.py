"""Pins the CPU oracle's GEMM, layout, autodiff and int8 routines (orc_gemm_bf16, orc_transpose,
orc_cast, orc_gelu_bwd, orc_mse_fwd_bwd, orc_quantize_rows_i8, orc_gemm_w8a8) with checks that
do not reuse their code: exact small-integer products, numpy f64 / int64 matmuls, scipy's erf,
central finite differences."""
import numpy as np
import pytest
from scipy.special import erf, erfc

from oracle import oracle
from vernondsl_amd import rng, spec

F32, BF16 = 0, 1


def bf16_rand(shape, seed, lo=-1.0, hi=1.0):
    return rng.f32_to_bf16(rng.uniform(seed, int(np.prod(shape)), lo, hi)).reshape(shape)


@pytest.mark.parametrize("ta,tb", [(0, 1), (0, 0), (1, 0), (1, 1)])
def test_gemm_layouts_vs_numpy_f64(ta, tb):
    M, N, K = 37, 45, 29
    A = bf16_rand((K, M) if ta else (M, K), 1)
    B = bf16_rand((N, K) if tb else (K, N), 2)
    Af = rng.bf16_to_f32(A).astype(np.float64)
    Bf = rng.bf16_to_f32(B).astype(np.float64)
    ref = (Af.T if ta else Af) @ (Bf.T if tb else Bf)
    got = oracle.gemm_bf16(A, B, ta, tb)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)


def test_gemm_exact_on_small_integers():
    r = np.random.default_rng(0)
    A = r.integers(-8, 9, (16, 64)).astype(np.float32)
    B = r.integers(-8, 9, (24, 64)).astype(np.float32)
    got = oracle.gemm_bf16(rng.f32_to_bf16(A), rng.f32_to_bf16(B), 0, 1)
    # brute force in Python integers
    ref = np.array([[sum(int(A[m, k]) * int(B[n, k]) for k in range(64)) for n in range(24)] for m in range(16)])
    assert np.array_equal(got, ref.astype(np.float32))


def test_gemm_epilogues():
    A, B = bf16_rand((20, 32), 3, -3, 3), bf16_rand((28, 32), 4, -3, 3)
    Af, Bf = rng.bf16_to_f32(A).astype(np.float64), rng.bf16_to_f32(B).astype(np.float64)
    pre_ref = Af @ Bf.T
    out, pre = oracle.gemm_bf16(A, B, 0, 1, c_dtype=BF16, epilogue=1, want_pre=True)
    np.testing.assert_allclose(pre, pre_ref, rtol=1e-6, atol=1e-6)
    gelu = 0.5 * pre_ref * (1 + erf(pre_ref / np.sqrt(2)))
    assert np.allclose(gelu, 0.5 * pre_ref * erfc(-pre_ref / np.sqrt(2)), rtol=1e-12, atol=1e-12)
    assert np.all(np.abs(rng.bf16_to_f32(out) - gelu) <= 2 ** -8 * np.abs(gelu) + 1e-6)
    relu = oracle.gemm_bf16(A, B, 0, 1, epilogue=2)
    np.testing.assert_allclose(relu, np.maximum(pre_ref, 0), rtol=1e-6, atol=1e-6)


def test_transpose_and_cast():
    x = rng.normal(5, 37 * 53).reshape(37, 53)
    assert np.array_equal(oracle.transpose(x), x.T)
    xb = rng.f32_to_bf16(x)
    assert np.array_equal(oracle.transpose(xb), xb.T)
    assert np.array_equal(oracle.cast(x, BF16), xb)
    assert np.array_equal(oracle.cast(xb, F32), rng.bf16_to_f32(xb))


def test_bf16_rounding_is_nearest_even():
    # bf16 keeps 7 mantissa bits: one ulp at 1.0 is 2^-7
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, 1.0 + 2 ** -9, 1.0 + 3 * 2 ** -8, -2.5, np.inf, -0.0],
                    np.float32)
    got = oracle.cast(vals, BF16)
    # 1 + 2^-8 is a tie between 1 (even) and 1 + 2^-7 (odd): 1.0; 1 + 3*2^-8 ties to 1 + 2^-6 (even)
    assert list(got) == [0x3F80, 0x3F80, 0x3F81, 0x3F80, 0x3F82, 0xC020, 0x7F80, 0x8000]
    assert np.array_equal(got, rng.f32_to_bf16(vals))


def test_gelu_fwd_known_values_and_odd_part_identity():
    """GELU(x) - GELU(-x) = x (Phi(x) + Phi(-x) = 1): a dropped term, a wrong sign or erf in
    place of erfc breaks it; plus closed-form values and bf16 in/out rounding."""
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    g = oracle.gelu_fwd(x).astype(np.float64)
    gm = oracle.gelu_fwd(-x).astype(np.float64)
    assert np.all(np.abs((g - gm) - x.astype(np.float64)) <= 2 * np.spacing(np.abs(x).astype(np.float32)) + 1e-30)
    # scipy's erfc (an implementation independent of the C library's) in the cancellation-free form
    ref = 0.5 * x.astype(np.float64) * erfc(-x.astype(np.float64) / np.sqrt(2))
    assert np.all(np.abs(g - ref) <= 1e-6 * np.abs(ref) + 1e-30)
    assert oracle.gelu_fwd(np.array([0.0, 1.0, -1.0], np.float32)).tolist() == [
        0.0, np.float32(0.8413447460685429), np.float32(-0.15865525393145707)]
    # bf16 input is widened exactly; bf16 output is the RNE of the f32 result
    xb = rng.f32_to_bf16(x)
    assert np.array_equal(oracle.gelu_fwd(xb), oracle.gelu_fwd(rng.bf16_to_f32(xb)))
    assert np.array_equal(oracle.gelu_fwd(x, y_bf16=True), rng.f32_to_bf16(oracle.gelu_fwd(x)))


def test_gelu_bwd_matches_finite_differences():
    pre = np.linspace(-4, 4, 64 * 48).astype(np.float32).reshape(64, 48)
    dh = np.ones_like(pre)
    da, da_t = oracle.gelu_bwd(dh, pre)
    p = pre.astype(np.float64)
    h = 1e-6
    gelu = lambda v: 0.5 * v * (1 + erf(v / np.sqrt(2)))  # noqa: E731
    fd = (gelu(p + h) - gelu(p - h)) / (2 * h)
    got = rng.bf16_to_f32(da).astype(np.float64)
    assert np.all(np.abs(got - fd) <= 2 ** -8 * np.abs(fd) + 1e-6)
    assert np.array_equal(da_t, da.T)


def test_gelu_grad_f32_matches_finite_differences():
    """The f32 GELU' (what the forward epilogue stores for the backward pass) against central
    differences of the f64 GELU, and equal to the f32 rounding of the backward's factor (dh = 1)."""
    pre = np.linspace(-6, 6, 4001).astype(np.float32)
    g = oracle.gelu_grad(pre).astype(np.float64)
    p = pre.astype(np.float64)
    h = 1e-5
    gelu = lambda v: 0.5 * v * (1 + erf(v / np.sqrt(2)))  # noqa: E731
    fd = (gelu(p + h) - gelu(p - h)) / (2 * h)
    assert np.all(np.abs(g - fd) <= 1e-7 * np.abs(fd) + 1e-9)
    da, _ = oracle.gelu_bwd(np.ones((1, pre.size), np.float32), pre.reshape(1, -1))
    assert np.array_equal(da[0], rng.f32_to_bf16(g.astype(np.float32)))
    assert oracle.gelu_grad(np.array([0.0], np.float32))[0] == np.float32(0.5)


def test_gelu_grad_keeps_relative_accuracy_for_negative_pre():
    pre = np.array([[-3.0, -5.0, -7.0, -9.0]], np.float32)
    da, _ = oracle.gelu_bwd(np.ones_like(pre), pre)
    v = pre.astype(np.float64)
    exact = 0.5 * erfc(-v / np.sqrt(2)) + v * np.exp(-v * v / 2) / np.sqrt(2 * np.pi)
    assert np.all(np.abs(rng.bf16_to_f32(da) - exact) <= 2 ** -8 * np.abs(exact))


def test_relu_bwd_is_a_select_and_add_is_one_f32_addition():
    """orc_relu_bwd against numpy's select (pre <= 0 and NaN give +0, infinities pass where pre >
    0), orc_add against numpy's f32 addition (one correctly rounded result), bf16 widened exactly."""
    r = np.random.default_rng(21)
    dh = r.standard_normal((9, 13)).astype(np.float32)
    pre = r.standard_normal((9, 13)).astype(np.float32)
    pre[0, :4] = [0.0, -0.0, np.nan, 1e-45]
    dh[1, :2] = [np.inf, -np.inf]
    pre[1, :2] = [-1.0, 2.0]
    da, da_t = oracle.relu_bwd(dh, pre)
    ref = oracle.cast(np.where(pre > 0, dh, np.float32(0)).astype(np.float32), oracle.BF16)
    assert np.array_equal(da, ref) and np.array_equal(da_t, ref.T)
    assert da[0, 0] == da[0, 1] == da[0, 2] == 0 and da[1, 0] == 0 and da[1, 1] == 0xFF80  # +0s, -inf kept
    a = r.standard_normal(1000).astype(np.float32)
    b = (r.standard_normal(1000) * 1e-3).astype(np.float32)
    assert np.array_equal(oracle.add(a, b), a + b)
    ab, bb = oracle.cast(a, oracle.BF16), oracle.cast(b, oracle.BF16)
    wide = rng.bf16_to_f32(ab) + rng.bf16_to_f32(bb)
    assert np.array_equal(oracle.add(ab, bb), wide)
    assert np.array_equal(oracle.add(ab, b, oracle.BF16), oracle.cast(rng.bf16_to_f32(ab) + b, oracle.BF16))


def test_mse_matches_finite_differences():
    y = rng.normal(7, 32 * 40).reshape(32, 40)
    t = rng.normal(8, 32 * 40).reshape(32, 40)
    loss, dy, dy_t = oracle.mse_fwd_bwd(y, t)
    d = y.astype(np.float64) - t
    assert abs(loss - np.mean(d * d)) <= 1e-6 * np.mean(d * d)
    # finite difference of the loss in one coordinate
    e = np.zeros_like(d)
    e[3, 5] = 1e-4
    fd = (np.mean((d + e) ** 2) - np.mean((d - e) ** 2)) / 2e-4
    assert abs(rng.bf16_to_f32(dy)[3, 5] - fd) <= 2 ** -8 * abs(fd)
    assert np.array_equal(dy_t, dy.T)


def test_quantize_rows():
    x = rng.f32_to_bf16(rng.normal(9, 16 * 300)).reshape(16, 300)
    x[3] = 0  # all-zero row
    q, s = oracle.quantize_rows_i8(x)
    xf = rng.bf16_to_f32(x)
    amax = np.abs(xf).max(axis=1)
    assert np.array_equal(s, (amax / np.float32(127)).astype(np.float32))
    assert (q[3] == 0).all() and s[3] == 0
    nz = s > 0
    ref = np.clip(np.rint(xf[nz] / s[nz, None]), -127, 127).astype(np.int8)  # f32 division, RNE
    assert np.array_equal(q[nz], ref)
    assert np.abs(q).max() == 127


def test_w8a8_exact_int_and_dequant_sequence():
    r = np.random.default_rng(1)
    M, N, K = 24, 40, 96
    xq = r.integers(-127, 128, (M, K)).astype(np.int8)
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    xs = r.uniform(0.001, 0.01, M).astype(np.float32)
    ws = r.uniform(0.005, 0.02, N).astype(np.float32)
    y, acc = oracle.gemm_w8a8(xq, xs, w, ws, out_dtype=F32, relu=True, want_acc=True)
    acc_ref = xq.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(acc, acc_ref.astype(np.int32))
    v = (acc_ref.astype(np.float32) * xs[:, None]).astype(np.float32) * ws[None, :]
    v = np.where(v > 0, v, np.float32(0)).astype(np.float32)
    assert np.array_equal(y, v)
    yb = oracle.gemm_w8a8(xq, xs, w, ws, out_dtype=BF16, relu=False)
    v2 = ((acc_ref.astype(np.float32) * xs[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32)
    assert np.array_equal(yb, rng.f32_to_bf16(v2))
    # the epilogue alone on given accumulators (what the full-size GPU check feeds it)
    assert np.array_equal(oracle.w8a8_dequant(acc_ref.astype(np.int32), xs, ws, relu=True, out_dtype=F32), y)
    assert np.array_equal(oracle.w8a8_dequant(acc_ref.astype(np.int32), xs, ws, relu=False), yb)


def test_w8a8_dequant_large_accumulators():
    """Accumulators of a K = 8192 layer reach 8192 * 127^2 > 2^24, where float(acc) rounds (RNE)."""
    r = np.random.default_rng(2)
    acc = r.integers(-8192 * 127 * 127, 8192 * 127 * 127 + 1, (16, 32)).astype(np.int32)
    acc[0, :4] = [2**24 + 1, -(2**24 + 3), 2**27 - 1, 0]
    xs = r.uniform(1e-4, 1e-2, 16).astype(np.float32)
    ws = r.uniform(0.005, 0.02, 32).astype(np.float32)
    a32 = acc.astype(np.float64).astype(np.float32)  # exact int -> f64, then one RNE rounding to f32
    assert a32[0, 0] == np.float32(2**24) and a32[0, 1] == np.float32(-(2**24 + 4))
    v = ((a32 * xs[:, None]).astype(np.float32) * ws[None, :]).astype(np.float32)
    assert np.array_equal(oracle.w8a8_dequant(acc, xs, ws, relu=False, out_dtype=F32), v)
    assert np.array_equal(oracle.w8a8_dequant(acc, xs, ws, relu=True), rng.f32_to_bf16(np.maximum(v, np.float32(0))))


def test_w8a8_config_generators():
    x, layers = spec.w8a8_inputs(batch=4, widths=(64, 64, 32))
    assert x.shape == (4, 64) and x.dtype == np.uint16
    (w0, s0), (w1, s1) = layers
    assert w0.shape == (64, 64) and w1.shape == (32, 64) and w0.dtype == np.int8
    assert w0.min() >= -127 and w0.max() <= 127
    assert s0.min() >= 0.005 and s0.max() < 0.02
