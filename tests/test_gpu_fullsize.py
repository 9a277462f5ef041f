"""Configs 4 and 5 at full size, every output element checked (not sampled rows).

Each op is fed the GPU's own inputs (the intermediates of the same step), so a wrong tile
anywhere in any GEMM fails:
- config 5 (int8, bit-exact): each layer's int32 accumulators come from an f64 matrix product of
  the int8 operands (numpy's BLAS on the host; exact, since every partial sum is an integer below
  2^53), and the oracle's own dequant epilogue (oracle.w8a8_dequant, the code of oracle.gemm_w8a8)
  turns them into the expected bf16 outputs; each quantisation is checked against the oracle;
- config 4 (bf16 GEMMs, f32 accumulate): each GEMM against numpy's fp32 product of the same bf16
  operands, with the bf16 GEMM tolerance 1e-2 (Frobenius-relative, and elementwise relative to
  (|A||B|)[m][n]); the GELU and MSE epilogues against the oracle.
The host products take well under a minute on the box's cores.
"""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, graph, kernels, rng, spec
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu


def _f32(bf16_bits):
    return rng.bf16_to_f32(bf16_bits)


def check_gemm(got, a, b, rel=1e-2, what=""):
    """got (f32) against a @ b (numpy fp32 product of f32 operands)."""
    ref = (a @ b).astype(np.float64)
    mag = (np.abs(a) @ np.abs(b)).astype(np.float64)
    d = got.astype(np.float64) - ref
    assert np.linalg.norm(d) <= rel * max(np.linalg.norm(ref), 1e-30), what
    bad = int(np.count_nonzero(np.abs(d) > rel * mag + 1e-30))
    assert bad == 0, f"{what}: {bad} elements outside the elementwise bound"


def test_w8a8_config5_every_element(dev, q):
    x, layers = spec.w8a8_inputs()
    g = graph.w8a8_infer_graph()
    exe = g.compile(dev)
    exe.write(q, "X", x)
    for li, (w, s) in enumerate(layers):
        exe.write(q, f"W{li}", w)
        exe.write(q, f"S{li}", s)
    step = exe.capture(q)
    step.launch(q)
    q.sync()
    quants = [op for op in g.ops if op.kind == "quantize"]
    gemms = [op for op in g.ops if op.kind in ("w8a8", "w8a8_packed")]
    assert len(quants) == len(gemms) == len(layers)
    h = x
    for li, (qop, gop) in enumerate(zip(quants, gemms)):
        xq, xs = exe.read(q, qop.outputs[0].name), exe.read(q, qop.outputs[1].name)
        rq, rs = oracle.quantize_rows_i8(h)
        assert np.array_equal(xs, rs) and np.array_equal(xq, rq), f"layer {li}: quantisation"
        w, ws = layers[li]
        acc = xq.astype(np.float64) @ w.astype(np.float64).T
        assert np.abs(acc).max() < 2**31 and np.array_equal(acc, np.rint(acc))
        ref = oracle.w8a8_dequant(acc.astype(np.int32), xs, ws, relu=gop.attrs["relu"])
        got = exe.read(q, gop.outputs[0].name)
        assert got.shape == ref.shape == (512, w.shape[0])
        bad = np.argwhere(got != ref)
        assert bad.size == 0, f"layer {li}: {len(bad)} outputs differ, first at {bad[:4].tolist()}"
        h = got
    step.destroy()
    exe.free()


def test_mlp_config4_every_element(dev, q):
    x, w1, w2, t = spec.mlp_inputs()
    g, _ = graph.mlp_train_graph()
    exe = g.compile(dev)
    for name, arr in (("X", x), ("W1", w1), ("W2", w2), ("T", t)):
        exe.write(q, name, arr)
    step = exe.capture(q)
    step.launch(q)
    q.sync()
    by_kind = {}
    for op in g.ops:
        by_kind.setdefault(op.kind, []).append(op)
    fwd1 = by_kind["linear"][0]
    mse = by_kind["linear_mse"][0]
    bwd = by_kind["gemm_mul_bwd"][0]
    rd = lambda v: exe.read(q, v.name)  # noqa: E731
    dgelu, h = rd(fwd1.attrs["dgelu"]), exe.read(q, "H")
    y, loss, dy = (rd(v) for v in mse.outputs[:3])
    da = rd(bwd.outputs[0])
    # the weight-gradient GEMMs read dY and dL/dpre as stored (K-major A): their transposes are
    # neither allocated nor written
    assert {mse.outputs[3].name, bwd.outputs[1].name} <= g.elided
    X, W1, W2 = _f32(x), _f32(w1), _f32(w2)
    # The step keeps GELU'(pre), not pre: the same forward GEMM with the plain GELU epilogue on the
    # step's own operands gives pre, and its H must equal the step's bit for bit.
    tp, th = Tensor(dev, pre_shape := (x.shape[0], w1.shape[0]), "f32"), Tensor(dev, pre_shape, "bf16")
    kernels.gemm_bf16_packed(q, exe.t["X"], exe.t[fwd1.attrs["packed"].name], th, _lib.EPI_GELU, tp)
    pre = tp.numpy(q)
    assert np.array_equal(th.numpy(q), h), "H from the GELU'-storing epilogue differs from the GELU one"
    tp.free()
    th.free()
    # forward: pre-activation, GELU (bf16, within one bf16 ulp of the oracle's libm GELU), GELU'
    # (within its approximation bound of the oracle's f64 GELU'), Y
    check_gemm(pre, X, W1.T, what="pre = X W1^T")
    dg_ref = oracle.gelu_grad(pre).astype(np.float64)
    err = np.abs(dgelu.astype(np.float64) - dg_ref) - (4e-7 * np.abs(dg_ref) + 2e-7)
    w = np.unravel_index(np.argmax(err), err.shape)
    assert err[w] <= 0, f"GELU'(pre) at {w}: pre {pre[w]!r} got {dgelu[w]!r} ref {dg_ref[w]!r}, {np.count_nonzero(err > 0)} over"
    h_ref = oracle.gelu_fwd(pre, y_bf16=True)
    ulps = np.abs(h.astype(np.int32) - h_ref.astype(np.int32))
    assert ulps.max() <= 1 and np.count_nonzero(ulps) <= 1e-3 * h.size, "H = GELU(pre)"
    H = _f32(h)
    check_gemm(y, H, W2.T, what="Y = H W2^T")
    # the loss and dL/dY from the GPU's Y: dY exact, the loss within f64-sum rounding
    r_loss, r_dy, r_dy_t = oracle.mse_fwd_bwd(y, t)
    assert np.array_equal(dy, r_dy)
    assert abs(float(loss[0]) - r_loss) <= 1e-6 * r_loss
    # weight gradient of W2 from the GPU's dY^T and H
    check_gemm(exe.read(q, "grad_W2"), np.ascontiguousarray(_f32(dy).T), H, what="dW2 = dY^T H")
    # dL/dpre = (dY W2) GELU'(pre): dY W2 from numpy in fp32, GELU' by the oracle; the bound is
    # the GEMM tolerance carried through |GELU'| <= 1.13, plus two bf16 roundings
    DY = _f32(dy)
    dh = DY @ W2
    da_ref, _ = oracle.gelu_bwd(dh, pre)
    mag = (np.abs(DY) @ np.abs(W2)).astype(np.float64) * 1.13
    got, ref = rng.bf16_to_f32(da).astype(np.float64), rng.bf16_to_f32(da_ref).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-2 * mag + 2.0**-7 * np.abs(ref)), "dL/dpre"
    # weight gradient of W1 from the GPU's dL/dpre^T and X
    check_gemm(exe.read(q, "grad_W1"), np.ascontiguousarray(_f32(da).T), X, what="dW1 = dA^T X")
    step.destroy()
    exe.free()
