"""Execution-graph construction and autodiff on the CPU (no device): the op sequence the
backward pass emits, shapes and layouts, and an f64 finite-difference pin of the composite
oracle (oracle.mlp_train_step) that the GPU graph is compared with."""
import numpy as np
import pytest
from scipy.special import erf

from oracle import oracle
from vernondsl_amd import graph, rng


def test_mlp_backward_op_sequence():
    g, grads = graph.mlp_train_graph(batch=64, d_in=32, hidden=48, d_out=16, prepare_transposes=False,
                                     fuse_gelu_backward=False, k_major_grads=False)
    kinds = [op.kind for op in g.ops]
    assert kinds == ["linear", "linear", "mse", "gemm", "gemm", "gelu_bwd", "gemm"]
    assert sorted(grads) == ["W1", "W2"]
    assert grads["W1"].shape == (48, 32) and grads["W2"].shape == (16, 48)
    assert grads["W1"].dtype == "f32"
    mse = g.ops[2]
    assert [v.shape for v in mse.outputs] == [(1,), (64, 16), (16, 64), mse.outputs[3].shape]
    dW2, dH, gb, dW1 = g.ops[3], g.ops[4], g.ops[5], g.ops[6]
    assert dW2.inputs[0].shape == (16, 64) and dW2.inputs[1].name == "H"   # dY^T [out][B], H [B][hid]
    assert dH.inputs[1].name == "W2" and dH.outputs[0].dtype == "f32" and not dH.attrs["trans_b"]
    assert gb.inputs[1] is g.ops[0].attrs["pre"]
    assert dW1.inputs[1].name == "X" and dW1.outputs[0].name == "grad_W1"
    assert not g.prepare_ops


def test_mlp_backward_prepared_transpose_and_fused_gelu():
    g, _ = graph.mlp_train_graph(batch=64, d_in=32, hidden=48, d_out=16, prepare_transposes=True,
                                 fuse_gelu_backward=False)
    assert [op.kind for op in g.ops] == ["linear", "linear", "mse", "gemm", "gemm", "gelu_bwd", "gemm"]
    # dH = dY W2 in the NT form on W2^T [hid][out], made by a prepare op (not on every step)
    dH = g.ops[4]
    assert dH.inputs[1].name == "W2.T" and dH.inputs[1].shape == (48, 16) and dH.attrs["trans_b"]
    assert [(op.kind, op.inputs[0].name, op.outputs[0].name) for op in g.prepare_ops] == [("transpose", "W2", "W2.T")]
    g, _ = graph.mlp_train_graph(batch=64, d_in=32, hidden=48, d_out=16, prepare_transposes=True,
                                 fuse_gelu_backward=True, k_major_grads=False)
    assert [op.kind for op in g.ops] == ["linear", "linear", "mse", "gemm", "gemm_gelu_bwd", "gemm"]
    dA, dW1 = g.ops[4], g.ops[5]
    # dL/dpre = (dY W2) * GELU'(pre) in one op
    assert dA.inputs[1].name == "W2.T" and dA.inputs[2] is g.ops[0].attrs["pre"]
    assert [v.shape for v in dA.outputs] == [(64, 48), (48, 64)] and dA.outputs[0].dtype == "bf16"
    assert dW1.inputs[0] is dA.outputs[1]


def test_mlp_stored_gelu_derivative():
    """The config-4 default: the forward GELU GEMM stores GELU'(pre) in place of pre and the fused
    backward GEMM multiplies by it; no value named pre remains, and the plain form keeps pre."""
    g, _ = graph.mlp_train_graph(batch=256, d_in=512, hidden=512, d_out=256)
    kinds = [op.kind for op in g.ops]
    assert kinds == ["linear", "linear_mse", "gemm", "gemm_mul_bwd", "gemm"]
    fwd, mul = g.ops[0], g.ops[3]
    dg = fwd.attrs["dgelu"]
    assert fwd.attrs["pre"] is None and fwd.outputs == [g.values["H"], dg] and dg.dtype == "f32"
    assert mul.inputs[1].name == "W2.T.packed" and mul.inputs[2] is dg and mul.outputs[1].shape == (512, 256)
    assert not any(n.startswith("pre#") for n in g.values)
    g2, _ = graph.mlp_train_graph(batch=256, d_in=512, hidden=512, d_out=256, store_gelu_deriv=False)
    assert [op.kind for op in g2.ops][3] == "gemm_gelu_bwd" and g2.ops[0].attrs["pre"] is not None


def test_mlp_packed_weights():
    """pack_weights: each forward linear op on a param reads a packed copy made by a prepare op;
    the backward ops still read the row-major weight."""
    g, _ = graph.mlp_train_graph(batch=64, d_in=512, hidden=512, d_out=256, pack_weights=True,
                                 prepare_transposes=False, fuse_gelu_backward=False)
    assert [(op.kind, op.inputs[0].name, op.outputs[0].name) for op in g.prepare_ops] == [
        ("pack_bf16", "W1", "W1.packed"), ("pack_bf16", "W2", "W2.packed")]
    lin = [op for op in g.ops if op.kind == "linear"]
    assert [op.attrs["packed"].name for op in lin] == ["W1.packed", "W2.packed"]
    assert [op.inputs[1].name for op in lin] == ["W1", "W2"]
    assert g.ops[4].inputs[1].name == "W2"  # dH = dY W2 uses the row-major weight
    g2, _ = graph.mlp_train_graph(batch=64, d_in=32, hidden=48, d_out=16, pack_weights=True,
                                  prepare_transposes=False)
    assert not g2.prepare_ops  # widths the packed GEMM does not take (K % 256) stay row-major


def test_mlp_default_graph_prepare_chain():
    """mlp_train_graph's default: packed forward weights, and the fused GELU-backward GEMM on W2^T
    packed (transpose, then pack: two prepare ops run in order)."""
    g, _ = graph.mlp_train_graph(batch=64, d_in=512, hidden=512, d_out=256, store_gelu_deriv=False)
    assert [op.kind for op in g.ops] == ["linear", "linear", "mse", "gemm", "gemm_gelu_bwd", "gemm"]
    assert [(op.kind, op.inputs[0].name, op.outputs[0].name) for op in g.prepare_ops] == [
        ("pack_bf16", "W1", "W1.packed"), ("pack_bf16", "W2", "W2.packed"), ("transpose", "W2", "W2.T"),
        ("pack_bf16", "W2.T", "W2.T.packed")]
    dA = g.ops[4]
    assert dA.inputs[1].name == "W2.T.packed" and dA.attrs["packed"]


def test_inference_graph_has_no_backward():
    g = graph.w8a8_infer_graph(batch=8, widths=(64, 64, 32))
    assert [op.kind for op in g.ops] == ["quantize", "w8a8", "quantize", "w8a8"]
    assert [op.attrs.get("relu") for op in g.ops if op.kind == "w8a8"] == [True, False]


def test_inference_graph_packs_weights():
    """Layers whose shape the packed int8 GEMM takes (in % 512, out % 32) read packed weights made
    by prepare ops, which are not part of the replayed step; others keep the row-major GEMM."""
    g = graph.w8a8_infer_graph(batch=8, widths=(512, 1024, 96, 64))
    assert [op.kind for op in g.ops] == ["quantize", "w8a8_packed", "quantize", "w8a8_packed", "quantize", "w8a8"]
    assert [op.kind for op in g.prepare_ops] == ["pack_w8a8", "pack_w8a8"]
    assert [op.inputs[0].name for op in g.prepare_ops] == ["W0", "W1"]
    for op, pre in zip([o for o in g.ops if o.kind == "w8a8_packed"], g.prepare_ops):
        assert op.inputs[2] is pre.outputs[0] and op.inputs[2].shape == pre.inputs[0].shape
    g2 = graph.Graph()
    x = g2.input("X", (8, 512), "bf16")
    g2.quant_linear(x, g2.param("W", (64, 512), "i8", False), g2.param("S", (64,), "f32", False), relu=True,
                    packed=False)
    assert [op.kind for op in g2.ops] == ["quantize", "w8a8"] and not g2.prepare_ops


def test_graph_rejects_bad_programs():
    g = graph.Graph()
    x = g.input("X", (4, 8), "bf16")
    w = g.param("W", (6, 9), "bf16")
    with pytest.raises(ValueError):
        g.linear(x, w)
    with pytest.raises(ValueError):
        g.input("X", (1,), "f32")
    y = g.linear(x, g.param("W2", (6, 8), "bf16"), out_dtype="f32")
    with pytest.raises(ValueError):
        g.backward(y)  # not a loss


def _mlp_f64(x, w1, w2, t):
    a = x @ w1.T
    h = 0.5 * a * (1 + erf(a / np.sqrt(2)))
    y = h @ w2.T
    return np.mean((y - t) ** 2)


def test_oracle_mlp_gradients_match_finite_differences():
    """Small MLP: the oracle composite's dW1/dW2 (bf16 roundings included) against central
    differences of the f64 loss; the tolerance covers the bf16 roundings of H, dY and dA."""
    B, D, Hd, O = 16, 8, 12, 6
    x = rng.f32_to_bf16(rng.normal(1, B * D)).reshape(B, D)
    w1 = rng.f32_to_bf16(rng.uniform(2, Hd * D, -0.5, 0.5)).reshape(Hd, D)
    w2 = rng.f32_to_bf16(rng.uniform(3, O * Hd, -0.5, 0.5)).reshape(O, Hd)
    t = rng.normal(4, B * O).reshape(B, O)
    r = oracle.mlp_train_step(x, w1, w2, t)
    X, W1, W2 = (rng.bf16_to_f32(a).astype(np.float64) for a in (x, w1, w2))
    T = t.astype(np.float64)
    assert abs(r["loss"] - _mlp_f64(X, W1, W2, T)) <= 1e-2 * _mlp_f64(X, W1, W2, T)
    eps = 1e-5
    for name, W in (("dW1", W1), ("dW2", W2)):
        fd = np.zeros_like(W)
        for idx in np.ndindex(W.shape):
            Wp, Wm = W.copy(), W.copy()
            Wp[idx] += eps
            Wm[idx] -= eps
            if name == "dW1":
                fd[idx] = (_mlp_f64(X, Wp, W2, T) - _mlp_f64(X, Wm, W2, T)) / (2 * eps)
            else:
                fd[idx] = (_mlp_f64(X, W1, Wp, T) - _mlp_f64(X, W1, Wm, T)) / (2 * eps)
        got = r[name].astype(np.float64)
        assert np.linalg.norm(got - fd) <= 2e-2 * np.linalg.norm(fd), name


def test_oracle_w8a8_forward_rows_independent():
    x = rng.f32_to_bf16(rng.normal(5, 6 * 64)).reshape(6, 64)
    layers = [(rng.int_uniform(6, 64 * 64, -127, 127).astype(np.int8).reshape(64, 64), rng.uniform(7, 64, 0.005, 0.02)),
              (rng.int_uniform(8, 32 * 64, -127, 127).astype(np.int8).reshape(32, 64), rng.uniform(9, 32, 0.005, 0.02))]
    full = oracle.w8a8_forward(x, layers)
    part = oracle.w8a8_forward(x[2:4], layers)
    assert np.array_equal(full[2:4], part)


def test_host_outputs_are_the_unread_results():
    """Buffers bound as VDSL_BIND_OUTPUT (streamed f32 GEMM results): exactly the values the step
    produces and nothing reads, never op scratch or anything a later op consumes."""
    g, _ = graph.mlp_train_graph()
    outs = g.host_outputs()
    assert {"grad_W1", "grad_W2", "Y", "loss"} <= outs
    read = {v.name for op in g.ops + g.prepare_ops for v in op.inputs}
    assert not (outs & read)
    assert all(g.values[n].kind != "scratch" for n in outs)
    assert "H" not in outs  # read by the output GEMM and the dW2 GEMM


def test_k_major_grads_elide_transposes():
    """The config-4 default: the weight-gradient GEMMs take dL/dY and dL/dpre as stored (trans_a),
    and their transposes, which nothing reads then, are elided; without the option they are read."""
    g, _ = graph.mlp_train_graph(batch=256, d_in=512, hidden=512, d_out=256)
    dW2, mul, dW1 = g.ops[2], g.ops[3], g.ops[4]
    mse = g.ops[1]
    assert dW2.attrs["trans_a"] and dW2.inputs[0] is mse.outputs[2] and dW2.inputs[0].shape == (256, 256)
    assert dW1.attrs["trans_a"] and dW1.inputs[0] is mul.outputs[0]
    assert g.elided == {mse.outputs[3].name, mul.outputs[1].name}
    assert not (g.elided & g.host_outputs())
    g2, _ = graph.mlp_train_graph(batch=256, d_in=512, hidden=512, d_out=256, k_major_grads=False)
    assert not g2.elided and not g2.ops[2].attrs["trans_a"] and g2.ops[2].inputs[0] is g2.ops[1].outputs[3]
    # the unfused form: the mse op's dY^T and the cast/transpose pair are dropped the same way
    g3, _ = graph.mlp_train_graph(batch=64, d_in=32, hidden=48, d_out=16, prepare_transposes=False,
                                  fuse_gelu_backward=False, pack_weights=False, fuse_mse=False, store_gelu_deriv=False)
    assert len(g3.elided) == 2 and all(n.startswith("dT_") for n in g3.elided)
    assert all(op.attrs["trans_a"] for op in g3.ops if op.kind == "gemm" and op.outputs[0].name.startswith("grad_"))


def test_fused_loss_without_y_elides_y():
    """keep_y=False: the fused output GEMM + loss does not store y, so y is elided (no buffer, and
    reading it raises) instead of an allocated buffer that is never written."""
    g, _ = graph.mlp_train_graph(batch=256, d_in=512, hidden=512, d_out=256, keep_y=False)
    lin = g.ops[1]
    assert lin.kind == "linear_mse"
    assert lin.outputs[0].name in g.elided and lin.outputs[0].name not in g.host_outputs()
    g2, _ = graph.mlp_train_graph(batch=256, d_in=512, hidden=512, d_out=256)
    assert g2.ops[1].outputs[0].name not in g2.elided


def residual_graph(B=16, D=8, Hd=8, O=6, **flags):
    """X -> H1 = relu(X W1^T) -> H2 = GELU(H1 WR^T) -> R = H1 + H2 -> H3 = GELU(R WR^T) -> Y = H3 W3^T
    -> MSE: H1 is read twice (a residual), WR by two layers (tied weights), ReLU and GELU both."""
    g = graph.Graph(**flags)
    x = g.input("X", (B, D), "bf16")
    w1 = g.param("W1", (Hd, D), "bf16")
    wr = g.param("WR", (Hd, Hd), "bf16")
    w3 = g.param("W3", (O, Hd), "bf16")
    t = g.input("T", (B, O), "f32")
    h1 = g.linear(x, w1, act="relu", name="H1")
    h2 = g.linear(h1, wr, act="gelu", name="H2")
    r = g.add(h1, h2, name="R")
    h3 = g.linear(r, wr, act="gelu", name="H3")
    y = g.linear(h3, w3, out_dtype="f32", name="Y")
    return g, g.backward(g.mse_loss(y, t))


def _residual_f64(X, W1, WR, W3, T):
    def gelu(a):
        return 0.5 * a * (1 + erf(a / np.sqrt(2)))
    h1 = np.maximum(X @ W1.T, 0)
    r = h1 + gelu(h1 @ WR.T)
    y = gelu(r @ WR.T) @ W3.T
    return np.mean((y - T) ** 2)


def residual_inputs(B=16, D=8, Hd=8, O=6, seed=30, w_range=0.6):
    x = rng.f32_to_bf16(rng.normal(seed, B * D)).reshape(B, D)
    w1 = rng.f32_to_bf16(rng.uniform(seed + 1, Hd * D, -w_range, w_range)).reshape(Hd, D)
    wr = rng.f32_to_bf16(rng.uniform(seed + 2, Hd * Hd, -w_range, w_range)).reshape(Hd, Hd)
    w3 = rng.f32_to_bf16(rng.uniform(seed + 3, O * Hd, -w_range, w_range)).reshape(O, Hd)
    t = rng.normal(seed + 4, B * O).reshape(B, O)
    return {"X": x, "W1": w1, "WR": wr, "W3": w3, "T": t}


def test_residual_graph_backward_structure():
    g, grads = residual_graph()
    kinds = [op.kind for op in g.ops]
    assert kinds[:6] == ["linear", "linear", "add", "linear", "linear", "mse"]
    assert sorted(grads) == ["W1", "W3", "WR"]
    assert grads["WR"].name == "grad_WR" and grads["WR"].producer.kind == "add"  # the tied weight's two terms
    terms = grads["WR"].producer.inputs
    assert all(t.producer.kind == "gemm" and t.name.startswith("dterm_WR") for t in terms)
    assert kinds.count("relu_bwd") == 1 and kinds.count("gelu_bwd") == 2
    # dL/dH1: the residual's term (dL/dR) plus the WR layer's dL/dH1, summed in f32 before relu_bwd
    relu = next(op for op in g.ops if op.kind == "relu_bwd")
    s = relu.inputs[0]
    assert s.dtype == "f32" and s.producer.kind == "add" and s.name.startswith("dsum_H1")
    assert grads["W1"].name == "grad_W1" and grads["W3"].name == "grad_W3"


def test_residual_graph_fusions_skip_values_read_twice():
    """With every fusion on, the GELU backward is fused only where its value has one reader (H3);
    the values read twice (H1, and R's gradient reaching H1 and H2) take the unfused rules."""
    flags = dict(prepare_transposes=True, fuse_gelu_backward=True, k_major_grads=True)
    g, grads = residual_graph(**flags)
    fused = [op for op in g.ops if op.kind == "gemm_gelu_bwd"]
    assert len(fused) == 1 and fused[0].inputs[2] is g.ops[3].attrs["pre"]  # H3's pre-activation
    assert sorted(grads) == ["W1", "W3", "WR"]
    g2 = graph.Graph(fuse_mse=True, pack_weights=True)
    x = g2.input("X", (128, 256), "bf16")
    y = g2.linear(x, g2.param("W", (256, 256), "bf16"), out_dtype="f32", name="Y")
    z = g2.add(y, y, name="Z")  # Y read by the loss and by another op: the loss stays unfused
    g2.backward(g2.mse_loss(y, g2.input("T", (128, 256), "f32")))
    assert [op.kind for op in g2.ops][:3] == ["linear", "add", "mse"] and z.name == "Z"


@pytest.mark.parametrize("flags", [{}, {"prepare_transposes": True, "fuse_gelu_backward": True, "k_major_grads": True}])
def test_residual_graph_gradients_match_finite_differences(flags):
    """The oracle run of the backward ops the graph emits against central differences of the f64
    loss: pins the add, relu, fan-out and tied-weight rules (a term dropped or overwritten fails)."""
    g, grads = residual_graph(**flags)
    feeds = residual_inputs()
    v = oracle.graph_step(g, feeds)
    X, W1, WR, W3 = (rng.bf16_to_f32(feeds[n]).astype(np.float64) for n in ("X", "W1", "WR", "W3"))
    T = feeds["T"].astype(np.float64)
    base = _residual_f64(X, W1, WR, W3, T)
    assert abs(float(v["loss"][0]) - base) <= 2e-2 * base
    eps = 1e-5
    for name, W in (("W1", W1), ("WR", WR), ("W3", W3)):
        fd = np.zeros_like(W)
        for idx in np.ndindex(W.shape):
            args = {"W1": W1, "WR": WR, "W3": W3}
            Wp, Wm = W.copy(), W.copy()
            Wp[idx] += eps
            Wm[idx] -= eps
            fd[idx] = (_residual_f64(X, **{**args, name: Wp}, T=T) - _residual_f64(X, **{**args, name: Wm}, T=T)) / (2 * eps)
        got = v[grads[name].name].astype(np.float64)
        assert np.linalg.norm(got - fd) <= 3e-2 * np.linalg.norm(fd), name
    # a graph that drops the residual's gradient term is caught: H1's gradient without it
    relu = next(op for op in g.ops if op.kind == "relu_bwd")
    terms = relu.inputs[0].producer.inputs
    assert len(terms) == 2 and not np.array_equal(v[terms[0].name], v[relu.inputs[0].name])
