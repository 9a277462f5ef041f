"""GPU execution graphs of configs 4 and 5, replayed as one hipGraph, against the CPU oracle.

Config 4 (bf16 MLP train step): small shapes are compared end to end with the oracle composite;
the full shape is checked op by op on sampled rows, each op fed the GPU's own inputs.
Config 5 (int8 inference): bit-exact.  Quantisation is per row, so every output row depends on
its input row only, and sampled rows of the full-size network are checked exactly.
Every graph test replays the graph several times, with eager work and synchronisation between
replays, and compares each replay with the eager run bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import graph, rng, spec

pytestmark = pytest.mark.gpu
BF16 = 1


def gemm_close(got, ref, mag, rel=1e-2):
    got, ref = got.astype(np.float64), ref.astype(np.float64)
    assert np.linalg.norm(got - ref) <= rel * max(np.linalg.norm(ref), 1e-30)
    assert np.all(np.abs(got - ref) <= rel * mag + 1e-30)


def bf16_close(a, b, floor=0.0):
    a, b = rng.bf16_to_f32(a).astype(np.float64), rng.bf16_to_f32(b).astype(np.float64)
    assert np.all(np.abs(a - b) <= 1e-2 * np.abs(b) + floor)


def loss_close(a, b):
    """The default graph forms the loss in the output GEMM's epilogue: the same f64 sum of squares
    in another order, so the f32 loss may differ from the unfused graph's in its last bit."""
    a, b = np.float32(a[0]), np.float32(b[0])
    return abs(float(a) - float(b)) <= 2 * float(np.spacing(b))


def absmm(a, b):
    return np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))


def run_mlp(dev, q, x, w1, w2, t, replays=3, **variant):
    B, D = x.shape
    Hd, O = w1.shape[0], w2.shape[0]
    g, grads = graph.mlp_train_graph(B, D, Hd, O, **variant)
    exe = g.compile(dev)
    for name, arr in (("X", x), ("W1", w1), ("W2", w2), ("T", t)):
        exe.write(q, name, arr)
    names = ["H", "Y", "loss", "grad_W1", "grad_W2"]
    exe.run(q)
    eager = {n: exe.read(q, n) for n in names}
    step = exe.capture(q)
    for _ in range(replays):
        for n in names:  # poison the outputs, then replay
            exe.t[n].buffer.fill_u32(q, 0x7FC07FC0)
        q.sync()
        step.launch(q)
        q.sync()
        for n in names:
            assert np.array_equal(exe.read(q, n), eager[n]), f"replay differs from eager run in {n}"
    step.destroy()
    out = dict(eager)
    fwd = g.ops[0]  # the GELU layer keeps pre, or GELU'(pre) in its place (store_gelu_deriv)
    if fwd.attrs["pre"] is not None:
        out["pre"] = exe.read(q, fwd.attrs["pre"].name)
    else:
        out["dgelu"] = exe.read(q, fwd.attrs["dgelu"].name)
    exe.free()
    return out


@pytest.mark.parametrize("d_in", [384, 512])  # 384: row-major W1 (not packable), 512: the default form
def test_mlp_small_end_to_end(dev, q, d_in):
    x, w1, w2, t = spec.mlp_inputs(batch=256, d_in=d_in, hidden=512, d_out=256)
    got = run_mlp(dev, q, x, w1, w2, t)
    ref = oracle.mlp_train_step(x, w1, w2, t)
    X, W1 = rng.bf16_to_f32(x), rng.bf16_to_f32(w1)
    if "dgelu" in got:  # GELU'(pre) kept instead of pre: within the pre bound through |GELU''| <= 0.8
        dg_ref = oracle.gelu_grad(ref["pre"]).astype(np.float64)
        assert np.all(np.abs(got["dgelu"] - dg_ref) <= 0.8e-2 * absmm(X, W1.T) + 4e-7 * np.abs(dg_ref) + 2e-7)
        got["pre"] = run_mlp(dev, q, x, w1, w2, t, replays=1, store_gelu_deriv=False)["pre"]
    gemm_close(got["pre"], ref["pre"], absmm(X, W1.T))
    assert abs(float(got["loss"][0]) - ref["loss"]) <= 1e-2 * ref["loss"]
    for n in ("grad_W1", "grad_W2"):
        r = ref["d" + n[5:]]
        a = got[n].astype(np.float64)
        assert np.linalg.norm(a - r) <= 1e-2 * np.linalg.norm(r), n


def test_mlp_graph_variants_identical(dev, q):
    """The prepared-transpose, fused-GELU-backward and packed-weight forms of the training step (and
    mlp_train_graph's default, all three) run the same products in the same order: every output
    equals the plain graph's bit for bit (each graph also replays equal to its eager run)."""
    x, w1, w2, t = spec.mlp_inputs(batch=256, d_in=512, hidden=512, d_out=256)
    plain = {"prepare_transposes": False, "fuse_gelu_backward": False, "pack_weights": False, "fuse_mse": False,
             "store_gelu_deriv": False}
    base = run_mlp(dev, q, x, w1, w2, t, replays=2, **plain)
    for variant in ({"prepare_transposes": True}, {"prepare_transposes": True, "fuse_gelu_backward": True},
                    {"pack_weights": True}, {"pack_weights": True, "fuse_mse": True},
                    {"prepare_transposes": True, "fuse_gelu_backward": True, "pack_weights": True}, {}):
        variant = {**plain, **variant} if variant else {}
        got = run_mlp(dev, q, x, w1, w2, t, replays=2, **variant)
        for n in ("H", "Y", "grad_W1", "grad_W2"):
            assert np.array_equal(got[n], base[n]), f"{variant}: {n} differs"
        if "pre" in got:
            assert np.array_equal(got["pre"], base["pre"]), f"{variant}: pre differs"
        assert loss_close(got["loss"], base["loss"]), variant


def test_mlp_rewritten_weights_reprepared(dev, q):
    """Writing W2 after a run re-runs the prepare chain that derives from it (W2 packed; W2^T, then
    W2^T packed): the next step equals the plain graph's step with the new W2, bit for bit."""
    x, w1, w2, t = spec.mlp_inputs(batch=256, d_in=512, hidden=512, d_out=256)
    w2b = np.ascontiguousarray(w2[::-1])
    plain = {"prepare_transposes": False, "fuse_gelu_backward": False, "pack_weights": False, "k_major_grads": False}
    ref = run_mlp(dev, q, x, w1, w2b, t, replays=1, **plain)
    g, _ = graph.mlp_train_graph(256, 512, 512, 256)
    assert len(g.prepare_ops) == 4
    exe = g.compile(dev)
    for name, arr in (("X", x), ("W1", w1), ("W2", w2), ("T", t)):
        exe.write(q, name, arr)
    exe.run(q)
    exe.write(q, "W2", w2b)
    step = exe.capture(q)
    step.launch(q)
    q.sync()
    for n in ("Y", "grad_W1", "grad_W2"):
        assert np.array_equal(exe.read(q, n), ref[n]), n
    assert loss_close(exe.read(q, "loss"), ref["loss"])
    step.destroy()
    exe.free()


def test_mlp_weights_written_after_capture_reach_the_replay(dev, q):
    """A param written after capture (a training loop's weight update): the captured step's next
    launch re-derives the packed W1, W2, W2^T and packed W2^T first, so the replay equals the plain
    graph's step on the new weights bit for bit; then again with the old weights restored."""
    x, w1, w2, t = spec.mlp_inputs(batch=256, d_in=512, hidden=512, d_out=256)
    w1b, w2b = np.ascontiguousarray(w1[:, ::-1]), np.ascontiguousarray(w2[::-1])
    plain = {"prepare_transposes": False, "fuse_gelu_backward": False, "pack_weights": False, "k_major_grads": False}
    ref_new = run_mlp(dev, q, x, w1b, w2b, t, replays=1, **plain)
    ref_old = run_mlp(dev, q, x, w1, w2, t, replays=1, **plain)
    g, _ = graph.mlp_train_graph(256, 512, 512, 256)
    exe = g.compile(dev)
    for name, arr in (("X", x), ("W1", w1), ("W2", w2), ("T", t)):
        exe.write(q, name, arr)
    step = exe.capture(q)
    step.launch(q)
    q.sync()
    names = ("H", "Y", "grad_W1", "grad_W2")
    for n in names:
        assert np.array_equal(exe.read(q, n), ref_old[n]), n
    assert loss_close(exe.read(q, "loss"), ref_old["loss"])
    for (a1, a2), ref in (((w1b, w2b), ref_new), ((w1, w2), ref_old)):
        exe.write(q, "W1", a1)
        exe.write(q, "W2", a2)
        for n in names:
            exe.t[n].buffer.fill_u32(q, 0x7FC07FC0)
        step.launch(q)
        q.sync()
        for n in names:
            assert np.array_equal(exe.read(q, n), ref[n]), n
        assert loss_close(exe.read(q, "loss"), ref["loss"])
    step.destroy()
    exe.free()


def test_mlp_config4_full_size(dev, q):
    """The full-size step with pre kept (the default graph, which keeps GELU'(pre) instead, is
    checked element by element in test_gpu_fullsize.py)."""
    x, w1, w2, t = spec.mlp_inputs()
    got = run_mlp(dev, q, x, w1, w2, t, replays=2, store_gelu_deriv=False)
    B = x.shape[0]
    rows = [0, 777, B - 1]
    X, W1, W2 = rng.bf16_to_f32(x), rng.bf16_to_f32(w1), rng.bf16_to_f32(w2)
    # forward, sampled rows
    for r in rows:
        h, pre = oracle.gemm_bf16(x, w1, 0, 1, c_dtype=BF16, epilogue=1, want_pre=True, row_range=(r, r + 1))
        gemm_close(got["pre"][r:r + 1], pre, absmm(X[r:r + 1], W1.T))
        y = oracle.gemm_bf16(got["H"], w2, 0, 1, row_range=(r, r + 1))
        gemm_close(got["Y"][r:r + 1], y, absmm(rng.bf16_to_f32(got["H"][r:r + 1]), W2.T))
    # loss and dY from the GPU's Y: dY is exact, the loss within f64-sum rounding
    loss, dy, dy_t = oracle.mse_fwd_bwd(got["Y"], t)
    assert abs(float(got["loss"][0]) - loss) <= 1e-6 * loss
    # weight gradients, sampled output rows, from the GPU's own intermediates
    for o in (0, 2048, 4095):
        dw2 = oracle.gemm_bf16(dy_t, got["H"], 0, 0, row_range=(o, o + 1))
        gemm_close(got["grad_W2"][o:o + 1], dw2, absmm(rng.bf16_to_f32(dy_t[o:o + 1]), rng.bf16_to_f32(got["H"])))
    dh = oracle.gemm_bf16(dy, w2, 0, 0)
    da, da_t = oracle.gelu_bwd(dh, got["pre"])
    for o in (0, 1234, 4095):
        dw1 = oracle.gemm_bf16(da_t, x, 0, 0, row_range=(o, o + 1))
        gemm_close(got["grad_W1"][o:o + 1], dw1, absmm(rng.bf16_to_f32(da_t[o:o + 1]), X), rel=2e-2)


def run_w8a8(dev, q, x, layers, replays=3):
    widths = (x.shape[1],) + tuple(w.shape[0] for w, _ in layers)
    g = graph.w8a8_infer_graph(x.shape[0], widths)
    exe = g.compile(dev)
    exe.write(q, "X", x)
    for li, (w, s) in enumerate(layers):
        exe.write(q, f"W{li}", w)
        exe.write(q, f"S{li}", s)
    exe.run(q)
    eager = exe.read(q, "Y")
    step = exe.capture(q)
    for _ in range(replays):
        exe.t["Y"].buffer.fill_u32(q, 0x7FC07FC0)
        q.sync()
        step.launch(q)
        q.sync()
        assert np.array_equal(exe.read(q, "Y"), eager)
    step.destroy()
    exe.free()
    return eager


def test_w8a8_small_bit_exact(dev, q):
    x, layers = spec.w8a8_inputs(batch=64, widths=(512, 384, 256, 128))
    got = run_w8a8(dev, q, x, layers)
    assert np.array_equal(got, oracle.w8a8_forward(x, layers))


def test_w8a8_config5_full_size_sampled_rows(dev, q):
    x, layers = spec.w8a8_inputs()
    got = run_w8a8(dev, q, x, layers, replays=2)
    assert got.shape == (512, 1024)
    rows = np.array([0, 1, 255, 256, 511])
    ref = oracle.w8a8_forward(x[rows], layers)
    assert np.array_equal(got[rows], ref)
    assert np.isfinite(rng.bf16_to_f32(got)).all()


def test_w8a8_rewritten_weights_are_repacked(dev, q):
    """A weight written after a run is packed again before the next run, and before a capture."""
    x, layers = spec.w8a8_inputs(batch=32, widths=(1024, 512, 256))
    g = graph.w8a8_infer_graph(32, (1024, 512, 256))
    assert [op.kind for op in g.ops].count("w8a8_packed") == 2
    exe = g.compile(dev)
    exe.write(q, "X", x)
    for li, (w, s) in enumerate(layers):
        exe.write(q, f"W{li}", w)
        exe.write(q, f"S{li}", s)
    exe.run(q)
    assert np.array_equal(exe.read(q, "Y"), oracle.w8a8_forward(x, layers))
    w0 = np.ascontiguousarray(layers[0][0][::-1])  # other weights, same shape
    layers2 = [(w0, layers[0][1])] + layers[1:]
    exe.write(q, "W0", w0)
    exe.run(q)
    assert np.array_equal(exe.read(q, "Y"), oracle.w8a8_forward(x, layers2))
    exe.write(q, "W0", layers[0][0])
    step = exe.capture(q)
    step.launch(q)
    q.sync()
    assert np.array_equal(exe.read(q, "Y"), oracle.w8a8_forward(x, layers))
    step.destroy()
    exe.free()


def test_elided_values_raise(dev, q):
    """A transposed gradient the graph elided has no buffer: reading or writing it names the reason."""
    g, _ = graph.mlp_train_graph(256, 512, 512, 256)
    exe = g.compile(dev)
    try:
        assert g.elided
        name = sorted(g.elided)[0]
        assert exe.t[name] is None
        with pytest.raises(KeyError, match="elided"):
            exe.read(q, name)
        with pytest.raises(KeyError, match="elided"):
            exe.write(q, name, np.zeros((1,), np.uint16))
    finally:
        exe.free()
    # keep_y=False: y is elided, and the step's loss and gradients are those of keep_y=True
    x, w1, w2, t = spec.mlp_inputs(batch=256, d_in=512, hidden=512, d_out=256)
    res = []
    for keep in (True, False):
        g, _ = graph.mlp_train_graph(256, 512, 512, 256, keep_y=keep)
        exe = g.compile(dev)
        try:
            for nm, arr in (("X", x), ("W1", w1), ("W2", w2), ("T", t)):
                exe.write(q, nm, arr)
            exe.run(q)
            res.append([exe.read(q, n) for n in ("loss", "grad_W1", "grad_W2")])
            if not keep:
                with pytest.raises(KeyError, match="keep_y"):
                    exe.read(q, "Y")
        finally:
            exe.free()
    for a, b in zip(*res):
        assert np.array_equal(a, b)


RES = dict(B=256, D=512, Hd=512, O=256)
FAST = {"prepare_transposes": True, "fuse_gelu_backward": True, "pack_weights": True, "fuse_mse": True,
        "store_gelu_deriv": True, "k_major_grads": True}


def run_residual(dev, q, feeds, replays=2, **flags):
    """The residual graph of tests/test_graph.py (ReLU, GELU, a residual add, a weight tied across
    two layers) on the device: eager run, then replays of its capture equal to it bit for bit."""
    from test_graph import residual_graph
    g, grads = residual_graph(**RES, **flags)
    exe = g.compile(dev)
    names = ["H1", "R", "loss"] + [grads[n].name for n in ("W1", "WR", "W3")]
    try:
        for n, a in feeds.items():
            exe.write(q, n, a)
        exe.run(q)
        eager = {n: exe.read(q, n) for n in names}
        step = exe.capture(q)
        for _ in range(replays):
            for n in names:
                exe.t[n].buffer.fill_u32(q, 0x7FC07FC0)
            q.sync()
            step.launch(q)
            q.sync()
            for n in names:
                assert np.array_equal(exe.read(q, n), eager[n]), f"replay differs from eager run in {n}"
        step.destroy()
    finally:
        exe.free()
    return g, eager


def test_residual_graph_against_the_oracle(dev, q):
    """Plain graph: every op against the oracle's run of the same ops (GEMM tolerances: f32
    accumulation against the oracle's f64 sums), the residual sum and the gradients summed over
    two readers included."""
    from test_graph import residual_inputs
    feeds = residual_inputs(**RES, w_range=0.08)
    g, got = run_residual(dev, q, feeds)
    ref = oracle.graph_step(g, feeds)
    X, W1 = rng.bf16_to_f32(feeds["X"]), rng.bf16_to_f32(feeds["W1"])
    bf16_close(got["H1"], ref["H1"], floor=1e-2 * absmm(X, W1.T).max())
    assert abs(float(got["loss"][0]) - float(ref["loss"][0])) <= 1e-2 * float(ref["loss"][0])
    for n in ("grad_W1", "grad_WR", "grad_W3"):
        a, r = got[n].astype(np.float64), ref[n].astype(np.float64)
        assert np.linalg.norm(a - r) <= 2e-2 * np.linalg.norm(r), n


def test_residual_graph_fused_forms_identical(dev, q):
    """Packed weights, prepared transposes, the fused GELU backward where it applies (H3) and the
    fused loss give the plain graph's values bit for bit (loss: last bit)."""
    from test_graph import residual_inputs
    feeds = residual_inputs(**RES, w_range=0.08)
    _, base = run_residual(dev, q, feeds, replays=1)
    for flags in ({"prepare_transposes": True, "fuse_gelu_backward": True}, {"pack_weights": True}, FAST):
        _, got = run_residual(dev, q, feeds, replays=1, **flags)
        for n in ("H1", "R", "grad_W1", "grad_WR", "grad_W3"):
            assert np.array_equal(got[n], base[n]), f"{flags}: {n} differs"
        assert loss_close(got["loss"], base["loss"]), flags
