"""GPU parity of the matrix vocabulary: mat2 / mat3 / mat4 operands of vdsl_op_map_chain_v
(source/README.md:34-37), ExtractComponentOp on a matrix (:41-42), the MATVEC / VECMAT products of
linalg.matvec (color.mlir:29-36), and vdsl_op_mat_transform for every matrix size.

Bar: bit-exact against the CPU oracle (the same separately rounded f32 products and sums in the same
order; components are moved, never rounded), in each of the chain's forms: the interpreter, the
kernel compiled at run time, and the automatic choice."""
import ctypes
import itertools

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, mapchain as mc
from vernondsl_amd._lib import lib
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(0x5EED0008)
LEAD = {"full": lambda r, c: (r, c), "row": lambda r, c: (c,), "col": lambda r, c: (r,), "scalar": lambda r, c: ()}


def _in_mode(mode, fn):
    _lib.call("vdsl_debug_map_chain_mode", mode)
    try:
        return fn()
    finally:
        _lib.call("vdsl_debug_map_chain_mode", 0)


def run_v(dev, q, prog, inputs, rows, cols):
    ts = [Tensor.from_numpy(dev, q, np.ascontiguousarray(a, np.float32)) for a in inputs]
    ow = len(prog.out_regs)
    out = Tensor(dev, (rows, cols, ow) if ow > 1 else (rows, cols), "f32")
    out.buffer.fill_u32(q, 0x7FC00001)
    kernels.map_chain_v(q, prog, ts, out)
    got = out.numpy(q)
    for t in ts + [out]:
        t.free()
    return got


def same_bits(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def check_all_forms(dev, q, prog, inputs, rows, cols):
    ref = oracle.map_chain_v(prog, inputs, rows, cols)
    for mode in (1, 2, 0):   # interpreter, compiled at run time, automatic
        got = _in_mode(mode, lambda: run_v(dev, q, prog, inputs, rows, cols))
        assert same_bits(got, ref), (mode, prog.code)
    return ref


@pytest.mark.parametrize("d", [2, 3, 4])
@pytest.mark.parametrize("bcast", ["full", "row", "col", "scalar"])
@pytest.mark.parametrize("shape", [(19, 261), (7, 1028)])
def test_products_and_extraction_bit_exact(dev, q, d, bcast, shape):
    """(19, 261): one whole block of 256 columns and a partial one, rows not 4-aligned (full mat3
    records then load per lane); (7, 1028): full mat3 and mat4 records staged through LDS in
    every whole block."""
    rows, cols = shape
    v = RNG.standard_normal((rows, cols, d)).astype(np.float32)
    m = RNG.standard_normal(LEAD[bcast](rows, cols) + (d, d)).astype(np.float32)
    V, M = mc.VecInput(0, d), mc.MatInput(1, d, bcast)
    outs = [M @ V, V @ M, M.T @ (M @ V), mc.vec(M[d - 1, 0], M[0, d - 1], M.component(d * d - 1), V.x)]
    for out in outs:
        check_all_forms(dev, q, mc.compile(out), [v, m], rows, cols)


@pytest.mark.parametrize("d", [2, 3, 4])
def test_small_integer_products_exact(dev, q, d):
    rows, cols = 33, 1030
    v = RNG.integers(-50, 51, (rows, cols, d)).astype(np.float32)
    m = RNG.integers(-9, 10, (rows, cols, d, d)).astype(np.float32)
    got = run_v(dev, q, mc.compile(mc.MatInput(1, d, "full") @ mc.VecInput(0, d)), [v, m], rows, cols)
    want = np.einsum("rcij,rcj->rci", m.astype(np.int64), v.astype(np.int64)).astype(np.float32)
    assert np.array_equal(got, want)


def test_products_of_zeros_are_positive_zero(dev, q):
    rows, cols = 4, 300
    for d in (2, 3, 4):
        v = np.zeros((rows, cols, d), np.float32)
        v[..., 0] = -0.0
        m = -np.ones((d, d), np.float32)
        for mode in (1, 2):
            got = _in_mode(mode, lambda: run_v(dev, q, mc.compile(mc.MatInput(1, d) @ mc.VecInput(0, d)), [v, m], rows, cols))
            assert np.all(got == 0) and not np.any(np.signbit(got))


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (1025, 513)])
def test_mvp_chain_equals_the_transform(dev, q, shape):
    """color.mlir:10-39 as one map chain: proj @ (view @ (model @ vec(pos, 1))) with mat4 uniforms."""
    rows, cols = shape
    pos = RNG.standard_normal((rows, cols, 3)).astype(np.float32)
    mats = RNG.standard_normal((3, 4, 4)).astype(np.float32)
    p = mc.VecInput(0, 3)
    model, view, proj = (mc.MatInput(k, 4) for k in (1, 2, 3))
    prog = mc.compile(proj @ (view @ (model @ mc.vec(p, 1.0))))
    ref = check_all_forms(dev, q, prog, [pos, *mats], rows, cols)
    assert same_bits(ref, oracle.vec_transform(pos.reshape(-1, 3), mats).reshape(rows, cols, 4))


def test_matrix_operand_errors(dev, q):
    x = Tensor(dev, (4, 4, 4), "f32")
    out = Tensor(dev, (4, 4), "f32")
    code = (_lib.MapInstr * 1)()
    code[0].op, code[0].dst, code[0].a, code[0].b, code[0].c = _lib.MAP_OPS["matvec"], 0, 0, 0, 0
    vin = (_lib.MapVInput * 1)()
    vin[0].buf, vin[0].bcast, vin[0].dtype, vin[0].width, vin[0].mat_dim = x.handle.value, 0, 0, 4, 0
    regs = (ctypes.c_int32 * 4)(0, 0, 0, 0)
    call = lambda n=1: lib.vdsl_op_map_chain_v(q.handle, 4, 4, code, n, vin, 1, regs, 1, out.handle)  # noqa: E731
    assert call() == -1 and b"matrix input" in lib.vdsl_last_error()   # a vec4 is not a mat2
    vin[0].mat_dim = 2
    assert call() == 0
    code[0].c = 2                     # row 2 of a mat2
    assert call() == -1
    code[0].c, code[0].ext[0] = 1, 8  # vector register out of range
    assert call() == -1
    code[0].ext[0], code[0].ext[1] = 1, 200   # past the mat2's vector: not read, accepted
    assert call() == 0
    vin[0].mat_dim = 3                # width must be mat_dim^2
    assert call() == -1
    vin[0].mat_dim, vin[0].width = 5, 25
    assert call() == -1
    vin[0].mat_dim, vin[0].width = 4, 16   # a mat4 per element needs 4 * 4 * 16 floats: x holds 64
    assert call() == -7
    # the scalar entry point has no matrix inputs
    sin = (_lib.MapInput * 1)()
    sin[0].buf, sin[0].bcast, sin[0].dtype = x.handle.value, 0, 0
    code[0].c = 0
    assert lib.vdsl_op_map_chain(q.handle, 4, 4, code, 1, sin, 1, 0, out.handle) == -1
    q.sync()
    x.free()
    out.free()


# ---- vdsl_op_mat_transform ---------------------------------------------------------------------------
@pytest.mark.parametrize("d", [2, 3, 4])
@pytest.mark.parametrize("full", [False, True])
@pytest.mark.parametrize("n", [1, 5, 1023, 1024, 4099, 100003])
def test_mat_transform_bit_exact(dev, q, d, full, n):
    w = d if full else d - 1
    pos = RNG.standard_normal((n, w)).astype(np.float32)
    for k in (1, 3):
        mats = RNG.standard_normal((k, d, d)).astype(np.float32)
        tp, tm = Tensor.from_numpy(dev, q, pos), Tensor.from_numpy(dev, q, mats)
        to, tv = Tensor(dev, (n, d), "f32"), Tensor(dev, (n, w), "f32")
        to.buffer.fill_u32(q, 0x7FC00001)
        tv.buffer.fill_u32(q, 0x7FC00001)
        kernels.mat_transform(q, tp, tm, to, tv if k == 3 else None)
        assert same_bits(to.numpy(q), oracle.mat_transform(pos, mats)), (d, w, k, n)
        if k == 3:
            assert same_bits(tv.numpy(q), pos)
        for t in (tp, tm, to, tv):
            t.free()


def test_mat_transform_exact_forms_and_errors(dev, q):
    n = 2000
    for d in (2, 3):
        pos = RNG.integers(-8, 9, (n, d - 1)).astype(np.float32)
        mats = RNG.integers(-4, 5, (3, d, d)).astype(np.float32)
        tp, tm, to = Tensor.from_numpy(dev, q, pos), Tensor.from_numpy(dev, q, mats), Tensor(dev, (n, d), "f32")
        kernels.mat_transform(q, tp, tm, to)
        v = np.concatenate([pos, np.ones((n, 1))], 1).astype(np.int64)
        for m in mats.astype(np.int64):
            v = v @ m.T
        assert np.array_equal(to.numpy(q), v.astype(np.float32))
        for perm in itertools.permutations(range(d)):
            P = Tensor.from_numpy(dev, q, np.eye(d, dtype=np.float32)[list(perm)][None])
            kernels.mat_transform(q, tp, P, to)
            ph = np.concatenate([pos, np.ones((n, 1), np.float32)], 1)
            assert np.array_equal(to.numpy(q), ph[:, list(perm)])
            P.free()
        h = lambda t: t.handle  # noqa: E731
        assert lib.vdsl_op_mat_transform(q.handle, n, d, d + 1, h(tp), 3, h(tm), h(to), None) == -1   # in_width
        assert lib.vdsl_op_mat_transform(q.handle, n, 5, d - 1, h(tp), 3, h(tm), h(to), None) == -1   # dim
        assert lib.vdsl_op_mat_transform(q.handle, n, d, d - 1, h(tp), 4, h(tm), h(to), None) == -1   # n_mats
        assert lib.vdsl_op_mat_transform(q.handle, n + 1, d, d - 1, h(tp), 3, h(tm), h(to), None) == -7
        assert lib.vdsl_op_mat_transform(q.handle, n, d, d - 1, h(tp), 3, h(tm), h(tp), None) in (-1, -7)
        assert lib.vdsl_op_mat_transform(q.handle, 0, d, d - 1, h(tp), 3, h(tm), h(to), None) == 0
        for t in (tp, tm, to):
            t.free()
