"""GPU parity of the vector vocabulary (vdsl_op_map_chain_v: vec2-4 operands, extract_component,
swizzle, from_elements; source/README.md:23-55) and of the MVP vertex transform
(vdsl_op_vec_transform; color.mlir:10-39) against the CPU oracle.

Bar: bit-exact for swizzles and extraction (components are moved, never rounded), for chains of
+, -, * (the same f32 operations in the same order), and for the vertex transform (the same
separately rounded products and sums); 1e-5 relative for chains with exp/tanh (the library's
branch-free forms against libm)."""
import ctypes
import itertools

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, mapchain as mc
from vernondsl_amd._lib import lib
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(0x5EED0007)


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


@pytest.mark.parametrize("w", [2, 3, 4])
@pytest.mark.parametrize("shape", [(1, 1), (7, 13), (64, 300), (513, 1027)])
def test_swizzles_bit_exact(dev, q, w, shape):
    rows, cols = shape
    x = RNG.standard_normal((rows, cols, w)).astype(np.float32)
    pats = ["".join("xyzw"[i] for i in p) for p in itertools.permutations(range(w))][:6]
    pats += ["x", "rg"[:w], "xx", ("zyx" if w >= 3 else "yx"), ("wzyx" if w == 4 else "yyyy"[:max(2, w)])]
    for pat in pats:
        prog = mc.compile(mc.VecInput(0, w).swizzle(pat))
        got = run_v(dev, q, prog, [x], rows, cols)
        ref = oracle.map_chain_v(prog, [x], rows, cols)
        assert np.array_equal(got, ref), (pat, shape)
        assert np.array_equal(got.reshape(rows, cols, -1), x[..., mc._components(pat, w)])


def test_from_elements_and_broadcast_vectors(dev, q):
    rows, cols = 37, 1029
    full = RNG.standard_normal((rows, cols, 3)).astype(np.float32)
    rowb = RNG.standard_normal((cols, 4)).astype(np.float32)
    colb = RNG.standard_normal((rows, 2)).astype(np.float32)
    sc = RNG.standard_normal(4).astype(np.float32)
    a, b, c, d = mc.VecInput(0, 3), mc.VecInput(1, 4, "row"), mc.VecInput(2, 2, "col"), mc.VecInput(3, 4, "scalar")
    for out in (mc.vec(a.x, b.a, c.y, d.w), mc.vec(a.zyx, 1.0), mc.vec(a.xy * c.yx + b.ba, a.z - d.x, 0.5),
                mc.vec(a.x * 2.0, b.g)):
        prog = mc.compile(out)
        ins = [full, rowb, colb, sc][:prog.n_inputs]
        got = run_v(dev, q, prog, ins, rows, cols)
        assert np.array_equal(got, oracle.map_chain_v(prog, ins, rows, cols))


def test_transcendental_vector_chain(dev, q):
    rows, cols = 129, 700
    p = RNG.standard_normal((rows, cols, 4)).astype(np.float32)
    v = mc.VecInput(0, 4)
    prog = mc.compile(mc.vec(mc.tanh(v.rgb * 0.75), mc.exp(-(v.a * v.a))))
    got = run_v(dev, q, prog, [p], rows, cols).astype(np.float64)
    ref = oracle.map_chain_v(prog, [p], rows, cols).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 * np.abs(ref) + 1e-30)


def test_width_one_vector_entry_equals_scalar_entry(dev, q):
    rows, cols = 33, 515
    x = RNG.standard_normal((rows, cols)).astype(np.float32)
    bias = RNG.standard_normal(cols).astype(np.float32)
    prog = mc.compile(mc.Input(0) * mc.Input(1, "row") - mc.Input(0) * 0.5)
    got = run_v(dev, q, prog, [x, bias], rows, cols)
    tx, tb, ty = Tensor.from_numpy(dev, q, x), Tensor.from_numpy(dev, q, bias), Tensor(dev, (rows, cols), "f32")
    kernels.map_chain(q, prog, [tx, tb], ty)
    assert np.array_equal(got, ty.numpy(q)) and np.array_equal(got, oracle.map_chain(prog, [x, bias], rows, cols))
    for t in (tx, tb, ty):
        t.free()


def test_vector_chain_errors(dev, q):
    x = Tensor(dev, (4, 4, 3), "f32")
    out = Tensor(dev, (4, 4, 2), "f32")
    code = (_lib.MapInstr * 1)()
    code[0].op, code[0].dst, code[0].a, code[0].c = _lib.MAP_OPS["load"], 0, 0, 3   # component 3 of a vec3
    vin = (_lib.MapVInput * 1)()
    vin[0].buf, vin[0].bcast, vin[0].dtype, vin[0].width = x.handle.value, 0, 0, 3
    regs = (ctypes.c_int32 * 4)(0, 0, 0, 0)
    assert lib.vdsl_op_map_chain_v(q.handle, 4, 4, code, 1, vin, 1, regs, 2, out.handle) == -1
    code[0].c = 2
    assert lib.vdsl_op_map_chain_v(q.handle, 4, 4, code, 1, vin, 1, regs, 3, out.handle) == -7   # out too small
    assert lib.vdsl_op_map_chain_v(q.handle, 4, 4, code, 1, vin, 1, regs, 5, out.handle) == -1   # out_width
    vin[0].width = 5
    assert lib.vdsl_op_map_chain_v(q.handle, 4, 4, code, 1, vin, 1, regs, 2, out.handle) == -1
    # the scalar entry point refuses a component other than 0
    sin = (_lib.MapInput * 1)()
    sin[0].buf, sin[0].bcast, sin[0].dtype = x.handle.value, 0, 0
    code[0].c = 1
    assert lib.vdsl_op_map_chain(q.handle, 4, 4, code, 1, sin, 1, 0, out.handle) == -1
    x.free()
    out.free()


# ---- vertex transform --------------------------------------------------------------------------
def _mats(k):
    return RNG.standard_normal((k, 4, 4)).astype(np.float32)


@pytest.mark.parametrize("w", [3, 4])
@pytest.mark.parametrize("k", [1, 2, 3])
@pytest.mark.parametrize("n", [1, 3, 4, 1021, 4096, 100003])
def test_vec_transform_bit_exact(dev, q, w, k, n):
    pos = RNG.standard_normal((n, w)).astype(np.float32)
    mats = _mats(k)
    tp, tm = Tensor.from_numpy(dev, q, pos), Tensor.from_numpy(dev, q, mats)
    to, tv = Tensor(dev, (n, 4), "f32"), Tensor(dev, (n, w), "f32")
    to.buffer.fill_u32(q, 0x7FC00001)
    kernels.vec_transform(q, tp, tm, to, tv if n % 2 else None)
    got = to.numpy(q)
    assert np.array_equal(got, oracle.vec_transform(pos, mats))
    if n % 2:
        assert np.array_equal(tv.numpy(q), pos)
    for t in (tp, tm, to, tv):
        t.free()


def test_vec_transform_exact_forms_and_errors(dev, q):
    n = 1000
    pos = RNG.integers(-8, 9, (n, 3)).astype(np.float32)
    mats = RNG.integers(-4, 5, (3, 4, 4)).astype(np.float32)
    tp, tm, to = Tensor.from_numpy(dev, q, pos), Tensor.from_numpy(dev, q, mats), Tensor(dev, (n, 4), "f32")
    kernels.vec_transform(q, tp, tm, to)
    v = np.concatenate([pos, np.ones((n, 1))], 1).astype(np.int64)
    for m in mats.astype(np.int64):
        v = v @ m.T
    assert np.array_equal(to.numpy(q), v.astype(np.float32))
    # -I on zero positions: +0, not -0
    z = Tensor.from_numpy(dev, q, np.zeros((8, 4), np.float32))
    mi = Tensor.from_numpy(dev, q, -np.eye(4, dtype=np.float32)[None])
    o8 = Tensor(dev, (8, 4), "f32")
    kernels.vec_transform(q, z, mi, o8)
    assert not np.any(np.signbit(o8.numpy(q)))
    assert lib.vdsl_op_vec_transform(q.handle, n, 2, tp.handle, 3, tm.handle, to.handle, None) == -1
    assert lib.vdsl_op_vec_transform(q.handle, n, 3, tp.handle, 4, tm.handle, to.handle, None) == -1
    assert lib.vdsl_op_vec_transform(q.handle, n + 1, 3, tp.handle, 3, tm.handle, to.handle, None) == -7
    assert lib.vdsl_op_vec_transform(q.handle, n, 3, tp.handle, 3, tm.handle, tp.handle, None) in (-1, -7)
    assert lib.vdsl_op_vec_transform(q.handle, 0, 3, tp.handle, 3, tm.handle, to.handle, None) == 0
    for t in (tp, tm, to, z, mi, o8):
        t.free()
