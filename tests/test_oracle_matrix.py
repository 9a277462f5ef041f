"""Pins of the oracle's matrix vocabulary: mat2 / mat3 / mat4 operands (source/README.md:34-37),
ExtractComponentOp on a matrix (:41-42), the matrix-vector products of linalg.matvec
(color.mlir:29-36) in vdsl_op_map_chain_v, and the vertex transform for every matrix size
(orc_mat_transform).  The checks do not restate the oracle's loops: identity, permutation and
power-of-two matrices are exact in f32; small-integer matrices and vectors are exact integer
arithmetic (numpy int64 matmul); a product of zeros accumulated into a zero-initialised output is
+0 whatever the signs (0 + (-0) = +0); random operands agree with numpy f64 within the n-term
rounding bound; extraction is numpy indexing; the transposed product equals the product with the
transposed matrix; and the map chain's MVP program equals the dedicated transform bit for bit."""
import itertools

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, mapchain as mc

RNG = np.random.default_rng(0x5EED0007)
U = 2.0 ** -24


def _mat_operand(bcast, rows, cols, d, gen):
    lead = {"full": (rows, cols), "row": (cols,), "col": (rows,), "scalar": ()}[bcast]
    return gen(lead + (d, d)).astype(np.float32)


def _broadcast(m, bcast, rows, cols):
    """The matrix operand seen per element: [rows][cols][d][d]."""
    d = m.shape[-1]
    if bcast == "full":
        return m
    if bcast == "row":
        return np.broadcast_to(m[None], (rows, cols, d, d))
    if bcast == "col":
        return np.broadcast_to(m[:, None], (rows, cols, d, d))
    return np.broadcast_to(m, (rows, cols, d, d))


def _run(out_vec, inputs, rows, cols):
    prog = mc.compile(out_vec)
    return prog, oracle.map_chain_v(prog, inputs, rows, cols)


@pytest.mark.parametrize("d", [2, 3, 4])
@pytest.mark.parametrize("bcast", ["full", "row", "col", "scalar"])
def test_extract_component_is_indexing(d, bcast):
    rows, cols = 5, 7
    m = _mat_operand(bcast, rows, cols, d, RNG.standard_normal)
    M = mc.MatInput(0, d, bcast)
    mb = _broadcast(m, bcast, rows, cols)
    for i, j in itertools.product(range(d), repeat=2):
        for e in (M[i, j], M.component(i * d + j), M[i][j], M.row(i)[j], M.col(j)[i], M.T[j, i]):
            got = oracle.map_chain_v(mc.compile(e), [m], rows, cols)
            assert np.array_equal(got, mb[..., i, j]), (i, j)


@pytest.mark.parametrize("d", [2, 3, 4])
def test_identity_and_permutation_matrices_are_exact(d):
    rows, cols = 6, 9
    v = RNG.standard_normal((rows, cols, d)).astype(np.float32)
    V = mc.VecInput(0, d)
    for perm in itertools.permutations(range(d)):
        P = np.eye(d, dtype=np.float32)[list(perm)]
        _, got = _run(mc.MatInput(1, d) @ V, [v, P], rows, cols)
        assert np.array_equal(got, v[..., list(perm)]), perm
        # v @ P = P^T v: the inverse permutation
        _, got = _run(V @ mc.MatInput(1, d), [v, P], rows, cols)
        assert np.array_equal(got, v[..., list(np.argsort(perm))]), perm


@pytest.mark.parametrize("d", [2, 3, 4])
def test_power_of_two_diagonal_is_exact(d):
    rows, cols = 4, 33
    v = RNG.standard_normal((rows, cols, d)).astype(np.float32)
    diag = np.float32([2.0, -0.5, 4.0, -0.125][:d])
    _, got = _run(mc.MatInput(1, d) @ mc.VecInput(0, d), [v, np.diag(diag)], rows, cols)
    assert np.array_equal(got, v * diag)


@pytest.mark.parametrize("d", [2, 3, 4])
@pytest.mark.parametrize("bcast", ["full", "row", "col", "scalar"])
def test_small_integers_are_exact_integer_arithmetic(d, bcast):
    rows, cols = 7, 10
    v = RNG.integers(-50, 51, (rows, cols, d)).astype(np.float32)
    m = _mat_operand(bcast, rows, cols, d, lambda s: RNG.integers(-9, 10, s))
    mb = _broadcast(m, bcast, rows, cols).astype(np.int64)
    vi = v.astype(np.int64)
    M, V = mc.MatInput(1, d, bcast), mc.VecInput(0, d)
    _, got = _run(M @ V, [v, m], rows, cols)
    assert np.array_equal(got, np.einsum("rcij,rcj->rci", mb, vi).astype(np.float32))
    _, got = _run(V @ M, [v, m], rows, cols)
    assert np.array_equal(got, np.einsum("rcji,rcj->rci", mb, vi).astype(np.float32))
    # chained: M (M v), two products per component, still exact (|values| < 2^24)
    _, got = _run(M @ (M @ V), [v, m], rows, cols)
    want = np.einsum("rcij,rcj->rci", mb, np.einsum("rcij,rcj->rci", mb, vi))
    assert np.array_equal(got, want.astype(np.float32))


def test_products_of_zeros_give_positive_zero():
    rows, cols = 2, 3
    v = np.zeros((rows, cols, 4), np.float32)
    v[..., 1] = -0.0
    for d in (2, 3, 4):
        m = -np.ones((d, d), np.float32)        # every product is -0 or +0 ... summed from +0
        _, got = _run(mc.MatInput(1, d) @ mc.VecInput(0, d), [np.ascontiguousarray(v[..., :d]), m], rows, cols)
        assert np.all(got == 0) and not np.any(np.signbit(got))
        _, got = _run(mc.VecInput(0, d) @ mc.MatInput(1, d), [np.ascontiguousarray(v[..., :d]), m], rows, cols)
        assert np.all(got == 0) and not np.any(np.signbit(got))


@pytest.mark.parametrize("d", [2, 3, 4])
@pytest.mark.parametrize("bcast", ["full", "col", "scalar"])
def test_random_products_within_rounding_of_f64(d, bcast):
    rows, cols = 16, 40
    v = RNG.standard_normal((rows, cols, d)).astype(np.float32)
    m = _mat_operand(bcast, rows, cols, d, RNG.standard_normal)
    mb = _broadcast(m, bcast, rows, cols).astype(np.float64)
    V, M = mc.VecInput(0, d), mc.MatInput(1, d, bcast)
    vd = v.astype(np.float64)
    gamma = d * U / (1 - d * U)   # d rounded products and d - 1 rounded sums (0 + p is exact)
    for expr, want, mag in (
        (M @ V, np.einsum("rcij,rcj->rci", mb, vd), np.einsum("rcij,rcj->rci", np.abs(mb), np.abs(vd))),
        (V @ M, np.einsum("rcji,rcj->rci", mb, vd), np.einsum("rcji,rcj->rci", np.abs(mb), np.abs(vd))),
    ):
        _, got = _run(expr, [v, m], rows, cols)
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= gamma * mag + 1e-45), float((err / (mag + 1e-30)).max())
        # the bound is not vacuous: the results are not all exactly the f64 values
        assert np.any(err > 0)


@pytest.mark.parametrize("d", [2, 3, 4])
def test_transposed_view_equals_transposed_matrix(d):
    rows, cols = 5, 8
    v = RNG.standard_normal((rows, cols, d)).astype(np.float32)
    m = RNG.standard_normal((rows, cols, d, d)).astype(np.float32)
    mt = np.ascontiguousarray(np.swapaxes(m, -1, -2))
    V = mc.VecInput(0, d)
    a = _run(mc.MatInput(1, d, "full").T @ V, [v, m], rows, cols)[1]
    b = _run(V @ mc.MatInput(1, d, "full"), [v, m], rows, cols)[1]
    c = _run(mc.MatInput(1, d, "full") @ V, [v, mt], rows, cols)[1]
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_mvp_program_matches_the_transform():
    """proj @ (view @ (model @ vec(pos, 1))) through the map chain equals orc_vec_transform."""
    rows, cols = 9, 31
    pos = RNG.standard_normal((rows, cols, 3)).astype(np.float32)
    mats = RNG.standard_normal((3, 4, 4)).astype(np.float32)
    p = mc.VecInput(0, 3)
    model, view, proj = (mc.MatInput(k, 4) for k in (1, 2, 3))
    prog, got = _run(proj @ (view @ (model @ mc.vec(p, 1.0))), [pos, *mats], rows, cols)
    assert len(prog.code) <= _lib.MAP_MAX_INSTR and max(max(c[1:5]) for c in prog.code) < _lib.MAP_MAX_REGS
    want = oracle.vec_transform(pos.reshape(-1, 3), mats).reshape(rows, cols, 4)
    assert np.array_equal(got, want)


# ---- the vertex transform for every matrix size ---------------------------------------------------
@pytest.mark.parametrize("d", [2, 3, 4])
def test_transform_identity_permutation_translation_exact(d):
    n = 301
    p = RNG.standard_normal((n, d - 1)).astype(np.float32)
    ph = np.concatenate([p, np.ones((n, 1), np.float32)], 1)
    eye = np.eye(d, dtype=np.float32)
    for k in (1, 2, 3):
        assert np.array_equal(oracle.mat_transform(p, np.stack([eye] * k)), ph)
    for perm in itertools.permutations(range(d)):
        assert np.array_equal(oracle.mat_transform(ph, eye[list(perm)][None]), ph[:, list(perm)])
    T = eye.copy()
    T[: d - 1, d - 1] = np.float32([0.25, -3.0, 8.0][: d - 1])
    S = np.diag(np.float32([2.0, -0.5, 4.0, 1.0][-d:] if d < 4 else [2.0, -0.5, 4.0, 1.0])).astype(np.float32)
    S[d - 1, d - 1] = 1.0
    got = oracle.mat_transform(p, np.stack([S, T]))
    want = ph * np.diag(S) + np.concatenate([T[: d - 1, d - 1], [0.0]]).astype(np.float32)
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("d", [2, 3, 4])
@pytest.mark.parametrize("full", [False, True])
def test_transform_small_integers_exact(d, full):
    n = 400
    w = d if full else d - 1
    p = RNG.integers(-8, 9, (n, w)).astype(np.float32)
    ms = RNG.integers(-4, 5, (3, d, d)).astype(np.float32)
    v = (p if full else np.concatenate([p, np.ones((n, 1), np.float32)], 1)).astype(np.int64)
    for m in ms.astype(np.int64):
        v = v @ m.T
    assert np.array_equal(oracle.mat_transform(p, ms), v.astype(np.float32))


@pytest.mark.parametrize("d", [2, 3, 4])
def test_transform_random_within_rounding_and_composes(d):
    n = 1500
    p = RNG.standard_normal((n, d)).astype(np.float32)
    ms = RNG.standard_normal((3, d, d)).astype(np.float32)
    o = oracle.mat_transform(p, ms).astype(np.float64)
    v, bound = p.astype(np.float64), np.zeros((n, d))
    for m in ms.astype(np.float64):
        bound = np.abs(v) @ np.abs(m.T) * 2 * d * U + bound @ np.abs(m.T)
        v = v @ m.T
    assert np.all(np.abs(o - v) <= bound * 1.01 + 1e-30)
    step = p
    for m in ms:
        step = oracle.mat_transform(step, m[None])
    assert np.array_equal(step, oracle.mat_transform(p, ms))


def test_vec_transform_is_the_mat4_case():
    p = RNG.standard_normal((77, 3)).astype(np.float32)
    ms = RNG.standard_normal((2, 4, 4)).astype(np.float32)
    assert np.array_equal(oracle.vec_transform(p, ms), oracle.mat_transform(p, ms))


# ---- front end ---------------------------------------------------------------------------------------
def test_compiled_products_use_vector_registers():
    V = mc.VecInput(0, 4)
    M = mc.MatInput(1, 4)
    prog = mc.compile(M @ V)
    loads = [c for c in prog.code if c[0] == "load"]
    prods = [c for c in prog.code if c[0] == "matvec"]
    assert len(loads) == 4 and len(prods) == 4
    vregs = [c[1] for c in loads]
    for row, c in enumerate(prods):
        assert c[2] == 1 and c[4] == row and [c[3], *c[6]] == vregs
    assert prog.dims == {0: 0, 1: 4} and prog.widths == {0: 4, 1: 16} and prog.bcast[1] == _lib.BCAST_SCALAR


def test_front_end_errors():
    with pytest.raises(ValueError):
        mc.MatInput(0, 5)
    with pytest.raises(ValueError):
        mc.MatInput(0, 3) @ mc.VecInput(1, 4)
    with pytest.raises(IndexError):
        mc.MatInput(0, 2)[2, 0]
    with pytest.raises(ValueError):   # one input read as a matrix and as a vector
        mc.compile(mc.vec(mc.MatInput(0, 2)[0, 0], mc.VecInput(0, 4).x))
