"""Pins of the oracle's vector vocabulary (vec2-4, extract_component, swizzle: source/README.md:23-55)
and of the MVP vertex transform (color.mlir:10-39), by closed forms that do not restate its loops:
swizzles are permutations (numpy fancy indexing), they compose as permutations, extracting after a
swizzle picks the permuted component; identity, permutation, power-of-two and translation matrices
transform exactly in f32; small-integer matrices and positions are exact integer arithmetic; a
zero position under -I gives +0 (the matvec accumulates into a zero-initialised output); random
inputs agree with f64 within the rounding bound of 4-term sums."""
import itertools

import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, mapchain as mc

RNG = np.random.default_rng(0x5EED0006)
SETS = ("xyzw", "rgba", "stpq")


def _vin(shape, w):
    return RNG.standard_normal(shape + ((w,) if w > 1 else ())).astype(np.float32)


@pytest.mark.parametrize("w", [1, 2, 3, 4])
def test_swizzle_is_fancy_indexing(w):
    rows, cols = 5, 9
    x = _vin((rows, cols), w)
    x3 = x.reshape(rows, cols, w)
    for n in range(1, 5):
        for idx in itertools.islice(itertools.product(range(w), repeat=n), 40):
            pat = "".join(SETS[len(idx) % 3][i] for i in idx)
            v = mc.VecInput(0, w)
            e = v.swizzle(pat)
            prog = mc.compile(e)
            got = oracle.map_chain_v(prog, [x], rows, cols)
            want = x3[..., list(idx)]
            assert np.array_equal(got.reshape(want.shape), want), pat


def test_swizzles_compose_as_permutations():
    rows, cols = 4, 6
    x = _vin((rows, cols), 4)
    for p in itertools.permutations(range(4)):
        for q in (p[::-1], (1, 0, 3, 2), (3, 3, 0, 1)):
            pp, qq = "".join("xyzw"[i] for i in p), "".join("rgba"[i] for i in q)
            first = oracle.map_chain_v(mc.compile(mc.VecInput(0, 4).swizzle(pp)), [x], rows, cols)
            second = oracle.map_chain_v(mc.compile(mc.VecInput(0, 4).swizzle(qq)), [first], rows, cols)
            once = oracle.map_chain_v(mc.compile(mc.VecInput(0, 4).swizzle(pp).swizzle(qq)), [x], rows, cols)
            composed = "".join("xyzw"[p[i]] for i in q)
            direct = oracle.map_chain_v(mc.compile(mc.VecInput(0, 4).swizzle(composed)), [x], rows, cols)
            assert np.array_equal(second, direct) and np.array_equal(once, direct), (pp, qq)


def test_extract_after_swizzle_picks_the_permuted_component():
    rows, cols = 3, 5
    x = _vin((rows, cols), 3)
    for pat in ("zyx", "xzy", "bgr", "rrg"):
        v = mc.VecInput(0, 3)
        sw = v.swizzle(pat)
        for i in range(3):
            a = oracle.map_chain_v(mc.compile(sw[i]), [x], rows, cols)
            b = oracle.map_chain_v(mc.compile(v.component(pat[i])), [x], rows, cols)
            assert np.array_equal(a, b) and np.array_equal(a, x[..., mc._components(pat, 3)[i]])


def test_broadcast_vector_operands():
    rows, cols = 6, 7
    full = _vin((rows, cols), 3)
    rowb = RNG.standard_normal((cols, 3)).astype(np.float32)
    colb = RNG.standard_normal((rows, 2)).astype(np.float32)
    sc = RNG.standard_normal(4).astype(np.float32)
    a, b = mc.VecInput(0, 3), mc.VecInput(1, 3, "row")
    c, d = mc.VecInput(2, 2, "col"), mc.VecInput(3, 4, "scalar")
    prog = mc.compile(mc.vec(a.x, b.z, c.y, d.w))
    got = oracle.map_chain_v(prog, [full, rowb, colb, sc], rows, cols)
    want = np.stack([full[..., 0], np.broadcast_to(rowb[:, 2], (rows, cols)),
                     np.broadcast_to(colb[:, 1:2], (rows, cols)), np.full((rows, cols), sc[3], np.float32)], -1)
    assert np.array_equal(got, want)


def test_width_one_vector_chain_equals_scalar_chain():
    rows, cols = 8, 16
    x = RNG.standard_normal((rows, cols)).astype(np.float32)
    bias = RNG.standard_normal(cols).astype(np.float32)
    e = mc.tanh(mc.Input(0) * 0.5 + 0.25) * mc.Input(1, "row") - mc.Input(0)
    prog = mc.compile(e)
    assert np.array_equal(oracle.map_chain_v(prog, [x, bias], rows, cols), oracle.map_chain(prog, [x, bias], rows, cols))


def test_vector_arithmetic_against_f64():
    rows, cols = 7, 11
    p = _vin((rows, cols), 3)
    col = RNG.standard_normal((cols, 4)).astype(np.float32)
    v, c = mc.VecInput(0, 3), mc.VecInput(1, 4, "row")
    out = mc.vec(v.zyx * 2.0 + c.rgb, mc.exp(-(v.x * v.x)))
    got = oracle.map_chain_v(mc.compile(out), [p, col], rows, cols).astype(np.float64)
    P, Cc = p.astype(np.float64), col.astype(np.float64)
    want = np.concatenate([P[..., ::-1] * 2 + Cc[None, :, :3], np.exp(-P[..., :1] ** 2)], -1)
    assert np.all(np.abs(got - want) <= 1e-6 * (np.abs(want) + 2 * np.abs(P[..., ::-1][..., [0, 0, 0, 0]]) + 1e-6))


# ---- vertex transform ------------------------------------------------------------------------------
def _pos(n, w=3, scale=1.0):
    return (RNG.standard_normal((n, w)) * scale).astype(np.float32)


def test_identity_and_permutation_matrices_are_exact():
    p = _pos(257)
    I = np.eye(4, dtype=np.float32)
    for k in (1, 2, 3):
        o = oracle.vec_transform(p, np.stack([I] * k))
        assert np.array_equal(o[:, :3], p) and np.all(o[:, 3] == 1.0)
    for perm in itertools.permutations(range(4)):
        P = I[list(perm)]
        o = oracle.vec_transform(p, P[None])
        v4 = np.concatenate([p, np.ones((len(p), 1), np.float32)], 1)
        assert np.array_equal(o, v4[:, list(perm)]), perm


def test_power_of_two_scaling_and_translation_are_exact():
    p = _pos(300)
    S = np.diag([2.0, 0.5, -4.0, 1.0]).astype(np.float32)
    T = np.eye(4, dtype=np.float32)
    T[:3, 3] = [0.25, -3.0, 8.0]
    o = oracle.vec_transform(p, np.stack([S, T]))
    # T (S v): the translation adds exactly to the scaled coordinates (one rounding, as numpy f32)
    want = np.stack([p[:, 0] * np.float32(2) + np.float32(0.25), p[:, 1] * np.float32(0.5) - np.float32(3),
                     p[:, 2] * np.float32(-4) + np.float32(8), np.ones(len(p), np.float32)], 1)
    assert np.array_equal(o, want)


def test_small_integers_are_exact_integer_arithmetic():
    n = 500
    p = RNG.integers(-8, 9, (n, 3)).astype(np.float32)
    ms = RNG.integers(-4, 5, (3, 4, 4)).astype(np.float32)
    o = oracle.vec_transform(p, ms)
    v = np.concatenate([p, np.ones((n, 1))], 1).astype(np.int64)
    for m in ms.astype(np.int64):   # |values| stay far below 2^24: every f32 step is exact
        v = v @ m.T
    assert np.array_equal(o.astype(np.int64), v) and np.array_equal(o, v.astype(np.float32))


def test_zero_initialised_accumulation_gives_positive_zero():
    p = np.zeros((4, 4), np.float32)
    o = oracle.vec_transform(p, -np.eye(4, dtype=np.float32)[None])
    assert np.all(o == 0) and not np.any(np.signbit(o))   # 0 + (-1 * 0) = +0, not -0


def test_random_chain_within_f32_rounding_of_f64():
    n = 2000
    p = _pos(n, 4)
    ms = RNG.standard_normal((3, 4, 4)).astype(np.float32)
    o = oracle.vec_transform(p, ms).astype(np.float64)
    v, bound = p.astype(np.float64), np.zeros((n, 4))
    for m in ms.astype(np.float64):
        # each output: 4 products and 4 sums rounded; the error carried from v scales with |M|
        bound = np.abs(v) @ np.abs(m.T) * 8 * 2.0 ** -24 + bound @ np.abs(m.T)
        v = v @ m.T
    assert np.all(np.abs(o - v) <= bound * 1.01 + 1e-30)
    # and the chain is the composition of single transforms
    step = p
    for m in ms:
        step = oracle.vec_transform(step, m[None])
    assert np.array_equal(step, oracle.vec_transform(p, ms))


def test_varying_widths_and_names():
    v = mc.VecInput(0, 2)
    with pytest.raises(ValueError):
        v.swizzle("xz")          # z is past a vec2
    with pytest.raises(ValueError):
        v.swizzle("xg")          # two component sets in one pattern
    with pytest.raises(AttributeError):
        v.xyzwx                  # five components
    assert _lib.MAP_MAX_INPUTS == 4
