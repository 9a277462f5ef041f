"""The row quantisation kernel's division-free rule, checked on the CPU.

quantize_rows_resident (vernondsl_amd/csrc/gemm_w8a8.hip) forms rint(x / s) as rint(x * rcp(s)) and
falls back to the IEEE division for any lane whose product lies within 2^-13 of a half-integer (and
for rows whose s is outside [2^-120, 2^120]).  This test restates that rule in numpy float32 (IEEE
round-to-nearest, like the kernel built with -ffp-contract=off) and checks that wherever the fast
path is kept it gives rint(fl(x / s)) exactly, with the reciprocal correctly rounded or off by one
ulp either way (v_rcp_f32's documented accuracy):
  - exhaustively for bf16 rows: every bf16 amax mantissa, every bf16 x with |x| <= amax over 48
    binades below it (further down x * rcp(s) < 2^-40 and both forms give 0);
  - for f32 rows: random amax and x, plus every x within 3 ulp of s * (k + 1/2), k = 0 .. 126, the
    inputs closest to a rounding tie.
The quotients x / s depend on x / amax only (s = amax / 127, scaled by powers of two), so amax in
[1, 2) stands for every binade where s is in the fast path's range.
"""
import numpy as np

F = np.float32
WINDOW = F(2.0 ** -13)


def _check(x, amax):
    """x, amax: float32 arrays of the same shape (|x| <= amax, amax in [1, 2))."""
    s = (amax / F(127.0)).astype(F)
    slow = np.rint((x / s).astype(F))
    r0 = (F(1.0) / s).astype(F)
    kept = 0
    for r in (r0, np.nextafter(r0, F(np.inf)), np.nextafter(r0, F(0.0))):
        q = (x * r).astype(F)
        t = np.rint(q)
        near = np.abs(np.abs((q - t).astype(F)) - F(0.5)) < WINDOW
        bad = (~near) & (t != slow)
        assert not bad.any(), f"fast path differs: x={x[bad][:4]} amax={amax[bad][:4]}"
        kept += int(np.count_nonzero(~near))
    return kept


def test_rule_exhaustive_bf16():
    mant = np.arange(128, dtype=np.uint32)
    amax_bits = (np.uint32(127) << 23) | (mant << 16)            # bf16 values in [1, 2)
    amax = amax_bits.view(F)
    exps = np.arange(127 - 47, 128, dtype=np.uint32)              # binades 2^-47 .. 2^0
    xb = ((exps[:, None] << 23) | (mant[None, :] << 16)).ravel()
    x_pos = xb.view(F)
    total = 0
    for a in amax:
        xs = x_pos[x_pos <= a]
        xs = np.concatenate([xs, -xs])
        total += _check(xs, np.full_like(xs, a))
    assert total > 1_000_000  # the fast path is the common case


def test_rule_f32_random_and_near_ties():
    g = np.random.default_rng(7)
    amax = (F(1.0) + g.random(20000, dtype=F)).astype(F)
    x = (amax * (g.random(20000, dtype=F) * F(2.0) - F(1.0))).astype(F)
    _check(x, amax)
    # inputs next to the ties s * (k + 1/2): the cases the window exists for
    a = (F(1.0) + g.random(300, dtype=F)).astype(F)
    s = (a / F(127.0)).astype(F)
    k = np.arange(127, dtype=F) + F(0.5)
    base = (s[:, None] * k[None, :]).astype(F)
    cand = [base]
    up, dn = base, base
    for _ in range(3):
        up, dn = np.nextafter(up, F(np.inf)), np.nextafter(dn, F(0.0))
        cand += [up, dn]
    xs = np.stack(cand).reshape(len(cand), -1)
    amx = np.broadcast_to(a[:, None], base.shape).ravel()
    for row in xs:
        ok = np.abs(row) <= amx
        _check(np.concatenate([row[ok], -row[ok]]), np.concatenate([amx[ok], amx[ok]]))


def test_rule_window_is_needed():
    """Without the fallback the product form would be wrong somewhere: exact ties exist."""
    a = F(127.0 / 64.0)                      # s = 1/64 exactly: x / s = 64 x
    x = np.array([F(1.5 / 64.0), F(2.5 / 64.0)], F)
    s = F(a / F(127.0))
    assert np.array_equal(np.rint((x / s).astype(F)), [2.0, 2.0])   # 1.5 -> 2, 2.5 -> 2 (half to even)
    q = (x * (F(1.0) / s)).astype(F)
    assert np.all(np.abs(np.abs(q - np.rint(q)) - F(0.5)) < WINDOW)  # both take the division
