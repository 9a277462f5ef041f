"""GPU parity of the packed-weight int8 GEMM (vdsl_op_gemm_w8a8_packed) and the weight packing.

Bar: bit-exact.  The int32 accumulators and the dequantised outputs must equal the CPU oracle's
(orc_gemm_w8a8 on the unpacked weights) and the row-major GPU kernel's, for shapes that take
every launch plan: 128 x 256 blocks (large M), 128 x 128 blocks (config-5 layers), 128 x 128
blocks with K split four ways (the 1024-wide last layer), 64 x 256 blocks with K split (M < 128),
and ragged M and N; and every plan forced on one ragged shape.  Calls
in a row on one workspace (left holding the previous call's partials) must not depend on its
contents.
"""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
F32, BF16 = 0, 1


def _operands(M, N, K, seed):
    r = np.random.default_rng(seed)
    xq = r.integers(-127, 128, (M, K)).astype(np.int8)
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    xs = r.uniform(0.001, 0.01, M).astype(np.float32)
    ws = r.uniform(0.005, 0.02, N).astype(np.float32)
    return xq, w, xs, ws


class Packed:
    """Device operands of one packed GEMM shape, with its own workspace (filled with a NaN-like
    pattern first: the kernels must not depend on its contents)."""

    def __init__(self, dev, q, M, N, K):
        self.M, self.N, self.K = M, N, K
        self.wsb = kernels.gemm_w8a8_packed_workspace_bytes(M, N, K)
        self.ws = Tensor(dev, (max(self.wsb, 4),), "i8")
        self.ws.buffer.fill_u32(q, 0x7FC07FC0)
        self.dev, self.q = dev, q

    def run(self, xq, w, xs, ws, relu, dt):
        dev, q, M, N, K = self.dev, self.q, self.M, self.N, self.K
        txq, tw, txs, tws = (Tensor.from_numpy(dev, q, a) for a in (xq, w, xs, ws))
        twp = Tensor(dev, (N, K), "i8")
        kernels.pack_w8a8_weights(q, tw, twp)
        ty, tacc = Tensor(dev, (M, N), dt), Tensor(dev, (M, N), "i32")
        ty.buffer.fill_u32(q, 0x7FC07FC0)
        kernels.gemm_w8a8_packed(q, txq, txs, twp, tws, ty, relu, tacc, self.ws if self.wsb else None)
        y, acc = ty.numpy(q), tacc.numpy(q)
        for t in (txq, tw, txs, tws, twp, ty, tacc):
            t.free()
        return y, acc

    def free(self):
        self.ws.free()


def test_pack_layout(dev, q):
    """The packed array is the register image of MFMA B fragments: unit (nb, kb) holds lane l's
    16 bytes w[32 nb + l % 32][32 kb + 16 (l // 32) ...]."""
    N, K = 96, 128
    w = np.random.default_rng(5).integers(-128, 128, (N, K)).astype(np.int8)
    tw, twp = Tensor.from_numpy(dev, q, w), Tensor(dev, (N, K), "i8")
    kernels.pack_w8a8_weights(q, tw, twp)
    got = twp.numpy(q).reshape(N // 32, K // 32, 64, 16)
    for nb in range(N // 32):
        for kb in range(K // 32):
            for lane in (0, 1, 31, 32, 33, 63):
                r, c = 32 * nb + lane % 32, 32 * kb + 16 * (lane // 32)
                assert np.array_equal(got[nb, kb, lane], w[r, c:c + 16]), (nb, kb, lane)
    # every byte of w appears exactly once
    assert np.array_equal(np.sort(got.reshape(-1)), np.sort(w.reshape(-1)))
    tw.free()
    twp.free()


@pytest.mark.parametrize("M,N,K,relu,dt", [(64, 256, 4096, True, "bf16"),   # 64x256 blocks, split 8
                                           (100, 96, 512, False, "f32"),    # ragged M, N < block, no split
                                           (130, 320, 2048, True, "bf16"),  # ragged M and N, split 4
                                           (256, 512, 1024, False, "f32"),  # split 2
                                           (1024, 8192, 512, True, "bf16"),  # 128x256 blocks
                                           (1000, 8224, 512, False, "f32"),  # 128x256, ragged
                                           (500, 8224, 512, True, "bf16"),    # 128x128, ragged M and N
                                           (512, 4096, 1024, False, "bf16")])  # 128x128, whole tiles
def test_packed_vs_oracle(dev, q, M, N, K, relu, dt):
    xq, w, xs, ws = _operands(M, N, K, M * 7 + N + K)
    p = Packed(dev, q, M, N, K)
    y, acc = p.run(xq, w, xs, ws, relu, dt)
    ry, racc = oracle.gemm_w8a8(xq, xs, w, ws, out_dtype=BF16 if dt == "bf16" else F32, relu=relu, want_acc=True)
    assert np.array_equal(acc, racc)
    assert np.array_equal(y, ry)
    p.free()


@pytest.mark.parametrize("M,N,K", [(512, 8192, 8192), (512, 1024, 8192)])
def test_packed_config5_shapes(dev, q, M, N, K):
    """Config-5 layer shapes: equal to the row-major kernel everywhere, to the oracle on sampled
    rows, and to an exact int64 product on a column slice of every row."""
    xq, w, xs, ws = _operands(M, N, K, N + K)
    p = Packed(dev, q, M, N, K)
    y, acc = p.run(xq, w, xs, ws, True, "bf16")
    txq, tw, txs, tws = (Tensor.from_numpy(dev, q, a) for a in (xq, w, xs, ws))
    ty, tacc = Tensor(dev, (M, N), "bf16"), Tensor(dev, (M, N), "i32")
    wsb = kernels.gemm_w8a8_workspace_bytes(M, N, K)
    twk = Tensor(dev, (max(1, wsb),), "i8")
    kernels.gemm_w8a8(q, txq, txs, tw, tws, ty, True, tacc, twk if wsb else None)
    assert np.array_equal(acc, tacc.numpy(q))
    assert np.array_equal(y, ty.numpy(q))
    rows = slice(0, 8)
    ry, racc = oracle.gemm_w8a8(xq[rows], xs[rows], w, ws, out_dtype=BF16, relu=True, want_acc=True)
    assert np.array_equal(acc[rows], racc)
    assert np.array_equal(y[rows], ry)
    cols = slice(N - 64, N)
    ref = xq.astype(np.int64) @ w[cols].astype(np.int64).T
    assert np.array_equal(acc[:, cols], ref.astype(np.int32))
    for t in (txq, tw, txs, tws, ty, tacc, twk):
        t.free()
    p.free()


def test_packed_calls_in_a_row(dev, q):
    """One workspace, three calls with different operands: each result is exact, whatever the
    call before left in the workspace."""
    M, N, K = 128, 512, 4096
    p = Packed(dev, q, M, N, K)
    assert p.wsb > 0
    for seed in (1, 2, 3):
        xq, w, xs, ws = _operands(M, N, K, seed)
        y, acc = p.run(xq, w, xs, ws, seed % 2 == 1, "bf16")
        ry, racc = oracle.gemm_w8a8(xq, xs, w, ws, out_dtype=BF16, relu=seed % 2 == 1, want_acc=True)
        assert np.array_equal(acc, racc), seed
        assert np.array_equal(y, ry), seed
    p.free()


def test_packed_shape_errors(dev, q):
    with pytest.raises(_lib.VdslError):
        kernels.gemm_w8a8_packed_workspace_bytes(64, 256, 4000)  # K % 512
    with pytest.raises(_lib.VdslError):
        kernels.gemm_w8a8_packed_workspace_bytes(64, 250, 4096)  # N % 32
    tw, twp = Tensor(dev, (40, 64), "i8"), Tensor(dev, (40, 64), "i8")
    with pytest.raises(_lib.VdslError):
        kernels.pack_w8a8_weights(q, tw, twp)  # N % 32
    tw.free()
    twp.free()


@pytest.mark.parametrize("cfg,split", [(0, 1), (0, 2), (1, 1), (1, 4), (2, 1), (2, 2), (3, 1), (3, 3), (3, 8), (4, 1),
                                       (4, 4), (5, 1), (5, 3), (6, 1), (6, 2)])
def test_every_forced_plan(dev, q, cfg, split):
    """Each tile configuration and K split, forced with vdsl_debug_w8a8_packed_plan on a shape
    ragged in M and N: bit-exact against the oracle (a split whose stages do not divide K is
    ignored by the library; K = 6144 divides by every split here)."""
    M, N, K = 200, 352, 6144
    xq, w, xs, ws = _operands(M, N, K, 31 * cfg + split)
    _lib.call("vdsl_debug_w8a8_packed_plan", cfg, split)
    try:
        p = Packed(dev, q, M, N, K)
        y, acc = p.run(xq, w, xs, ws, True, "bf16")
        p.free()
    finally:
        _lib.call("vdsl_debug_w8a8_packed_plan", -1, 0)
    ry, racc = oracle.gemm_w8a8(xq, xs, w, ws, out_dtype=BF16, relu=True, want_acc=True)
    assert np.array_equal(acc, racc)
    assert np.array_equal(y, ry)
