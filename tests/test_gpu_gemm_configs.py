"""Every GEMM tile configuration of the library, forced one at a time with vdsl_debug_gemm_config.

The per-shape choice runs only a few configurations in the other tests; this file runs all of them
on shapes with ragged edge tiles in both directions (rows and columns past M and N are clamped in
the direct-to-LDS loops, masked in the register-staged ones) and a K that every configuration
accepts.  bf16: every configuration accumulates the same k-steps in the same order with the same
MFMA, so each output must equal the per-shape choice's bit for bit, and that one is checked
against the oracle at the bf16 GEMM tolerance.  int8 (including the split-K configurations, which
these small outputs select): accumulators and outputs bit-exact against the oracle.
"""
import numpy as np
import pytest

from oracle import oracle
from vernondsl_amd import _lib, kernels, rng
from vernondsl_amd._lib import call
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
BF16 = 1
N_BF16_CONFIGS = 27  # gemm_bf16.hip: register-staged 0..13, direct-to-LDS 14..22, 128-byte stages 23..26
N_W8A8_CONFIGS = 23  # gemm_w8a8.hip: register-staged 0..13, direct-to-LDS 14..19, 128-byte stages 20..22


@pytest.fixture
def forced_config():
    yield lambda c: call("vdsl_debug_gemm_config", c)
    call("vdsl_debug_gemm_config", -1)


def run_bf16(dev, q, tA, tB, M, N, K, gelu):
    out = Tensor(dev, (M, N), "bf16" if gelu else "f32")
    out.buffer.fill_u32(q, 0x7FC07FC0)
    pre = Tensor(dev, (M, N), "f32") if gelu else None
    if pre is not None:
        pre.buffer.fill_u32(q, 0x7FC07FC0)
    kernels.gemm_bf16(q, tA, tB, out, False, True, _lib.EPI_GELU if gelu else _lib.EPI_NONE, pre)
    res = (out.numpy(q), pre.numpy(q) if pre is not None else None)
    out.free()
    if pre is not None:
        pre.free()
    return res


@pytest.mark.parametrize("M,N,K", [(300, 520, 256), (129, 258, 128)])
def test_every_bf16_config_matches(dev, q, forced_config, M, N, K):
    A = rng.f32_to_bf16(rng.uniform(71, M * K, -1, 1)).reshape(M, K)
    B = rng.f32_to_bf16(rng.uniform(72, N * K, -1, 1)).reshape(N, K)
    tA, tB = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16")
    try:
        forced_config(-1)
        base = {g: run_bf16(dev, q, tA, tB, M, N, K, g) for g in (False, True)}
        ref_f32 = oracle.gemm_bf16(A, B, False, True)
        got = base[False][0].astype(np.float64)
        mag = np.abs(rng.bf16_to_f32(A).astype(np.float64)) @ np.abs(rng.bf16_to_f32(B).astype(np.float64)).T
        assert np.all(np.abs(got - ref_f32) <= 1e-2 * mag + 1e-30)
        assert np.array_equal(base[True][1], base[False][0])  # pre-activation == plain product
        for c in range(N_BF16_CONFIGS):
            forced_config(c)
            for g in (False, True):
                out, pre = run_bf16(dev, q, tA, tB, M, N, K, g)
                assert np.array_equal(out, base[g][0]), f"config {c} gelu={g}: output differs"
                if g:
                    assert np.array_equal(pre, base[g][1]), f"config {c}: pre-activation differs"
    finally:
        tA.free()
        tB.free()


@pytest.mark.parametrize("M,N,K", [(300, 512, 256), (256, 768, 192), (129, 258, 128)])
def test_bf16_nn_k_major_b_matches_nt(dev, q, forced_config, M, N, K):
    """B stored [K][N] (trans_b = 0): with N % 256 == 0 the 256-wide direct-to-LDS configurations
    (15, and 23 when K % 64 == 0) read B K-major with transposing LDS reads instead of transposing
    it first; every output equals the NT product of the host-transposed B under the same
    configuration, bit for bit (same k-steps, same order).  N = 258 takes the transpose path."""
    A = rng.f32_to_bf16(rng.uniform(81, M * K, -1, 1)).reshape(M, K)
    B = rng.f32_to_bf16(rng.uniform(82, K * N, -1, 1)).reshape(K, N)
    tA, tB = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16")
    tBt = Tensor.from_numpy(dev, q, np.ascontiguousarray(B.T), "bf16")
    ws = Tensor(dev, (max(1, kernels.gemm_bf16_workspace_bytes(False, False, M, N, K)),), "i8")
    try:
        for c in (-1, 15, 23):
            forced_config(c)
            for gelu in (False, True):
                outs = []
                for tb, src in ((False, tB), (True, tBt)):
                    ws.buffer.fill_u32(q, 0xA5A5A5A5)
                    out = Tensor(dev, (M, N), "bf16" if gelu else "f32")
                    pre = Tensor(dev, (M, N), "f32") if gelu else None
                    for t in (out, pre):
                        if t is not None:
                            t.buffer.fill_u32(q, 0x7FC07FC0)
                    kernels.gemm_bf16(q, tA, src, out, False, tb, _lib.EPI_GELU if gelu else _lib.EPI_NONE, pre,
                                      None if tb else ws)
                    outs.append((out.numpy(q), pre.numpy(q) if pre is not None else None))
                    if not tb and c in (15, 23) and N % 256 == 0:  # the K-major kernel ran: no transpose into ws
                        assert np.all(ws.numpy(q).view(np.uint32) == 0xA5A5A5A5), f"config {c}: B was transposed"
                    out.free()
                    if pre is not None:
                        pre.free()
                (o_nn, p_nn), (o_nt, p_nt) = outs
                assert np.array_equal(o_nn, o_nt), f"config {c} gelu={gelu}: NN output differs from NT"
                if gelu:
                    assert np.array_equal(p_nn, p_nt), f"config {c}: NN pre-activation differs from NT"
        forced_config(-1)
        ref = oracle.gemm_bf16(A, B, False, False)
        out = Tensor(dev, (M, N), "f32")
        kernels.gemm_bf16(q, tA, tB, out, False, False, _lib.EPI_NONE, None, ws)
        mag = np.abs(rng.bf16_to_f32(A).astype(np.float64)) @ np.abs(rng.bf16_to_f32(B).astype(np.float64))
        assert np.all(np.abs(out.numpy(q).astype(np.float64) - ref) <= 1e-2 * mag + 1e-30)
        out.free()
    finally:
        for t in (tA, tB, tBt, ws):
            t.free()


def gelu_bwd_pair(dev, q, tA, tB, tpre, M, N, fused):
    """(da, da_t) from the fused GEMM + GELU backward, or from the plain GEMM (f32) followed by
    the GELU backward op."""
    da, da_t = Tensor(dev, (M, N), "bf16"), Tensor(dev, (N, M), "bf16")
    for t in (da, da_t):
        t.buffer.fill_u32(q, 0x7FC07FC0)
    if fused:
        kernels.gemm_bf16_gelu_bwd(q, tA, tB, tpre, da, da_t)
    else:
        dh = Tensor(dev, (M, N), "f32")
        kernels.gemm_bf16(q, tA, tB, dh, False, True, _lib.EPI_NONE)
        kernels.gelu_bwd(q, dh, tpre, da, da_t)
        dh.free()
    res = (da.numpy(q), da_t.numpy(q))
    da.free()
    da_t.free()
    return res


@pytest.mark.parametrize("M,N,K", [(256, 512, 256), (300, 520, 256), (129, 258, 128)])
def test_every_bf16_config_gelu_bwd_fused(dev, q, forced_config, M, N, K):
    """The fused dL/dpre = (A B^T) * GELU'(pre) equals the GEMM followed by the GELU backward op,
    bit for bit, under every tile configuration (whole tiles with M % 8 == 0 take the LDS-staged
    epilogue with the transposed store, the others the per-element one)."""
    A = rng.f32_to_bf16(rng.uniform(81, M * K, -1, 1)).reshape(M, K)
    B = rng.f32_to_bf16(rng.uniform(82, N * K, -1, 1)).reshape(N, K)
    pre = (rng.normal(83, M * N) * 2.0).astype(np.float32).reshape(M, N)
    tA, tB, tpre = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16"), Tensor.from_numpy(dev, q, pre)
    try:
        forced_config(-1)
        base = gelu_bwd_pair(dev, q, tA, tB, tpre, M, N, fused=False)
        assert np.array_equal(base[1], base[0].T)
        for c in [-1] + list(range(N_BF16_CONFIGS)):
            forced_config(c)
            got = gelu_bwd_pair(dev, q, tA, tB, tpre, M, N, fused=True)
            assert np.array_equal(got[0], base[0]), f"config {c}: da differs"
            assert np.array_equal(got[1], base[1]), f"config {c}: da_t differs"
    finally:
        for t in (tA, tB, tpre):
            t.free()


@pytest.mark.parametrize("M,N,K", [(300, 520, 1024), (64, 1000, 512)])
def test_every_w8a8_config_bit_exact(dev, q, forced_config, M, N, K):
    r = np.random.default_rng(M * 7 + N + K)
    xq = r.integers(-127, 128, (M, K)).astype(np.int8)
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    xs = r.uniform(0.001, 0.01, M).astype(np.float32)
    ws = r.uniform(0.005, 0.02, N).astype(np.float32)
    ry, racc = oracle.gemm_w8a8(xq, xs, w, ws, out_dtype=BF16, relu=True, want_acc=True)
    ts = [Tensor.from_numpy(dev, q, a) for a in (xq, w, xs, ws)]
    txq, tw, txs, tws = ts
    try:
        for c in [-1] + list(range(N_W8A8_CONFIGS)):
            forced_config(c)
            wsb = kernels.gemm_w8a8_workspace_bytes(M, N, K)  # depends on the configuration
            ty, tacc = Tensor(dev, (M, N), "bf16"), Tensor(dev, (M, N), "i32")
            twk = Tensor(dev, (max(1, wsb),), "i8") if wsb else None
            tacc.buffer.fill_u32(q, 0xDEADBEEF)
            kernels.gemm_w8a8(q, txq, txs, tw, tws, ty, True, tacc, twk)
            assert np.array_equal(tacc.numpy(q), racc), f"config {c}: int32 accumulators differ"
            assert np.array_equal(ty.numpy(q), ry), f"config {c}: outputs differ"
            for t in (ty, tacc, twk):
                if t is not None:
                    t.free()
    finally:
        for t in ts:
            t.free()


@pytest.mark.parametrize("M,N,K", [(512, 512, 256), (300, 512, 256), (256, 768, 192)])
def test_streamed_f32_output_matches(dev, q, forced_config, M, N, K):
    """An f32 result bound as VDSL_BIND_OUTPUT leaves the LDS-staged epilogue through streaming
    stores: the same bits as a storage-buffer result under every configuration, in the NT form,
    the K-major NN form and the packed-weight form."""
    A = rng.f32_to_bf16(rng.uniform(91, M * K, -1, 1)).reshape(M, K)
    B = rng.f32_to_bf16(rng.uniform(92, N * K, -1, 1)).reshape(N, K)
    tA, tB = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16")
    tBkn = Tensor.from_numpy(dev, q, np.ascontiguousarray(B.T), "bf16")
    ws = Tensor(dev, (max(1, kernels.gemm_bf16_workspace_bytes(False, False, M, N, K)),), "i8")

    def run(src, tb, binding, packed=False):
        out = Tensor(dev, (M, N), "f32", binding)
        out.buffer.fill_u32(q, 0x7FC07FC0)
        if packed:
            kernels.gemm_bf16_packed(q, tA, src, out)
        else:
            kernels.gemm_bf16(q, tA, src, out, False, tb, _lib.EPI_NONE, None, None if tb else ws)
        r = out.numpy(q)
        out.free()
        return r

    try:
        for c in [-1] + list(range(N_BF16_CONFIGS)):
            forced_config(c)
            for src, tb in ((tB, True), (tBkn, False)):
                plain = run(src, tb, _lib.BIND_STORAGE_BUFFER)
                streamed = run(src, tb, _lib.BIND_OUTPUT)
                assert np.array_equal(plain, streamed), f"config {c} trans_b={tb}: streamed output differs"
        forced_config(-1)
        if K % 256 == 0 and N % 32 == 0:
            tBp = Tensor(dev, (N, K), "bf16")
            kernels.pack_bf16_weights(q, tB, tBp)
            plain = run(tBp, True, _lib.BIND_STORAGE_BUFFER, packed=True)
            assert np.array_equal(plain, run(tBp, True, _lib.BIND_OUTPUT, packed=True)), "packed: streamed output differs"
            assert np.array_equal(plain, run(tB, True, _lib.BIND_STORAGE_BUFFER)), "packed differs from NT"
            tBp.free()
    finally:
        for t in (tA, tB, tBkn, ws):
            t.free()


@pytest.mark.parametrize("M,N,K", [(512, 512, 256), (256, 768, 192), (1024, 512, 512), (300, 512, 256)])
def test_bf16_tn_k_major_a_matches_nt(dev, q, forced_config, M, N, K):
    """A stored [K][M] (trans_a = 1) and B stored [K][N]: the 256 x 256 direct-to-LDS configuration
    (15) reads both operands K-major when M and N are multiples of 256, with no transpose into the
    workspace; every output equals the NT product of the host-transposed operands under the same
    configuration, bit for bit.  M = 300 takes the transpose path."""
    A = rng.f32_to_bf16(rng.uniform(95, K * M, -1, 1)).reshape(K, M)   # stored [K][M]
    B = rng.f32_to_bf16(rng.uniform(96, K * N, -1, 1)).reshape(K, N)   # stored [K][N]
    tA, tB = Tensor.from_numpy(dev, q, A, "bf16"), Tensor.from_numpy(dev, q, B, "bf16")
    tAt = Tensor.from_numpy(dev, q, np.ascontiguousarray(A.T), "bf16")
    tBt = Tensor.from_numpy(dev, q, np.ascontiguousarray(B.T), "bf16")
    ws = Tensor(dev, (max(1, kernels.gemm_bf16_workspace_bytes(True, False, M, N, K)),), "i8")
    try:
        for c in (-1, 15, 14, 23):
            forced_config(c)
            ws.buffer.fill_u32(q, 0xA5A5A5A5)
            out = Tensor(dev, (M, N), "f32")
            kernels.gemm_bf16(q, tA, tB, out, True, False, _lib.EPI_NONE, None, ws)
            got = out.numpy(q)
            if c == 15 and M % 256 == 0 and N % 256 == 0:
                assert np.all(ws.numpy(q).view(np.uint32) == 0xA5A5A5A5), "K-major A: an operand was transposed"
            out.buffer.fill_u32(q, 0x7FC07FC0)
            kernels.gemm_bf16(q, tAt, tBt, out, False, True, _lib.EPI_NONE, None, None)
            assert np.array_equal(got, out.numpy(q)), f"config {c}: TN output differs from NT"
            out.free()
        forced_config(-1)
        ref = oracle.gemm_bf16(np.ascontiguousarray(A.T), B, False, False)
        out = Tensor(dev, (M, N), "f32")
        forced_config(15)
        kernels.gemm_bf16(q, tA, tB, out, True, False, _lib.EPI_NONE, None, ws)
        mag = np.abs(rng.bf16_to_f32(A).astype(np.float64)).T @ np.abs(rng.bf16_to_f32(B).astype(np.float64))
        assert np.all(np.abs(out.numpy(q).astype(np.float64) - ref) <= 1e-2 * mag + 1e-30)
        out.free()
    finally:
        for t in (tA, tB, tAt, tBt, ws):
            t.free()
