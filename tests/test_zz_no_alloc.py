"""The allocation-free int8 GEMM (vdsl_op_gemm_w8a8_packed_noalloc), called through the C ABI,
against vdsl_op_gemm_w8a8_packed with a caller-provided workspace: bit for bit (int32
accumulators and dequantised outputs).

Two calls in a row that both split K, so both run through the library's scratch array: config 5's
last layer (512 x 1024 x 8192) with its K split 8 ways (forced with vdsl_debug_w8a8_packed_plan:
the full 16 MiB), then a smaller input (256 x 512 x 4096, 4 MiB) that leaves most of the first
call's partials in place; then the first shape in its own plan (8 MiB), and an unsplit shape that
needs no scratch.  A launch plan that needs more scratch than the array holds is refused before
anything is enqueued."""
import ctypes as C

import numpy as np
import pytest

from vernondsl_amd import _lib, kernels
from vernondsl_amd._lib import call, lib
from vernondsl_amd.rhi import Tensor

pytestmark = pytest.mark.gpu
SCRATCH = 16 << 20  # VDSL_W8A8_NOALLOC_SCRATCH_BYTES
UNSUPPORTED = -5


def _case(dev, q, M, N, K, seed, relu, dt, plan=None):
    if plan is not None:
        call("vdsl_debug_w8a8_packed_plan", *plan)
        try:
            return _case(dev, q, M, N, K, seed, relu, dt)
        finally:
            call("vdsl_debug_w8a8_packed_plan", -1, 0)
    r = np.random.default_rng(seed)
    xq = r.integers(-127, 128, (M, K)).astype(np.int8)
    w = r.integers(-127, 128, (N, K)).astype(np.int8)
    xs = r.uniform(0.001, 0.01, M).astype(np.float32)
    ws = r.uniform(0.005, 0.02, N).astype(np.float32)
    txq, tw, txs, tws = (Tensor.from_numpy(dev, q, a) for a in (xq, w, xs, ws))
    twp = Tensor(dev, (N, K), "i8")
    kernels.pack_w8a8_weights(q, tw, twp)
    wsb = kernels.gemm_w8a8_packed_workspace_bytes(M, N, K)
    assert wsb <= SCRATCH
    work = Tensor(dev, (max(wsb, 4),), "i8")
    work.buffer.fill_u32(q, 0x7FC07FC0)
    outs = []
    for fn in ("vdsl_op_gemm_w8a8_packed", "vdsl_op_gemm_w8a8_packed_noalloc"):
        ty, tacc = Tensor(dev, (M, N), dt), Tensor(dev, (M, N), "i32")
        ty.buffer.fill_u32(q, 0x7FC07FC0)
        tacc.buffer.fill_u32(q, 0x7FC07FC0)
        args = [q.handle, M, N, K, txq.handle, txs.handle, twp.handle, tws.handle, ty.handle, ty.dtype,
                int(relu), tacc.handle]
        if fn == "vdsl_op_gemm_w8a8_packed":
            args.append(work.handle if wsb else None)
        print(f"no_alloc: {fn} M={M} N={N} K={K} scratch={wsb}", flush=True)
        call(fn, *args)
        outs.append((ty.numpy(q), tacc.numpy(q)))
        ty.free()
        tacc.free()
    for t in (txq, tw, txs, tws, twp, work):
        t.free()
    (y0, a0), (y1, a1) = outs
    assert np.array_equal(a1, a0), "int32 accumulators differ"
    assert np.array_equal(y1, y0), "dequantised outputs differ"
    return wsb


def test_noalloc_matches_workspace_entry_point(dev, q):
    assert _case(dev, q, 512, 1024, 8192, 1, relu=False, dt="bf16", plan=(3, 8)) == SCRATCH
    assert _case(dev, q, 256, 512, 4096, 2, relu=True, dt="f32") == 4 << 20
    assert _case(dev, q, 512, 1024, 8192, 3, relu=True, dt="bf16") == 8 << 20
    assert _case(dev, q, 2048, 2048, 512, 4, relu=True, dt="bf16") == 0


def test_noalloc_refuses_plans_beyond_the_scratch_array(dev, q):
    M, N, K = 8256, 256, 1024  # forced: 65 tiles of 128 x 256, K split 2: 65 * 2 * 128 KiB > 16 MiB
    call("vdsl_debug_w8a8_packed_plan", 0, 2)
    txq, twp, ty = Tensor(dev, (M, K), "i8"), Tensor(dev, (N, K), "i8"), Tensor(dev, (M, N), "bf16")
    txs, tws = Tensor(dev, (M,), "f32"), Tensor(dev, (N,), "f32")
    try:
        need = kernels.gemm_w8a8_packed_workspace_bytes(M, N, K)
        assert need > SCRATCH
        st = lib.vdsl_op_gemm_w8a8_packed_noalloc(q.handle, M, N, K, txq.handle, txs.handle, twp.handle,
                                                  tws.handle, ty.handle, _lib.BF16, 1, None)
        msg = lib.vdsl_last_error().decode()
        assert st == UNSUPPORTED and str(need) in msg and "16777216" in msg, (st, msg)
    finally:
        call("vdsl_debug_w8a8_packed_plan", -1, 0)
        for t in (txq, twp, ty, txs, tws):
            t.free()
