"""The RHI device on a real GPU: transfers at byte offsets, fills and copies, zero-byte buffers,
binding-kind enforcement, handle lifetime, allocation-failure injection, graph-capture misuse and
replay, and event timing.

Every error case here is rejected by the library's host-side checks before any HIP call is
made, so no case hands the device an invalid access.
"""
import ctypes as C

import numpy as np
import pytest

from vernondsl_amd import _lib, graph, kernels
from vernondsl_amd._lib import VdslError, call, lib
from vernondsl_amd.rhi import Buffer, Device, Event, Queue, Tensor

pytestmark = pytest.mark.gpu

INVALID_ARG, INVALID_HANDLE, OOM, CAPTURE, SHAPE = -1, -2, -3, -6, -7


def status(fn, *args):
    """Raw C-ABI status of one call, with the thread's last error message."""
    st = getattr(lib, fn)(*args)
    msg = lib.vdsl_last_error()
    return st, (msg.decode() if msg else "")


def read_bytes(q, buf, offset, n):
    out = np.empty(n, np.uint8)
    call("vdsl_buffer_read", q.handle, buf.handle, offset, out.ctypes.data_as(C.c_void_p), n)
    return out


def write_bytes(q, buf, offset, data):
    data = np.ascontiguousarray(data, np.uint8)
    call("vdsl_buffer_write", q.handle, buf.handle, offset, data.ctypes.data_as(C.c_void_p), data.nbytes)


def test_device_info_is_gfx950(dev):
    info = dev.info()
    assert info["arch"].split(":")[0] == "gfx950", info
    assert info["wavefront_size"] == 64
    assert info["compute_units"] >= 32
    assert info["lds_bytes_per_block"] >= 64 * 1024
    assert info["hbm_bytes"] >= 128 * 2**30


def test_transfers_fills_and_copies_at_offsets(dev, q):
    rng = np.random.default_rng(11)
    n = 4099                                  # odd size: no multiple-of-4 assumption anywhere
    a, b = Buffer(dev, n), Buffer(dev, n)
    try:
        host = rng.integers(0, 256, n, dtype=np.uint8)
        write_bytes(q, a, 0, host)
        assert np.array_equal(read_bytes(q, a, 0, n), host)
        patch = rng.integers(0, 256, 1001, dtype=np.uint8)
        write_bytes(q, a, 3, patch)           # unaligned offset and length
        host[3:1004] = patch
        assert np.array_equal(read_bytes(q, a, 0, n), host)
        assert np.array_equal(read_bytes(q, a, 1001, 7), host[1001:1008])

        a.fill_u32(q, 0xDEADBEEF, offset=8, nbytes=64)
        host[8:72] = np.frombuffer(np.full(16, 0xDEADBEEF, np.uint32).tobytes(), np.uint8)
        assert np.array_equal(read_bytes(q, a, 0, n), host)

        b.fill_u32(q, 0, offset=0, nbytes=4096)
        write_bytes(q, b, 4096, np.zeros(3, np.uint8))
        call("vdsl_buffer_copy", q.handle, b.handle, 5, a.handle, 17, 2000)
        ref = np.zeros(n, np.uint8)
        ref[5:2005] = host[17:2017]
        assert np.array_equal(read_bytes(q, b, 0, n), ref)

        # zero-byte transfers at the end of the buffer are no-ops, not range errors
        for fn, args in (("vdsl_buffer_write", (q.handle, a.handle, n, None, 0)),
                         ("vdsl_buffer_read", (q.handle, a.handle, n, None, 0)),
                         ("vdsl_buffer_copy", (q.handle, b.handle, n, a.handle, n, 0)),
                         ("vdsl_buffer_fill_u32", (q.handle, a.handle, 0, 0, 7))):
            assert status(fn, *args)[0] == 0, fn
        assert np.array_equal(read_bytes(q, a, 0, n), host)
    finally:
        a.free()
        b.free()


def test_range_and_argument_errors(dev, q):
    a, b = Buffer(dev, 4096), Buffer(dev, 64)
    tmp = np.zeros(16, np.uint8)
    p = tmp.ctypes.data_as(C.c_void_p)
    try:
        cases = [
            ("vdsl_buffer_write", (q.handle, a.handle, 4090, p, 10), SHAPE, "exceeds"),
            ("vdsl_buffer_write", (q.handle, a.handle, 4097, p, 0), SHAPE, "exceeds"),
            ("vdsl_buffer_read", (q.handle, a.handle, 1, p, 2**64 - 1), SHAPE, "exceeds"),  # no wrap-around
            ("vdsl_buffer_write", (q.handle, a.handle, 0, None, 4), INVALID_ARG, "src is null"),
            ("vdsl_buffer_read", (q.handle, a.handle, 0, None, 4), INVALID_ARG, "dst is null"),
            ("vdsl_buffer_fill_u32", (q.handle, a.handle, 2, 8, 0), INVALID_ARG, "multiples of 4"),
            ("vdsl_buffer_fill_u32", (q.handle, a.handle, 0, 6, 0), INVALID_ARG, "multiples of 4"),
            ("vdsl_buffer_fill_u32", (q.handle, a.handle, 4092, 8, 0), SHAPE, "exceeds"),
            ("vdsl_buffer_copy", (q.handle, b.handle, 0, a.handle, 0, 65), SHAPE, "exceeds"),
            ("vdsl_buffer_copy", (q.handle, a.handle, 0, b.handle, 60, 8), SHAPE, "exceeds"),
        ]
        for fn, args, want, text in cases:
            st, msg = status(fn, *args)
            assert st == want and text in msg, (fn, args[2:], st, msg)
        # a rejected call leaves the buffer untouched
        a.fill_u32(q, 0x01020304)
        status("vdsl_buffer_fill_u32", q.handle, a.handle, 4092, 8, 0)
        assert np.all(np.frombuffer(read_bytes(q, a, 0, 4096).tobytes(), np.uint32) == 0x01020304)
    finally:
        a.free()
        b.free()


def test_zero_byte_buffer(dev, q):
    z = Buffer(dev, 0)
    try:
        size = C.c_size_t(99)
        call("vdsl_buffer_size", z.handle, C.byref(size))
        assert size.value == 0
        assert z.address() == 0
        assert status("vdsl_buffer_write", q.handle, z.handle, 0, None, 0)[0] == 0
        assert status("vdsl_buffer_read", q.handle, z.handle, 1, None, 0)[0] == SHAPE
        assert status("vdsl_buffer_fill_u32", q.handle, z.handle, 0, 0, 0)[0] == 0
        # an op with an empty output grid accepts the empty buffer
        p = kernels.escape_time_params(ni=0, nj=5)
        call("vdsl_op_escape_time", q.handle, C.byref(p), z.handle)
        q.sync()
    finally:
        z.free()


def test_uniform_constant_is_read_only_on_device(dev, q):
    """Host writes initialise a uniform_constant buffer; device-side writes into it are rejected."""
    uc = Buffer(dev, 256, binding="uniform_constant")
    sb = Buffer(dev, 256)
    try:
        kind = C.c_int(-1)
        call("vdsl_buffer_binding", uc.handle, C.byref(kind))
        assert kind.value == _lib.BIND_UNIFORM_CONSTANT
        data = np.arange(256, dtype=np.uint8)
        write_bytes(q, uc, 0, data)
        assert np.array_equal(read_bytes(q, uc, 0, 256), data)
        st, msg = status("vdsl_buffer_fill_u32", q.handle, uc.handle, 0, 256, 0)
        assert st == INVALID_ARG and "uniform_constant" in msg
        st, msg = status("vdsl_buffer_copy", q.handle, uc.handle, 0, sb.handle, 0, 16)
        assert st == INVALID_ARG and "uniform_constant" in msg
        call("vdsl_buffer_copy", q.handle, sb.handle, 0, uc.handle, 0, 256)  # reading it is fine
        assert np.array_equal(read_bytes(q, sb, 0, 256), data)
        p = kernels.escape_time_params(ni=8, nj=8)
        st, msg = status("vdsl_op_escape_time", q.handle, C.byref(p), uc.handle)
        assert st == INVALID_ARG and "uniform_constant" in msg
        assert np.array_equal(read_bytes(q, uc, 0, 256), data)
    finally:
        uc.free()
        sb.free()


def test_op_output_too_small_is_a_shape_error(dev, q):
    out = Buffer(dev, 8 * 8 * 4 - 4)
    try:
        p = kernels.escape_time_params(ni=8, nj=8)
        st, msg = status("vdsl_op_escape_time", q.handle, C.byref(p), out.handle)
        assert st == SHAPE and "holds 252 bytes, op needs 256" in msg
    finally:
        out.free()


def test_overflowing_extents_are_shape_errors_before_any_launch(dev, q):
    """Extents whose byte size wraps size_t (rows * cols * element size >= 2^64) must be refused
    by the host-side size check; a wrapped size would pass a small buffer and the kernel would
    read past it.  Every call below returns before it enqueues anything."""
    b = Buffer(dev, 4096)
    try:
        h = b.handle
        big = 1 << 62                      # x 4 bytes = 2^64
        cases = [
            ("vdsl_op_row_reduce_softmax", q.handle, 1, big, _lib.F32, h, None, None, None),
            ("vdsl_op_col_reduce", q.handle, big, 1, _lib.F32, h, None, None),
            ("vdsl_op_transpose", q.handle, big, 2, _lib.BF16, h, b.handle),
            ("vdsl_op_cast", q.handle, big, _lib.F32, h, _lib.BF16, h),
            ("vdsl_op_gelu_fwd", q.handle, big, _lib.F32, h, _lib.F32, h),
            ("vdsl_op_gelu_bwd", q.handle, 1 << 40, 1 << 40, h, h, h, None),
            ("vdsl_op_mse_fwd_bwd", q.handle, 1 << 40, 1 << 40, h, h, h, None, None, h),
            ("vdsl_op_quantize_rows_i8", q.handle, 1, big, _lib.F32, h, h, h),
        ]
        for fn, *args in cases:
            st, msg = status(fn, *args)
            assert st == SHAPE and "overflows" in msg, (fn, st, msg)
        # the map chain sizes its output from rows * cols
        prog = (_lib.MapInstr * 1)()
        prog[0].op, prog[0].dst = _lib.MAP_OPS["const"], 0
        st, msg = status("vdsl_op_map_chain", q.handle, 1 << 40, 1 << 40, prog, 1, None, 0, 0, h)
        assert st == SHAPE and "overflows" in msg, msg
        st, msg = status("vdsl_op_map_chain", q.handle, -1, 4, prog, 1, None, 0, 0, h)
        assert st == INVALID_ARG
    finally:
        b.free()


def test_stale_and_double_freed_handles(dev, q):
    b = Buffer(dev, 64)
    h = C.c_void_p(b.handle.value)
    b.free()
    st, msg = status("vdsl_buffer_free", h)
    assert st == INVALID_HANDLE and "invalid buffer handle" in msg
    st, _ = status("vdsl_buffer_write", q.handle, h, 0, None, 0)
    assert st == INVALID_HANDLE
    # a buffer handle is not a queue handle, and vice versa
    b2 = Buffer(dev, 64)
    try:
        assert status("vdsl_queue_sync", b2.handle)[0] == INVALID_HANDLE
        assert status("vdsl_buffer_free", q.handle)[0] == INVALID_HANDLE
    finally:
        b2.free()


def test_device_close_requires_release_and_rejects_foreign_handles(dev, q):
    d2 = Device(0)                       # a second handle on the same GPU: a distinct device
    q2 = Queue(d2)
    b2 = Buffer(d2, 64)
    ev = Event(d2)
    st, msg = status("vdsl_device_close", d2.handle)
    assert st == INVALID_ARG and "still owns 3" in msg
    # objects of one device handle are not accepted with another's queue
    st, msg = status("vdsl_buffer_fill_u32", q.handle, b2.handle, 0, 64, 0)
    assert st == INVALID_ARG and "another device" in msg
    b1 = Buffer(dev, 64)
    try:
        st, msg = status("vdsl_buffer_copy", q2.handle, b2.handle, 0, b1.handle, 0, 64)
        assert st == INVALID_ARG and "another device" in msg
        with q.capture() as rec:
            b1.fill_u32(q, 5)
        st, msg = status("vdsl_graph_launch", rec.graph.handle, q2.handle)
        assert st == INVALID_ARG and "different devices" in msg
        rec.graph.destroy()
    finally:
        b1.free()
    b2.free()
    ev.destroy()
    q2.destroy()
    h = C.c_void_p(d2.handle.value)
    d2.close()
    assert status("vdsl_device_close", h)[0] == INVALID_HANDLE


def test_allocation_failure_injection_leaves_nothing_behind(dev):
    """With injection at n, the n+1-th allocation fails with VDSL_ERR_OUT_OF_MEMORY; an executable
    graph whose allocation fails part-way releases what it had allocated, so its device closes."""
    d2 = Device(0)
    try:
        call("vdsl_debug_fail_alloc_after", 2)
        b1, b2 = Buffer(d2, 16), Buffer(d2, 16)
        with pytest.raises(VdslError) as ei:
            Buffer(d2, 16)
        assert ei.value.status == OOM and "injected" in ei.value.message
        call("vdsl_debug_fail_alloc_after", -1)
        b1.free()
        b2.free()
        g, _ = graph.mlp_train_graph(64, 64, 64, 64)
        exe = g.compile(d2)
        n_alloc = sum(t is not None for t in exe.t.values()) + (exe.workspace is not None)  # elided values allocate nothing
        exe.free()
        for k in sorted({0, 1, n_alloc // 2, n_alloc - 1}):  # first, second, a middle and the last
            call("vdsl_debug_fail_alloc_after", k)
            try:
                with pytest.raises(VdslError) as ei:
                    g.compile(d2)
            finally:
                call("vdsl_debug_fail_alloc_after", -1)
            assert ei.value.status == OOM
            st, msg = status("vdsl_device_close", d2.handle)
            assert st == 0, f"allocation failure after {k} allocations: {msg}"
            d2.handle = None
            d2 = Device(0)
    finally:
        call("vdsl_debug_fail_alloc_after", -1)
        d2.close()
    b = Buffer(dev, 16)  # injection is off again
    b.free()


def test_real_allocation_failure_does_not_fail_the_next_launch(dev, q):
    """A hipMalloc that fails leaves HIP's per-thread last error set; the library clears it, so the
    next op's launch check does not report that failure against its own kernel."""
    with pytest.raises(VdslError) as ei:
        Buffer(dev, 1 << 62)
    assert ei.value.status == OOM
    t = Tensor.from_numpy(dev, q, np.arange(64, dtype=np.float32))
    t.buffer.fill_u32(q, 0x3F800000)  # a kernel launch right after the failure
    assert np.all(t.numpy(q) == 1.0)
    t.free()


def test_capture_misuse_is_rejected_and_capture_survives(dev):
    q2 = Queue(dev)
    buf = Buffer(dev, 1024)
    out = np.zeros(16, np.uint8)
    p = out.ctypes.data_as(C.c_void_p)
    try:
        st, msg = status("vdsl_graph_end", q2.handle, None)
        assert st == CAPTURE and "without graph_begin" in msg
        with q2.capture() as rec0:
            buf.fill_u32(q2, 1)
        g0 = rec0.graph

        q2.begin_graph()
        try:
            buf.fill_u32(q2, 0xABCD1234, offset=0, nbytes=512)
            for fn, args, text in (
                ("vdsl_graph_begin", (q2.handle,), "already capturing"),
                ("vdsl_buffer_write", (q2.handle, buf.handle, 0, p, 16), "host transfers"),
                ("vdsl_buffer_read", (q2.handle, buf.handle, 0, p, 16), "host transfers"),
                ("vdsl_queue_sync", (q2.handle,), "capturing queue"),
                ("vdsl_queue_destroy", (q2.handle,), "capturing"),
                ("vdsl_graph_launch", (g0.handle, q2.handle), "capturing queue"),
            ):
                st, msg = status(fn, *args)
                assert st == CAPTURE and text in msg, (fn, st, msg)
            buf.fill_u32(q2, 0x55667788, offset=512, nbytes=512)
        finally:
            g1 = q2.end_graph()
        buf.fill_u32(q2, 0)
        q2.sync()
        g1.launch(q2)
        q2.sync()
        words = np.frombuffer(read_bytes(q2, buf, 0, 1024).tobytes(), np.uint32)
        assert np.all(words[:128] == 0xABCD1234) and np.all(words[128:] == 0x55667788)
        g0.launch(q2)
        q2.sync()
        assert np.all(np.frombuffer(read_bytes(q2, buf, 0, 1024).tobytes(), np.uint32) == 1)
        h1 = C.c_void_p(g1.handle.value)
        g0.destroy()
        g1.destroy()
        st, msg = status("vdsl_graph_launch", h1, q2.handle)
        assert st == INVALID_HANDLE and "invalid graph handle" in msg
    finally:
        buf.free()
        q2.destroy()


def test_graph_of_fill_and_copy_replays(dev, q):
    """A recorded fill (a kernel, not a memset node) and device copy, replayed with eager work and
    synchronisation between replays; every replay checked against the expected bytes."""
    a, b = Buffer(dev, 8192), Buffer(dev, 8192)
    try:
        with q.capture() as rec:
            a.fill_u32(q, 0xA5A5A5A5, offset=1024, nbytes=2048)
            call("vdsl_buffer_copy", q.handle, b.handle, 3, a.handle, 1000, 3000)
        g = rec.graph
        for rep in range(4):
            a.fill_u32(q, rep)               # eager poison between replays
            b.fill_u32(q, 0xFFFFFFFF)
            q.sync()
            g.launch(q)
            q.sync()
            ah = np.frombuffer(read_bytes(q, a, 0, 8192).tobytes(), np.uint32)
            want_a = np.full(2048, rep, np.uint32)
            want_a[256:768] = 0xA5A5A5A5
            assert np.array_equal(ah, want_a), rep
            bb = read_bytes(q, b, 0, 8192)
            ab = read_bytes(q, a, 0, 8192)
            assert np.array_equal(bb[3:3003], ab[1000:4000]), rep
            assert np.all(bb[:3] == 0xFF) and np.all(bb[3003:] == 0xFF), rep
        g.destroy()
    finally:
        a.free()
        b.free()


def test_events_time_device_work(dev, q):
    """Elapsed time of a 256 MiB fill is positive, finite and no shorter than writing at 30 TB/s
    would take (beyond both HBM and the last-level cache)."""
    big = Tensor(dev, (64 * 2**20,), "f32")
    e0, e1 = Event(dev), Event(dev)
    try:
        big.buffer.fill_u32(q, 0)
        q.sync()
        e0.record(q)
        big.buffer.fill_u32(q, 0x3F800000)
        e1.record(q)
        ms = e0.elapsed_ms(e1)
        assert 256 * 2**20 / 30.0e12 * 1e3 <= ms < 1000.0, ms
        got = big.numpy(q)
        assert got[0] == 1.0 and got[-1] == 1.0 and got[12345678] == 1.0
        st, _ = status("vdsl_event_elapsed_ms", e0.handle, e1.handle, None)
        assert st == INVALID_ARG
    finally:
        e0.destroy()
        e1.destroy()
        big.free()
