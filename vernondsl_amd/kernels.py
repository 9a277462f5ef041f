"""Op-class calls on the HIP device, one function per `vdsl_op_*` entry point of include/vdsl.h.

Each function checks operand shapes and dtypes on the host before anything is enqueued (the C
ABI checks buffer sizes again), then enqueues the op on `q` and returns without waiting.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from ._lib import call
from .mapchain import Program
from .rhi import Queue, Tensor, dtype_code


def _h(t):
    return None if t is None else t.handle


def _expect(t: Tensor, shape, dtype, name):
    if t is None:
        return
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {t.shape}, expected {tuple(shape)}")
    if t.dtype != dtype_code(dtype):
        raise ValueError(f"{name}: dtype {t.dtype}, expected {dtype}")


# ---- op class 1: escape-time iterative map (fractal.py:16-25) -------------------------------
def escape_time_params(**kw) -> _lib.EscapeTimeParams:
    p = _lib.EscapeTimeParams()
    defaults = dict(family=_lib.ESC_MANDELBROT, escape_test=_lib.ESC_MAG2_GT, rounding=_lib.ESC_ROUND_FMA,
                    out_kind=_lib.ESC_OUT_I32_COUNT, max_iter=256, bound=4.0,
                    re_den=1.0, re_off=0.0, re_scale=1.0, re_post=0.0,
                    im_den=1.0, im_off=0.0, im_scale=1.0, im_post=0.0,
                    c_re=0.0, c_im=0.0, out_base=0.0, out_scale=1.0)
    defaults.update(kw)
    for k, v in defaults.items():
        setattr(p, k, v)
    return p


def escape_time(q: Queue, p: _lib.EscapeTimeParams, out: Tensor):
    dt = "i32" if p.out_kind == _lib.ESC_OUT_I32_COUNT else "f32"
    _expect(out, (p.ni, p.nj), dt, "out")
    call("vdsl_op_escape_time", q.handle, C.byref(p), out.handle)


# ---- op class 2: fused map chain --------------------------------------------------------------
def map_chain(q: Queue, prog: Program, inputs, out: Tensor):
    """inputs[k] is the Tensor for Input(k); its broadcast comes from the program."""
    rows, cols = out.shape
    if len(inputs) != prog.n_inputs:
        raise ValueError(f"program reads {prog.n_inputs} inputs, {len(inputs)} given")
    arr = (_lib.MapInput * max(1, len(inputs)))()
    for k, t in enumerate(inputs):
        bc = prog.bcast[k]
        want = {_lib.BCAST_FULL: (rows, cols), _lib.BCAST_ROW: (cols,), _lib.BCAST_COL: (rows,), _lib.BCAST_SCALAR: (1,)}[bc]
        _expect(t, want, "f32", f"input{k}")
        arr[k].buf, arr[k].bcast, arr[k].dtype = t.handle.value, bc, _lib.F32
    _expect(out, (rows, cols), "f32", "out")
    code = prog.instr_array()
    call("vdsl_op_map_chain", q.handle, rows, cols, code, len(prog.code), arr, len(inputs), prog.out_reg, out.handle)


def map_chain_v(q: Queue, prog: Program, inputs, out: Tensor):
    """A chain over vector operands (vdsl_op_map_chain_v).  inputs[k] is the Tensor of input k:
    [rows][cols][w] for a full input of width w > 1 ([rows][cols] when w = 1), [cols][w] / [rows][w]
    / [w] when broadcast.  out: [rows][cols][len(prog.out_regs)] ([rows][cols] for one component)."""
    rows, cols = out.shape[:2]
    ow = len(prog.out_regs)
    _expect(out, (rows, cols, ow) if ow > 1 else (rows, cols), "f32", "out")
    if len(inputs) != prog.n_inputs:
        raise ValueError(f"program reads {prog.n_inputs} inputs, {len(inputs)} given")
    arr = (_lib.MapVInput * max(1, len(inputs)))()
    for k, t in enumerate(inputs):
        bc, w, d = prog.bcast[k], prog.widths[k], prog.dims.get(k, 0)
        want = {_lib.BCAST_FULL: (rows, cols), _lib.BCAST_ROW: (cols,), _lib.BCAST_COL: (rows,), _lib.BCAST_SCALAR: ()}[bc]
        if d:
            want = want + (d, d)
        elif w > 1 or bc == _lib.BCAST_SCALAR:
            want = want + (w,)
        _expect(t, want, "f32", f"input{k}")
        arr[k].buf, arr[k].bcast, arr[k].dtype, arr[k].width, arr[k].mat_dim = t.handle.value, bc, _lib.F32, w, d
    regs = (C.c_int32 * 4)(*(prog.out_regs + [0] * (4 - ow)))
    call("vdsl_op_map_chain_v", q.handle, rows, cols, prog.instr_array(), len(prog.code), arr, len(inputs), regs, ow,
         out.handle)


# ---- vertex transform (color.mlir:10-39) ----------------------------------------------------------
def vec_transform(q: Queue, pos: Tensor, mats: Tensor, out: Tensor, varying: Tensor | None = None):
    """out [n][4] = M_k ... M_1 vec4(pos, 1) for pos [n][3] (or M... pos for [n][4]); mats [k][4][4]
    row-major (model, view, proj order), k = 1..3; varying (optional) [n][3|4] = pos."""
    n, w = pos.shape
    nm = mats.shape[0]
    _expect(pos, (n, w), "f32", "pos")
    _expect(mats, (nm, 4, 4), "f32", "mats")
    _expect(out, (n, 4), "f32", "out")
    _expect(varying, (n, w), "f32", "varying")
    call("vdsl_op_vec_transform", q.handle, n, w, pos.handle, nm, mats.handle, out.handle, _h(varying))


def mat_transform(q: Queue, pos: Tensor, mats: Tensor, out: Tensor, varying: Tensor | None = None):
    """out [n][d] = M_k ... M_1 vec(pos, 1) for pos [n][d-1] (or M... pos for [n][d]); mats [k][d][d]
    row-major, d = 2, 3 or 4, k = 1..3; varying (optional) [n][d-1|d] = pos."""
    n, w = pos.shape
    nm, d = mats.shape[0], mats.shape[1]
    _expect(pos, (n, w), "f32", "pos")
    _expect(mats, (nm, d, d), "f32", "mats")
    _expect(out, (n, d), "f32", "out")
    _expect(varying, (n, w), "f32", "varying")
    call("vdsl_op_mat_transform", q.handle, n, d, w, pos.handle, nm, mats.handle, out.handle, _h(varying))


# ---- op class 3: row reductions + softmax ------------------------------------------------------
def row_reduce_softmax(q: Queue, x: Tensor, row_sum=None, row_max=None, softmax=None):
    rows, cols = x.shape
    _expect(row_sum, (rows,), "f32", "row_sum")
    _expect(row_max, (rows,), "f32", "row_max")
    _expect(softmax, (rows, cols), x.dtype, "softmax")
    call("vdsl_op_row_reduce_softmax", q.handle, rows, cols, x.dtype, x.handle, _h(row_sum), _h(row_max), _h(softmax))


def col_reduce(q: Queue, x: Tensor, col_sum=None, col_max=None):
    rows, cols = x.shape
    _expect(col_sum, (cols,), "f32", "col_sum")
    _expect(col_max, (cols,), "f32", "col_max")
    call("vdsl_op_col_reduce", q.handle, rows, cols, x.dtype, x.handle, _h(col_sum), _h(col_max))


# ---- op class 4: bf16 GEMM + layout + autodiff blocks ------------------------------------------
def gemm_bf16_workspace_bytes(trans_a, trans_b, M, N, K) -> int:
    n = C.c_size_t()
    call("vdsl_gemm_bf16_workspace_bytes", int(trans_a), int(trans_b), M, N, K, C.byref(n))
    return n.value


def gemm_bf16(q: Queue, A: Tensor, B: Tensor, Cout: Tensor, trans_a=False, trans_b=False,
              epilogue=_lib.EPI_NONE, pre_act=None, workspace=None):
    if trans_a:
        K, M = A.shape
    else:
        M, K = A.shape
    if trans_b:
        N, K2 = B.shape
    else:
        K2, N = B.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    _expect(A, A.shape, "bf16", "A")
    _expect(B, B.shape, "bf16", "B")
    if Cout.shape != (M, N):
        raise ValueError(f"C: shape {Cout.shape}, expected {(M, N)}")
    _expect(pre_act, (M, N), "f32", "pre_act")
    call("vdsl_op_gemm_bf16", q.handle, int(trans_a), int(trans_b), M, N, K, A.handle, B.handle, Cout.handle,
         Cout.dtype, int(epilogue), _h(pre_act), _h(workspace))


def gemm_bf16_mse_packed(q: Queue, A: Tensor, Bp: Tensor, T: Tensor, Y, loss: Tensor, dy: Tensor, dy_t=None,
                         partials: Tensor = None):
    """Y = A Bp^T fused with loss = mean((Y - T)^2), dy = bf16(2 (Y - T) / n), dy_t = dy^T
    (vdsl_op_gemm_bf16_mse_packed); Y (f32) and dy_t may be None.  Bp: packed [N][K] weights."""
    M, K = A.shape
    N = Bp.shape[0]
    _expect(A, (M, K), "bf16", "A")
    _expect(Bp, (N, K), "bf16", "Bp")
    _expect(T, (M, N), "f32", "T")
    _expect(Y, (M, N), "f32", "Y")
    _expect(loss, (1,), "f32", "loss")
    _expect(dy, (M, N), "bf16", "dy")
    _expect(dy_t, (N, M), "bf16", "dy_t")
    call("vdsl_op_gemm_bf16_mse_packed", q.handle, M, N, K, A.handle, Bp.handle, T.handle, _h(Y), loss.handle, dy.handle,
         _h(dy_t), partials.handle)


def pack_bf16_weights(q: Queue, w: Tensor, wp: Tensor):
    """Writes w (bf16 [N][K]) into wp in the MFMA fragment order gemm_bf16_packed reads."""
    N, K = w.shape
    _expect(w, (N, K), "bf16", "w")
    _expect(wp, (N, K), "bf16", "wp")
    call("vdsl_op_pack_bf16_weights", q.handle, N, K, w.handle, wp.handle)


def gemm_bf16_packed(q: Queue, A: Tensor, Bp: Tensor, Cout: Tensor, epilogue=_lib.EPI_NONE, pre_act=None):
    """gemm_bf16(A, B, trans_b=True) with B packed by pack_bf16_weights (Bp keeps the logical
    shape [N][K]); bit-identical results."""
    M, K = A.shape
    N, K2 = Bp.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    _expect(A, (M, K), "bf16", "A")
    _expect(Bp, (N, K), "bf16", "Bp")
    if Cout.shape != (M, N):
        raise ValueError(f"C: shape {Cout.shape}, expected {(M, N)}")
    _expect(pre_act, (M, N), "f32", "pre_act")
    call("vdsl_op_gemm_bf16_packed", q.handle, M, N, K, A.handle, Bp.handle, Cout.handle, Cout.dtype, int(epilogue),
         _h(pre_act))


def transpose(q: Queue, src: Tensor, dst: Tensor):
    rows, cols = src.shape
    _expect(dst, (cols, rows), src.dtype, "dst")
    call("vdsl_op_transpose", q.handle, rows, cols, src.dtype, src.handle, dst.handle)


def cast(q: Queue, src: Tensor, dst: Tensor):
    if src.numel != dst.numel:
        raise ValueError("cast: element counts differ")
    call("vdsl_op_cast", q.handle, src.numel, src.dtype, src.handle, dst.dtype, dst.handle)


def gelu_fwd(q: Queue, x: Tensor, y: Tensor):
    """y = GELU(x) elementwise (exact-erf form); x, y f32 or bf16 of one element count."""
    if x.numel != y.numel:
        raise ValueError(f"gelu_fwd: x has {x.numel} elements, y {y.numel}")
    call("vdsl_op_gelu_fwd", q.handle, x.numel, x.dtype, x.handle, y.dtype, y.handle)


def gelu_bwd(q: Queue, dh: Tensor, pre: Tensor, da: Tensor, da_t=None, act: str = "gelu"):
    """da = bf16(dh * act'(pre)) (+ its transpose da_t); act "gelu" or "relu"."""
    rows, cols = dh.shape
    _expect(dh, (rows, cols), "f32", "dh")
    _expect(pre, (rows, cols), "f32", "pre")
    _expect(da, (rows, cols), "bf16", "da")
    _expect(da_t, (cols, rows), "bf16", "da_t")
    fn = {"gelu": "vdsl_op_gelu_bwd", "relu": "vdsl_op_relu_bwd"}[act]
    call(fn, q.handle, rows, cols, dh.handle, pre.handle, da.handle, _h(da_t))


def add(q: Queue, a: Tensor, b: Tensor, out: Tensor):
    """out = a + b elementwise (f32 or bf16 each; one f32 addition rounded to out's dtype)."""
    if not (a.numel == b.numel == out.numel):
        raise ValueError(f"add: {a.numel}, {b.numel} and {out.numel} elements")
    call("vdsl_op_add", q.handle, out.numel, a.dtype, a.handle, b.dtype, b.handle, out.dtype, out.handle)


def gemm_bf16_gelu_bwd(q: Queue, A: Tensor, B: Tensor, pre: Tensor, da: Tensor, da_t=None, packed=False):
    """da = (A B^T) * GELU'(pre) as bf16 (and da_t = da^T): the GEMM forming dL/dy fused with the
    GELU backward (A bf16 [M][K], B bf16 [N][K] - packed by pack_bf16_weights if `packed` -, pre
    f32 [M][N])."""
    M, K = A.shape
    N, K2 = B.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    _expect(A, (M, K), "bf16", "A")
    _expect(B, (N, K), "bf16", "B")
    _expect(pre, (M, N), "f32", "pre")
    _expect(da, (M, N), "bf16", "da")
    _expect(da_t, (N, M), "bf16", "da_t")
    call("vdsl_op_gemm_bf16_gelu_bwd_packed" if packed else "vdsl_op_gemm_bf16_gelu_bwd", q.handle, M, N, K, A.handle,
         B.handle, pre.handle, da.handle, _h(da_t))


def gemm_bf16_mul_packed(q: Queue, A: Tensor, Bp: Tensor, g: Tensor, c: Tensor, c_t=None):
    """c = bf16((A Bp^T) * g) (and c_t = c^T): the GEMM forming dL/dh fused with the multiply by a
    stored local derivative g (f32 [M][N], e.g. GELU'(pre) from a forward GEMM with the
    EPI_GELU_DERIV epilogue).  Bp: packed [N][K] weights."""
    M, K = A.shape
    N, K2 = Bp.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    _expect(A, (M, K), "bf16", "A")
    _expect(Bp, (N, K), "bf16", "Bp")
    _expect(g, (M, N), "f32", "g")
    _expect(c, (M, N), "bf16", "c")
    _expect(c_t, (N, M), "bf16", "c_t")
    call("vdsl_op_gemm_bf16_mul_packed", q.handle, M, N, K, A.handle, Bp.handle, g.handle, c.handle, _h(c_t))


def pixel_program(q: Queue, prog, inputs, out: Tensor | None, grid=None):
    """Runs a compiled per-pixel program (vernondsl_amd.pixprog.PixelProgram) over out's [ni][nj]
    grid: out f32 [ni][nj] or [ni][nj][out_width] (the program stores registers) or i32 [ni][nj]
    (it stores its loop count); inputs: f32 fields [ni][nj] or [ni][nj][in_widths[k]], read at
    each pixel, or of their own extents [in_rows[k]][in_cols[k]] (gathered, or scatter-added
    into).  A program that stores nothing (pixprog.OUT_NONE) takes out None and grid (ni, nj)."""
    if prog.out_kind == 3:
        if out is not None or grid is None or len(grid) != 2:
            raise ValueError("a program that stores nothing takes out=None and grid=(ni, nj)")
        ni, nj = (int(v) for v in grid)
    else:
        if out is None or len(out.shape) not in (2, 3):
            raise ValueError("out must be a 2-D field of scalars or vectors")
        ni, nj = out.shape[:2]
        if grid is not None and tuple(grid) != (ni, nj):
            raise ValueError(f"grid {tuple(grid)} is not out's [{ni}][{nj}]")

    def field_shape(w, r=ni, c=nj):
        return (r, c) if w == 1 else (r, c, w)

    if prog.out_kind in (1, 2):  # the loop count, or an int32 field
        _expect(out, (ni, nj), "i32", "out")
    elif prog.out_kind != 3:
        _expect(out, field_shape(prog.out_width), "f32", "out")
    for k, t in enumerate(inputs):
        r, c = (prog.in_rows[k], prog.in_cols[k]) if prog.in_rows[k] else (ni, nj)  # an input of its own extents
        _expect(t, field_shape(prog.in_widths[k], r, c), "i32" if prog.in_dtypes[k] == _lib.I32 else "f32", f"input{k}")
    hs = (C.c_void_p * max(1, len(inputs)))(*[t.handle for t in inputs])
    call("vdsl_op_pixel_program", q.handle, ni, nj, C.byref(prog), hs, len(inputs), _h(out))


def mse_partials_count(rows, cols) -> int:
    return int(_lib.lib.vdsl_mse_partials_count(rows, cols))


def mse_fwd_bwd(q: Queue, y: Tensor, t: Tensor, loss: Tensor, dy: Tensor, dy_t, partials: Tensor):
    rows, cols = y.shape
    _expect(t, (rows, cols), "f32", "t")
    _expect(loss, (1,), "f32", "loss")
    _expect(dy, (rows, cols), "bf16", "dy")
    _expect(dy_t, (cols, rows), "bf16", "dy_t")
    call("vdsl_op_mse_fwd_bwd", q.handle, rows, cols, y.handle, t.handle, loss.handle, dy.handle, _h(dy_t),
         partials.handle)


# ---- op class 5: int8 W8A8 -----------------------------------------------------------------------
def quantize_rows_i8(q: Queue, x: Tensor, qx: Tensor, scale: Tensor):
    rows, cols = x.shape
    _expect(qx, (rows, cols), "i8", "qx")
    _expect(scale, (rows,), "f32", "scale")
    call("vdsl_op_quantize_rows_i8", q.handle, rows, cols, x.dtype, x.handle, qx.handle, scale.handle)


def gemm_w8a8_workspace_bytes(M, N, K) -> int:
    n = C.c_size_t()
    call("vdsl_gemm_w8a8_workspace_bytes", M, N, K, C.byref(n))
    return n.value


def gemm_w8a8(q: Queue, xq: Tensor, x_scale: Tensor, w: Tensor, w_scale: Tensor, y: Tensor, relu=False,
              acc_out=None, workspace=None):
    M, K = xq.shape
    N, K2 = w.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    _expect(xq, (M, K), "i8", "xq")
    _expect(w, (N, K), "i8", "w")
    _expect(x_scale, (M,), "f32", "x_scale")
    _expect(w_scale, (N,), "f32", "w_scale")
    if y.shape != (M, N):
        raise ValueError(f"y: shape {y.shape}, expected {(M, N)}")
    _expect(acc_out, (M, N), "i32", "acc_out")
    call("vdsl_op_gemm_w8a8", q.handle, M, N, K, xq.handle, x_scale.handle, w.handle, w_scale.handle, y.handle,
         y.dtype, int(bool(relu)), _h(acc_out), _h(workspace))


def pack_w8a8_weights(q: Queue, w: Tensor, wp: Tensor):
    """Writes w (int8 [N][K]) into wp in the MFMA fragment order gemm_w8a8_packed reads."""
    N, K = w.shape
    _expect(w, (N, K), "i8", "w")
    _expect(wp, (N, K), "i8", "wp")
    call("vdsl_op_pack_w8a8_weights", q.handle, N, K, w.handle, wp.handle)


def gemm_w8a8_packed_workspace_bytes(M, N, K) -> int:
    n = C.c_size_t()
    call("vdsl_gemm_w8a8_packed_workspace_bytes", M, N, K, C.byref(n))
    return n.value


def gemm_w8a8_packed(q: Queue, xq: Tensor, x_scale: Tensor, wp: Tensor, w_scale: Tensor, y: Tensor, relu=False,
                     acc_out=None, workspace=None):
    """gemm_w8a8 with weights packed by pack_w8a8_weights (wp keeps the logical shape [N][K]).
    workspace: gemm_w8a8_packed_workspace_bytes(M, N, K) bytes (split-K partials)."""
    M, K = xq.shape
    N, K2 = wp.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    _expect(xq, (M, K), "i8", "xq")
    _expect(wp, (N, K), "i8", "wp")
    _expect(x_scale, (M,), "f32", "x_scale")
    _expect(w_scale, (N,), "f32", "w_scale")
    if y.shape != (M, N):
        raise ValueError(f"y: shape {y.shape}, expected {(M, N)}")
    _expect(acc_out, (M, N), "i32", "acc_out")
    call("vdsl_op_gemm_w8a8_packed", q.handle, M, N, K, xq.handle, x_scale.handle, wp.handle, w_scale.handle,
         y.handle, y.dtype, int(bool(relu)), _h(acc_out), _h(workspace))


def gemm_w8a8_packed_noalloc(q: Queue, xq: Tensor, x_scale: Tensor, wp: Tensor, w_scale: Tensor, y: Tensor,
                             relu=False, acc_out=None):
    """gemm_w8a8_packed without a workspace (vdsl_op_gemm_w8a8_packed_noalloc): the split-K
    partials live in the library's own per-GPU array, so the call allocates nothing.  Calls that
    overlap in time on one GPU share that array and race."""
    M, K = xq.shape
    N, K2 = wp.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    _expect(xq, (M, K), "i8", "xq")
    _expect(wp, (N, K), "i8", "wp")
    _expect(x_scale, (M,), "f32", "x_scale")
    _expect(w_scale, (N,), "f32", "w_scale")
    if y.shape != (M, N):
        raise ValueError(f"y: shape {y.shape}, expected {(M, N)}")
    _expect(acc_out, (M, N), "i32", "acc_out")
    call("vdsl_op_gemm_w8a8_packed_noalloc", q.handle, M, N, K, xq.handle, x_scale.handle, wp.handle,
         w_scale.handle, y.handle, y.dtype, int(bool(relu)), _h(acc_out))
