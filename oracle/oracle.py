"""ctypes wrapper of liboracle.so (vdsl_oracle.c): numpy arrays in, numpy arrays out.

TEST INFRASTRUCTURE: the parity checker and the timed CPU baseline.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.  It never touches the GPU.
Each wrapper names the C function (and through it the reference lines) it calls.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, BF16, I8, I32 = 0, 1, 2, 3
# vdsl_map_opcode values (include/vdsl.h)
MAP_OPS = {
    "load": 1, "const": 2, "mov": 3, "neg": 4, "abs": 5, "square": 6, "exp": 7, "log": 8,
    "tanh": 9, "sigmoid": 10, "relu": 11, "sqrt": 12, "recip": 13, "add": 14, "sub": 15,
    "mul": 16, "div": 17, "max": 18, "min": 19, "fma": 20, "mul_imm": 21, "add_imm": 22,
    "matvec": 23, "vecmat": 24,
}


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    return C.CDLL(LIB_PATH)


_lib = _load()
_vp = C.c_void_p
_i64 = C.c_int64


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class EscapeTimeParams(C.Structure):
    # Same layout as vdsl_escape_time_params (include/vdsl.h).
    _fields_ = [
        ("ni", C.c_int32), ("nj", C.c_int32), ("family", C.c_int32), ("escape_test", C.c_int32),
        ("rounding", C.c_int32), ("out_kind", C.c_int32), ("max_iter", C.c_int32), ("bound", C.c_float),
        ("re_den", C.c_float), ("re_off", C.c_float), ("re_scale", C.c_float), ("re_post", C.c_float),
        ("im_den", C.c_float), ("im_off", C.c_float), ("im_scale", C.c_float), ("im_post", C.c_float),
        ("c_re", C.c_float), ("c_im", C.c_float), ("out_base", C.c_float), ("out_scale", C.c_float),
    ]


class MapInstr(C.Structure):
    _fields_ = [
        ("op", C.c_uint8), ("dst", C.c_uint8), ("a", C.c_uint8), ("b", C.c_uint8), ("c", C.c_uint8),
        ("ext", C.c_uint8 * 3), ("imm", C.c_float),
    ]


_lib.orc_escape_time_rows.argtypes = [C.POINTER(EscapeTimeParams), _vp, C.c_int, C.c_int]
_lib.orc_map_chain_rows.argtypes = [_i64, _i64, C.POINTER(MapInstr), C.c_int, C.POINTER(_vp), C.POINTER(C.c_int),
                                    C.c_int, C.c_int, _vp, _i64, _i64]
_lib.orc_map_chain_v_rows.argtypes = [_i64, _i64, C.POINTER(MapInstr), C.c_int, C.POINTER(_vp), C.POINTER(C.c_int),
                                      C.POINTER(C.c_int), C.c_int, C.POINTER(C.c_int), C.c_int, _vp, _i64, _i64]
_lib.orc_vec_transform.argtypes = [_i64, C.c_int, _vp, C.c_int, _vp, _vp]
_lib.orc_mat_transform.argtypes = [_i64, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp]
_lib.orc_row_reduce_softmax_rows.argtypes = [_i64, _i64, C.c_int, _vp, _vp, _vp, _vp, _i64, _i64]
_lib.orc_col_reduce.argtypes = [_i64, _i64, C.c_int, _vp, _vp, _vp]
_lib.orc_gemm_bf16_rows.argtypes = [C.c_int, C.c_int, _i64, _i64, _i64, _vp, _vp, _vp, C.c_int, C.c_int, _vp, _i64, _i64]
_lib.orc_transpose.argtypes = [_i64, _i64, C.c_int, _vp, _vp]
_lib.orc_cast.argtypes = [_i64, C.c_int, _vp, C.c_int, _vp]
_lib.orc_gelu_fwd.argtypes = [_i64, C.c_int, _vp, C.c_int, _vp]
_lib.orc_gelu_bwd.argtypes = [_i64, _i64, _vp, _vp, _vp, _vp]
_lib.orc_relu_bwd.argtypes = [_i64, _i64, _vp, _vp, _vp, _vp]
_lib.orc_add.argtypes = [_i64, C.c_int, _vp, C.c_int, _vp, C.c_int, _vp]
_lib.orc_gelu_grad.argtypes = [_i64, _vp, _vp]
_lib.orc_pixel_program_rows.argtypes = [_vp, _i64, _i64, C.POINTER(_vp), _vp, _i64, _i64]
_lib.orc_mse_fwd_bwd.argtypes = [_i64, _i64, _vp, _vp, _vp, _vp, _vp]
_lib.orc_quantize_rows_i8.argtypes = [_i64, _i64, C.c_int, _vp, _vp, _vp]
_lib.orc_gemm_w8a8_rows.argtypes = [_i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, _vp, _i64, _i64]
_lib.orc_w8a8_dequant.argtypes = [_i64, _i64, _vp, _vp, _vp, _vp, C.c_int, C.c_int]
_lib.orc_num_threads.restype = C.c_int
_lib.orc_set_num_threads.argtypes = [C.c_int]


def num_threads() -> int:
    return _lib.orc_num_threads()


def set_num_threads(n: int):
    _lib.orc_set_num_threads(int(n))


def _dt(a: np.ndarray) -> int:
    return BF16 if a.dtype == np.uint16 else F32


# ---- escape time: orc_escape_time (fractal.py:11-25) ----------------------------------------
def escape_time(params: dict, rows=None) -> np.ndarray:
    """Full grid, or only rows [r0, r1) when rows=(r0, r1) (the result then has r1 - r0 rows)."""
    p = EscapeTimeParams(**params)
    r0, r1 = rows if rows else (0, p.ni)
    dt = np.int32 if p.out_kind == 0 else np.float32
    out = np.zeros((p.ni, p.nj), dtype=dt)
    _lib.orc_escape_time_rows(C.byref(p), _p(out), r0, r1)
    return out[r0:r1]


# ---- map chain: orc_map_chain -------------------------------------------------------------------
def _instrs(code_list):
    """vdsl_map_instr array from (op, dst, a, b, c, imm[, ext]) tuples; ext (three registers) is
    given only by MATVEC / VECMAT."""
    code = (MapInstr * max(1, len(code_list)))()
    for i, ins in enumerate(code_list):
        op, dst, a, b, c, imm = ins[:6]
        code[i].op, code[i].dst, code[i].a, code[i].b, code[i].c, code[i].imm = MAP_OPS[op], dst, a, b, c, imm
        for k, r in enumerate(ins[6] if len(ins) > 6 else ()):
            code[i].ext[k] = r
    return code


def map_chain(prog, inputs, rows: int, cols: int, row_range=None) -> np.ndarray:
    """prog: vernondsl_amd.mapchain.Program (its code list and broadcasts)."""
    code = _instrs(prog.code)
    arrs = [np.ascontiguousarray(x, dtype=np.float32) for x in inputs]
    ptrs = (_vp * max(1, len(arrs)))(*[a.ctypes.data for a in arrs])
    bc = (C.c_int * max(1, len(arrs)))(*[prog.bcast[k] for k in range(len(arrs))])
    r0, r1 = row_range if row_range else (0, rows)
    out = np.zeros((r1 - r0, cols), dtype=np.float32)
    # The C routine indexes output rows absolutely; shift the base pointer by -r0 rows.
    base = out.ctypes.data - r0 * cols * 4
    _lib.orc_map_chain_rows(rows, cols, code, len(prog.code), ptrs, bc, len(arrs), prog.out_reg, _vp(base), r0, r1)
    return out


def map_chain_v(prog, inputs, rows: int, cols: int, row_range=None) -> np.ndarray:
    """Vector-operand chain (orc_map_chain_v_rows): prog carries widths and out_regs; returns
    [rows][cols][len(out_regs)] (or [rows][cols] for one output component) for rows [r0, r1)."""
    code = _instrs(prog.code)
    arrs = [np.ascontiguousarray(x, dtype=np.float32) for x in inputs]
    n = max(1, len(arrs))
    ptrs = (_vp * n)(*[a.ctypes.data for a in arrs])
    bc = (C.c_int * n)(*[prog.bcast[k] for k in range(len(arrs))])
    wd = (C.c_int * n)(*[prog.widths[k] for k in range(len(arrs))])
    ow = len(prog.out_regs)
    regs = (C.c_int * 4)(*(list(prog.out_regs) + [0] * (4 - ow)))
    r0, r1 = row_range if row_range else (0, rows)
    out = np.zeros((r1 - r0, cols, ow), dtype=np.float32)
    base = out.ctypes.data - r0 * cols * ow * 4
    _lib.orc_map_chain_v_rows(rows, cols, code, len(prog.code), ptrs, bc, wd, len(arrs), regs, ow, _vp(base), r0, r1)
    return out if ow > 1 else out[:, :, 0]


def pixel_program(prog, ni: int, nj: int, inputs=(), rows=None) -> np.ndarray:
    """orc_pixel_program_rows: prog is a vernondsl_amd.pixprog.PixelProgram (the C struct);
    inputs: f32 [ni][nj] (one component) or [ni][nj][w] arrays, w = prog.in_widths[k], or int32
    [ni][nj] (prog.in_dtypes[k] = VDSL_I32); returns f32 [rows][nj] or [rows][nj][out_width], or
    int32 [rows][nj] (the count or an int32 field; rows: (r0, r1), default all), or None for a
    program that stores nothing.  An input the program scatter-adds into is updated in place: it
    must be a C-contiguous array of its dtype (float32 / int32)."""
    total = prog.n_pre + prog.n_test + prog.n_body + prog.n_post
    targets = {prog.code[pc].a for pc in range(total) if prog.code[pc].op in (44, 46, 47, 48)}  # scatter add / max / min, store
    for k in targets:
        want = np.int32 if prog.in_dtypes[k] == 3 else np.float32
        a = inputs[k]
        if not (isinstance(a, np.ndarray) and a.dtype == want and a.flags.c_contiguous and a.flags.writeable):
            raise ValueError(f"input {k} is scatter-added into: pass a writable C-contiguous {np.dtype(want).name} array")
    ins = [np.ascontiguousarray(a, np.int32 if prog.in_dtypes[k] == 3 else np.float32) for k, a in enumerate(inputs)]
    for k, a in enumerate(ins):
        w = prog.in_widths[k]
        rk, ck = (prog.in_rows[k], prog.in_cols[k]) if prog.in_rows[k] else (ni, nj)  # an input of its own extents
        if a.shape != ((rk, ck) if w == 1 else (rk, ck, w)) and a.shape != (rk, ck, w):
            raise ValueError(f"input {k} of shape {a.shape}, expected {(rk, ck, w)}")
    r0, r1 = rows if rows else (0, ni)
    int_out = prog.out_kind in (1, 2)  # the loop count, or a value stored to an int32 field
    shape = (r1 - r0, nj) if int_out or prog.out_width == 1 else (r1 - r0, nj, prog.out_width)
    out = np.zeros(shape, np.int32 if int_out else np.float32)
    ptrs = (_vp * max(1, len(ins)))(*[a.ctypes.data for a in ins])
    _lib.orc_pixel_program_rows(C.addressof(prog), ni, nj, ptrs, _p(out), r0, r1)
    return None if prog.out_kind == 3 else out


def mat_transform(pos: np.ndarray, mats: np.ndarray) -> np.ndarray:
    """orc_mat_transform: mats f32 [k][d][d] (d = 2..4), pos f32 [n][d-1|d] -> f32 [n][d]."""
    pos = np.ascontiguousarray(pos, np.float32)
    mats = np.ascontiguousarray(mats, np.float32)
    n, w = pos.shape
    d = mats.shape[1]
    out = np.empty((n, d), np.float32)
    _lib.orc_mat_transform(n, d, w, _p(pos), mats.shape[0], _p(mats), _p(out))
    return out


def vec_transform(pos: np.ndarray, mats: np.ndarray) -> np.ndarray:
    """orc_vec_transform: pos f32 [n][3|4], mats f32 [k][4][4] -> f32 [n][4]."""
    pos = np.ascontiguousarray(pos, np.float32)
    mats = np.ascontiguousarray(mats, np.float32)
    n, w = pos.shape
    out = np.empty((n, 4), np.float32)
    _lib.orc_vec_transform(n, w, _p(pos), mats.shape[0], _p(mats), _p(out))
    return out


# ---- row reduce + softmax: orc_row_reduce_softmax ----------------------------------------------
def row_reduce_softmax(x: np.ndarray, row_range=None):
    """Returns (row_sum f32, row_max f32, softmax in x's dtype) for rows [r0, r1)."""
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    r0, r1 = row_range if row_range else (0, rows)
    n = r1 - r0
    s = np.zeros(n, np.float32)
    m = np.zeros(n, np.float32)
    sm = np.zeros((n, cols), x.dtype)
    _lib.orc_row_reduce_softmax_rows(rows, cols, _dt(x), _p(x), _vp(s.ctypes.data - r0 * 4),
                                     _vp(m.ctypes.data - r0 * 4), _vp(sm.ctypes.data - r0 * cols * x.itemsize), r0, r1)
    return s, m, sm


def col_reduce(x: np.ndarray):
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    s = np.zeros(cols, np.float32)
    m = np.zeros(cols, np.float32)
    _lib.orc_col_reduce(rows, cols, _dt(x), _p(x), _p(s), _p(m))
    return s, m


# ---- bf16 GEMM and friends: orc_gemm_bf16 etc. -----------------------------------------------------
def gemm_bf16(A: np.ndarray, B: np.ndarray, trans_a=False, trans_b=False, c_dtype=F32, epilogue=0,
              want_pre=False, row_range=None):
    A = np.ascontiguousarray(A, dtype=np.uint16)
    B = np.ascontiguousarray(B, dtype=np.uint16)
    if trans_a:
        K, M = A.shape
    else:
        M, K = A.shape
    N = B.shape[0] if trans_b else B.shape[1]
    r0, r1 = row_range if row_range else (0, M)
    Cm = np.zeros((r1 - r0, N), np.uint16 if c_dtype == BF16 else np.float32)
    pre = np.zeros((r1 - r0, N), np.float32) if want_pre else None
    es = Cm.itemsize
    _lib.orc_gemm_bf16_rows(int(trans_a), int(trans_b), M, N, K, _p(A), _p(B), _vp(Cm.ctypes.data - r0 * N * es),
                            c_dtype, epilogue, None if pre is None else _vp(pre.ctypes.data - r0 * N * 4), r0, r1)
    return (Cm, pre) if want_pre else Cm


def transpose(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    out = np.zeros((cols, rows), x.dtype)
    _lib.orc_transpose(rows, cols, _dt(x), _p(x), _p(out))
    return out


def cast(x: np.ndarray, dst_dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    out = np.zeros(x.shape, np.uint16 if dst_dtype == BF16 else np.float32)
    _lib.orc_cast(x.size, _dt(x), _p(x), dst_dtype, _p(out))
    return out


def gelu_fwd(x: np.ndarray, y_bf16: bool = False):
    """GELU(x) elementwise; x f32, or uint16 holding bf16; returns f32 or (y_bf16) uint16 bf16."""
    x = np.ascontiguousarray(x)
    xd = 1 if x.dtype == np.uint16 else 0
    if xd == 0:
        x = x.astype(np.float32, copy=False)
    y = np.zeros(x.shape, np.uint16 if y_bf16 else np.float32)
    _lib.orc_gelu_fwd(x.size, xd, _p(x), 1 if y_bf16 else 0, _p(y))
    return y


def gelu_bwd(dh: np.ndarray, pre: np.ndarray):
    dh = np.ascontiguousarray(dh, np.float32)
    pre = np.ascontiguousarray(pre, np.float32)
    rows, cols = dh.shape
    da = np.zeros((rows, cols), np.uint16)
    da_t = np.zeros((cols, rows), np.uint16)
    _lib.orc_gelu_bwd(rows, cols, _p(dh), _p(pre), _p(da), _p(da_t))
    return da, da_t


def relu_bwd(dh: np.ndarray, pre: np.ndarray):
    dh = np.ascontiguousarray(dh, np.float32)
    pre = np.ascontiguousarray(pre, np.float32)
    rows, cols = dh.shape
    da = np.zeros((rows, cols), np.uint16)
    da_t = np.zeros((cols, rows), np.uint16)
    _lib.orc_relu_bwd(rows, cols, _p(dh), _p(pre), _p(da), _p(da_t))
    return da, da_t


def add(a: np.ndarray, b: np.ndarray, out_dtype: int = F32) -> np.ndarray:
    """a + b elementwise; a, b f32 or uint16 holding bf16; returns f32 or uint16 bf16."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    if a.size != b.size:
        raise ValueError("add: sizes differ")
    out = np.zeros(a.shape, np.uint16 if out_dtype == BF16 else np.float32)
    _lib.orc_add(a.size, _dt(a), _p(a), _dt(b), _p(b), out_dtype, _p(out))
    return out


def gelu_grad(x: np.ndarray) -> np.ndarray:
    """GELU'(x) elementwise, f32 in and out."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(x.shape, np.float32)
    _lib.orc_gelu_grad(x.size, _p(x), _p(y))
    return y


def mse_fwd_bwd(y: np.ndarray, t: np.ndarray):
    y = np.ascontiguousarray(y, np.float32)
    t = np.ascontiguousarray(t, np.float32)
    rows, cols = y.shape
    loss = np.zeros(1, np.float32)
    dy = np.zeros((rows, cols), np.uint16)
    dy_t = np.zeros((cols, rows), np.uint16)
    _lib.orc_mse_fwd_bwd(rows, cols, _p(y), _p(t), _p(loss), _p(dy), _p(dy_t))
    return float(loss[0]), dy, dy_t


# ---- int8 W8A8: orc_quantize_rows_i8 / orc_gemm_w8a8 -----------------------------------------------
def quantize_rows_i8(x: np.ndarray):
    x = np.ascontiguousarray(x)
    rows, cols = x.shape
    q = np.zeros((rows, cols), np.int8)
    s = np.zeros(rows, np.float32)
    _lib.orc_quantize_rows_i8(rows, cols, _dt(x), _p(x), _p(q), _p(s))
    return q, s


def gemm_w8a8(xq, xs, w, ws, out_dtype=BF16, relu=False, want_acc=False, row_range=None):
    xq = np.ascontiguousarray(xq, np.int8)
    w = np.ascontiguousarray(w, np.int8)
    xs = np.ascontiguousarray(xs, np.float32)
    ws = np.ascontiguousarray(ws, np.float32)
    M, K = xq.shape
    N = w.shape[0]
    r0, r1 = row_range if row_range else (0, M)
    y = np.zeros((r1 - r0, N), np.uint16 if out_dtype == BF16 else np.float32)
    acc = np.zeros((r1 - r0, N), np.int32) if want_acc else None
    _lib.orc_gemm_w8a8_rows(M, N, K, _p(xq), _p(xs), _p(w), _p(ws), _vp(y.ctypes.data - r0 * N * y.itemsize), out_dtype,
                            int(relu), None if acc is None else _vp(acc.ctypes.data - r0 * N * 4), r0, r1)
    return (y, acc) if want_acc else y


def w8a8_dequant(acc, xs, ws, relu=False, out_dtype=BF16):
    """The dequant epilogue of gemm_w8a8 on given int32 accumulators acc [M][N]."""
    acc = np.ascontiguousarray(acc, np.int32)
    xs = np.ascontiguousarray(xs, np.float32)
    ws = np.ascontiguousarray(ws, np.float32)
    M, N = acc.shape
    y = np.zeros((M, N), np.uint16 if out_dtype == BF16 else np.float32)
    _lib.orc_w8a8_dequant(M, N, _p(acc), _p(xs), _p(ws), _p(y), out_dtype, int(relu))
    return y


# ---- composite programs of configs 4 and 5 (built from the routines above) --------------------
GELU = 1


def mlp_train_step(x, w1, w2, t, batch_rows=None):
    """Config 4 forward + backward with the same roundings as the HIP graph:
    H = bf16(GELU(X W1^T)) (pre-activation kept in f32), Y = H W2^T (f32), loss = mean((Y - T)^2),
    dY = bf16((Y - T) 2/n), dW2 = dY^T H, dH = dY W2 (f32), dA = bf16(dH GELU'(pre)), dW1 = dA^T X."""
    h, pre = gemm_bf16(x, w1, False, True, c_dtype=BF16, epilogue=GELU, want_pre=True)
    y = gemm_bf16(h, w2, False, True)
    loss, dy, dy_t = mse_fwd_bwd(y, t)
    dw2 = gemm_bf16(dy_t, h, False, False)
    dh = gemm_bf16(dy, w2, False, False)
    da, da_t = gelu_bwd(dh, pre)
    dw1 = gemm_bf16(da_t, x, False, False)
    return {"H": h, "pre": pre, "Y": y, "loss": loss, "dY": dy, "dW2": dw2, "dH": dh, "dA": da, "dW1": dw1}


def w8a8_forward(x, layers):
    """Config 5 forward: per layer quantise rows, int8 GEMM, dequant, ReLU except after the last."""
    h = x
    for li, (w, s) in enumerate(layers):
        xq, xs = quantize_rows_i8(h)
        h = gemm_w8a8(xq, xs, w, s, out_dtype=BF16, relu=li < len(layers) - 1)
    return h


def graph_step(g, feeds: dict) -> dict:
    """Runs an execution graph's prepare ops and step ops (vernondsl_amd.graph.Graph: ops with
    .kind, .inputs, .outputs, .attrs; values with .name, .dtype) on the routines above, with the
    roundings the device ops document, and returns {value name: array} (bf16 as uint16).  A
    packed weight holds the weight itself here (packing only reorders bytes for the device).
    feeds: the inputs and params by name."""
    v = dict(feeds)
    code = {"f32": F32, "bf16": BF16}
    epi = {"none": 0, "gelu": GELU, "relu": 2}

    def nt(a, b, dtype=F32, e=0, pre=False):
        return gemm_bf16(v[a.name], v[b.name], False, True, c_dtype=dtype, epilogue=e, want_pre=pre)

    for op in g.prepare_ops:
        src = v[op.inputs[0].name]
        v[op.outputs[0].name] = transpose(src) if op.kind == "transpose" else src
    for op in g.ops:
        ins, outs, k = op.inputs, op.outputs, op.kind
        if k == "linear":
            y, pre = nt(ins[0], ins[1], code[outs[0].dtype], epi[op.attrs["act"]], True)
            v[outs[0].name] = y
            if op.attrs.get("pre") is not None:
                v[op.attrs["pre"].name] = pre
            if op.attrs.get("dgelu") is not None:
                v[op.attrs["dgelu"].name] = gelu_grad(pre)
        elif k == "gemm":
            v[outs[0].name] = gemm_bf16(v[ins[0].name], v[ins[1].name], op.attrs["trans_a"], op.attrs["trans_b"])
        elif k in ("mse", "linear_mse"):
            if k == "linear_mse":
                v[outs[0].name] = nt(ins[0], ins[1])
                y, t, outs = v[outs[0].name], v[ins[2].name], outs[1:]
            else:
                y, t = v[ins[0].name], v[ins[1].name]
            loss, dy, dy_t = mse_fwd_bwd(y, t)
            v[outs[0].name] = np.array([loss], np.float32)
            if len(outs) > 1:
                v[outs[1].name], v[outs[2].name] = dy, dy_t
        elif k in ("gelu_bwd", "relu_bwd"):
            v[outs[0].name], v[outs[1].name] = (gelu_bwd if k == "gelu_bwd" else relu_bwd)(v[ins[0].name], v[ins[1].name])
        elif k == "gemm_gelu_bwd":
            v[outs[0].name], v[outs[1].name] = gelu_bwd(nt(ins[0], ins[1]), v[ins[2].name])
        elif k == "gemm_mul_bwd":  # dh * GELU'(pre), GELU'(pre) stored by the forward GEMM
            da = cast((nt(ins[0], ins[1]) * v[ins[2].name]).astype(np.float32), BF16)
            v[outs[0].name], v[outs[1].name] = da, transpose(da)
        elif k == "cast":
            v[outs[0].name] = cast(v[ins[0].name], code[outs[0].dtype])
        elif k == "transpose":
            v[outs[0].name] = transpose(v[ins[0].name])
        elif k == "add":
            v[outs[0].name] = add(v[ins[0].name], v[ins[1].name], code[outs[0].dtype])
        else:
            raise NotImplementedError(k)
    return v
