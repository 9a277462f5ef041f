"""Taichi-subset front end: the API surface `fractal.py` uses, lowered onto the HIP device.

`python -m vernondsl_amd.run prog.py` makes `import taichi as ti` resolve to this module, so a
program written against Taichi's API for the escape-time op class runs unchanged.  The surface
follows what the reference program calls (fractal.py):

    ti.init(arch=...)                     :5    -> the HIP device (every arch maps to it)
    ti.field(dtype=float, shape=(W, H))   :8    -> a device tensor, f32 (Taichi's default float)
    @ti.func                              :11   -> inlined where it is called
    @ti.kernel, typed scalar arguments    :16-17
    for i, j in field: ...                :18   -> one launch of vdsl_op_escape_time
    ti.Vector([...]) with * + [k], ti.cos, .norm()   :13,19,20,22,23
    ti.GUI(name, res) .set_image .show    :28,32,33 -> headless: frames are read back and counted

Kernels are not executed in Python.  Each call lowers the kernel's AST with a small symbolic
interpreter (no eval/exec of the program text): scalar arithmetic on Python values is folded in
f32 (Taichi's default float type), and the body must have the escape-time shape

    for i, j in F:
        c = <Vector, pixel map or constant>    z = <Vector, pixel map or constant>
        k = 0
        while <|z| test> and k < MAX:           (either order of the two tests)
            z = <complex square of z> + c
            k += 1
        F[i, j] = <k, or a + k * b / a - k * b>

A body of any other shape raises TaichiLoweringError naming what did not match; there is no CPU
fallback.  Accepted complex squares are the ones equal bit for bit to (zr*zr - zi*zi, (zi*zr)*2):
`z[0]**2 - z[1]**2`, `z[0]*z[0] - z[1]*z[1]`, and `z[1]*z[0]*2` / `z[0]*z[1]*2` / `2*(z[0]*z[1])` /
`z[0]*z[1] + z[0]*z[1]` for the imaginary part (`(2*z[0])*z[1]` is refused: it rounds differently
when the product is subnormal).
"""
from __future__ import annotations

import ast
import inspect
import math
import textwrap

import numpy as np

from . import _lib

# ---- types and archs ------------------------------------------------------------------------
f32 = float32 = "f32"
i32 = int32 = "i32"
f64 = float64 = "f64"
cpu = "cpu"
gpu = "gpu"
cuda = "cuda"
vulkan = "vulkan"
opengl = "opengl"
gles = "gles"
metal = "metal"
dx11 = "dx11"
amdgpu = "amdgpu"
hip = "hip"

_state = {"device": None, "queue": None, "arch": None, "frames": 0}


class TaichiLoweringError(RuntimeError):
    """The kernel body is not one this backend lowers."""


def init(arch=None, default_fp=None, **_kw):
    """Selects the backend (fractal.py:5).  Every arch runs on the HIP device; the device itself is
    opened on the first launch, so programs can be lowered on a host without a GPU."""
    if default_fp not in (None, f32, float):
        raise TaichiLoweringError("only f32 is supported as default_fp")
    _state["arch"] = arch


def _device():
    if _state["device"] is None:
        from .rhi import Device, Queue
        _state["device"] = Device(0)
        _state["queue"] = Queue(_state["device"])
    return _state["device"], _state["queue"]


class Field:
    """A dense 2-D field (fractal.py:8).  Storage is a device tensor, allocated on first use."""

    def __init__(self, dtype, shape):
        if dtype in (float, f32, None):
            self.dtype = f32
        elif dtype in (int, i32):
            self.dtype = i32
        else:
            raise TaichiLoweringError(f"field dtype {dtype!r}: only f32 and i32 fields are supported")
        if isinstance(shape, int):
            shape = (shape,)
        self.shape = tuple(int(s) for s in shape)
        self._tensor = None

    def tensor(self):
        if self._tensor is None:
            from .rhi import Tensor
            dev, _ = _device()
            self._tensor = Tensor(dev, self.shape, self.dtype)
        return self._tensor

    def to_numpy(self):
        _, q = _device()
        return self.tensor().numpy(q)

    def __getitem__(self, idx):
        return self.to_numpy()[idx]


def field(dtype=float, shape=None, **_kw):
    return Field(dtype, shape)


def func(fn):
    fn._vdsl_ti_func = True
    return fn


def kernel(fn):
    return Kernel(fn)


class Vector:  # only meaningful inside kernels, where the lowering interprets it
    def __init__(self, *_a, **_k):
        raise TaichiLoweringError("ti.Vector is only available inside @ti.kernel / @ti.func code")


def cos(x):
    return np.cos(np.float32(x), dtype=np.float32)


def sin(x):
    return np.sin(np.float32(x), dtype=np.float32)


class GUI:
    """Headless stand-in for ti.GUI (fractal.py:28,32,33): set_image reads the field back (the
    device->host boundary of the reference's frame loop), show() counts frames.  After
    `frame_limit` frames (set by the runner) show() raises FrameLimitReached."""

    frame_limit = None

    def __init__(self, name="", res=None, **_kw):
        self.name = name
        self.res = res
        self.last_image = None
        self.frames = 0

    def set_image(self, img):
        self.last_image = img.to_numpy() if isinstance(img, Field) else np.asarray(img)

    def show(self, *_a):
        self.frames += 1
        _state["frames"] += 1
        _state["last_gui"] = self
        if GUI.frame_limit is not None and self.frames >= GUI.frame_limit:
            raise FrameLimitReached(self)

    @property
    def running(self):
        return True


class FrameLimitReached(Exception):
    def __init__(self, gui):
        super().__init__(f"{gui.frames} frames")
        self.gui = gui


# ---- kernels ---------------------------------------------------------------------------------
class Kernel:
    def __init__(self, fn):
        self.fn = fn
        src = textwrap.dedent(inspect.getsource(fn))
        mod = ast.parse(src)
        self.fdef = next(n for n in mod.body if isinstance(n, ast.FunctionDef))
        self.arg_names = [a.arg for a in self.fdef.args.args]
        self.arg_types = [_annotation(a.annotation) for a in self.fdef.args.args]

    def lower(self, *args):
        env = dict(self.fn.__globals__)
        for name, typ, val in zip(self.arg_names, self.arg_types, args):
            env[name] = _coerce(typ, val)
        return lower_escape_time(self.fdef, _FuncResolver(env), env)

    def __call__(self, *args):
        fld, params = self.lower(*args)
        from . import kernels
        _, q = _device()
        p = kernels.escape_time_params(**params)
        kernels.escape_time(q, p, fld.tensor())


def _annotation(node):
    if node is None:
        return None
    if isinstance(node, ast.Name):
        return {"float": f32, "int": i32, "f32": f32, "i32": i32}.get(node.id, node.id)
    if isinstance(node, ast.Attribute):
        return {"f32": f32, "i32": i32, "float32": f32, "int32": i32}.get(node.attr, node.attr)
    return None


def _coerce(typ, val):
    if typ == f32:
        return np.float32(val)
    if typ == i32:
        return int(val)
    return val


class _FuncResolver:
    """Finds @ti.func definitions: by function object (programs being run) or by AST (text)."""

    def __init__(self, env, func_asts=None):
        self.env = env
        self.func_asts = func_asts or {}

    def get(self, name):
        if name in self.func_asts:
            return self.func_asts[name]
        obj = self.env.get(name)
        if obj is not None and getattr(obj, "_vdsl_ti_func", False):
            src = textwrap.dedent(inspect.getsource(obj))
            return next(n for n in ast.parse(src).body if isinstance(n, ast.FunctionDef))
        return None


# ---- symbolic values -------------------------------------------------------------------------
class Sym:
    """An expression tree node: op in {'i', 'j', 'zr', 'zi', 'k', 'add', 'sub', 'mul', 'div',
    'neg', 'pow', 'norm', 'dot'}; args are Syms or numbers."""

    def __init__(self, op, *args):
        self.op, self.args = op, args

    def __repr__(self):
        return f"{self.op}({', '.join(map(repr, self.args))})"


class Vec:
    def __init__(self, comps):
        self.comps = list(comps)


def _is_num(v):
    return isinstance(v, (int, float, np.floating, np.integer)) and not isinstance(v, bool)


def _f32(v):
    return np.float32(v)


def _binop(op, a, b):
    if isinstance(a, Vec) or isinstance(b, Vec):
        if isinstance(a, Vec) and isinstance(b, Vec):
            if len(a.comps) != len(b.comps):
                raise TaichiLoweringError("vector length mismatch")
            return Vec([_binop(op, x, y) for x, y in zip(a.comps, b.comps)])
        if isinstance(a, Vec):
            return Vec([_binop(op, x, b) for x in a.comps])
        return Vec([_binop(op, a, y) for y in b.comps])
    if _is_num(a) and _is_num(b):
        # Taichi folds scalar arithmetic in its default float type (f32) unless both are ints
        if isinstance(a, (int, np.integer)) and isinstance(b, (int, np.integer)) and op != "div":
            return {"add": a + b, "sub": a - b, "mul": a * b, "pow": a ** b}[op]
        x, y = _f32(a), _f32(b)
        with np.errstate(all="ignore"):
            return {"add": x + y, "sub": x - y, "mul": x * y, "div": x / y, "pow": x ** y}[op]
    return Sym(op, a, b)


class _Interp:
    """Evaluates kernel / func ASTs over numbers, Syms and Vecs."""

    def __init__(self, env, funcs):
        self.env = env
        self.funcs = funcs

    def expr(self, n, local):
        if isinstance(n, ast.Constant):
            return n.value
        if isinstance(n, ast.Name):
            if n.id in local:
                return local[n.id]
            if n.id in self.env:
                return self.env[n.id]
            raise TaichiLoweringError(f"unknown name {n.id!r}")
        if isinstance(n, ast.BinOp):
            ops = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div", ast.Pow: "pow"}
            if type(n.op) not in ops:
                raise TaichiLoweringError(f"operator {type(n.op).__name__} is not supported")
            return _binop(ops[type(n.op)], self.expr(n.left, local), self.expr(n.right, local))
        if isinstance(n, ast.UnaryOp) and isinstance(n.op, ast.USub):
            v = self.expr(n.operand, local)
            if isinstance(v, Vec):
                return Vec([(-_f32(c) if _is_num(c) else Sym("neg", c)) for c in v.comps])
            return -_f32(v) if _is_num(v) else Sym("neg", v)
        if isinstance(n, ast.Subscript):
            base = self.expr(n.value, local)
            idx = self.expr(n.slice, local)
            if isinstance(base, Vec) and isinstance(idx, int):
                return base.comps[idx]
            raise TaichiLoweringError("only constant vector indexing is supported in expressions")
        if isinstance(n, ast.Attribute):
            base = self.expr(n.value, local)
            return getattr(base, n.attr) if not isinstance(base, (Vec, Sym)) else (base, n.attr)
        if isinstance(n, ast.List) or isinstance(n, ast.Tuple):
            return [self.expr(e, local) for e in n.elts]
        if isinstance(n, ast.Call):
            return self.call(n, local)
        raise TaichiLoweringError(f"expression {ast.dump(n)[:60]} is not supported")

    def call(self, n, local):
        f = n.func
        # method calls on vectors: z.norm(), z.norm_sqr(), z.dot(w)
        if isinstance(f, ast.Attribute):
            base = self.expr(f.value, local)
            if isinstance(base, Vec):
                if f.attr == "norm":
                    return Sym("norm", base)
                if f.attr == "norm_sqr":
                    return Sym("dot", base, base)
                if f.attr == "dot":
                    other = self.expr(n.args[0], local)
                    return Sym("dot", base, other)
                raise TaichiLoweringError(f"vector method {f.attr!r} is not supported")
            if f.attr == "Vector":
                comps = self.expr(n.args[0], local)
                return Vec(comps)
            if f.attr in ("cos", "sin"):
                a = self.expr(n.args[0], local)
                if not _is_num(a):
                    raise TaichiLoweringError(f"ti.{f.attr} of a per-pixel value is not supported")
                return (cos if f.attr == "cos" else sin)(a)
            raise TaichiLoweringError(f"call {f.attr!r} is not supported")
        if isinstance(f, ast.Name):
            fdef = self.funcs.get(f.id)
            if fdef is None:
                obj = self.env.get(f.id)
                if obj in (float,):
                    return _f32(self.expr(n.args[0], local))
                if obj in (int,):
                    return int(self.expr(n.args[0], local))
                raise TaichiLoweringError(f"call of {f.id!r}: only @ti.func functions are inlined")
            args = [self.expr(a, local) for a in n.args]
            sub = dict(zip([a.arg for a in fdef.args.args], args))
            for st in fdef.body:
                if isinstance(st, ast.Return):
                    return self.expr(st.value, sub)
                if isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Name):
                    sub[st.targets[0].id] = self.expr(st.value, sub)
                    continue
                if isinstance(st, ast.Expr) and isinstance(st.value, ast.Constant):
                    continue  # docstring
                raise TaichiLoweringError(f"statement in @ti.func {f.id!r} is not supported")
            raise TaichiLoweringError(f"@ti.func {f.id!r} returns nothing")
        raise TaichiLoweringError("unsupported call")


# ---- pattern matching --------------------------------------------------------------------------
def _match_coord(e, var):
    """((var / den) + off) * scale + post  ->  (den, off, scale, post); each part optional."""
    post = 0.0
    if isinstance(e, Sym) and e.op in ("add", "sub") and _is_num(e.args[1]):
        post = float(e.args[1]) if e.op == "add" else -float(_f32(e.args[1]))
        e = e.args[0]
    scale = 1.0
    if isinstance(e, Sym) and e.op == "mul":
        if _is_num(e.args[1]):
            scale, e = float(e.args[1]), e.args[0]
        elif _is_num(e.args[0]):
            scale, e = float(e.args[0]), e.args[1]
    off = 0.0
    if isinstance(e, Sym) and e.op in ("add", "sub") and _is_num(e.args[1]):
        off = float(e.args[1]) if e.op == "add" else -float(_f32(e.args[1]))
        e = e.args[0]
    if isinstance(e, Sym) and e.op == "div" and isinstance(e.args[0], Sym) and e.args[0].op == var and _is_num(e.args[1]):
        return float(e.args[1]), off, scale, post
    if isinstance(e, Sym) and e.op == var:
        return 1.0, off, scale, post
    raise TaichiLoweringError(f"pixel coordinate {e!r} is not of the form ((index / n) + a) * b + c")


def _is(e, op, *args):
    return isinstance(e, Sym) and e.op == op and len(e.args) == len(args) and all(
        (a is None) or (isinstance(a, str) and isinstance(x, Sym) and x.op == a) or (_is_num(a) and _is_num(x) and float(x) == a)
        for x, a in zip(e.args, args))


def _is_sq(e, v):
    return _is(e, "mul", v, v) or _is(e, "pow", v, 2)


def _is_zr_zi(e):
    return _is(e, "mul", "zr", "zi") or _is(e, "mul", "zi", "zr")


def _match_complex_square(re_e, im_e):
    if not (isinstance(re_e, Sym) and re_e.op == "sub" and _is_sq(re_e.args[0], "zr") and _is_sq(re_e.args[1], "zi")):
        raise TaichiLoweringError(f"real part {re_e!r} is not zr*zr - zi*zi")
    ok = (isinstance(im_e, Sym) and im_e.op == "mul" and (
        (_is_zr_zi(im_e.args[0]) and _is_num(im_e.args[1]) and float(im_e.args[1]) == 2.0) or
        (_is_num(im_e.args[0]) and float(im_e.args[0]) == 2.0 and _is_zr_zi(im_e.args[1]))))
    ok = ok or (isinstance(im_e, Sym) and im_e.op == "add" and _is_zr_zi(im_e.args[0]) and _is_zr_zi(im_e.args[1]))
    if not ok:
        raise TaichiLoweringError(f"imaginary part {im_e!r} is not 2*zr*zi")


def lower_escape_time(fdef: ast.FunctionDef, funcs, env) -> tuple:
    """Lowers one @ti.kernel to (field, vdsl_escape_time_params as a dict)."""
    body = [s for s in fdef.body if not (isinstance(s, ast.Expr) and isinstance(s.value, ast.Constant))]
    if len(body) != 1 or not isinstance(body[0], ast.For):
        raise TaichiLoweringError("the kernel body must be one struct-for `for i, j in field:`")
    loop = body[0]
    if not (isinstance(loop.target, ast.Tuple) and len(loop.target.elts) == 2):
        raise TaichiLoweringError("the struct-for must bind two indices (a 2-D field)")
    iname, jname = (e.id for e in loop.target.elts)
    interp = _Interp(env, funcs)
    fld = interp.expr(loop.iter, {})
    if not isinstance(fld, Field) or len(fld.shape) != 2:
        raise TaichiLoweringError("the struct-for must iterate a 2-D ti.field")
    local = {iname: Sym("i"), jname: Sym("j")}
    params = dict(ni=fld.shape[0], nj=fld.shape[1])
    state = {}
    stmts = list(loop.body)
    counter = None
    while stmts:
        st = stmts.pop(0)
        if isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Name):
            v = interp.expr(st.value, local)
            local[st.targets[0].id] = v
            if _is_num(v) and float(v) == 0 and isinstance(st.value, ast.Constant) and isinstance(st.value.value, int):
                counter = st.targets[0].id
            continue
        if isinstance(st, ast.While):
            state["while"] = st
            _lower_while(st, interp, local, counter, params)
            counter_name = params.pop("_counter")
            local[counter_name] = Sym("k")
            continue
        if isinstance(st, ast.Assign) and isinstance(st.targets[0], ast.Subscript):
            tgt = st.targets[0]
            if interp.expr(tgt.value, local) is not fld:
                raise TaichiLoweringError("the store must write the iterated field")
            idx = tgt.slice
            if not (isinstance(idx, ast.Tuple) and [e.id for e in idx.elts] == [iname, jname]):
                raise TaichiLoweringError("the store must write field[i, j]")
            _lower_store(interp.expr(st.value, local), fld, params)
            state["store"] = True
            continue
        raise TaichiLoweringError(f"statement at line {getattr(st, 'lineno', '?')} is not supported")
    if "while" not in state or "store" not in state:
        raise TaichiLoweringError("the struct-for needs an escape loop and a store of the count")
    return fld, params


def _lower_while(st, interp, local, counter, params):
    # condition: a BoolOp `and` of a magnitude test and a counter bound, in either order
    tests = st.test.values if isinstance(st.test, ast.BoolOp) and isinstance(st.test.op, ast.And) else [st.test]
    if len(tests) != 2:
        raise TaichiLoweringError("the while condition must be `<|z| test> and <counter> < max`")
    zname = None
    for t in tests:
        if not (isinstance(t, ast.Compare) and len(t.ops) == 1):
            raise TaichiLoweringError("each while test must be one comparison")
        left = t.left
        if isinstance(left, ast.Name) and left.id == counter:
            if not isinstance(t.ops[0], ast.Lt):
                raise TaichiLoweringError("the counter test must be `counter < max`")
            params["max_iter"] = int(interp.expr(t.comparators[0], local))
            continue
        is_method = isinstance(left, ast.Call) and isinstance(left.func, ast.Attribute) and isinstance(left.func.value, ast.Name)
        zv = local.get(left.func.value.id) if is_method else None
        if not isinstance(zv, Vec):
            raise TaichiLoweringError("the magnitude test must call .norm()/.norm_sqr()/.dot() on the iterated vector")
        zname = left.func.value.id
        meth = left.func.attr
        bound = float(_f32(interp.expr(t.comparators[0], local)))
        op = type(t.ops[0])
        if meth == "norm" and op is ast.Lt:
            params.update(escape_test=_lib.ESC_NORM_GE, bound=bound)
        elif meth in ("norm_sqr", "dot") and op is ast.LtE:
            if meth == "dot":
                arg = t.left.args[0]
                if not (isinstance(arg, ast.Name) and arg.id == zname):
                    raise TaichiLoweringError("z.dot(w) needs w = z")
            params.update(escape_test=_lib.ESC_MAG2_GT, bound=bound)
        else:
            raise TaichiLoweringError("supported tests: z.norm() < r, z.norm_sqr() <= r2, z.dot(z) <= r2")
    if zname is None or "max_iter" not in params:
        raise TaichiLoweringError("the while condition needs both a magnitude test and a counter bound")
    # body: z = f(z) + c ; counter += 1
    body = list(st.body)
    if len(body) != 2:
        raise TaichiLoweringError("the while body must be `z = sq(z) + c` and `counter += 1`")
    upd, inc = body
    if not (isinstance(inc, ast.AugAssign) and isinstance(inc.op, ast.Add) and isinstance(inc.target, ast.Name)
            and inc.target.id == counter and isinstance(inc.value, ast.Constant) and inc.value.value == 1):
        raise TaichiLoweringError("the loop must count with `counter += 1` after the update")
    if not (isinstance(upd, ast.Assign) and isinstance(upd.targets[0], ast.Name) and upd.targets[0].id == zname):
        raise TaichiLoweringError("the loop must update the tested vector first")
    z0 = local[zname]
    sym_local = dict(local)
    sym_local[zname] = Vec([Sym("zr"), Sym("zi")])
    new = interp.expr(upd.value, sym_local)
    if not (isinstance(new, Vec) and len(new.comps) == 2):
        raise TaichiLoweringError("the update must produce a 2-vector")
    re_e, im_e = new.comps
    if not (isinstance(re_e, Sym) and re_e.op == "add" and isinstance(im_e, Sym) and im_e.op == "add"):
        raise TaichiLoweringError("the update must be `square(z) + c`")
    _match_complex_square(re_e.args[0], im_e.args[0])
    c_re, c_im = re_e.args[1], im_e.args[1]
    # Julia: c constant, z0 from the pixel; Mandelbrot: z0 = 0, c from the pixel
    if _is_num(c_re) and _is_num(c_im):
        params.update(family=_lib.ESC_JULIA, c_re=float(_f32(c_re)), c_im=float(_f32(c_im)))
        src = z0
    else:
        if not (isinstance(z0, Vec) and all(_is_num(v) and float(v) == 0.0 for v in z0.comps)):
            raise TaichiLoweringError("with a per-pixel c the iteration must start from z = 0")
        params.update(family=_lib.ESC_MANDELBROT)
        src = Vec([c_re, c_im])
    if not isinstance(src, Vec) or len(src.comps) != 2:
        raise TaichiLoweringError("the pixel map must be a 2-vector")
    for comp, var, key in ((src.comps[0], "i", "re"), (src.comps[1], "j", "im")):
        den, off, scale, post = _match_coord(comp, var)
        params.update({f"{key}_den": den, f"{key}_off": off, f"{key}_scale": scale, f"{key}_post": post})
    params["rounding"] = _lib.ESC_ROUND_SEPARATE
    params["_counter"] = counter


def _lower_store(v, fld, params):
    if isinstance(v, Sym) and v.op == "k":
        params.update(out_kind=_lib.ESC_OUT_I32_COUNT if fld.dtype == i32 else _lib.ESC_OUT_F32_AFFINE,
                      out_base=0.0, out_scale=1.0)
    else:
        if fld.dtype != f32:
            raise TaichiLoweringError("an i32 field stores the raw count")
        base, scale = 0.0, 1.0
        if isinstance(v, Sym) and v.op in ("add", "sub") and _is_num(v.args[0]):      # a +- k*b
            base = float(_f32(v.args[0]))
            sign = -1.0 if v.op == "sub" else 1.0
            term = v.args[1]
        elif isinstance(v, Sym) and v.op in ("add", "sub") and _is_num(v.args[1]):    # k*b +- a
            base = float(_f32(v.args[1])) * (-1.0 if v.op == "sub" else 1.0)
            sign, term = 1.0, v.args[0]
        else:
            sign, term = 1.0, v
        if _is(term, "mul", "k", None) and _is_num(term.args[1]):
            scale = sign * float(_f32(term.args[1]))
        elif _is(term, "mul", None, "k") and _is_num(term.args[0]):
            scale = sign * float(_f32(term.args[0]))
        else:
            raise TaichiLoweringError(f"store {v!r} is not a + k * b")
        params.update(out_kind=_lib.ESC_OUT_F32_AFFINE, out_base=base, out_scale=scale)
    if params["out_kind"] == _lib.ESC_OUT_I32_COUNT and fld.dtype != i32:
        raise TaichiLoweringError("storing the raw count needs an i32 field")


# ---- lowering from program text (no execution) -----------------------------------------------------
def lower_source(text: str, kernel_name: str, args: dict) -> tuple:
    """Lowers `kernel_name` of a Taichi program given as text, without running it: module-level
    constants and fields are evaluated statically (literals, arithmetic, ti.field calls)."""
    mod = ast.parse(text)
    env = {"float": float, "int": int}
    tinames = set()
    for st in mod.body:
        if isinstance(st, ast.Import):
            for a in st.names:
                if a.name == "taichi":
                    tinames.add(a.asname or "taichi")
    import sys as _sys
    for name in tinames:
        env[name] = _sys.modules[__name__]
    funcs, kern = {}, None
    interp = _Interp(env, _FuncResolver(env, funcs))
    for st in mod.body:
        if isinstance(st, ast.FunctionDef):
            decos = {d.attr if isinstance(d, ast.Attribute) else getattr(d, "id", "") for d in st.decorator_list}
            if "func" in decos:
                funcs[st.name] = st
            if "kernel" in decos and st.name == kernel_name:
                kern = st
        elif (isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Tuple)
              and isinstance(st.value, ast.Tuple) and len(st.targets[0].elts) == len(st.value.elts)):
            for t, v in zip(st.targets[0].elts, st.value.elts):  # W, H = 400, 300
                if isinstance(t, ast.Name):
                    try:
                        env[t.id] = interp.expr(v, {})
                    except TaichiLoweringError:
                        pass
        elif isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Name):
            v = st.value
            if isinstance(v, ast.Call) and isinstance(v.func, ast.Attribute) and v.func.attr == "field":
                kw = {k.arg: k.value for k in v.keywords}
                shape = interp.expr(kw["shape"], {})
                dt = kw.get("dtype")
                dtype = f32 if dt is None or (isinstance(dt, ast.Name) and dt.id == "float") else (
                    i32 if (isinstance(dt, ast.Name) and dt.id == "int") or getattr(dt, "attr", "") in ("i32", "int32") else f32)
                env[st.targets[0].id] = Field(dtype, shape)
            else:
                try:
                    env[st.targets[0].id] = interp.expr(v, {})
                except TaichiLoweringError:
                    pass  # not a constant (GUI objects and the like)
    if kern is None:
        raise TaichiLoweringError(f"no @ti.kernel named {kernel_name!r}")
    for a in kern.args.args:
        if a.arg in args:
            env[a.arg] = _coerce(_annotation(a.annotation), args[a.arg])
    return lower_escape_time(kern, _FuncResolver(env, funcs), env)


# math helpers programs sometimes use at module level
pi = math.pi
