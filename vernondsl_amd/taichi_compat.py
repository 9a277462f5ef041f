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

Bodies of any other shape are lowered by the general path to a per-pixel register program
(vernondsl_amd.pixprog, run by vdsl_op_pixel_program, compiled at run time for the program): any
expression of the pixel indices, scalar kernel arguments, other 2-D f32 fields read at [i, j]
and constants, with loops - a `while <test> and <counter> < MAX:` check-then-update
loop whose body ends with `counter += 1`, or a `for k in range(N)` / `range(A, B)` loop (a
perfect nest of them runs as one loop over its trips; N may be an integer expression of the
pixel), whose test and body may read the counter or k (from the loop's trip), with `break` and
`continue` in the body or its ifs (`continue` not in a while loop, where it would skip the
increment), `@ti.func` calls (statements before a final return), `ti.types.vector` values,
swizzles, integer bit operations (`& | ^ << >> ~`) of bounded integers; a body of several loops runs as parts joined by hidden per-pixel fields - and stores
`F[i, j] = <value>` (an i32 field stores the loop counter) into one or more fields of the loop's
shape: a body storing several fields becomes one program per stored field, run in an order in
which no program loads a field that an earlier one stored (a snapshot copy where the programs
load each other's fields; a load at [i, j] after the body's own store reads the stored value, as
in Taichi); a kernel of several top-level struct-fors runs their lowerings one after another.
1-D fields and struct-fors (`for i in x:`, `for i in range(N):`) run as one row of the grid, 3-D
ones ([A][B][C], `for i, j, k in u:`) as the grid [A B][C]; 0-D fields (`shape=()`) are read and
added into as `s[None]`.  `F[idx] += v` / `-= v` at an index other than the loop's (and
`ti.atomic_add(F[idx], v)` as a statement; `ti.atomic_max` / `atomic_min` alike) is Taichi's atomic
add: a scatter-add of the program,
dropped where an index falls outside F, with idx a tuple or a vector expression such as
`base + offset` (`.cast(int)` / `int()` truncate); a field added into is neither read nor stored
by the same struct-for, and adds inside an if happen only where the branch runs.  `F[idx] = v` at
another index is a plain store there (with ti.ndrange((a, b), ...) interiors and boundary loops).
Kernel-scope scalars set to constants before the struct-fors and `+=` / `-=` in them are Taichi's
reductions; `return name` returns one from the call.  `ti.random()` draws from a counter-based
generator whose state advances once per kernel call.  `ti.Matrix`
values (`@`, `outer_product`, `trace`, `determinant`, `transpose`) and 2 x 2 matrix fields lower
to their scalar operations; `for I in ti.grouped(F)` binds I to the index vector.  A lowering called again with the same arguments is replayed as one
recorded hipGraph.  What neither path lowers raises
TaichiLoweringError naming what did not match; there is no CPU fallback.  Accepted complex squares are the ones equal bit for bit to (zr*zr - zi*zi, (zi*zr)*2):
`z[0]**2 - z[1]**2`, `z[0]*z[0] - z[1]*z[1]`, and `z[1]*z[0]*2` / `z[0]*z[1]*2` / `2*(z[0]*z[1])` /
`z[0]*z[1] + z[0]*z[1]` for the imaginary part (`(2*z[0])*z[1]` is refused: it rounds differently
when the product is subnormal).
"""
from __future__ import annotations

import ast
import collections
import copy
import inspect
import itertools
import os
import math as _pymath
import sys
import textwrap
import types as _pytypes

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
    """A dense 2-D field (fractal.py:8), or a 0-D (shape ()), 1-D or 3-D one, of scalars or of
    vectors of `width` f32 components (ti.Vector.field).  Storage is a device tensor ([W][H],
    [N], [1] for 0-D, plus [width] for vectors), allocated and zeroed on first use."""

    def __init__(self, dtype, shape, width=1, mat=None):
        self.mat = tuple(mat) if mat else None  # (n, m) for a field of n x m matrices (row-major components)
        if dtype in (float, f32, None):
            self.dtype = f32
        elif dtype in (int, i32):
            self.dtype = i32
        else:
            raise TaichiLoweringError(f"field dtype {dtype!r}: only f32 and i32 fields are supported")
        if isinstance(shape, int):
            shape = (shape,)
        self.shape = tuple(int(s) for s in (shape if shape is not None else ()))
        self.width = int(width)
        if not 1 <= self.width <= 4 or (self.width > 1 and self.dtype != f32):
            raise TaichiLoweringError("vector fields hold 1 to 4 f32 components")
        self._tensor = None
        self._snap = None
        self._grid = None

    def snapshot(self):
        """A hidden field of this one's type and shape, made once: the copy of its values taken
        before a struct-for's programs when one of them stores it and another loads it."""
        if self._snap is None:
            self._snap = Field(self.dtype, self.shape, self.width, self.mat)
        return self._snap

    def tensor(self):
        if self._tensor is None:
            from .rhi import Tensor
            dev, q = _device()
            shape = self.shape or (1,)  # a 0-D field holds one element
            t = Tensor(dev, shape if self.width == 1 else shape + (self.width,), self.dtype)
            t.buffer.fill_u32(q, 0)  # a Taichi field starts zeroed
            self._tensor = t
        return self._tensor

    def grid_tensor(self):
        """The tensor as a per-pixel program grid: a 1-D field of n elements is one row, [1][n]; a
        3-D field [A][B][C] is [A B][C] (the same bytes); a 0-D field is [1][1]."""
        t = self.tensor()
        if self._grid is None or self._grid[0] is not t:
            if len(self.shape) <= 1:
                g = t.view((1,) + t.shape)
            elif len(self.shape) == 3:
                g = t.view((self.shape[0] * self.shape[1],) + t.shape[2:])
            else:
                g = t
            self._grid = (t, g)  # made once: kernels launch many times
        return self._grid[1]

    def to_numpy(self):
        _, q = _device()
        a = self.tensor().numpy(q)
        return a.reshape(a.shape[1:]) if not self.shape else a

    def from_numpy(self, arr):
        """Sets every element from an array of the field's shape (and component count)."""
        want = self.shape if self.width == 1 else self.shape + (self.width,)
        a = np.array(arr, np.int32 if self.dtype == i32 else np.float32, order="C")  # keeps a 0-D shape
        if a.shape != want:
            raise ValueError(f"from_numpy: array of shape {a.shape}, the field is {want}")
        _, q = _device()
        self.tensor().buffer.write(q, a.reshape(-1))

    def fill(self, value):
        """Sets every element (every component) to value."""
        bits = np.array([value], np.int32 if self.dtype == i32 else np.float32).view(np.uint32)[0]
        _, q = _device()
        self.tensor().buffer.fill_u32(q, int(bits))

    def __getitem__(self, idx):
        return self.to_numpy()[() if idx is None else idx]

    def __setitem__(self, idx, value):
        a = self.to_numpy()
        a[() if idx is None else idx] = value
        self.from_numpy(a)


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

    @staticmethod
    def field(n, dtype=float, shape=None, **_kw):
        """ti.Vector.field(n, dtype, shape): a 2-D field of n-component f32 vectors."""
        return Field(dtype, shape, width=n)


class Matrix:  # only meaningful inside kernels, where the lowering interprets it
    def __init__(self, *_a, **_k):
        raise TaichiLoweringError("ti.Matrix is only available inside @ti.kernel / @ti.func code")

    @staticmethod
    def field(n, m, dtype=float, shape=None, **_kw):
        """ti.Matrix.field(n, m, dtype, shape): a field of n x m f32 matrices (n m <= 4), stored
        row-major as n m components per element."""
        if n * m > 4:
            raise TaichiLoweringError("matrix fields hold at most 4 components (2 x 2)")
        return Field(dtype, shape, width=n * m, mat=(n, m))


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

    def circles(self, pos, radius=1, color=0xFFFFFF, **_kw):
        """Headless: the frame's content is the positions drawn (an [N][2] array, or a field of
        2-vectors read back)."""
        self.last_image = pos.to_numpy() if isinstance(pos, Field) else np.asarray(pos)

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
        self._cache = collections.OrderedDict()  # argument values -> Lowered, most recent last

    CACHE_SIZE = 64

    def lower(self, *args) -> "Lowered":
        """The kernel lowered for these argument values, from a per-kernel cache of the last
        CACHE_SIZE argument tuples.  Module-level values the body reads are taken at the first
        lowering for given arguments, as Taichi takes Python globals as compile-time constants."""
        vals = tuple(_coerce(typ, val) for typ, val in zip(self.arg_types, args))
        try:
            key = (len(args),) + tuple((type(v).__name__, v) for v in vals)
            hit = self._cache.get(key)
        except TypeError:  # an unhashable argument: lowered every call
            key, hit = None, None
        if hit is not None:
            self._cache.move_to_end(key)
            return hit
        env = dict(self.fn.__globals__)
        for name, val in zip(self.arg_names, vals):
            env[name] = val
        funcs = _FuncResolver(env)
        low = _with_rng_advance(lower_kernel(self.fdef, funcs, env), self.fdef, funcs, env)
        if key is not None:
            self._cache[key] = low
            while len(self._cache) > self.CACHE_SIZE:
                self._cache.popitem(last=False)
        return low

    # Calls of one lowering (one argument tuple) made eagerly before its launches are recorded as
    # one hipGraph, replayed by the calls after (VDSL_TI_GRAPHS=0: always eager).  A kernel called
    # every frame or substep then costs one graph launch instead of one launch per program (the
    # mpm88 example's substep: 12 programs, 32 us of device time, ~325 us launched one by one).
    GRAPH_AFTER = 2

    def __call__(self, *args):
        low = self.lower(*args)
        _, q = _device()
        graph = getattr(low, "graph", None)
        if graph:
            graph.launch(q)
            return self._result(low)
        self._launch(low, q)
        low.calls = getattr(low, "calls", 0) + 1
        if graph is None and low.calls >= self.GRAPH_AFTER and os.environ.get("VDSL_TI_GRAPHS", "1") != "0":
            # record (not run) the same launches; every program is compiled by now
            try:
                with q.capture() as rec:
                    self._launch(low, q)
                low.graph = rec.graph
            except Exception:  # an op that cannot be recorded: this lowering stays eager
                low.graph = False
        return self._result(low)

    @staticmethod
    def _result(low):
        """The value `return name` names (its hidden 0-D field, read back), or None."""
        ret = getattr(low, "ret", None)
        if ret is None:
            return None
        v = ret.to_numpy()[()]
        return int(v) if ret.dtype == i32 else float(v)

    @staticmethod
    def _launch(low, q):
        from . import kernels
        for op in low.ops():
            if op.kind == "copy":
                op.field.tensor().buffer.copy_from(q, op.inputs[0].tensor().buffer)
            elif op.kind == "escape_time":
                kernels.escape_time(q, kernels.escape_time_params(**op.params), op.field.tensor())
            else:
                out = op.field.grid_tensor() if op.field is not None else None  # None: scatter-adds only
                kernels.pixel_program(q, op.program, [f.grid_tensor() for f in op.inputs], out, grid=op.grid)


_RNG = {}


def _rng_state():
    """The global generator state of ti.random (an int32 0-D field, made once)."""
    if "field" not in _RNG:
        _RNG["field"] = Field(i32, ())
    return _RNG["field"]


def _with_rng_advance(low, fdef, funcs, env):
    """low, followed (when one of its programs draws ti.random numbers) by a program adding 1 to
    the generator state, so that the next call draws other numbers."""
    if not any(getattr(op, "uses_rng", False) for op in low.ops()):
        return low
    env2 = dict(env)
    env2["__vdsl_rng"] = _rng_state()
    body = [ast.AugAssign(target=ast.Subscript(value=ast.Name(id="__vdsl_rng", ctx=ast.Load()), slice=ast.Constant(value=None),
                                               ctx=ast.Store()), op=ast.Add(), value=ast.Constant(value=1), lineno=0)]
    loop = ast.For(target=ast.Name(id="__vdsl_r", ctx=ast.Store()), iter=ast.Call(func=ast.Name(id="range", ctx=ast.Load()),
                   args=[ast.Constant(value=1)], keywords=[]), body=body, orelse=[], lineno=0)
    inc = lower_pixel_program(ast.FunctionDef(name=fdef.name, args=fdef.args, body=[loop], decorator_list=[], returns=None,
                                              type_comment=None), funcs, env2)
    out = Lowered("sequence", low.field, parts=[low, inc])
    out.ret = getattr(low, "ret", None)
    return out


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
        return self.text(4)

    def text(self, depth):
        """The expression as text, subexpressions below `depth` levels written as `...` (the tree
        shares subexpressions, so written out in full it can grow exponentially)."""
        if depth <= 0:
            return "..."
        return f"{self.op}({', '.join(a.text(depth - 1) if isinstance(a, Sym) else repr(a) for a in self.args)})"


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
            if isinstance(n.op, (ast.FloorDiv, ast.Mod)):  # of integers (extents, module constants)
                x, y = self.expr(n.left, local), self.expr(n.right, local)
                if not all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) for v in (x, y)) or y == 0:
                    raise TaichiLoweringError(f"{type(n.op).__name__} is supported here for integer constants only")
                return x // y if isinstance(n.op, ast.FloorDiv) else x % y
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
    if fld.width != 1:
        raise TaichiLoweringError("the escape-time op stores one value per pixel (a field of scalars)")
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
    """Lowers `kernel_name` of a Taichi program given as text, without running it, to the
    escape-time op: (field, vdsl_escape_time_params as a dict).  Module-level constants and fields
    are evaluated statically (literals, arithmetic, ti.field calls)."""
    kern, funcs, env = _parse_source(text, kernel_name, args)
    return lower_escape_time(kern, _FuncResolver(env, funcs), env)


def lower_source_kernel(text: str, kernel_name: str, args: dict, general: bool = False) -> "Lowered":
    """As lower_source, by either path (escape-time op, else the general per-pixel program);
    general=True takes the general path even for bodies of the escape-time form."""
    kern, funcs, env = _parse_source(text, kernel_name, args)
    return lower_kernel(kern, _FuncResolver(env, funcs), env, general=general)


def _parse_source(text: str, kernel_name: str, args: dict):
    mod = ast.parse(text)
    env = {"float": float, "int": int}
    tinames = set()
    import sys as _sys
    for st in mod.body:
        if isinstance(st, ast.Import):
            for a in st.names:
                if a.name == "taichi":
                    tinames.add(a.asname or "taichi")
                elif a.name == "taichi.math" and a.asname:
                    env[a.asname] = math
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
                is_vec = isinstance(v.func.value, ast.Attribute) and v.func.value.attr == "Vector"
                is_mat = isinstance(v.func.value, ast.Attribute) and v.func.value.attr == "Matrix"
                pos = list(v.args)
                width, mat = 1, None
                if is_vec:  # ti.Vector.field(n, dtype, shape)
                    width = interp.expr(kw["n"] if "n" in kw else pos.pop(0), {})
                elif is_mat:  # ti.Matrix.field(n, m, dtype, shape)
                    mat = (interp.expr(kw["n"] if "n" in kw else pos.pop(0), {}),
                           interp.expr(kw["m"] if "m" in kw else pos.pop(0), {}))
                    width = mat[0] * mat[1]
                elif "n" in kw:
                    raise TaichiLoweringError("ti.field takes no component count")
                if "dtype" not in kw and pos:  # ti.field(dtype, shape)
                    kw["dtype"] = pos.pop(0)
                if "shape" not in kw and pos:
                    kw["shape"] = pos.pop(0)
                shape = interp.expr(kw["shape"], {})
                dt = kw.get("dtype")
                dtype = f32 if dt is None or (isinstance(dt, ast.Name) and dt.id == "float") else (
                    i32 if (isinstance(dt, ast.Name) and dt.id == "int") or getattr(dt, "attr", "") in ("i32", "int32") else f32)
                env[st.targets[0].id] = Field(dtype, shape, width=int(width), mat=mat)
            elif (isinstance(v, ast.Call) and isinstance(v.func, ast.Attribute) and v.func.attr == "vector"
                  and isinstance(v.func.value, ast.Attribute) and v.func.value.attr == "types" and v.args):
                env[st.targets[0].id] = _VectorType(interp.expr(v.args[0], {}))  # vec3 = ti.types.vector(3, float)
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
    return kern, funcs, env


# math helpers programs sometimes use at module level
pi = _pymath.pi

# ti.math (also importable as taichi.math under the runner): names only; inside kernels the
# lowering interprets the calls (vec2-4, clamp, mix, smoothstep, length, normalize, dot, cross,
# fract, sign, step and the scalar functions).
math = _pytypes.ModuleType("taichi.math")
math.pi = _pymath.pi
math.e = _pymath.e
for _name in ("vec2", "vec3", "vec4", "clamp", "mix", "smoothstep", "length", "normalize", "dot", "cross", "fract",
              "sign", "step", "sqrt", "exp", "log", "sin", "cos", "tanh", "floor", "ceil", "min", "max", "mod", "log2",
              "atan2", "asin", "acos", "atan", "tan", "pow", "round"):
    setattr(math, _name, _name)  # placeholders: only meaningful inside kernels


class _VectorType:
    """ti.types.vector(n, dtype) / ti.math.vec2-4: inside kernels a constructor of n-vectors
    (one scalar fills every component; vectors and scalars are laid out in order)."""
    def __init__(self, n, dtype=float):
        self.n, self.dtype = int(n), dtype


def _matrix_type(n, m, dtype=float):
    raise TaichiLoweringError("ti.types.matrix is not supported; use ti.Matrix values")


types = _pytypes.ModuleType("taichi.types")  # ti.types
types.vector = _VectorType
types.matrix = _matrix_type
for _name in ("reflect", "isnan", "isinf"):
    setattr(math, _name, _name)


def ndrange(*extents):
    """ti.ndrange(W, H): the index space of a struct-for that is not over a field."""
    return tuple(int(e) for e in extents)


def static(v):
    """ti.static(range(N)): a loop unrolled when the kernel is lowered."""
    return v


def template():
    return None


# ---- the general path: any struct-for body as a per-pixel register program ---------------------------
class Lowered:
    """A lowered kernel: kind "escape_time" (field, params for vdsl_op_escape_time),
    "pixel_program" (field, program for vdsl_op_pixel_program, input fields it reads or
    scatter-adds into, grid: its [ni][nj]; field None for a program of scatter-adds alone), "copy"
    (field = a copy of inputs[0]), or "sequence" (parts: Lowered ops run in order; a kernel of
    several struct-fors, or a struct-for storing several fields)."""

    def __init__(self, kind, field, params=None, program=None, inputs=(), parts=()):
        self.kind, self.field, self.params, self.program, self.inputs = kind, field, params, program, list(inputs)
        self.parts = list(parts)
        self.reads = list(inputs)  # the input fields a pixel program loads
        self.grid = None

    def ops(self):
        """The escape-time and pixel-program ops this kernel runs, in order."""
        return [o for p in self.parts for o in p.ops()] if self.kind == "sequence" else [self]

    def substitute(self, old, new):
        """Reads field `new` wherever this program read `old` (same type and shape)."""
        self.inputs = [new if f is old else f for f in self.inputs]
        self.reads = [new if f is old else f for f in self.reads]


def lower_kernel(fdef: ast.FunctionDef, funcs, env, general: bool = False) -> Lowered:
    """Each top-level struct-for of the kernel, in order (a Taichi kernel runs them one after
    another, each a parallel loop): the escape-time op for bodies of that form (its hand-tuned
    kernel; not when general), else the general per-pixel program(s); TaichiLoweringError when
    neither lowers one."""
    body = [s for s in fdef.body if not (isinstance(s, ast.Expr) and isinstance(s.value, ast.Constant))]
    if any(not isinstance(s, ast.For) for s in body) and len(body) > 1:
        return _lower_with_reducers(fdef, body, funcs, env, general)
    if len(body) > 1 and all(isinstance(s, ast.For) for s in body):
        parts = []
        for loop in body:
            sub = ast.FunctionDef(name=fdef.name, args=fdef.args, body=[loop], decorator_list=[], returns=None,
                                  type_comment=None)
            parts.append(lower_kernel(sub, funcs, env, general))
        return Lowered("sequence", parts[0].field, parts=parts)
    if general:
        return lower_pixel_program(fdef, funcs, env)
    try:
        fld, params = lower_escape_time(fdef, funcs, env)
        return Lowered("escape_time", fld, params=params)
    except TaichiLoweringError as e1:
        try:
            return lower_pixel_program(fdef, funcs, env)
        except TaichiLoweringError as e2:
            raise TaichiLoweringError(f"{e2} (and not of the escape-time form: {e1})") from None


def _lower_with_reducers(fdef, body, funcs, env, general):
    """A kernel body with kernel-scope scalars around its struct-fors, Taichi's reduction idiom:

        e = 0.0
        for i in x:
            e += f(x[i])          (+= / -= only: Taichi makes them atomic adds)
        return e

    Each such scalar becomes a hidden 0-D field: one store of its initial value, then
    scatter-adds at a constant index (summed per block), and `return` names the field whose
    value the call returns (Lowered.ret)."""
    env2 = dict(env)
    fields, loops, ret = {}, [], None
    interp = _PixInterp(env, funcs, None, None, "_", None)

    class Use(ast.NodeTransformer):  # a kernel-scope name inside a loop: its hidden field's element
        def visit_Name(self, nd):
            if nd.id in fields:
                return ast.copy_location(ast.Subscript(value=ast.Name(id=fields[nd.id][0], ctx=ast.Load()),
                                                       slice=ast.Constant(value=None), ctx=nd.ctx), nd)
            return nd

    for k, st in enumerate(body):
        if isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Name) \
                and not any(isinstance(s2, ast.For) for s2 in body[:k]):
            try:
                v = interp.expr(st.value, {})
            except (TaichiLoweringError, TypeError, AttributeError):
                v = None
            if not _is_num(v):
                raise TaichiLoweringError("a kernel-scope variable starts from a constant")
            nm = st.targets[0].id
            hidden = f"__vdsl_red_{nm}"
            fld = Field(i32 if isinstance(v, (int, np.integer)) and not isinstance(v, bool) else f32, ())
            env2[hidden] = fld
            fields[nm] = (hidden, fld)
            init = ast.For(target=ast.Name(id="__vdsl_r", ctx=ast.Store()), iter=ast.Call(
                func=ast.Name(id="range", ctx=ast.Load()), args=[ast.Constant(value=1)], keywords=[]), orelse=[],
                lineno=0, body=[ast.Assign(targets=[ast.Subscript(value=ast.Name(id=hidden, ctx=ast.Load()),
                                                                  slice=ast.Constant(value=None), ctx=ast.Store())],
                                           value=ast.Constant(value=v.item() if hasattr(v, "item") else v), lineno=0)])
            loops.append(init)
        elif isinstance(st, ast.For):
            loops.append(Use().visit(copy.deepcopy(st)))
        elif isinstance(st, ast.Return) and st is body[-1] and isinstance(st.value, ast.Name) and st.value.id in fields:
            ret = fields[st.value.id][1]
        else:
            raise TaichiLoweringError(f"statement at line {getattr(st, 'lineno', '?')} of the kernel body: a kernel holds "
                                      "struct-fors, kernel-scope scalars set to constants before them, and `return name`")
    if not loops:
        raise TaichiLoweringError("the kernel has no struct-for")
    parts = []
    for loop in loops:
        sub = ast.FunctionDef(name=fdef.name, args=fdef.args, body=[loop], decorator_list=[], returns=None, type_comment=None)
        parts.append(lower_kernel(sub, funcs, env2, general))
    low = Lowered("sequence", parts[0].field, parts=parts)
    low.ret = ret
    return low


class _PVec:
    """A small vector (ti.Vector) of per-pixel values: numbers or pixprog Nodes."""

    def __init__(self, comps):
        self.comps = list(comps)


class _PMat:
    """A small matrix (ti.Matrix) of per-pixel values, as rows of numbers or pixprog Nodes."""

    def __init__(self, rows):
        self.rows = [list(r) for r in rows]
        if not self.rows or any(len(r) != len(self.rows[0]) for r in self.rows) or not self.rows[0]:
            raise TaichiLoweringError("a matrix has rows of one length")

    @property
    def shape(self):
        return len(self.rows), len(self.rows[0])

    def flat(self):
        return [x for r in self.rows for x in r]

    @staticmethod
    def of(flat, n, m):
        return _PMat([flat[i * m:(i + 1) * m] for i in range(n)])


_BIT_OPS = {ast.BitAnd: "band", ast.BitOr: "bor", ast.BitXor: "bxor", ast.LShift: "shl", ast.RShift: "shr"}
_UNARY_FUNCS = {"sqrt": "sqrt", "exp": "exp", "log": "log", "sin": "sin", "cos": "cos", "tanh": "tanh", "abs": "abs",
                "floor": "floor", "asin": "asin", "acos": "acos", "atan": "atan", "tan": "tan", "round": "round"}
def _skey(fld):
    """The local-scope key of the value the body has stored to fld[i, j] (read back by a later read
    of fld[i, j] in the same body)."""
    return ("__store__", id(fld))


def _is_skey(k):
    return isinstance(k, tuple) and len(k) == 2 and k[0] == "__store__"
_MATH_FUNCS = ("vec2", "vec3", "vec4", "clamp", "mix", "smoothstep", "length", "normalize", "dot", "cross", "fract",
               "step", "sign")


class _PixInterp:
    """Evaluates a struct-for body over numbers (folded in f32 as Taichi's default float, ints
    kept exact), pixprog Nodes and _PVec vectors."""

    def __init__(self, env, funcs, b, fld, iname, jname, kname=None):
        from . import pixprog
        self.pp = pixprog
        self.env, self.funcs, self.b = env, funcs, b
        self.fld, self.iname, self.jname = fld, iname, jname
        # the struct-for's indices: one (1-D), two (2-D) or three (3-D)
        self.names = [iname] if jname is None else [iname, jname] if kname is None else [iname, jname, kname]
        self.stored = []  # fields the body stores to at [i, j], in the order of their first store
        self.fields = {}  # id -> Field, for the store keys
        self.shape = fld.shape if isinstance(fld, Field) else None  # the struct-for's index space
        self.inputs = []  # Fields read at [i, j], in LOAD order
        self.in_extents = []  # per input: None (the struct-for's grid), or its own grid (rows, cols)
        self.bools = set()  # ids of Nodes known to hold 1.0 / 0.0 (comparisons and their logic)
        # ids of Nodes known to hold integers (the indices and +, -, *, %, // of them and of integer
        # constants) -> a bound on their magnitude.  The program computes in f32 registers, where
        # integers are exact up to 2^24: an integer expression that may go beyond is refused, since
        # Taichi evaluates it in int32 and the results would differ.
        self.ibound = {}
        self.in_loop = False
        self.unroll = True  # unroll short range loops whose variable is read (False: keep them loops)
        self.targets = []  # fields the body scatter-adds into (also in inputs, never read)
        self.scatters = []  # their adds (pixprog scatter_add effects), in program order
        self.pred = None  # inside if branches: the condition under which a statement runs
        self.rng, self.draws = False, {}  # ti.random: used; draws met per call site

    # -- values
    def node(self, v):
        if isinstance(v, self.pp.Node):
            return v
        if _is_num(v):
            return self.b.const(_f32(v))
        raise TaichiLoweringError(f"{v!r} is not a per-pixel scalar")

    _INT_EXACT = 1 << 24

    def _ib(self, v):
        """Magnitude bound of an integer value (a Python int or a tracked Node), else None."""
        if isinstance(v, (int, np.integer)) and not isinstance(v, bool):
            return abs(int(v))
        return self.ibound.get(id(v)) if isinstance(v, self.pp.Node) else None

    def _int_result(self, r, bound, what):
        if bound is not None and isinstance(r, self.pp.Node):
            if bound > self._INT_EXACT:
                raise TaichiLoweringError(
                    f"integer expression ({what}) may reach {bound}, beyond 2^24: per-pixel programs compute in f32, "
                    "where integers are exact only up to 2^24, while Taichi computes it in int32")
            self.ibound[id(r)] = bound
        return r

    def arith(self, op, x, y):
        r = self._arith(op, x, y)
        bx, by = self._ib(x), self._ib(y)
        if bx is not None and by is not None and op in ("add", "sub", "mul"):
            return self._int_result(r, bx * by if op == "mul" else bx + by, op)
        return r

    def _arith(self, op, x, y):
        if isinstance(x, _PMat) or isinstance(y, _PMat):
            # element by element (Taichi's * of two matrices is too; @ is the product)
            if isinstance(x, _PVec) or isinstance(y, _PVec):
                raise TaichiLoweringError("a matrix and a vector combine with @, not element by element")
            if isinstance(x, _PMat) and isinstance(y, _PMat) and x.shape != y.shape:
                raise TaichiLoweringError(f"matrix shapes {x.shape} and {y.shape} differ")
            n, m = (x if isinstance(x, _PMat) else y).shape
            xf = x.flat() if isinstance(x, _PMat) else [x] * (n * m)
            yf = y.flat() if isinstance(y, _PMat) else [y] * (n * m)
            return _PMat.of([self.arith(op, a, c) for a, c in zip(xf, yf)], n, m)
        if isinstance(x, _PVec) or isinstance(y, _PVec):
            xs = x.comps if isinstance(x, _PVec) else None
            ys = y.comps if isinstance(y, _PVec) else None
            if xs is not None and ys is not None and len(xs) != len(ys):
                raise TaichiLoweringError("vector length mismatch")
            n = len(xs if xs is not None else ys)
            return _PVec([self.arith(op, xs[k] if xs is not None else x, ys[k] if ys is not None else y) for k in range(n)])
        if _is_num(x) and _is_num(y):
            if op == "pow":
                return _binop("pow", x, y)
            return _binop(op, x, y)
        if op == "pow":
            if not (isinstance(y, (int, np.integer)) and 1 <= int(y) <= 8):
                return self.b.op("powf", self.node(x), self.node(y))  # the math library's powf
            r = x
            for _ in range(int(y) - 1):
                r = self.b.op("mul", self.node(r), self.node(x))
            return r
        return self.b.op(op, self.node(x), self.node(y))

    def unary(self, fn, x):
        if isinstance(x, _PVec):
            return _PVec([self.unary(fn, c) for c in x.comps])
        if isinstance(x, _PMat):
            return _PMat.of([self.unary(fn, c) for c in x.flat()], *x.shape)
        if isinstance(x, (int, np.integer)) and not isinstance(x, bool) and fn in ("neg", "abs"):
            return -int(x) if fn == "neg" else abs(int(x))  # integers stay exact integers
        if _is_num(x):
            v = np.float32(x)
            with np.errstate(all="ignore"):
                return {"neg": -v, "abs": np.abs(v), "sqrt": np.sqrt(v), "exp": np.exp(v), "log": np.log(v), "sin": np.sin(v),
                        "cos": np.cos(v), "tanh": np.tanh(v), "floor": np.floor(v), "trunc": np.trunc(v),
                        "asin": np.arcsin(v), "acos": np.arccos(v), "atan": np.arctan(v), "tan": np.tan(v),
                        "recip": np.float32(1.0) / v,
                        "round": np.float32(np.copysign(np.floor(np.abs(np.float64(v)) + 0.5), v))}[fn]
        r = self.b.op(fn, x)
        bx = self._ib(x)
        return self._int_result(r, bx, fn) if fn in ("neg", "abs", "floor", "round") and bx is not None else r

    def matmul(self, a, c):
        """a @ c for matrices and vectors (a vector is a column, or a row on the left): each
        element a[i][0] c[0][j] + a[i][1] c[1][j] + ..., summed in that order."""
        def rows(v, left):
            if isinstance(v, _PMat):
                return v.rows
            if isinstance(v, _PVec):
                return [list(v.comps)] if left else [[x] for x in v.comps]
            raise TaichiLoweringError("@ takes matrices and vectors")
        ra, rc = rows(a, True), rows(c, False)
        if len(ra[0]) != len(rc):
            raise TaichiLoweringError(f"@ of a {len(ra)} x {len(ra[0])} and a {len(rc)} x {len(rc[0])} operand")
        out = []
        for i in range(len(ra)):
            row = []
            for j in range(len(rc[0])):
                acc = self.arith("mul", ra[i][0], rc[0][j])
                for k in range(1, len(rc)):
                    acc = self.arith("add", acc, self.arith("mul", ra[i][k], rc[k][j]))
                row.append(acc)
            out.append(row)
        if isinstance(c, _PVec):
            return _PVec([r[0] for r in out])
        if isinstance(a, _PVec):
            return _PVec(out[0])
        return _PMat(out)

    def mat_method(self, mat, name, args):
        n, m = mat.shape
        if name == "transpose":
            return _PMat([[mat.rows[i][j] for i in range(n)] for j in range(m)])
        if name == "trace":
            if n != m:
                raise TaichiLoweringError("trace of a square matrix")
            acc = mat.rows[0][0]
            for i in range(1, n):
                acc = self.arith("add", acc, mat.rows[i][i])
            return acc
        if name == "determinant":
            r = mat.rows
            if (n, m) == (1, 1):
                return r[0][0]
            if (n, m) == (2, 2):
                return self.arith("sub", self.arith("mul", r[0][0], r[1][1]), self.arith("mul", r[0][1], r[1][0]))
            if (n, m) == (3, 3):
                def minor(a, b, c, d):
                    return self.arith("sub", self.arith("mul", a, d), self.arith("mul", b, c))
                t0 = self.arith("mul", r[0][0], minor(r[1][1], r[1][2], r[2][1], r[2][2]))
                t1 = self.arith("mul", r[0][1], minor(r[1][0], r[1][2], r[2][0], r[2][2]))
                t2 = self.arith("mul", r[0][2], minor(r[1][0], r[1][1], r[2][0], r[2][1]))
                return self.arith("add", self.arith("sub", t0, t1), t2)
            raise TaichiLoweringError("determinant of a 1 x 1, 2 x 2 or 3 x 3 matrix")
        if name in ("norm", "norm_sqr"):
            f = _PVec(mat.flat())
            return self.dot(f, f) if name == "norm_sqr" else self.unary("sqrt", self.dot(f, f))
        raise TaichiLoweringError(f"matrix method {name!r} is not supported")

    def dot(self, a, c):
        if not (isinstance(a, _PVec) and isinstance(c, _PVec) and len(a.comps) == len(c.comps)):
            raise TaichiLoweringError("dot needs two vectors of one length")
        acc = self.arith("mul", a.comps[0], c.comps[0])
        for x, y in zip(a.comps[1:], c.comps[1:]):
            acc = self.arith("add", acc, self.arith("mul", x, y))
        return acc

    # -- expressions
    def expr(self, n, local):
        if isinstance(n, ast.Constant):
            if isinstance(n.value, bool):  # True / False are the integers 1 / 0, as in Taichi
                return int(n.value)
            if not isinstance(n.value, (int, float)):
                raise TaichiLoweringError(f"constant {n.value!r} is not a number")
            return n.value
        if isinstance(n, ast.Name):
            if n.id in local:
                v = local[n.id]
                if v is _UNREADABLE:
                    raise TaichiLoweringError(f"{n.id!r} can only be read after the loop (the loop counter)")
                if v is _ONE_BRANCH:
                    raise TaichiLoweringError(f"{n.id!r} is assigned in one branch of an if only")
                return v
            if n.id in self.env:
                return self.env[n.id]
            if n.id in _BUILTINS:  # int / float as values (a .cast(int) argument)
                return _BUILTINS[n.id]
            raise TaichiLoweringError(f"unknown name {n.id!r}")
        if isinstance(n, ast.BinOp):
            ops = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div", ast.Pow: "pow"}
            x, y = self.expr(n.left, local), self.expr(n.right, local)
            if isinstance(n.op, (ast.Mod, ast.FloorDiv)):
                return self.floor_op(type(n.op) is ast.Mod, x, y)
            if isinstance(n.op, ast.MatMult):
                return self.matmul(x, y)
            if type(n.op) in _BIT_OPS:
                return self.bit_op(_BIT_OPS[type(n.op)], x, y)
            if type(n.op) not in ops:
                raise TaichiLoweringError(f"operator {type(n.op).__name__} is not supported")
            return self.arith(ops[type(n.op)], x, y)
        if isinstance(n, ast.UnaryOp):
            v = self.expr(n.operand, local)
            if isinstance(n.op, ast.USub):
                return self.unary("neg", v)
            if isinstance(n.op, ast.Invert):  # ~x = -x - 1 of an integer
                if isinstance(v, (int, np.integer)) and not isinstance(v, bool):
                    return ~int(v)
                if self._ib(v) is None:
                    raise TaichiLoweringError("~ takes integers of a known bound")
                return self.arith("sub", self.unary("neg", v), 1)
            if isinstance(n.op, ast.UAdd):
                return v
            if isinstance(n.op, ast.Not):
                return self.logic_not(v)
            raise TaichiLoweringError(f"unary {type(n.op).__name__} is not supported")
        if isinstance(n, ast.Compare):
            return self.compare(n, local)
        if isinstance(n, ast.BoolOp):
            vals = [self.expr(v, local) for v in n.values]
            return self.logic("and" if isinstance(n.op, ast.And) else "or", vals)
        if isinstance(n, ast.IfExp):
            return self.select(self.expr(n.test, local), self.expr(n.body, local), self.expr(n.orelse, local))
        if isinstance(n, ast.Subscript):
            base = self.expr(n.value, local)
            if isinstance(base, Field):
                return self.field_read(base, n.slice, local)
            idx = self.expr(n.slice, local)
            if isinstance(base, _PVec) and isinstance(idx, (int, np.integer)) and -len(base.comps) <= idx < len(base.comps):
                return base.comps[int(idx)]
            if isinstance(base, list) and isinstance(idx, (int, np.integer)) and -len(base) <= idx < len(base):
                return base[int(idx)]  # a Python list of values (w[i] of a list of weight vectors)
            if isinstance(base, _PMat) and isinstance(idx, list) and len(idx) == 2 and \
                    all(isinstance(k, (int, np.integer)) for k in idx):
                return base.rows[int(idx[0])][int(idx[1])]
            raise TaichiLoweringError("only constant vector indexing and field[i, j] reads are supported")
        if isinstance(n, ast.Attribute):
            base = self.expr(n.value, local)
            if isinstance(base, _PVec) and n.attr == "n":
                return len(base.comps)
            if isinstance(base, _PVec) and 1 <= len(n.attr) <= 4 and \
                    (set(n.attr) <= set("xyzw") or set(n.attr) <= set("rgba")):
                names = "xyzw" if set(n.attr) <= set("xyzw") else "rgba"
                ks = [names.index(ch) for ch in n.attr]
                if max(ks) >= len(base.comps):
                    raise TaichiLoweringError(f"vector has no component {n.attr!r}")
                return base.comps[ks[0]] if len(ks) == 1 else _PVec([base.comps[k] for k in ks])
            if isinstance(base, (_PVec, self.pp.Node)):
                return (base, n.attr)
            return getattr(base, n.attr)
        if isinstance(n, (ast.List, ast.Tuple)):
            return [self.expr(e, local) for e in n.elts]
        if isinstance(n, ast.Call):
            return self.call(n, local)
        raise TaichiLoweringError(f"expression {ast.dump(n)[:60]} is not supported")

    def _elts(self, idx):
        """The index expressions of a subscript: field[i, j] of a 2-D struct-for, field[i] of a 1-D one."""
        elts = list(idx.elts) if isinstance(idx, ast.Tuple) else [idx]
        if len(elts) != len(self.names):
            raise TaichiLoweringError(f"fields of this struct-for are {len(self.names)}-D: index them as "
                                      f"field[{', '.join(self.names)}]")
        return elts

    def _is_here(self, idx):
        return [getattr(e, "id", None) for e in self._elts(idx)] == self.names

    def _at_here(self, fld, idx):
        """fld[idx] is this pixel's element of a field of the struct-for's shape."""
        elts = list(idx.elts) if isinstance(idx, ast.Tuple) else [idx]
        return tuple(fld.shape) == tuple(self.shape) and [getattr(e, "id", None) for e in elts] == self.names

    def _here(self):
        """The subscript of this pixel: (i, j), i, or (i, j, k)."""
        if len(self.names) == 1:
            return ast.Name(id=self.iname, ctx=ast.Load())
        return ast.Tuple(elts=[ast.Name(id=n, ctx=ast.Load()) for n in self.names], ctx=ast.Load())

    def field_read(self, fld, idx, local):
        """fld[idx] as _field_read gives it; a field of matrices as a matrix."""
        v = self._field_read(fld, idx, local)
        if fld.mat and isinstance(v, _PVec):
            return _PMat.of(v.comps, *fld.mat)
        return v

    def _field_read(self, fld, idx, local):
        """fld[i, j] (this pixel), or fld[e1, e2] at per-pixel indices (a stencil or gather read,
        clamped to the field, whose shape must be the struct-for's); fld[i] / fld[e] in a 1-D
        struct-for, which runs as one row (row index 0)."""
        if fld in self.targets:
            raise TaichiLoweringError("a field scatter-added into is also read in the same struct-for")
        own = tuple(fld.shape) != tuple(self.shape)  # a field of another shape: gathered in its own grid
        elts = list(idx.elts) if isinstance(idx, ast.Tuple) else [idx]
        here = not own and [getattr(e, "id", None) for e in elts] == self.names
        if here and _skey(fld) in local:
            return local[_skey(fld)]  # the value this pixel stored earlier in the body
        if fld not in self.inputs:
            if len(self.inputs) == self.pp.MAX_INPUTS:
                raise TaichiLoweringError(f"at most {self.pp.MAX_INPUTS} fields can be read")
            self.inputs.append(fld)
            self.in_extents.append(_grid_of(fld.shape) if own else None)
        k = self.inputs.index(fld)
        if here:
            if fld.width == 1:
                return self.b.load(k)
            return _PVec([self.b.load(k, c) for c in range(fld.width)])
        vals = self._index_values(fld, idx, local)
        if len(vals) == 0:  # a 0-D field
            row, col = 0.0, 0.0
        elif len(vals) == 1:
            row, col = 0.0, vals[0]
        elif len(vals) == 3:
            # [A][B][C] runs as [A B][C]: the row A-index * B + B-index, each clamped to its own
            # axis and truncated first (so an index past one axis does not run into the next)
            a, b2, col = vals

            def axis(v, n):
                return self.unary("floor", self.minmax("min", [self.minmax("max", [v, 0.0]), float(n - 1)]))
            row = self.arith("add", self.arith("mul", axis(a, fld.shape[0]), float(fld.shape[1])), axis(b2, fld.shape[1]))
        else:
            row, col = vals
        row, col = self.node(row), self.node(col)
        if fld.width == 1:
            return self.b.load_at(k, row, col)
        return _PVec([self.b.load_at(k, row, col, c) for c in range(fld.width)])

    def call(self, n, local):
        f = n.func
        if isinstance(f, ast.Attribute):
            base = self.expr(f.value, local)
            if isinstance(base, _PVec):
                if f.attr == "norm":
                    return self.unary("sqrt", self.dot(base, base))
                if f.attr == "norm_sqr":
                    return self.dot(base, base)
                if f.attr == "dot":
                    return self.dot(base, self.expr(n.args[0], local))
                if f.attr == "normalized":
                    return self.normalize(base)
                if f.attr == "sum":  # ((c0 + c1) + c2) + ...
                    acc = base.comps[0]
                    for c in base.comps[1:]:
                        acc = self.arith("add", acc, c)
                    return acc
                if f.attr in ("max", "min"):
                    return self.minmax(f.attr, list(base.comps))
                if f.attr == "cross":
                    return self.cross(base, self.expr(n.args[0], local))
                if f.attr == "cast":
                    return self.cast(base, self.expr(n.args[0], local))
                if f.attr == "outer_product":
                    c = self.expr(n.args[0], local)
                    if not isinstance(c, _PVec):
                        raise TaichiLoweringError("outer_product takes a vector")
                    return _PMat([[self.arith("mul", a, d) for d in c.comps] for a in base.comps])
                raise TaichiLoweringError(f"vector method {f.attr!r} is not supported")
            if isinstance(base, _PMat):
                if f.attr == "cast":
                    return self.cast(base, self.expr(n.args[0], local))
                return self.mat_method(base, f.attr, [self.expr(a, local) for a in n.args])
            if base is Matrix or base is Vector:  # ti.Matrix.zero / identity, ti.Vector.zero / one
                vals = [self.expr(a, local) for a in n.args[1:]]
                if not all(isinstance(v, (int, np.integer)) for v in vals):
                    raise TaichiLoweringError(f"ti.{base.__name__}.{f.attr} takes (dtype, sizes)")
                if base is Vector and f.attr in ("zero", "one") and len(vals) == 1:
                    return _PVec([0.0 if f.attr == "zero" else 1.0] * int(vals[0]))
                if base is Matrix and f.attr == "zero" and len(vals) == 2:
                    return _PMat([[0.0] * int(vals[1]) for _ in range(int(vals[0]))])
                if base is Matrix and f.attr == "identity" and len(vals) == 1:
                    k = int(vals[0])
                    return _PMat([[1.0 if i == j else 0.0 for j in range(k)] for i in range(k)])
                raise TaichiLoweringError(f"ti.{base.__name__}.{f.attr} is not supported")
            if f.attr == "Matrix":
                rows = self.expr(n.args[0], local)
                if not isinstance(rows, list) or not all(isinstance(r, (list, _PVec)) for r in rows):
                    raise TaichiLoweringError("ti.Matrix takes a list of rows")
                return _PMat([r.comps if isinstance(r, _PVec) else r for r in rows])
            if f.attr == "Vector":
                comps = self.expr(n.args[0], local)
                if not isinstance(comps, list) or any(isinstance(c, _PVec) for c in comps):
                    raise TaichiLoweringError("ti.Vector takes a list of scalars")
                return _PVec(comps)
            if f.attr in _UNARY_FUNCS:
                return self.unary(_UNARY_FUNCS[f.attr], self.expr(n.args[0], local))
            if f.attr == "select":
                if len(n.args) != 3:
                    raise TaichiLoweringError("ti.select takes (condition, if_true, if_false)")
                return self.select(*[self.expr(a, local) for a in n.args])
            if f.attr in _MATH_FUNCS:
                return self.math_call(f.attr, [self.expr(a, local) for a in n.args])
            if f.attr == "ceil":
                return self.unary("neg", self.unary("floor", self.unary("neg", self.expr(n.args[0], local))))
            if f.attr in ("max", "min"):
                return self.minmax(f.attr, [self.expr(a, local) for a in n.args])
            if f.attr == "cast":
                if len(n.args) != 2:
                    raise TaichiLoweringError("ti.cast takes (value, dtype)")
                return self.cast(self.expr(n.args[0], local), self.expr(n.args[1], local))
            if f.attr in ("atomic_add", "atomic_sub", "atomic_max", "atomic_min"):
                raise TaichiLoweringError(f"ti.{f.attr} is supported as a statement (its old value is not returned)")
            if f.attr == "random":
                return self.random(n, local)
            if f.attr in ("f32", "float32") and len(n.args) == 1:
                v = self.expr(n.args[0], local)
                return _f32(v) if _is_num(v) else v
            if f.attr in ("i32", "int32") and len(n.args) == 1:
                return self.cast(self.expr(n.args[0], local), int)
            if f.attr == "reflect" and len(n.args) == 2:  # x - 2 dot(n, x) n
                x, nn = (self.expr(a, local) for a in n.args)
                return self.arith("sub", x, self.arith("mul", self.arith("mul", 2.0, self.dot(nn, x)), nn))
            if f.attr in ("isnan", "isinf") and len(n.args) == 1:
                def test(v):
                    if _is_num(v):
                        return int(np.isnan(_f32(v)) if f.attr == "isnan" else np.isinf(_f32(v)))
                    if f.attr == "isnan":
                        return self.b.op("ne", v, v)
                    return self.b.op("eq", self.b.op("abs", v), float("inf"))
                return self.elementwise(test, self.expr(n.args[0], local))
            if f.attr == "static" and len(n.args) == 1:  # `if ti.static(cond):` decided when lowering
                return self.expr(n.args[0], local)
            if f.attr == "rsqrt" and len(n.args) == 1:  # 1 / sqrt(x), both exactly rounded
                return self.unary("recip", self.unary("sqrt", self.expr(n.args[0], local)))
            if f.attr == "log2" and len(n.args) == 1:  # log(x) / ln 2
                return self.arith("mul", self.unary("log", self.expr(n.args[0], local)), _f32(1.0 / _pymath.log(2.0)))
            if f.attr == "mod" and len(n.args) == 2:  # taichi.math.mod: x - y floor(x / y), GLSL's mod
                x, y = (self.expr(a, local) for a in n.args)
                return self.arith("sub", x, self.arith("mul", y, self.unary("floor", self.arith("div", x, y))))
            if f.attr in ("atan2", "pow"):
                if len(n.args) != 2:
                    raise TaichiLoweringError(f"ti.{f.attr} takes two values")
                kind = "atan2" if f.attr == "atan2" else "powf"
                x, y = (self.expr(a, local) for a in n.args)

                def fn2(a, c):
                    if _is_num(a) and _is_num(c):
                        with np.errstate(all="ignore"):
                            return (np.arctan2 if kind == "atan2" else np.power)(_f32(a), _f32(c))
                    return self.b.op(kind, self.node(a), self.node(c))
                return self.elementwise(fn2, x, y)
            raise TaichiLoweringError(f"call {f.attr!r} is not supported")
        if isinstance(f, ast.Name):
            fdef = self.funcs.get(f.id)
            if fdef is None:
                obj = self.env.get(f.id, _BUILTINS.get(f.id))
                if obj is abs:
                    return self.unary("abs", self.expr(n.args[0], local))
                if obj in (max, min):
                    return self.minmax(obj.__name__, [self.expr(a, local) for a in n.args])
                if obj is float:
                    v = self.expr(n.args[0], local)
                    return _f32(v) if _is_num(v) else v
                if obj is int:
                    return self.cast(self.expr(n.args[0], local), int)
                if isinstance(obj, _VectorType):
                    vals = [self.expr(a, local) for a in n.args]
                    if len(vals) == 1 and not isinstance(vals[0], (_PVec, list)):
                        return _PVec([vals[0]] * obj.n)
                    comps = [c for v in vals for c in (v.comps if isinstance(v, _PVec) else v if isinstance(v, list) else [v])]
                    if len(comps) != obj.n:
                        raise TaichiLoweringError(f"a {obj.n}-vector made of {len(comps)} components")
                    return _PVec(comps)
                raise TaichiLoweringError(f"call of {f.id!r}: only @ti.func functions are inlined")
            args = [self.expr(a, local) for a in n.args]
            # the function's own scope, sharing the caller's view of the fields it has stored
            sub = {k: v for k, v in local.items() if _is_skey(k)}
            sub.update(zip([a.arg for a in fdef.args.args], args))
            body = [st for st in fdef.body if not (isinstance(st, ast.Expr) and isinstance(st.value, ast.Constant))]
            if any(isinstance(nd, ast.Return) for st in body[:-1] for nd in ast.walk(st)) or \
                    any(isinstance(nd, ast.Return) for st in body[-1:] if not isinstance(st, ast.Return) for nd in ast.walk(st)):
                raise TaichiLoweringError(f"@ti.func {f.id!r}: a return must be its last statement")
            for st in body:
                if isinstance(st, ast.Return):
                    for k, v in sub.items():
                        if _is_skey(k):
                            local[k] = v
                    return self.expr(st.value, sub) if st.value is not None else None
                if not self.assign(st, sub):
                    raise TaichiLoweringError(f"statement at line {getattr(st, 'lineno', '?')} in @ti.func {f.id!r} "
                                              "is not supported")
            for k, v in sub.items():
                if _is_skey(k):
                    local[k] = v
            return None
        raise TaichiLoweringError("unsupported call")

    def random(self, n, local):
        """ti.random() / ti.random(float): a uniform number in [0, 1), a function of the global
        generator state (a hidden 0-D field, advanced once per kernel call), this pixel and the
        draw: the call's place in the source and how often the lowering has met it (static loops
        unroll one call into several draws)."""
        if n.args:
            dt = self.expr(n.args[0], local)
            if dt not in (float, f32):
                raise TaichiLoweringError("ti.random gives f32 numbers here (ti.random() or ti.random(float))")
        site = (getattr(n, "lineno", 0) % 4096) * 64 + getattr(n, "col_offset", 0) % 64
        occ = self.draws.get(site, 0)
        self.draws[site] = occ + 1
        seed = self._field_read(_rng_state(), ast.Constant(value=None), local)
        self.rng = True
        return self.b.random(seed, site * 64 + occ % 64)

    def cast(self, v, dtype):
        """ti.cast / .cast / int(): to an integer type truncates toward zero (Taichi's float ->
        int conversion), to a float type keeps the value."""
        if isinstance(v, _PVec):
            return _PVec([self.cast(c, dtype) for c in v.comps])
        if isinstance(v, _PMat):
            return _PMat.of([self.cast(c, dtype) for c in v.flat()], *v.shape)
        if dtype in (float, f32, f64):
            return _f32(v) if _is_num(v) and not isinstance(v, (int, np.integer)) else v
        if dtype not in (int, i32):
            raise TaichiLoweringError(f"cast to {dtype!r}: only int / ti.i32 and float / ti.f32")
        if isinstance(v, (int, np.integer)) and not isinstance(v, bool):
            return int(v)
        if _is_num(v):
            x = float(_f32(v))
            if x != x or abs(x) >= 2.0 ** 31:
                raise TaichiLoweringError(f"int({x}) is outside int32")
            return int(x)
        if self._ib(v) is not None:
            return v  # already an integer
        return self.unary("trunc", v)

    def _index_values(self, fld, idx, local):
        """The index values of fld[idx]: one per axis of fld (a tuple of expressions, one
        expression, or one vector expression such as base + offset); () for a 0-D field."""
        if not fld.shape:
            if not ((isinstance(idx, ast.Constant) and idx.value is None) or (isinstance(idx, ast.Tuple) and not idx.elts)):
                raise TaichiLoweringError("a 0-D field is indexed as field[None]")
            return []
        elts = list(idx.elts) if isinstance(idx, ast.Tuple) else [idx]
        vals = [self.expr(e, local) for e in elts]
        if len(vals) == 1 and isinstance(vals[0], _PVec):
            vals = list(vals[0].comps)
        if len(vals) != len(fld.shape):
            raise TaichiLoweringError(f"a field of shape {fld.shape} is indexed with {len(vals)} indices")
        if any(isinstance(v, (_PVec, list)) for v in vals):
            raise TaichiLoweringError("field indices are scalars")
        return vals

    def scatter(self, fld, idx, value, local, negate=False, op="add"):
        """fld[idx] += value (-= with negate) at an index other than this pixel's: Taichi's atomic
        add, an effect of the program (pixprog scatter_add), dropped where an index falls outside
        fld.  The field must be neither stored nor read in the same struct-for (its reads would
        race with the adds)."""
        if self.in_loop:
            raise TaichiLoweringError("a scatter-add (field[...] += v at another index) inside a runtime loop is not supported")
        if fld in self.stored:
            raise TaichiLoweringError("a field is both stored at the loop index and scatter-added into in one struct-for")
        if fld in self.inputs and fld not in self.targets:
            raise TaichiLoweringError("a field scatter-added into is also read in the same struct-for")
        vals = self._index_values(fld, idx, local)
        if len(vals) == 0:
            row, col = 0.0, 0.0
        elif len(vals) == 1:
            row, col = 0.0, vals[0]
        elif len(vals) == 2:
            row, col = vals
        else:
            # [A][B][C] as [A B][C]: the row a * B + b where 0 <= a < A and 0 <= b < B, else -1 (the
            # add is dropped); each axis truncated first, so b past B does not reach the next a
            a, b2, col = vals
            A, B = fld.shape[0], fld.shape[1]
            a, b2 = self.cast(a, int), self.cast(b2, int)
            ok = self.logic("and", [self.cmp_value("le", 0.0, a), self.cmp_value("lt", a, float(A)),
                                    self.cmp_value("le", 0.0, b2), self.cmp_value("lt", b2, float(B))])
            row = self.select(ok, self.arith("add", self.arith("mul", a, float(B)), b2), -1.0)
        v = _PVec(value) if isinstance(value, list) else value
        if isinstance(v, _PMat):
            if fld.mat != v.shape:
                raise TaichiLoweringError("a matrix is added into a field of matrices of its shape")
            v = _PVec(v.flat())
        if fld.width == 1:
            if isinstance(v, _PVec):
                raise TaichiLoweringError("a field of scalars takes a scalar")
            comps = [v]
        elif isinstance(v, _PVec):
            if len(v.comps) != fld.width:
                raise TaichiLoweringError(f"a field of {fld.width}-vectors takes {fld.width} components")
            comps = v.comps
        else:
            comps = [v] * fld.width
        if fld not in self.inputs:
            if len(self.inputs) == self.pp.MAX_INPUTS:
                raise TaichiLoweringError(f"at most {self.pp.MAX_INPUTS} fields can be read or scatter-added into")
            self.inputs.append(fld)
            self.in_extents.append(_grid_of(fld.shape) if tuple(fld.shape) != tuple(self.shape) else None)
        if fld not in self.targets:
            self.targets.append(fld)
        k = self.inputs.index(fld)
        if self.pred is not None:  # in an if branch: a row of -1 drops the add where it does not run
            row = self.select(self.pred, row, -1.0)
        r, c = self.node(row), self.node(col)
        for q, x in enumerate(comps):
            if negate:
                x = self.unary("neg", x)
            self.scatters.append(self.b.scatter_add(k, r, c, self.node(x), q, op=op))

    def minmax(self, which, vals):
        if len(vals) < 2:
            raise TaichiLoweringError(f"{which} needs two or more values")
        acc = vals[0]
        for v in vals[1:]:
            acc = self.elementwise(lambda x, y: self._minmax2(which, x, y), acc, v)
        return acc

    def _minmax2(self, which, x, y):
        if _is_num(x) and _is_num(y):
            return (max if which == "max" else min)(_f32(x), _f32(y))
        return self.b.op(which, self.node(x), self.node(y))

    def elementwise(self, fn, *vals):
        """fn over scalars, or per component where some of vals are vectors (scalars broadcast)."""
        vecs = [v for v in vals if isinstance(v, _PVec)]
        if not vecs:
            return fn(*vals)
        n = len(vecs[0].comps)
        if any(len(v.comps) != n for v in vecs):
            raise TaichiLoweringError("vector length mismatch")
        return _PVec([fn(*[v.comps[k] if isinstance(v, _PVec) else v for v in vals]) for k in range(n)])

    def normalize(self, v):
        """v * (1 / |v|), as Taichi's Matrix.normalized forms it."""
        if not isinstance(v, _PVec):
            raise TaichiLoweringError("normalize takes a vector")
        inv = self.arith("div", 1.0, self.unary("sqrt", self.dot(v, v)))
        return _PVec([self.arith("mul", c, inv) for c in v.comps])

    def cross(self, a, c):
        if not (isinstance(a, _PVec) and isinstance(c, _PVec) and len(a.comps) == len(c.comps) == 3):
            raise TaichiLoweringError("cross takes two 3-vectors")
        x, y = a.comps, c.comps
        comp = lambda i, j: self.arith("sub", self.arith("mul", x[i], y[j]), self.arith("mul", x[j], y[i]))
        return _PVec([comp(1, 2), comp(2, 0), comp(0, 1)])

    def math_call(self, name, args):
        """ti.math's functions, written out in the operations Taichi's definitions use."""
        if name in ("vec2", "vec3", "vec4"):
            comps = []
            for a in args:
                comps.extend(a.comps if isinstance(a, _PVec) else [a])
            want = int(name[3])
            if len(comps) == 1:
                comps = comps * want
            if len(comps) != want:
                raise TaichiLoweringError(f"{name} of {len(comps)} components")
            return _PVec(comps)
        if name == "clamp":
            x, lo, hi = args
            return self.minmax("min", [self.minmax("max", [x, lo]), hi])
        if name == "mix":  # x * (1 - a) + y * a
            x, y, a = args
            return self.arith("add", self.arith("mul", x, self.arith("sub", 1.0, a)), self.arith("mul", y, a))
        if name == "smoothstep":  # t = clamp((x - e0) / (e1 - e0), 0, 1); t * t * (3 - 2 t)
            e0, e1, x = args
            t = self.math_call("clamp", [self.arith("div", self.arith("sub", x, e0), self.arith("sub", e1, e0)), 0.0, 1.0])
            return self.arith("mul", self.arith("mul", t, t), self.arith("sub", 3.0, self.arith("mul", 2.0, t)))
        if name == "length":
            return self.unary("sqrt", self.dot(args[0], args[0]))
        if name == "normalize":
            return self.normalize(args[0])
        if name == "dot":
            return self.dot(args[0], args[1])
        if name == "cross":
            return self.cross(args[0], args[1])
        if name == "fract":
            return self.arith("sub", args[0], self.unary("floor", args[0]))
        if name == "step":  # 0 where x < edge, else 1
            edge, x = args
            return self.elementwise(lambda e, v: self.select(self.cmp_value("lt", v, e), 0.0, 1.0), edge, x)
        if name == "sign":
            return self.elementwise(
                lambda v: self.select(self.cmp_value("lt", 0.0, v), 1.0, self.select(self.cmp_value("lt", v, 0.0), -1.0, 0.0)),
                args[0])
        raise TaichiLoweringError(f"ti.math.{name} is not supported")

    def cmp_value(self, kind, a, c):
        if _is_num(a) and _is_num(c):
            fa, fc = _f32(a), _f32(c)
            return int({"lt": fa < fc, "le": fa <= fc, "eq": fa == fc, "ne": fa != fc}[kind])
        return self._bool(self.b.op(kind, self.node(a), self.node(c)))

    # -- conditions: comparisons give 1.0 / 0.0; a value is true where it is not 0 (NaN is true)
    def _bool(self, n):
        self.bools.add(id(n))
        return n

    def truth(self, v):
        if isinstance(v, _PVec):
            raise TaichiLoweringError("a vector is not a condition")
        if _is_num(v):
            return 1 if _f32(v) != 0 else 0
        if id(v) in self.bools:
            return v
        return self._bool(self.b.op("ne", v, 0.0))

    def compare(self, n, local):
        ops = {ast.Lt: ("lt", False), ast.LtE: ("le", False), ast.Gt: ("lt", True), ast.GtE: ("le", True),
               ast.Eq: ("eq", False), ast.NotEq: ("ne", False)}
        terms, left = [], self.expr(n.left, local)
        for op, rhs_n in zip(n.ops, n.comparators):
            if type(op) not in ops:
                raise TaichiLoweringError(f"comparison {type(op).__name__} is not supported")
            right = self.expr(rhs_n, local)
            if isinstance(left, _PVec) or isinstance(right, _PVec):
                raise TaichiLoweringError("comparisons are of scalars")
            kind, swap = ops[type(op)]
            a, c = (right, left) if swap else (left, right)
            if _is_num(a) and _is_num(c):
                fa, fc = _f32(a), _f32(c)
                terms.append(int({"lt": fa < fc, "le": fa <= fc, "eq": fa == fc, "ne": fa != fc}[kind]))
            else:
                terms.append(self._bool(self.b.op(kind, self.node(a), self.node(c))))
            left = right
        return self.logic("and", terms)

    def logic(self, which, vals):
        acc = self.truth(vals[0])
        for v in vals[1:]:
            t = self.truth(v)
            if _is_num(acc) and _is_num(t):
                acc = (acc and t) if which == "and" else (acc or t)
            elif _is_num(acc) or _is_num(t):
                k, other = (acc, t) if _is_num(acc) else (t, acc)
                if which == "and":
                    acc = other if k else 0
                else:
                    acc = 1 if k else other
            else:
                acc = self._bool(self.b.op("mul" if which == "and" else "max", acc, t))
        return acc

    def logic_not(self, v):
        t = self.truth(v)
        if _is_num(t):
            return 1 - t
        return self._bool(self.b.op("eq", t, 0.0))

    def select(self, c, x, y):
        if isinstance(x, _PMat) or isinstance(y, _PMat):
            if not (isinstance(x, _PMat) and isinstance(y, _PMat) and x.shape == y.shape):
                raise TaichiLoweringError("a conditional picks between two matrices of one shape")
            return _PMat.of([self.select(c, a, d) for a, d in zip(x.flat(), y.flat())], *x.shape)
        if isinstance(x, _PVec) or isinstance(y, _PVec):
            if not (isinstance(x, _PVec) and isinstance(y, _PVec) and len(x.comps) == len(y.comps)):
                raise TaichiLoweringError("a conditional picks between two vectors of one length or two scalars")
            return _PVec([self.select(c, a, d) for a, d in zip(x.comps, y.comps)])
        if isinstance(c, _PVec):
            raise TaichiLoweringError("a vector is not a condition")
        if _is_num(c):
            return x if _f32(c) != 0 else y
        if x is y or (_is_num(x) and _is_num(y) and _f32(x).tobytes() == _f32(y).tobytes()):
            return x
        r = self.b.op("select", c, self.node(x), self.node(y))
        if id(self.node(x)) in self.bools and id(self.node(y)) in self.bools:
            self.bools.add(id(r))
        return r

    def bit_op(self, op, x, y):
        """&, |, ^, << and >> of integers (int32 operations, >> arithmetic): folded when both are
        known, else the bit opcodes on values whose bound keeps them exact in f32 registers."""
        if isinstance(x, _PVec) or isinstance(y, _PVec):
            return self.elementwise(lambda a, c: self.bit_op(op, a, c), x, y)
        ints = all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) for v in (x, y))
        if ints:
            a, c = int(x), int(y)
            return {"band": a & c, "bor": a | c, "bxor": a ^ c, "shl": a << (c & 31), "shr": a >> (c & 31)}[op]
        bx, by = self._ib(x), self._ib(y)
        if bx is None or by is None:
            raise TaichiLoweringError("bit operations take integers of a known bound below 2^24 (indices, loop variables, "
                                      "constants and integer arithmetic of them)")
        if op == "shl":
            if not isinstance(y, (int, np.integer)):
                raise TaichiLoweringError("x << n needs n known when the kernel is lowered")
            bound = bx << (int(y) & 31)
        elif op == "shr":
            bound = bx
        else:  # two's complement operands in [-2^k, 2^k) give results in the same range
            bound = 1 << max(bx, by).bit_length()
        r = self.b.op(op, self.node(x), self.node(y))
        return self._int_result(r, bound, {"band": "&", "bor": "|", "bxor": "^", "shl": "<<", "shr": ">>"}[op])

    def floor_op(self, mod, x, y):
        """x % y (floored, the sign of y) and x // y, as x - floor(x / y) * y and floor(x / y)."""
        if isinstance(x, _PVec) or isinstance(y, _PVec):
            raise TaichiLoweringError("% and // are of scalars")
        if isinstance(x, (int, np.integer)) and isinstance(y, (int, np.integer)) and not isinstance(x, bool):
            if y == 0:
                raise TaichiLoweringError("integer division by zero")
            return x % y if mod else x // y
        bx, by = self._ib(x), self._ib(y)
        if bx is not None and by is not None:
            # floor(x / y) of integers below 2^24 in magnitude is exact in f32 (the quotient cannot
            # round up to the next integer), and so is x - q * y; the results are integers again
            self._int_result(x, bx, "the dividend of % or //") if isinstance(x, self.pp.Node) else None
            q = self.b.op("floor", self.node(self._arith("div", x, y)))
            self.ibound[id(q)] = bx
            if not mod:
                return q
            return self._int_result(self._arith("sub", x, self._arith("mul", q, y)), max(by - 1, 0), "%")
        q = self.unary("floor", self.arith("div", x, y))
        return self.arith("sub", x, self.arith("mul", q, y)) if mod else q

    # -- statements
    def if_stmt(self, st, local):
        """Both branches are evaluated; each name either assigns afterwards takes the branch's value
        by a select on the condition (a store in one branch only keeps the field's value in the
        other)."""
        c = self.expr(st.test, local)
        if isinstance(c, _PVec):
            raise TaichiLoweringError("a vector is not a condition")
        if _is_num(c):  # a condition known when the kernel is lowered
            for s2 in (st.body if _f32(c) != 0 else st.orelse):
                if not self.assign(s2, local):
                    raise TaichiLoweringError(f"statement at line {getattr(s2, 'lineno', '?')} is not supported")
            return
        branches = []
        outer = self.pred
        for stmts, cond in ((st.body, self.truth(c)), (st.orelse, self.logic_not(c))):
            loc = dict(local)
            # scatter-adds in a branch happen only where its condition holds
            self.pred = cond if outer is None else self.logic("and", [outer, cond])
            try:
                for s2 in stmts:
                    if not self.assign(s2, loc):
                        raise TaichiLoweringError(f"statement at line {getattr(s2, 'lineno', '?')} in an if is not supported")
            finally:
                self.pred = outer
            branches.append(loc)
        lt, lf = branches
        for nm in list(dict.fromkeys(list(lt) + list(lf))):
            vt, vf = lt.get(nm, _ONE_BRANCH), lf.get(nm, _ONE_BRANCH)
            if vt is vf:
                local[nm] = vt
                continue
            if _is_skey(nm):  # the field keeps its value where a branch does not store
                keep = local.get(nm)
                if keep is None:
                    keep = self._field_read(self.fields[nm[1]], self._here(), {})
                vt = keep if vt is _ONE_BRANCH else vt
                vf = keep if vf is _ONE_BRANCH else vf
            elif vt is _ONE_BRANCH or vf is _ONE_BRANCH or vt is _UNREADABLE or vf is _UNREADABLE:
                local[nm] = _ONE_BRANCH
                continue
            local[nm] = self.select(c, vt, vf)

    def static_values(self, st, local):
        """The values of `for v in ti.static(...)` (a loop unrolled when the kernel is lowered), or
        None for any other statement."""
        if not isinstance(st, ast.For):
            return None
        it = st.iter
        if not (isinstance(it, ast.Call) and len(it.args) == 1 and
                ((isinstance(it.func, ast.Attribute) and it.func.attr == "static") or
                 (isinstance(it.func, ast.Name) and it.func.id == "static"))):
            # `for k in range(N)` whose body reads k (a component index, say) and holds no other
            # loop: unrolled as well, which runs the same statements in the same order; N is
            # bounded by the program size.  A loop around another loop stays a loop (a nest of
            # range loops runs as one loop over its trips), so nests do not multiply the program.
            if (self.unroll and isinstance(it, ast.Call) and isinstance(it.func, ast.Name) and it.func.id == "range"
                    and isinstance(st.target, ast.Name)
                    and not any(isinstance(nd, (ast.For, ast.While)) for s2 in st.body for nd in ast.walk(s2))
                    and not any(_jumps(st.body))
                    and any(isinstance(nd, ast.Name) and nd.id == st.target.id and isinstance(nd.ctx, ast.Load)
                            for s2 in st.body for nd in ast.walk(s2))):
                bounds = [self.expr(a, local) for a in it.args]
                if all(isinstance(v, (int, np.integer)) for v in bounds) and len(range(*map(int, bounds))) <= 32:
                    return list(range(*[int(v) for v in bounds]))
            return None
        inner = it.args[0]
        if isinstance(inner, ast.Call) and isinstance(inner.func, ast.Name) and inner.func.id == "range":
            bounds = [self.expr(a, local) for a in inner.args]
            if not all(isinstance(v, (int, np.integer)) for v in bounds):
                raise TaichiLoweringError("ti.static(range(...)) needs integer constants")
            return list(range(*[int(v) for v in bounds]))
        if isinstance(inner, ast.Call) and ((isinstance(inner.func, ast.Attribute) and inner.func.attr == "ndrange") or
                                            (isinstance(inner.func, ast.Name) and inner.func.id == "ndrange")):
            # ti.static(ti.ndrange(A, B, ...)): every index tuple, the last index fastest; an
            # extent is n (0 .. n-1) or a pair (lo, hi)
            axes = []
            for a in inner.args:
                v = self.expr(a, local)
                if isinstance(v, (int, np.integer)) and not isinstance(v, bool):
                    axes.append(range(int(v)))
                elif isinstance(v, list) and len(v) == 2 and all(isinstance(x, (int, np.integer)) for x in v):
                    axes.append(range(int(v[0]), int(v[1])))
                else:
                    raise TaichiLoweringError("ti.static(ti.ndrange(...)) needs integer extents")
            return [tuple(t) for t in itertools.product(*axes)]
        vals = self.expr(inner, local)
        if isinstance(vals, _PVec):
            return list(vals.comps)
        if isinstance(vals, (list, tuple)):
            return list(vals)
        raise TaichiLoweringError("ti.static loops over range(...) or a list of values")

    def store_here(self, target, v, local):
        """target[i, j] = v (this pixel's element; kept as the stored value, components flat)."""
        if self.in_loop:
            raise TaichiLoweringError("a store inside the loop is not supported (store after it)")
        if isinstance(v, list):
            v = _PVec(v)
        if isinstance(v, _PMat):
            if target.mat != v.shape:
                raise TaichiLoweringError(f"a {v.shape[0]} x {v.shape[1]} matrix stored to a field of "
                                          f"{'matrices ' + str(target.mat) if target.mat else 'vectors or scalars'}")
            v = _PVec(v.flat())
        if target.width == 1:
            if isinstance(v, _PVec):
                raise TaichiLoweringError("a field of scalars stores a scalar")
        elif not isinstance(v, _PVec):
            v = _PVec([v] * target.width)  # a scalar fills every component
        elif len(v.comps) != target.width:
            raise TaichiLoweringError(f"a field of {target.width}-vectors stores {target.width} components")
        if target in self.targets:
            raise TaichiLoweringError("a field is both stored at the loop index and scatter-added into in one struct-for")
        if target not in self.stored:
            self.stored.append(target)
            self.fields[id(target)] = target
        local[_skey(target)] = v

    def element_component_assign(self, st, tgt, local):
        """field[i, j].y op= v, field[i, j][k] op= v, field[i, j][a, b] = v (a matrix field): this
        pixel's element with one component replaced, stored again."""
        sub = tgt.value
        fld = self.expr(sub.value, local)
        if not (isinstance(fld, Field) and self._at_here(fld, sub.slice)):
            raise TaichiLoweringError("a component is assigned in this pixel's element of a field (field[i, j].x = v)")
        cur = self._field_read(fld, sub.slice, local)
        comps = list(cur.comps) if isinstance(cur, _PVec) else [cur]
        if isinstance(tgt, ast.Attribute):
            if tgt.attr not in ("x", "y", "z", "w") or "xyzw".index(tgt.attr) >= len(comps):
                raise TaichiLoweringError(f"the field's elements have no component {tgt.attr!r}")
            k = "xyzw".index(tgt.attr)
        else:
            idx = self.expr(tgt.slice, local)
            if fld.mat and isinstance(idx, list) and len(idx) == 2 and all(isinstance(x, (int, np.integer)) for x in idx):
                k = int(idx[0]) * fld.mat[1] + int(idx[1])
            elif isinstance(idx, (int, np.integer)) and 0 <= idx < len(comps):
                k = int(idx)
            else:
                raise TaichiLoweringError("a field element's component is set at a constant index")
        val = self.expr(st.value, local)
        if isinstance(st, ast.AugAssign):
            ops = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div"}
            if type(st.op) not in ops:
                raise TaichiLoweringError(f"augmented {type(st.op).__name__} is not supported")
            val = self.arith(ops[type(st.op)], comps[k], val)
        if isinstance(val, (_PVec, _PMat)):
            raise TaichiLoweringError("a component takes a scalar")
        comps[k] = val
        self.store_here(fld, _PVec(comps) if len(comps) > 1 else comps[0], local)
        return True

    def component_assign(self, st, tgt, local):
        """v[k] = x, v.x = x, v[k] += x on a local vector (M[a, b] on a local matrix): a new value
        with that component replaced."""
        name = tgt.value.id
        vec = local[name]
        if isinstance(vec, _PMat):
            idx = self.expr(tgt.slice, local) if isinstance(tgt, ast.Subscript) else None
            if not (isinstance(idx, list) and len(idx) == 2 and all(isinstance(x, (int, np.integer)) for x in idx)):
                raise TaichiLoweringError("a matrix component is set as M[a, b] at constant indices")
            a, c = int(idx[0]), int(idx[1])
            val = self.expr(st.value, local)
            if isinstance(st, ast.AugAssign):
                ops = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div"}
                if type(st.op) not in ops:
                    raise TaichiLoweringError(f"augmented {type(st.op).__name__} is not supported")
                val = self.arith(ops[type(st.op)], vec.rows[a][c], val)
            rows = [list(r) for r in vec.rows]
            rows[a][c] = val
            local[name] = _PMat(rows)
            return True
        if isinstance(tgt, ast.Attribute):
            if tgt.attr not in ("x", "y", "z", "w"):
                raise TaichiLoweringError(f"vector has no component {tgt.attr!r}")
            k = "xyzw".index(tgt.attr)
        else:
            k = self.expr(tgt.slice, local)
        if not isinstance(k, (int, np.integer)) or not -len(vec.comps) <= k < len(vec.comps):
            raise TaichiLoweringError("a vector component is set at a constant index")
        val = self.expr(st.value, local)
        if isinstance(st, ast.AugAssign):
            ops = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div"}
            if type(st.op) not in ops:
                raise TaichiLoweringError(f"augmented {type(st.op).__name__} is not supported")
            val = self.arith(ops[type(st.op)], vec.comps[int(k)], val)
        if isinstance(val, _PVec):
            raise TaichiLoweringError("a vector component takes a scalar")
        comps = list(vec.comps)
        comps[int(k)] = val
        local[name] = _PVec(comps)
        return True

    def assign(self, st, local):
        if isinstance(st, ast.Assign) and len(st.targets) > 1:  # a = b = value
            return all(self.assign(ast.Assign(targets=[t], value=st.value, lineno=getattr(st, "lineno", 0)), local)
                       for t in st.targets)
        if isinstance(st, ast.If):
            self.if_stmt(st, local)
            return True
        vals = self.static_values(st, local)
        if vals is not None:
            tnames = [st.target.id] if isinstance(st.target, ast.Name) else \
                [e.id for e in st.target.elts] if isinstance(st.target, ast.Tuple) and \
                all(isinstance(e, ast.Name) for e in st.target.elts) else None
            if tnames is None or st.orelse:
                raise TaichiLoweringError("a ti.static loop binds names and has no else")
            for v in vals:
                if len(tnames) == 1:
                    local[tnames[0]] = v
                else:
                    if not isinstance(v, tuple) or len(v) != len(tnames):
                        raise TaichiLoweringError(f"a ti.static loop over {len(tnames)} names needs tuples of that many values")
                    local.update(zip(tnames, v))
                for s2 in st.body:
                    if not self.assign(s2, local):
                        raise TaichiLoweringError(f"statement at line {getattr(s2, 'lineno', '?')} is not supported")
            return True
        if (isinstance(st, (ast.Assign, ast.AugAssign)) and isinstance(getattr(st, "target", None) or st.targets[0],
                                                                       (ast.Subscript, ast.Attribute))):
            tgt = st.target if isinstance(st, ast.AugAssign) else st.targets[0]
            if isinstance(tgt.value, ast.Name) and isinstance(local.get(tgt.value.id), (_PVec, _PMat)):
                return self.component_assign(st, tgt, local)
            if isinstance(tgt.value, ast.Subscript) and isinstance(self.expr(tgt.value.value, local), Field):
                return self.element_component_assign(st, tgt, local)
        if isinstance(st, ast.Expr) and isinstance(st.value, ast.Call):
            # ti.atomic_add(field[idx], v) / ti.atomic_sub as a statement: field[idx] += v / -= v
            fn = st.value.func
            name = fn.attr if isinstance(fn, ast.Attribute) else fn.id if isinstance(fn, ast.Name) else None
            if name in ("atomic_add", "atomic_sub", "atomic_max", "atomic_min"):
                args = st.value.args
                if len(args) != 2 or not isinstance(args[0], ast.Subscript):
                    raise TaichiLoweringError(f"ti.{name} takes (field[index], value)")
                if name in ("atomic_add", "atomic_sub"):
                    op = ast.Add() if name == "atomic_add" else ast.Sub()
                    return self.assign(ast.AugAssign(target=args[0], op=op, value=args[1],
                                                     lineno=getattr(st, "lineno", 0)), local)
                which = name[len("atomic_"):]
                fld = self.expr(args[0].value, local)
                if not isinstance(fld, Field):
                    raise TaichiLoweringError(f"ti.{name} takes a field element")
                val = self.expr(args[1], local)
                if self._at_here(fld, args[0].slice):  # this pixel's element: a plain max / min and store
                    cur = self._field_read(fld, args[0].slice, local)
                    if isinstance(val, list):
                        val = _PVec(val)
                    self.store_here(fld, self.elementwise(lambda a, c: self.minmax(which, [a, c]), cur, val), local)
                else:
                    self.scatter(fld, args[0].slice, val, local, op=which)
                return True
            return False
        if isinstance(st, ast.AugAssign) and isinstance(st.target, ast.Subscript):
            base = self.expr(st.target.value, local)
            if isinstance(base, Field) and not self._at_here(base, st.target.slice):
                # at another index: Taichi's atomic add
                if not isinstance(st.op, (ast.Add, ast.Sub)):
                    raise TaichiLoweringError(f"augmented {type(st.op).__name__} at another index than the loop's "
                                              "(only += and -=, Taichi's atomic adds)")
                self.scatter(base, st.target.slice, self.expr(st.value, local), local, negate=isinstance(st.op, ast.Sub))
                return True
            # field[i, j] op= v is field[i, j] = field[i, j] op v (the read sees an earlier store)
            return self.assign(ast.Assign(targets=[st.target], value=ast.BinOp(
                left=ast.Subscript(value=st.target.value, slice=st.target.slice, ctx=ast.Load()), op=st.op,
                right=st.value), lineno=getattr(st, "lineno", 0)), local)
        if isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Subscript):
            tgt = st.targets[0]
            target = self.expr(tgt.value, local)
            if not isinstance(target, Field):
                raise TaichiLoweringError("the body stores to fields (field[...] = v)")
            if not self._at_here(target, tgt.slice):  # another element: a store at computed indices
                self.scatter(target, tgt.slice, self.expr(st.value, local), local, op="store")
                return True
            self.store_here(target, self.expr(st.value, local), local)
            return True
        if isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Name):
            local[st.targets[0].id] = self.expr(st.value, local)
            return True
        if (isinstance(st, ast.Assign) and len(st.targets) == 1 and isinstance(st.targets[0], ast.Tuple)
                and all(isinstance(t, ast.Name) for t in st.targets[0].elts)):
            vals = self.expr(st.value, local)  # every right-hand value first: a parallel assignment
            names = [t.id for t in st.targets[0].elts]
            if isinstance(vals, _PVec):
                vals = vals.comps
            if not isinstance(vals, list) or len(vals) != len(names):
                raise TaichiLoweringError("tuple assignment of a different number of values")
            for nm, v in zip(names, vals):
                local[nm] = v
            return True
        if isinstance(st, ast.AugAssign) and isinstance(st.target, ast.Name):
            ops = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div"}
            if type(st.op) not in ops:
                raise TaichiLoweringError(f"augmented {type(st.op).__name__} is not supported")
            cur = self.expr(st.target, local)
            local[st.target.id] = self.arith(ops[type(st.op)], cur, self.expr(st.value, local))
            return True
        return False


_UNREADABLE = object()  # the loop counter inside the loop
_ONE_BRANCH = object()  # a name an if statement assigns in one branch only


_BUILTINS = {"abs": abs, "max": max, "min": min, "float": float, "int": int}


def _assigned_names(stmts):
    out = []
    for st in stmts:
        if isinstance(st, (ast.If, ast.For)):  # if branches; unrolled loops (their variable too)
            names = [st.target.id] if isinstance(st, ast.For) and isinstance(st.target, ast.Name) else \
                [e.id for e in st.target.elts if isinstance(e, ast.Name)] if isinstance(st, ast.For) and \
                isinstance(st.target, ast.Tuple) else []
            for nm in names + _assigned_names(st.body) + _assigned_names(st.orelse):
                if nm not in out:
                    out.append(nm)
        elif isinstance(st, ast.Assign):
            for t in st.targets:
                for e in (t.elts if isinstance(t, ast.Tuple) else [t]):
                    if isinstance(e, ast.Name) and e.id not in out:
                        out.append(e.id)
        elif isinstance(st, ast.AugAssign) and isinstance(st.target, ast.Name) and st.target.id not in out:
            out.append(st.target.id)
    return out


def lower_pixel_program(fdef: ast.FunctionDef, funcs, env, depth=0, unroll=True) -> Lowered:
    """Lowers one @ti.kernel struct-for body to per-pixel programs (vernondsl_amd.pixprog): one
    program when the body stores one field; when it stores several, one program per stored field
    (each evaluates the whole body and stores its field; the other stores stay local, so a later
    read of such a field at [i, j] sees the stored value), as a "sequence" in which no program
    loads a field from memory after another program of the sequence has stored it (the loads see
    the values from before the loop, as Taichi's do at [i, j]).  The programs are ordered so that
    a program loading a field runs before the one storing it; where they load each other's fields
    (x from v and v from x, as a particle update does), one such field is first copied to a
    snapshot (Field.snapshot) that the other programs load instead."""
    split = _split_at_second_loop(fdef, funcs, env, depth, unroll)
    if split is not None:
        return split
    try:
        low, stored, scatters = _lower_pixel_one(fdef, funcs, env, None, unroll)
        if low is not None:
            return low
        parts = {id(f): _lower_pixel_one(fdef, funcs, env, f, unroll)[0] for f in stored}
        if scatters:  # the body's scatter-adds run once, as a program of their own
            parts[id(_SCATTERS)] = _lower_pixel_one(fdef, funcs, env, _SCATTERS, unroll)[0]
            stored = stored + [_SCATTERS]
    except TaichiLoweringError as e:
        if not str(e).startswith("the program needs more than"):
            raise
        # a program too large for the device form (instructions or registers): first with short
        # range loops kept as loops rather than unrolled, then as two parts split at a statement
        # in the middle of the body
        if unroll:
            try:
                return lower_pixel_program(fdef, funcs, env, depth, unroll=False)
            except TaichiLoweringError as e2:
                if not str(e2).startswith("the program needs more than") and "does not split" not in str(e2):
                    raise
        expanded = _expand_static_loops(fdef, funcs, env)  # so that the split can fall between iterations
        if expanded is not None:
            fdef = expanded
        stmts = _struct_for(fdef, funcs, env)[4]
        if len(stmts) < 2:
            raise
        return _split_body(fdef, funcs, env, len(stmts) // 2, depth)

    def loaded_by_other(f, among):  # some other program still to run loads f
        return any(g is not f and f in parts[id(g)].reads for g in among)

    order, copies, pending = [], [], list(stored)
    while pending:
        ready = [f for f in pending if not loaded_by_other(f, pending)]
        if ready:
            order.append(ready[0])
            pending.remove(ready[0])
            continue
        f = next(f for f in pending if loaded_by_other(f, pending))
        snap = f.snapshot()  # (never the scatter-adds' entry: no program loads it)
        copies.append(Lowered("copy", snap, inputs=[f]))
        for g in pending:
            if g is not f:
                parts[id(g)].substitute(f, snap)
    return Lowered("sequence", stored[0], parts=copies + [parts[id(f)] for f in order])


def _struct_for(fdef: ast.FunctionDef, funcs, env, unroll=True):
    """The struct-for of a kernel body set up for interpretation: (the loop, the interpreter, its
    Builder, the locals holding the indices, the body's statements)."""
    from . import pixprog as pp
    body = [s for s in fdef.body if not (isinstance(s, ast.Expr) and isinstance(s.value, ast.Constant))]
    if len(body) != 1 or not isinstance(body[0], ast.For):
        raise TaichiLoweringError("the kernel body must be one struct-for `for i, j in field:` (or `for i in field:`)")
    loop = _ungroup(body[0], env, funcs)
    kname = None
    if isinstance(loop.target, ast.Tuple) and len(loop.target.elts) == 2:
        iname, jname = (e.id for e in loop.target.elts)
    elif isinstance(loop.target, ast.Tuple) and len(loop.target.elts) == 3:
        iname, jname, kname = (e.id for e in loop.target.elts)  # a 3-D struct-for
    elif isinstance(loop.target, ast.Name):
        iname, jname = loop.target.id, None  # a 1-D struct-for
    else:
        raise TaichiLoweringError("the struct-for must bind one, two or three indices (a 1-D, 2-D or 3-D field)")
    dims = 1 if jname is None else 2 if kname is None else 3
    b = pp.Builder()
    it0 = _PixInterp(env, funcs, b, None, iname, jname, kname)
    it = loop.iter
    fname = it.func.attr if isinstance(it, ast.Call) and isinstance(it.func, ast.Attribute) else \
        it.func.id if isinstance(it, ast.Call) and isinstance(it.func, ast.Name) else None
    offsets = (0,) * dims
    if fname in ("ndrange", "range"):  # ti.ndrange(W, H) / ti.ndrange((a, b), ...) / range(N) / range(A, B)
        vals = [it0.expr(a, {}) for a in it.args]
        if fname == "range":
            vals = [vals] if len(vals) == 2 else vals
        bounds = []
        for v in vals:
            if isinstance(v, (int, np.integer)) and not isinstance(v, bool):
                bounds.append((0, int(v)))
            elif isinstance(v, (list, tuple)) and len(v) == 2 and all(isinstance(x, (int, np.integer)) for x in v):
                bounds.append((int(v[0]), int(v[1])))
            else:
                bounds = None
                break
        if bounds is None or len(bounds) != dims or (fname == "range" and len(it.args) not in (1, 2)):
            raise TaichiLoweringError(f"the loop needs {dims} integer extent(s) for its {dims} index(es): "
                                      "ti.ndrange(W, H), ti.ndrange((a, b), (c, d)), range(N) or range(A, B)")
        ip = _PixInterp(env, funcs, b, None, iname, jname, kname)
        ip.shape = tuple(max(hi - lo, 0) for lo, hi in bounds)
        offsets = tuple(lo for lo, _ in bounds)
    else:
        fld = it0.expr(it, {})
        if not isinstance(fld, Field) or len(fld.shape) != dims:
            raise TaichiLoweringError(f"the struct-for binds {dims} index(es): it must iterate a {dims}-D ti.field, "
                                      "ti.ndrange or range")
        ip = _PixInterp(env, funcs, b, fld, iname, jname, kname)
    ip.unroll = unroll
    # a 1-D struct-for runs as one row of the program grid: its index is the column index; a 3-D
    # one [A][B][C] as the grid [A B][C]: i = row // B, j = row % B (exact integer operations), k
    # the column
    shape = ip.shape if ip.shape is not None else ip.fld.shape
    if dims == 3:
        if shape[0] * shape[1] > _PixInterp._INT_EXACT:
            raise TaichiLoweringError("a 3-D struct-for needs A * B <= 2^24 for its [A][B][C] extents")
        row = b.index(0)
        ip.ibound[id(row)] = max(shape[0] * shape[1] - 1, 0)
        local = {iname: ip.floor_op(False, row, shape[1]), jname: ip.floor_op(True, row, shape[1]), kname: b.index(1)}
        ip.ibound[id(local[kname])] = max(int(shape[2]) - 1, 0)
    else:
        local = {iname: b.index(0), jname: b.index(1)} if dims == 2 else {iname: b.index(1)}
        for nm, ext in zip(ip.names, shape):
            ip.ibound[id(local[nm])] = max(int(ext) - 1, 0)
    for nm, lo in zip(ip.names, offsets):  # ti.ndrange((a, b), ...): the index runs from a
        if lo:
            local[nm] = ip.arith("add", local[nm], lo)
    stmts = [s for s in loop.body if not (isinstance(s, ast.Expr) and isinstance(s.value, ast.Constant)) and not isinstance(s, ast.Pass)]
    return loop, ip, b, local, stmts


def _ungroup(loop, env, funcs):
    """`for I in ti.grouped(F): ...` as `for i0, i1 in F: I = ti.Vector([i0, i1]); ...`, with
    F[I] written F[i0, i1] (so it is this pixel's element); other loops unchanged."""
    it = loop.iter
    if not (isinstance(it, ast.Call) and len(it.args) == 1 and isinstance(loop.target, ast.Name) and (
            (isinstance(it.func, ast.Attribute) and it.func.attr == "grouped") or
            (isinstance(it.func, ast.Name) and it.func.id == "grouped"))):
        return loop
    fld = _PixInterp(env, funcs, None, None, "_", None).expr(it.args[0], {})
    shape = fld.shape if isinstance(fld, Field) else tuple(fld) if isinstance(fld, (list, tuple)) else None
    if not shape or not 1 <= len(shape) <= 3:
        raise TaichiLoweringError("ti.grouped takes a 1-D, 2-D or 3-D field or ti.ndrange")
    grp = loop.target.id
    names = [f"__vdsl_{grp}{k}" for k in range(len(shape))]

    class Sub(ast.NodeTransformer):
        def visit_Subscript(self, nd):
            self.generic_visit(nd)
            if isinstance(nd.slice, ast.Name) and nd.slice.id == grp:
                nd.slice = ast.Tuple(elts=[ast.Name(id=n, ctx=ast.Load()) for n in names], ctx=ast.Load()) \
                    if len(names) > 1 else ast.Name(id=names[0], ctx=ast.Load())
            return nd
    body = [Sub().visit(copy.deepcopy(st)) for st in loop.body]
    bind = ast.Assign(targets=[ast.Name(id=grp, ctx=ast.Store())], lineno=0, value=ast.Call(
        func=ast.Attribute(value=ast.Name(id="__vdsl_ti", ctx=ast.Load()), attr="Vector"),
        args=[ast.List(elts=[ast.Name(id=n, ctx=ast.Load()) for n in names], ctx=ast.Load())], keywords=[]))
    env.setdefault("__vdsl_ti", sys.modules[__name__])
    target = ast.Tuple(elts=[ast.Name(id=n, ctx=ast.Store()) for n in names], ctx=ast.Store()) if len(names) > 1 \
        else ast.Name(id=names[0], ctx=ast.Store())
    return ast.For(target=target, iter=it.args[0], body=[bind] + body, orelse=[], lineno=getattr(loop, "lineno", 0))


def _grid_of(shape):
    """The per-pixel program grid of a field of `shape`: [1][1] (0-D), [1][N], [R][C], or [A B][C]."""
    if len(shape) == 0:
        return (1, 1)
    if len(shape) == 1:
        return (1, shape[0])
    if len(shape) == 3:
        return (shape[0] * shape[1], shape[2])
    return tuple(shape)


def _is_runtime_loop(st, ip, local) -> bool:
    if not isinstance(st, (ast.While, ast.For)):
        return False
    try:
        return ip.static_values(st, local) is None
    except TaichiLoweringError:
        return True


def _run_stmts(ip, b, local, stmts):
    """Interprets a struct-for body (at most one runtime loop): (initial states, test, new states,
    max_iter, whether there is a loop)."""
    init, test, new_state, max_iter, has_loop = {}, None, {}, 0, False
    for st in stmts:
        if _is_runtime_loop(st, ip, local):
            if has_loop:
                raise TaichiLoweringError("at most one loop per struct-for body")
            if any(_is_skey(k) for k in local):
                raise TaichiLoweringError("the store field[i, j] = ... must come after the loop")
            has_loop = True
            init, test, new_state, max_iter = _lower_loop(st, ip, local, b)
            continue
        if ip.assign(st, local):
            continue
        raise TaichiLoweringError(f"statement at line {getattr(st, 'lineno', '?')} is not supported")
    return init, test, new_state, max_iter, has_loop


def _split_at_second_loop(fdef: ast.FunctionDef, funcs, env, depth=0, unroll=True):
    """A struct-for body with two or more runtime loops, split before the second loop
    (_split_body); None for a body with at most one runtime loop."""
    loop, ip, b, local, stmts = _struct_for(fdef, funcs, env, unroll)
    loops = [k for k, st in enumerate(stmts) if _is_runtime_loop(st, ip, local)]
    if len(loops) < 2:
        return None
    return _split_body(fdef, funcs, env, loops[1], depth, unroll)


def _split_body(fdef: ast.FunctionDef, funcs, env, at, depth, unroll=True):
    """The struct-for body as two parts run one after the other: its statements before `at`, then
    the rest.  The values the second part reads from the first go through hidden per-pixel fields
    of the struct-for's shape (their components packed four to a field; plain numbers are passed
    as constants), which the first part stores and the second reads at the pixel."""
    if depth > 8:
        raise TaichiLoweringError("the struct-for body does not split into programs that fit the device form")
    loop, ip, b, local, stmts = _struct_for(fdef, funcs, env, unroll)
    part1, part2 = stmts[:at], stmts[at:]
    _run_stmts(ip, b, local, part1)  # a dry run: the kinds of the values the second part reads
    reads2 = _reads_before_writes(part2)
    passed = []  # (name, value) of the locals the second part reads
    for nm, v in local.items():
        if not (isinstance(nm, str) and nm in reads2 and nm not in ip.names):
            continue
        if v is _UNREADABLE or v is _ONE_BRANCH:
            continue
        if _leaves(v) is None:
            raise TaichiLoweringError(f"{nm!r} holds a value that cannot pass between the parts of a split body")
        passed.append((nm, v))
    shape = ip.shape if ip.shape is not None else ip.fld.shape
    env2 = dict(env)
    env2["__vdsl_ti"] = sys.modules[__name__]
    # every per-pixel scalar to pass, in order (numbers are written into the second part)
    flat = [(nm, path) for nm, v in passed for path, x in _leaves(v) if not _is_num(x)]
    fields, stores, slot = [], [], {}
    serial = sum(1 for nm in env2 if str(nm).startswith("__vdsl_tmp"))  # names of earlier splits stay bound
    for k in range(0, len(flat), 4):
        group = flat[k:k + 4]
        name = f"__vdsl_tmp{serial + k // 4}"
        env2[name] = Field(f32, shape, len(group))
        fields.append(name)
        for q, key in enumerate(group):
            slot[key] = (name, q, len(group))
    here = ast.Name(id=ip.iname, ctx=ast.Load()) if len(ip.names) == 1 else \
        ast.Tuple(elts=[ast.Name(id=n, ctx=ast.Load()) for n in ip.names], ctx=ast.Load())

    for name in fields:
        members = sorted((q, key) for key, (fn, q, _) in slot.items() if fn == name)
        vals = [_access(nm, path) for _, (nm, path) in members]
        value = vals[0] if len(vals) == 1 else ast.Call(func=ast.Attribute(value=ast.Name(id="__vdsl_ti", ctx=ast.Load()), attr="Vector"),
                                                         args=[ast.List(elts=vals, ctx=ast.Load())], keywords=[])
        stores.append(ast.Assign(targets=[ast.Subscript(value=ast.Name(id=name, ctx=ast.Load()), slice=here, ctx=ast.Store())],
                                 value=value, lineno=0))

    def read(nm, path):
        fn, q, width = slot[(nm, path)]
        whole = ast.Subscript(value=ast.Name(id=fn, ctx=ast.Load()), slice=here, ctx=ast.Load())
        return whole if width == 1 else ast.Subscript(value=whole, slice=ast.Constant(value=q), ctx=ast.Load())

    prelude = []
    for nm, v in passed:
        leaf = dict(_leaves(v))

        def leaf_ast(path, nm=nm, leaf=leaf):
            x = leaf[path]
            if _is_num(x):
                return ast.Constant(value=int(x) if isinstance(x, (int, np.integer)) and not isinstance(x, bool)
                                    else float(_f32(x)))
            return read(nm, path)
        prelude.append(ast.Assign(targets=[ast.Name(id=nm, ctx=ast.Store())], value=_rebuild(v, leaf_ast), lineno=0))

    def kernel_of(body):
        f = ast.For(target=loop.target, iter=loop.iter, body=body, orelse=[], lineno=getattr(loop, "lineno", 0))
        return ast.FunctionDef(name=fdef.name, args=fdef.args, body=[f], decorator_list=[], returns=None, type_comment=None)

    if not stores and not any((isinstance(nd, ast.Subscript) and isinstance(nd.ctx, ast.Store)) or _is_atomic_call(nd)
                              for st in part1 for nd in ast.walk(st)):
        # the first part passes nothing on and stores nothing: only its loop's cost would remain
        return lower_pixel_program(kernel_of(prelude + part2), funcs, env2, depth + 1, unroll)
    first = lower_pixel_program(kernel_of(part1 + stores), funcs, env2, depth + 1, unroll)
    second = lower_pixel_program(kernel_of(prelude + part2), funcs, env2, depth + 1, unroll)
    return Lowered("sequence", second.field, parts=[first, second])


def _reads_before_writes(stmts):
    """The names a statement list reads before it assigns them (a statement's own reads count
    before its assignments; a compound statement's reads all count)."""
    assigned, reads = set(), set()
    for st in stmts:
        for nd in ast.walk(st):
            if isinstance(nd, ast.Name) and isinstance(getattr(nd, "ctx", ast.Load()), ast.Load) and nd.id not in assigned:
                reads.add(nd.id)
        if isinstance(st, ast.AugAssign) and isinstance(st.target, ast.Name):
            reads.add(st.target.id) if st.target.id not in assigned else None
        if isinstance(st, (ast.Assign, ast.AugAssign)):
            for t in (st.targets if isinstance(st, ast.Assign) else [st.target]):
                for e in (t.elts if isinstance(t, ast.Tuple) else [t]):
                    if isinstance(e, ast.Name):
                        assigned.add(e.id)
    return reads


def _leaves(v, path=()):
    """The scalar leaves of a value one part of a split body passes to the next: [(path, value)],
    a path step being an index (a list or vector component) or a pair (a matrix element); None
    for a value not made of scalars, vectors, matrices and lists of them."""
    if isinstance(v, _PMat):
        n, m = v.shape
        return [(path + ((a, c),), v.rows[a][c]) for a in range(n) for c in range(m)]
    if isinstance(v, _PVec):
        return [(path + (k,), c) for k, c in enumerate(v.comps)]
    if isinstance(v, list):
        out = []
        for k, e in enumerate(v):
            sub = _leaves(e, path + (k,))
            if sub is None:
                return None
            out += sub
        return out
    from . import pixprog
    if _is_num(v) or isinstance(v, pixprog.Node):
        return [(path, v)]
    return None


def _access(name, path):
    """The expression name[...] along a leaf path (a matrix element as M[a, b])."""
    node = ast.Name(id=name, ctx=ast.Load())
    for step in path:
        idx = ast.Tuple(elts=[ast.Constant(value=step[0]), ast.Constant(value=step[1])], ctx=ast.Load()) \
            if isinstance(step, tuple) else ast.Constant(value=step)
        node = ast.Subscript(value=node, slice=idx, ctx=ast.Load())
    return node


def _rebuild(v, leaf_ast, path=()):
    """An expression of v's structure (ti.Matrix, ti.Vector, lists) with leaf_ast(path) at each
    scalar."""
    ti_ = ast.Name(id="__vdsl_ti", ctx=ast.Load())
    if isinstance(v, _PMat):
        n, m = v.shape
        rows = [ast.List(elts=[leaf_ast(path + ((a, c),)) for c in range(m)], ctx=ast.Load()) for a in range(n)]
        return ast.Call(func=ast.Attribute(value=ti_, attr="Matrix"), args=[ast.List(elts=rows, ctx=ast.Load())], keywords=[])
    if isinstance(v, _PVec):
        return ast.Call(func=ast.Attribute(value=ti_, attr="Vector"),
                        args=[ast.List(elts=[leaf_ast(path + (k,)) for k in range(len(v.comps))], ctx=ast.Load())],
                        keywords=[])
    if isinstance(v, list):
        return ast.List(elts=[_rebuild(e, leaf_ast, path + (k,)) for k, e in enumerate(v)], ctx=ast.Load())
    return leaf_ast(path)


def _expand_static_loops(fdef: ast.FunctionDef, funcs, env):
    """fdef with each top-level static loop of its struct-for body (ti.static, or a short range
    loop that is unrolled anyway) over constant values written out iteration by iteration (the
    loop's names bound by assignments, then a copy of its body), so that a body too large for one
    program can be split between iterations; None if there is no such loop."""
    loop, ip, b, local, stmts = _struct_for(fdef, funcs, env)
    out, changed = [], False
    for st in stmts:
        vals = None
        if isinstance(st, ast.For) and not st.orelse:
            try:
                vals = ip.static_values(st, local)
            except TaichiLoweringError:
                vals = None
        names = [st.target.id] if isinstance(getattr(st, "target", None), ast.Name) else \
            [e.id for e in st.target.elts] if isinstance(getattr(st, "target", None), ast.Tuple) and \
            all(isinstance(e, ast.Name) for e in st.target.elts) else None

        def const(x):
            return isinstance(x, (int, float, np.integer, np.floating)) and not isinstance(x, bool)
        ok = vals is not None and names is not None and all(
            (len(names) == 1 and const(v)) or (isinstance(v, tuple) and len(v) == len(names) and all(map(const, v)))
            for v in vals)
        if not ok:
            out.append(st)
            continue
        for v in vals:
            for nm, x in zip(names, v if isinstance(v, tuple) else (v,)):
                out.append(ast.Assign(targets=[ast.Name(id=nm, ctx=ast.Store())], lineno=0,
                                      value=ast.Constant(value=int(x) if isinstance(x, (int, np.integer)) else float(x))))
            out.extend(copy.deepcopy(st.body))
        changed = True
    if not changed:
        return None
    f = ast.For(target=loop.target, iter=loop.iter, body=out, orelse=[], lineno=getattr(loop, "lineno", 0))
    return ast.FunctionDef(name=fdef.name, args=fdef.args, body=[f], decorator_list=[], returns=None, type_comment=None)


_SCATTERS = object()  # the target of the program that runs a body's scatter-adds on their own


def _is_atomic_call(nd) -> bool:
    """ti.atomic_add(...) / ti.atomic_sub(...) (a scatter-add statement)."""
    if not isinstance(nd, ast.Call):
        return False
    f = nd.func
    return (f.attr if isinstance(f, ast.Attribute) else f.id if isinstance(f, ast.Name) else None) in (
        "atomic_add", "atomic_sub", "atomic_max", "atomic_min")


def _lower_pixel_one(fdef: ast.FunctionDef, funcs, env, target, unroll=True):
    """(Lowered program storing `target`, the fields the body stores, whether the body
    scatter-adds); target None: the only field the body stores, with the body's scatter-adds
    (Lowered None when it stores several); target _SCATTERS: a program of the scatter-adds alone,
    storing nothing."""
    from . import pixprog as pp
    loop, ip, b, local, stmts = _struct_for(fdef, funcs, env, unroll)
    init, test, new_state, max_iter, has_loop = _run_stmts(ip, b, local, stmts)
    if not ip.stored and not ip.scatters:
        raise TaichiLoweringError("the struct-for body must store field[i, j] = ... or scatter-add (field[...] += v)")
    effects = []
    if target is None:
        if len(ip.stored) > 1:
            return None, ip.stored, bool(ip.scatters)
        target = ip.stored[0] if ip.stored else _SCATTERS
        effects = ip.scatters
    elif target is _SCATTERS:
        effects = ip.scatters
    fld = None if target is _SCATTERS else target
    v = None if fld is None else local[_skey(target)]
    out_i32 = False
    if fld is None:
        out = None
    elif fld.dtype == i32:
        if isinstance(v, pp.Node) and v.kind == "count":
            out = pp.COUNT
        else:  # any value, truncated as Taichi's int field assignment does
            out, out_i32 = (v if isinstance(v, pp.Node) else float(_f32(v))), True
    elif isinstance(v, _PVec):
        out = [c if isinstance(c, pp.Node) else float(_f32(c)) for c in v.comps]
    else:
        out = v if isinstance(v, pp.Node) else float(_f32(v))
    try:
        prog = pp.compile_program(b, init=init, test=test, body=new_state, max_iter=max_iter, out=out, loop=has_loop,
                                  in_widths=[f.width for f in ip.inputs],
                                  in_dtypes=[pp.I32 if f.dtype == i32 else pp.F32 for f in ip.inputs], out_i32=out_i32,
                                  in_extents=ip.in_extents, effects=effects)
    except pp.ProgramError as e:
        raise TaichiLoweringError(str(e)) from None
    # the fields this program loads (an input that only dead code reads is not one)
    roots = list(init.values()) + list(new_state.values()) + (list(test[1:]) if test else [])
    roots += out if isinstance(out, list) else [out]
    roots += effects
    todo, seen, live = [n for n in roots if isinstance(n, pp.Node)], set(), set()
    while todo:
        n = todo.pop()
        if id(n) not in seen:
            seen.add(id(n))
            if n.kind in ("load", "load_at"):
                live.add(n.val[0])
            todo.extend(n.args)
    low = Lowered("pixel_program", fld, program=prog, inputs=ip.inputs)
    low.reads = [f for k, f in enumerate(ip.inputs) if k in live]
    low.grid = _grid_of(ip.shape if ip.shape is not None else ip.fld.shape)
    low.uses_rng = ip.rng
    return low, ip.stored, bool(ip.scatters)


def _is_range(it) -> bool:
    return (isinstance(it, ast.Call) and isinstance(it.func, ast.Name) and it.func.id == "range"
            and len(it.args) in (1, 2))


def _range_bounds(it, ip, local):
    """(first, end) of range(N) / range(A, B) with integer constant arguments, else None."""
    try:
        vals = [ip.expr(a, local) for a in it.args]
    except TaichiLoweringError:
        return None
    if not all(isinstance(v, (int, np.integer)) and not isinstance(v, bool) for v in vals):
        return None
    return (int(vals[0]), int(vals[1])) if len(vals) == 2 else (0, int(vals[0]))


_BRK, _SKIP = "__vdsl_break", "__vdsl_skip"  # hidden locals of a loop with break / continue


def _jumps(stmts):
    """(break, continue) among the statements at this loop's level: in if branches, not in the
    bodies of inner loops (which they leave instead)."""
    brk = cont = False
    for st in stmts:
        if isinstance(st, ast.Break):
            brk = True
        elif isinstance(st, ast.Continue):
            cont = True
        elif isinstance(st, ast.If):
            b2, c2 = _jumps(st.body + st.orelse)
            brk, cont = brk or b2, cont or c2
    return brk, cont


def _without_jumps(stmts):
    """The loop body with break / continue as assignments to flags: a jump sets the trip's skip
    flag (break also the loop's break flag, which the loop's test reads before the next trip),
    and the statements after one that may jump run under `if skip == 0`, so they take effect
    only on lanes that did not jump."""
    def flag(name):
        return ast.Assign(targets=[ast.Name(id=name, ctx=ast.Store())], value=ast.Constant(value=1), lineno=0)
    out = []
    for k, st in enumerate(stmts):
        if isinstance(st, (ast.Break, ast.Continue)):
            out.append(flag(_SKIP))
            if isinstance(st, ast.Break):
                out.append(flag(_BRK))
            return out  # what follows an unconditional jump never runs
        if isinstance(st, ast.If) and any(_jumps([st])):
            out.append(ast.If(test=st.test, body=_without_jumps(st.body), orelse=_without_jumps(st.orelse),
                              lineno=getattr(st, "lineno", 0)))
            rest = _without_jumps(stmts[k + 1:])
            if rest:
                live = ast.Compare(left=ast.Name(id=_SKIP, ctx=ast.Load()), ops=[ast.Eq()],
                                   comparators=[ast.Constant(value=0)])
                out.append(ast.If(test=live, body=rest, orelse=[], lineno=getattr(st, "lineno", 0)))
            return out
        out.append(st)
    return out


def _lower_loop(st, ip: _PixInterp, local: dict, b):
    """One loop of the body: (initial states, test, new states, max_iter); rebinds `local` to the
    values after the loop (states, and the counter as the loop's count)."""
    from . import pixprog as pp
    counter, nest, dyn_n = None, [], None
    if isinstance(st, ast.For):
        # a perfect nest of range loops (each body is just the next loop) runs as one loop over
        # the product of the extents, its variables recovered from the trip, the innermost fastest
        loops = [st]
        while True:
            inner = [s for s in loops[-1].body
                     if not (isinstance(s, ast.Expr) and isinstance(s.value, ast.Constant)) and not isinstance(s, ast.Pass)]
            if not (len(inner) == 1 and isinstance(inner[0], ast.For) and _is_range(inner[0].iter)
                    and not _jumps(inner[0].body)[0]  # a break leaves the inner loop only
                    and _range_bounds(inner[0].iter, ip, local) is not None
                    and ip.static_values(inner[0], local) is None):
                break
            loops.append(inner[0])
        for lp in loops:
            if not _is_range(lp.iter):
                raise TaichiLoweringError("the inner loop must be `for k in range(N)`, `for k in range(A, B)` or a while loop")
            bounds = _range_bounds(lp.iter, ip, local)
            if bounds is None and len(loops) == 1 and len(lp.iter.args) == 1:
                # range(N) with N an integer expression of the pixel: a loop of at most N's bound
                # trips whose test is `k < N` (lanes leave it at their own N)
                n = ip.expr(lp.iter.args[0], local)
                bnd = ip._ib(n) if isinstance(n, pp.Node) else None
                if bnd is not None:
                    dyn_n, bounds = n, (0, bnd)
            if bounds is None:
                raise TaichiLoweringError("range(...) of a loop needs integer constants, or range(N) an integer expression "
                                          "of the indices and constants")
            nest.append((lp.target.id if isinstance(lp.target, ast.Name) else None, bounds[0], max(bounds[1] - bounds[0], 0)))
        max_iter = 1
        for _, _, ext in nest:
            max_iter *= ext
        loop_body = list(loops[-1].body)
        test = None
    else:
        tests = st.test.values if isinstance(st.test, ast.BoolOp) and isinstance(st.test.op, ast.And) else [st.test]
        loop_body = list(st.body)
        inc = loop_body[-1] if loop_body else None
        if not (isinstance(inc, ast.AugAssign) and isinstance(inc.op, ast.Add) and isinstance(inc.target, ast.Name)
                and isinstance(inc.value, ast.Constant) and inc.value.value == 1):
            raise TaichiLoweringError("a while loop must end with `counter += 1`")
        counter = inc.target.id
        if not (counter in local and _is_num(local[counter]) and isinstance(local[counter], (int, np.integer))
                and int(local[counter]) == 0):
            raise TaichiLoweringError("the loop counter must start at 0")
        loop_body = loop_body[:-1]
        max_iter, test_cmp = None, []
        for t in tests:
            if isinstance(t, ast.Compare) and len(t.ops) == 1 and isinstance(t.left, ast.Name) and t.left.id == counter:
                if not isinstance(t.ops[0], (ast.Lt, ast.LtE)):
                    raise TaichiLoweringError("the counter test must be `counter < MAX` or `counter <= MAX`")
                m = ip.expr(t.comparators[0], local)
                if not isinstance(m, (int, np.integer)):
                    raise TaichiLoweringError("the counter bound must be an integer constant")
                max_iter = int(m) + (1 if isinstance(t.ops[0], ast.LtE) else 0)
            else:
                test_cmp.append(t)
        if max_iter is None:
            raise TaichiLoweringError("the while condition needs a bound `counter < MAX`")
        if _jumps(loop_body)[1]:
            raise TaichiLoweringError("continue in a while loop would skip its `counter += 1`")
        test = test_cmp or None
        max_iter = max(0, max_iter)
    # break / continue: flags (a loop state and a per-trip value); the loop runs while the break
    # flag is clear, the check made before each trip as the loop's other tests are
    brk, cont = _jumps(loop_body)
    if brk or cont:
        loop_body = [ast.Assign(targets=[ast.Name(id=_SKIP, ctx=ast.Store())], value=ast.Constant(value=0), lineno=0)] \
            + _without_jumps(loop_body)
    if brk:
        local[_BRK] = 0
        clear = ast.Compare(left=ast.Name(id=_BRK, ctx=ast.Load()), ops=[ast.Eq()], comparators=[ast.Constant(value=0)])
        test = (test or []) + [clear]
    # loop-carried state: names assigned in the body that exist before the loop
    assigned = _assigned_names(loop_body)
    for nm in [counter] + [v for v, _, _ in nest]:
        if nm is not None and nm in assigned:
            raise TaichiLoweringError(f"the loop variable {nm!r} is assigned in the loop: the counter of a while loop "
                                      "changes only by its final `+= 1`, a range loop's variable not at all")
    state = [nm for nm in assigned if nm in local and nm != counter]
    init, names = {}, {}
    body_local = dict(local)
    # inside the loop the counter of a while loop and the variable of `for k in range(N)` are the
    # loop's trip (the same on every lane still in the loop), exact while N - 1 <= 2^24
    trip = b.trip() if max_iter - 1 <= _PixInterp._INT_EXACT else _UNREADABLE
    if trip is not _UNREADABLE:
        ip.ibound[id(trip)] = max(int(max_iter) - 1, 0)
    if counter is not None:
        body_local[counter] = trip
    rest = trip  # the trips of the loops not yet given their variables
    for k in range(len(nest) - 1, -1, -1):
        nm, first, ext = nest[k]
        if trip is _UNREADABLE:
            idx = _UNREADABLE
        elif k == 0:
            idx = rest
        else:
            idx = ip.floor_op(True, rest, ext)
            rest = ip.floor_op(False, rest, ext)
        if nm is not None:
            body_local[nm] = idx if (idx is _UNREADABLE or first == 0) else ip.arith("add", idx, first)
    for nm in state:
        v = local[nm]
        if isinstance(v, _PVec):
            comps = []
            for c, cv in enumerate(v.comps):
                key = f"{nm}.{c}"
                init[key] = cv if isinstance(cv, pp.Node) else _f32(cv)
                comps.append(b.state(key))
            names[nm] = (len(v.comps),)
            body_local[nm] = _PVec(comps)
        elif _is_num(v) or isinstance(v, pp.Node):
            init[nm] = v if isinstance(v, pp.Node) else _f32(v)
            names[nm] = ()
            body_local[nm] = b.state(nm)
        else:
            raise TaichiLoweringError(f"loop state {nm!r} must be a number or a vector")
    for nm in assigned:
        if nm not in state and nm != counter:
            body_local.pop(nm, None)  # defined inside the loop: read before assignment is an error
    test_out = None
    if dyn_n is not None:
        if trip is _UNREADABLE:
            raise TaichiLoweringError("range(N) of a per-pixel N needs N below 2^24")
        test_out = ("lt", trip, dyn_n)
    if test is not None:
        ops = {ast.Lt: "lt", ast.LtE: "le", ast.Gt: "gt", ast.GtE: "ge"}
        one = test[0]
        if (len(test) == 1 and dyn_n is None and isinstance(one, ast.Compare) and len(one.ops) == 1
                and type(one.ops[0]) in ops):
            lhs, rhs = ip.expr(one.left, body_local), ip.expr(one.comparators[0], body_local)
            if isinstance(lhs, _PVec) or isinstance(rhs, _PVec):
                raise TaichiLoweringError("the loop test compares scalars")
            test_out = (ops[type(one.ops[0])], lhs, rhs)
        else:  # any other condition: its truth value (1 / 0) against 0.5
            terms = [ip.expr(e, body_local) for e in test]
            if dyn_n is not None:
                terms = [b.op("lt", trip, dyn_n)] + terms
            t = ip.logic("and", terms)
            test_out = ("gt", t, 0.5)
    ip.in_loop = True
    try:
        for s2 in loop_body:
            if not ip.assign(s2, body_local):
                raise TaichiLoweringError(f"statement at line {getattr(s2, 'lineno', '?')} in the loop is not supported")
    finally:
        ip.in_loop = False
    new_state = {}
    for nm, shape in names.items():
        v = body_local[nm]
        if shape:
            if not (isinstance(v, _PVec) and len(v.comps) == shape[0]):
                raise TaichiLoweringError(f"loop state {nm!r} changes its vector length")
            for c, cv in enumerate(v.comps):
                new_state[f"{nm}.{c}"] = cv
        else:
            if isinstance(v, _PVec):
                raise TaichiLoweringError(f"loop state {nm!r} changes from a scalar to a vector")
            new_state[nm] = v
    # after the loop: states hold their final values, the counter the loop's count
    for nm, shape in names.items():
        local[nm] = _PVec([b.state(f"{nm}.{c}") for c in range(shape[0])]) if shape else b.state(nm)
    if counter is not None:
        # a trip that broke out did not reach its `counter += 1`
        local[counter] = ip.arith("sub", b.count(), b.state(_BRK)) if brk else b.count()
    for nm in assigned:
        if nm not in state and nm != counter:
            local.pop(nm, None)
    return init, test_out, new_state, max_iter
