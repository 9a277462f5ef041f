"""Map-chain front end: elementwise expressions -> vdsl_map_instr register programs.

    x = mc.Input(0)                    # [rows][cols]
    bias = mc.Input(1, bcast="row")    # [cols], shared by every row
    y = mc.tanh(x * 0.75 + (-0.25)) * mc.exp(-(x * x)) + bias
    prog = mc.compile(y)               # instructions, out_reg, input broadcasts

compile() walks the expression depth-first (left operand first), loads each input once (common
sub-expressions are shared), and gives every value the lowest register free at its definition,
after releasing the registers of operands that die there.  The output is deterministic, so the
library's compile-time specialisations (map_chain.hip) are keyed on exactly these programs.

Vector operands follow the vernon dialect's vocabulary (source/README.md:23-55): a VecInput holds
vec2-vec4 elements (AoS); `v.r` / `v.component("r")` is ExtractComponentOp, `v.bgr` /
`v.swizzle("bgr")` is SwizzleOp (component sets xyzw, rgba, stpq, not mixed in one pattern), and
`vec(...)` builds a vector from scalars and vectors (tensor.from_elements, color.mlir:21).
Arithmetic on vectors is per component; a scalar operand applies to every component:

    pos = mc.VecInput(0, 3)                       # [rows][cols][3]
    out = mc.vec(pos.zyx * 2.0, 1.0)              # [rows][cols][4], w = 1
    prog = mc.compile(out)                        # prog.out_regs: one register per component

A MatInput holds mat2-mat4 elements (!vernon.mat2-4, row-major AoS; a uniform by default, as the
mat4 uniforms of color.mlir:5-7).  `M @ v` is linalg.matvec (color.mlir:29-36), `v @ M` the row
vector times M, `M.T` the transposed view, `M[i, j]` / `M.component(k)` ExtractComponentOp on a
matrix, `M[i]` / `M.row(i)` / `M.col(j)` vectors of components:

    model, view, proj = (mc.MatInput(k, 4) for k in (1, 2, 3))
    gl_position = proj @ (view @ (model @ mc.vec(pos, 1.0)))
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import _lib

_BCAST = {"full": _lib.BCAST_FULL, "row": _lib.BCAST_ROW, "col": _lib.BCAST_COL, "scalar": _lib.BCAST_SCALAR}
UNARY = ("neg", "abs", "square", "exp", "log", "tanh", "sigmoid", "relu", "sqrt", "recip")
BINARY = ("add", "sub", "mul", "div", "max", "min")


class Expr:
    op: str
    args: tuple
    imm: float

    def __init__(self, op, args=(), imm=0.0):
        self.op, self.args, self.imm = op, tuple(args), float(imm)

    def key(self):
        return (self.op, tuple(a.key() for a in self.args), self.imm)

    # arithmetic -----------------------------------------------------------------------------
    def __add__(self, o):
        return Expr("add_imm", (self,), o) if isinstance(o, (int, float)) else Expr("add", (self, _e(o)))

    def __radd__(self, o):
        return self.__add__(o)

    def __sub__(self, o):
        return Expr("add_imm", (self,), -float(o)) if isinstance(o, (int, float)) else Expr("sub", (self, _e(o)))

    def __rsub__(self, o):
        return Expr("sub", (_e(o), self))

    def __mul__(self, o):
        if isinstance(o, (int, float)):
            return Expr("mul_imm", (self,), o)
        o = _e(o)
        if o is self or o.key() == self.key():
            return Expr("square", (self,))
        return Expr("mul", (self, o))

    def __rmul__(self, o):
        return self.__mul__(o)

    def __truediv__(self, o):
        return Expr("div", (self, _e(o)))

    def __rtruediv__(self, o):
        return Expr("div", (_e(o), self))

    def __neg__(self):
        return Expr("neg", (self,))


class Input(Expr):
    def __init__(self, index: int, bcast: str = "full", width: int = 1, comp: int = 0, mat_dim: int = 0):
        if not 0 <= index < _lib.MAP_MAX_INPUTS:
            raise ValueError("input index out of range")
        super().__init__("load", (), 0.0)
        self.index = index
        self.bcast = _BCAST[bcast] if isinstance(bcast, str) else bcast
        self.width = width
        self.comp = comp
        self.mat_dim = mat_dim

    def key(self):
        # the operand's type is part of the key, so that one input read under two types is not
        # merged into one load (compile() then rejects it)
        return ("load", self.index, self.comp, self.bcast, self.width, self.mat_dim)


_SETS = ("xyzw", "rgba", "stpq")


def _components(pattern: str, width: int) -> list:
    """Component indices of a swizzle pattern over a vector of `width` components."""
    if not 1 <= len(pattern) <= 4:
        raise ValueError(f"swizzle {pattern!r}: 1 to 4 components")
    for s in _SETS:
        if all(ch in s for ch in pattern):
            idx = [s.index(ch) for ch in pattern]
            if max(idx) >= width:
                raise ValueError(f"swizzle {pattern!r} reads past a vec{width}")
            return idx
    raise ValueError(f"swizzle {pattern!r}: components must come from one of {', '.join(_SETS)}")


class Vec:
    """A vector value: one scalar Expr per component (vec2-vec4)."""

    def __init__(self, comps):
        comps = [_e(c) for c in comps]
        if not 1 <= len(comps) <= 4:
            raise ValueError("vectors have 1 to 4 components")
        self.comps = comps

    @property
    def width(self):
        return len(self.comps)

    def __getitem__(self, i: int) -> Expr:
        return self.comps[i]

    def component(self, c) -> Expr:
        """ExtractComponentOp: component `c` ("x"/"r"/... or an index)."""
        return self.comps[_components(c, self.width)[0] if isinstance(c, str) else c]

    def swizzle(self, pattern: str):
        """SwizzleOp: the components named by `pattern`, in its order (one name gives a scalar)."""
        idx = _components(pattern, self.width)
        return self.comps[idx[0]] if len(idx) == 1 else Vec([self.comps[i] for i in idx])

    def __getattr__(self, name):
        if name.startswith("_") or not name.isalpha():
            raise AttributeError(name)
        try:
            return self.swizzle(name)
        except ValueError as e:
            raise AttributeError(str(e)) from None

    def _zip(self, o, fn):
        if isinstance(o, Vec):
            if o.width != self.width:
                raise ValueError(f"vec{self.width} and vec{o.width} operands")
            return Vec([fn(a, b) for a, b in zip(self.comps, o.comps)])
        return Vec([fn(a, o) for a in self.comps])

    def __add__(self, o):
        return self._zip(o, lambda a, b: a + b)

    def __radd__(self, o):
        return self._zip(o, lambda a, b: b + a)

    def __sub__(self, o):
        return self._zip(o, lambda a, b: a - b)

    def __rsub__(self, o):
        return self._zip(o, lambda a, b: _e(b) - a)

    def __mul__(self, o):
        return self._zip(o, lambda a, b: a * b)

    def __rmul__(self, o):
        return self._zip(o, lambda a, b: b * a if isinstance(b, Expr) else a * b)

    def __truediv__(self, o):
        return self._zip(o, lambda a, b: a / b)

    def __neg__(self):
        return Vec([-a for a in self.comps])


class VecInput(Vec):
    """Input `index` whose elements are vec`width` (AoS: [rows][cols][width] for a full input,
    [cols][width] row-broadcast, [rows][width] column-broadcast, [width] scalar)."""

    def __init__(self, index: int, width: int, bcast: str = "full"):
        if not 1 <= width <= 4:
            raise ValueError("vector inputs have 1 to 4 components")
        super().__init__([Input(index, bcast, width, c) for c in range(width)])
        self.index = index


class MatVec(Expr):
    """One component of a matrix-vector product: row `row` of matrix input `mat` times the vector
    (op "matvec", linalg.matvec), or the vector times column `row` (op "vecmat")."""

    def __init__(self, op: str, mat: "MatInput", row: int, comps):
        super().__init__(op, comps, 0.0)
        self.mat, self.row = mat, row

    def key(self):
        return (self.op, self.mat.index, self.row, tuple(a.key() for a in self.args))


class MatInput:
    """Input `index` whose elements are dim x dim matrices (mat2 / mat3 / mat4), row-major AoS:
    [rows][cols][dim][dim] for a full input, [cols][dim][dim] row-broadcast, [rows][dim][dim]
    column-broadcast, [dim][dim] for a uniform (bcast "scalar", the default).  `transposed` views
    the same operand as its transpose (no data moves: products and extraction swap indices)."""

    def __init__(self, index: int, dim: int, bcast: str = "scalar", transposed: bool = False):
        if dim not in (2, 3, 4):
            raise ValueError("matrix inputs are mat2, mat3 or mat4")
        if not 0 <= index < _lib.MAP_MAX_INPUTS:
            raise ValueError("input index out of range")
        self.index, self.dim, self.transposed = index, dim, transposed
        self.bcast = _BCAST[bcast] if isinstance(bcast, str) else bcast

    @property
    def T(self) -> "MatInput":
        m = MatInput(self.index, self.dim, "full", not self.transposed)
        m.bcast = self.bcast
        return m

    def _flat(self, i: int, j: int) -> int:
        d = self.dim
        if not (0 <= i < d and 0 <= j < d):
            raise IndexError(f"mat{d} index ({i}, {j}) out of range")
        return j * d + i if self.transposed else i * d + j

    def _load(self, flat: int) -> Input:
        return Input(self.index, self.bcast, self.dim * self.dim, flat, self.dim)

    def component(self, k) -> Expr:
        """ExtractComponentOp on a matrix: component k of the row-major view (k = i * dim + j), or
        k = (i, j)."""
        i, j = k if isinstance(k, tuple) else divmod(int(k), self.dim)
        return self._load(self._flat(i, j))

    def row(self, i: int) -> Vec:
        return Vec([self.component((i, j)) for j in range(self.dim)])

    def col(self, j: int) -> Vec:
        return Vec([self.component((i, j)) for i in range(self.dim)])

    def __getitem__(self, k):
        return self.component(k) if isinstance(k, tuple) else self.row(k)

    def _product(self, v, left: bool) -> Vec:
        v = v if isinstance(v, Vec) else Vec(v)
        if v.width != self.dim:
            raise ValueError(f"mat{self.dim} times a vec{v.width}")
        # M v takes rows of M; v M (= M^T v) takes its columns; the transposed view swaps them.
        rows_of_stored = left != self.transposed
        op = "matvec" if rows_of_stored else "vecmat"
        return Vec([MatVec(op, self, i, v.comps) for i in range(self.dim)])

    def __matmul__(self, v) -> Vec:
        """M @ v: linalg.matvec, out[i] = ((0 + M[i][0] v0) + M[i][1] v1) + ..."""
        return self._product(v, True)

    def __rmatmul__(self, v) -> Vec:
        """v @ M: out[j] = ((0 + v0 M[0][j]) + v1 M[1][j]) + ..."""
        return self._product(v, False)


def matvec(m: MatInput, v) -> Vec:
    """linalg.matvec (color.mlir:29-36): m @ v."""
    return m @ v


def vec(*parts) -> Vec:
    """tensor.from_elements: a vector from scalars (Expr or numbers) and vectors, in order."""
    comps = []
    for p in parts:
        comps.extend(p.comps if isinstance(p, Vec) else [_e(p)])
    return Vec(comps)


def const(v: float) -> Expr:
    return Expr("const", (), v)


def _e(o) -> Expr:
    return o if isinstance(o, Expr) else const(float(o))


def _unary(name):
    def f(x):
        if isinstance(x, Vec):
            return Vec([Expr(name, (c,)) for c in x.comps])
        return Expr(name, (_e(x),))
    f.__name__ = name
    return f


for _n in UNARY:
    globals()[_n] = _unary(_n)


def maximum(a, b):
    return Expr("max", (_e(a), _e(b)))


def minimum(a, b):
    return Expr("min", (_e(a), _e(b)))


def fma(a, b, c):
    """a * b + c with one rounding."""
    return Expr("fma", (_e(a), _e(b), _e(c)))


@dataclass
class Program:
    # (op, dst, a, b, c, imm), plus ext (the registers of vector components 1..3) for MATVEC /
    # VECMAT; a LOAD's c is its component
    code: list = field(default_factory=list)
    out_reg: int = 0
    bcast: dict = field(default_factory=dict)  # input index -> broadcast code
    widths: dict = field(default_factory=dict)  # input index -> components per element (1..4, or dim^2)
    out_regs: list = field(default_factory=list)  # one register per output component
    dims: dict = field(default_factory=dict)  # input index -> matrix dimension (0: a vector)

    @property
    def is_vector(self) -> bool:
        return len(self.out_regs) > 1 or any(w > 1 for w in self.widths.values())

    @property
    def n_inputs(self) -> int:
        return (max(self.bcast) + 1) if self.bcast else 0

    def instr_array(self):
        arr = (_lib.MapInstr * max(1, len(self.code)))()
        for i, ins in enumerate(self.code):
            op, dst, a, b, c, imm = ins[:6]
            arr[i].op, arr[i].dst, arr[i].a, arr[i].b, arr[i].c, arr[i].imm = _lib.MAP_OPS[op], dst, a, b, c, imm
            for k, r in enumerate(ins[6] if len(ins) > 6 else ()):
                arr[i].ext[k] = r
        return arr


def compile(expr) -> Program:  # noqa: A001 - mirrors the DSL verb
    """An Expr compiles to a scalar-output program; a Vec to one output register per component."""
    outs = list(expr.comps) if isinstance(expr, Vec) else [expr]
    # Deduplicate nodes and count uses.
    nodes, uses, order = {}, {}, []

    def visit(e):
        k = e.key()
        if k in nodes:
            uses[k] += 1
            return
        nodes[k] = e
        uses[k] = 1
        for a in e.args:
            visit(a)
        order.append(k)

    for o in outs:
        visit(o)
    reg_of, free, prog = {}, list(range(_lib.MAP_MAX_REGS)), Program()
    remaining = dict(uses)
    for o in outs:  # an output's register stays live to the end
        remaining[o.key()] += 1

    def emit(k):
        e = nodes[k]
        srcs = [reg_of[a.key()] for a in e.args]
        for a in e.args:  # operands whose last use is here release their registers first
            ak = a.key()
            remaining[ak] -= 1
            if remaining[ak] == 0:
                free.append(reg_of[ak])
        free.sort()
        if not free:
            raise ValueError(f"expression needs more than {_lib.MAP_MAX_REGS} live registers")
        dst = free.pop(0)
        reg_of[k] = dst

        def declare(index, bcast, width, dim):
            if (prog.bcast.get(index, bcast) != bcast or prog.widths.get(index, width) != width
                    or prog.dims.get(index, dim) != dim):
                raise ValueError(f"input {index} is read with two different broadcasts, widths or types")
            prog.bcast[index], prog.widths[index], prog.dims[index] = bcast, width, dim

        if e.op == "load":
            declare(e.index, e.bcast, e.width, e.mat_dim)
            prog.code.append(("load", dst, e.index, 0, e.comp, 0.0))
        elif e.op in ("matvec", "vecmat"):
            m = e.mat
            declare(m.index, m.bcast, m.dim * m.dim, m.dim)
            ext = tuple(srcs[1:] + [0] * (4 - len(srcs)))
            prog.code.append((e.op, dst, m.index, srcs[0], e.row, 0.0, ext))
        else:
            srcs = srcs + [0] * (3 - len(srcs))
            prog.code.append((e.op, dst, srcs[0], srcs[1], srcs[2], e.imm))

    for k in order:
        emit(k)
    if len(prog.code) > _lib.MAP_MAX_INSTR:
        raise ValueError(f"chain has {len(prog.code)} instructions; the limit is {_lib.MAP_MAX_INSTR}")
    prog.out_regs = [reg_of[o.key()] for o in outs]
    prog.out_reg = prog.out_regs[0]
    for i in range(prog.n_inputs):
        prog.bcast.setdefault(i, _lib.BCAST_FULL)
        prog.widths.setdefault(i, 1)
        prog.dims.setdefault(i, 0)
    return prog
