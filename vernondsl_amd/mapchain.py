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
    def __init__(self, index: int, bcast: str = "full", width: int = 1, comp: int = 0):
        if not 0 <= index < _lib.MAP_MAX_INPUTS:
            raise ValueError("input index out of range")
        super().__init__("load", (), 0.0)
        self.index = index
        self.bcast = _BCAST[bcast] if isinstance(bcast, str) else bcast
        self.width = width
        self.comp = comp

    def key(self):
        return ("load", self.index) if self.width == 1 else ("load", self.index, self.comp)


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
    code: list = field(default_factory=list)   # (op, dst, a, b, c, imm); a LOAD's c is its component
    out_reg: int = 0
    bcast: dict = field(default_factory=dict)  # input index -> broadcast code
    widths: dict = field(default_factory=dict)  # input index -> components per element (1..4)
    out_regs: list = field(default_factory=list)  # one register per output component

    @property
    def is_vector(self) -> bool:
        return len(self.out_regs) > 1 or any(w > 1 for w in self.widths.values())

    @property
    def n_inputs(self) -> int:
        return (max(self.bcast) + 1) if self.bcast else 0

    def instr_array(self):
        arr = (_lib.MapInstr * max(1, len(self.code)))()
        for i, (op, dst, a, b, c, imm) in enumerate(self.code):
            arr[i].op, arr[i].dst, arr[i].a, arr[i].b, arr[i].c, arr[i].imm = _lib.MAP_OPS[op], dst, a, b, c, imm
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
        srcs = srcs + [0] * (3 - len(srcs))
        if e.op == "load":
            if prog.bcast.get(e.index, e.bcast) != e.bcast or prog.widths.get(e.index, e.width) != e.width:
                raise ValueError(f"input {e.index} is read with two different broadcasts or widths")
            prog.bcast[e.index] = e.bcast
            prog.widths[e.index] = e.width
            prog.code.append(("load", dst, e.index, 0, e.comp, 0.0))
        else:
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
    return prog
