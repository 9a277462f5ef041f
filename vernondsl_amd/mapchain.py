"""Map-chain front end: elementwise expressions -> vdsl_map_instr register programs.

    x = mc.Input(0)                    # [rows][cols]
    bias = mc.Input(1, bcast="row")    # [cols], shared by every row
    y = mc.tanh(x * 0.75 + (-0.25)) * mc.exp(-(x * x)) + bias
    prog = mc.compile(y)               # instructions, out_reg, input broadcasts

compile() walks the expression depth-first (left operand first), loads each input once (common
sub-expressions are shared), and gives every value the lowest register free at its definition,
after releasing the registers of operands that die there.  The output is deterministic, so the
library's compile-time specialisations (map_chain.hip) are keyed on exactly these programs.
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
    def __init__(self, index: int, bcast: str = "full"):
        if not 0 <= index < _lib.MAP_MAX_INPUTS:
            raise ValueError("input index out of range")
        super().__init__("load", (), 0.0)
        self.index = index
        self.bcast = _BCAST[bcast]

    def key(self):
        return ("load", self.index)


def const(v: float) -> Expr:
    return Expr("const", (), v)


def _e(o) -> Expr:
    return o if isinstance(o, Expr) else const(float(o))


def _unary(name):
    def f(x):
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
    code: list = field(default_factory=list)   # (op, dst, a, b, c, imm)
    out_reg: int = 0
    bcast: dict = field(default_factory=dict)  # input index -> broadcast code

    @property
    def n_inputs(self) -> int:
        return (max(self.bcast) + 1) if self.bcast else 0

    def instr_array(self):
        arr = (_lib.MapInstr * max(1, len(self.code)))()
        for i, (op, dst, a, b, c, imm) in enumerate(self.code):
            arr[i].op, arr[i].dst, arr[i].a, arr[i].b, arr[i].c, arr[i].imm = _lib.MAP_OPS[op], dst, a, b, c, imm
        return arr


def compile(expr: Expr) -> Program:  # noqa: A001 - mirrors the DSL verb
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

    visit(expr)
    reg_of, free, prog = {}, list(range(_lib.MAP_MAX_REGS)), Program()
    remaining = dict(uses)

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
            prog.bcast[e.index] = e.bcast
            prog.code.append(("load", dst, e.index, 0, 0, 0.0))
        else:
            prog.code.append((e.op, dst, srcs[0], srcs[1], srcs[2], e.imm))

    for k in order:
        emit(k)
    if len(prog.code) > _lib.MAP_MAX_INSTR:
        raise ValueError(f"chain has {len(prog.code)} instructions; the limit is {_lib.MAP_MAX_INSTR}")
    prog.out_reg = reg_of[expr.key()]
    for i in range(prog.n_inputs):
        prog.bcast.setdefault(i, _lib.BCAST_FULL)
    return prog
