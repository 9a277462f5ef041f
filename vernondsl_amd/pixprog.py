"""Compiler of per-pixel programs to vdsl_pixel_program (include/vdsl.h).

A per-pixel program is what the body of a Taichi struct-for over a 2-D field computes for one pixel
(the reference's `paint`, fractal.py:16-25, is one): values are expression DAGs over the pixel
indices, other fields read at the same pixel, constants and, inside its one check-then-update loop
(fractal.py:22-24), the loop-carried state.  `compile_program` lowers such a program to the four
sections the device runs (pre, loop test, loop body, post) on 32 f32 registers:

    b = Builder()
    c_re = b.op("add", b.op("mul", b.op("div", b.index(0), 1024.0), 3.0), -2.0)   # any DAG
    prog = compile_program(b, init={"zr": 0.0, "zi": 0.0}, test=("le", mag, 4.0),
                           body={"zr": ..., "zi": ...}, max_iter=256, out=COUNT)

Every operation rounds once in f32 where it is written, as the device and the CPU oracle run it:
`a - c` for a constant c is emitted as a + (-c) and `a * c` as a multiply by an immediate (both
exact rewrites), a division stays a division.  Constants are folded in f32 before they get here.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

MAX_INSTR, MAX_REGS, MAX_INPUTS = 256, 32, 8
OP = dict(_lib.MAP_OPS)
OP.update({"index": 32, "cos": 33, "sin": 34, "count": 35, "lt": 36, "le": 37, "eq": 38, "ne": 39, "select": 40,
           "floor": 41, "load_at": 42, "trip": 43, "atomic_add": 44, "trunc": 45, "atomic_max": 46, "atomic_min": 47,
           "store_at": 48, "random": 49, "atan2": 50, "asin": 51, "acos": 52, "atan": 53, "tan": 54, "powf": 55,
           "band": 56, "bor": 57, "bxor": 58, "shl": 59, "shr": 60, "round": 61})
SCATTERS = ("atomic_add", "atomic_max", "atomic_min", "store_at")  # effect nodes: no result register
TESTS = {"none": 0, "lt": 1, "le": 2, "gt": 3, "ge": 4}
OUT_REG, OUT_COUNT, OUT_I32, OUT_NONE = 0, 1, 2, 3
F32, I32 = _lib.F32, _lib.I32  # input dtypes (vdsl_dtype)
COUNT = "count"  # compile_program(out=COUNT): store the loop's update count (an int32 field)

UNARY = ("neg", "abs", "sqrt", "exp", "log", "tanh", "sigmoid", "cos", "sin", "recip", "square", "floor", "trunc",
         "asin", "acos", "atan", "tan", "round")
BINARY = ("add", "sub", "mul", "div", "max", "min", "lt", "le", "eq", "ne", "atan2", "powf",
          "band", "bor", "bxor", "shl", "shr")  # comparisons give 1.0 / 0.0; bit operations of int32 values
TERNARY = ("fma", "select")  # select(c, a, b): a where c != 0 (NaN included), else b


class PixelProgram(C.Structure):
    # Same layout as vdsl_pixel_program (include/vdsl.h).
    _fields_ = [("n_pre", C.c_int32), ("n_test", C.c_int32), ("n_body", C.c_int32), ("n_post", C.c_int32),
                ("loop", C.c_int32), ("max_iter", C.c_int32), ("test", C.c_int32), ("test_a", C.c_int32),
                ("test_b", C.c_int32), ("out_kind", C.c_int32), ("out_width", C.c_int32), ("out_regs", C.c_int32 * 4),
                ("in_widths", C.c_int32 * MAX_INPUTS), ("in_dtypes", C.c_int32 * MAX_INPUTS),
                ("in_rows", C.c_int32 * MAX_INPUTS), ("in_cols", C.c_int32 * MAX_INPUTS),
                ("code", _lib.MapInstr * MAX_INSTR)]


class ProgramError(ValueError):
    """The program does not fit the device form (too many registers or instructions, bad ops)."""


class Node:
    """A hash-consed expression node: kind in const / index / load / state / count / <op>."""
    __slots__ = ("kind", "args", "val", "key", "deps")

    def __repr__(self):
        return self.text(4)

    def text(self, depth):
        """The expression as text, subexpressions below `depth` levels written as `...` (nodes are
        shared, so written out in full the text can grow exponentially)."""
        if self.kind == "const":
            return repr(float(self.val))
        if self.kind in ("index", "load", "state"):
            return f"{self.kind}({self.val})"
        if self.kind in ("count", "trip"):
            return self.kind
        if depth <= 0:
            return "..."
        return f"{self.kind}({', '.join(a.text(depth - 1) for a in self.args)})"


class Builder:
    """Makes expression nodes; identical expressions are one node (so they are computed once)."""

    def __init__(self):
        self._nodes = {}

    def _node(self, kind, args=(), val=None):
        key = (kind, tuple(id(a) for a in args), None if val is None else (val if kind != "const" else np.float32(val).tobytes()))
        n = self._nodes.get(key)
        if n is None:
            n = Node()
            n.kind, n.args, n.val, n.key = kind, tuple(args), val, key
            deps = set()
            if kind in ("state", "count", "trip"):
                deps.add(kind)
            for a in args:
                deps |= a.deps
            n.deps = frozenset(deps)
            self._nodes[key] = n
        return n

    def const(self, v) -> Node:
        return self._node("const", val=np.float32(v))

    def index(self, axis: int) -> Node:
        return self._node("index", val=int(axis))

    def load(self, k: int, component: int = 0) -> Node:
        """Component `component` of input field k at this pixel."""
        if not 0 <= k < MAX_INPUTS:
            raise ProgramError(f"at most {MAX_INPUTS} input fields")
        if not 0 <= component < 4:
            raise ProgramError("a field has at most 4 components")
        return self._node("load", val=(int(k), int(component)))

    def load_at(self, k: int, row, col, component: int = 0) -> Node:
        """Component `component` of input field k at [row][col] (per-pixel values, clamped to the
        field when the program runs)."""
        if not 0 <= k < MAX_INPUTS:
            raise ProgramError(f"at most {MAX_INPUTS} input fields")
        args = tuple(a if isinstance(a, Node) else self.const(a) for a in (row, col))
        return self._node("load_at", args, val=(int(k), int(component)))

    def scatter_add(self, k: int, row, col, value, component: int = 0, op: str = "add") -> Node:
        """The effect `input k [row][col] (component) += value` (an atomic add; op "max" / "min":
        the element becomes the max / min of itself and value; dropped where the indices fall
        outside field k), for compile_program(effects=...)."""
        if op not in ("add", "max", "min", "store"):
            raise ProgramError(f"unknown scatter op {op!r}")
        if not 0 <= k < MAX_INPUTS:
            raise ProgramError(f"at most {MAX_INPUTS} input fields")
        if not 0 <= component < 4:
            raise ProgramError("a field has at most 4 components")
        args = tuple(a if isinstance(a, Node) else self.const(a) for a in (row, col, value))
        # never merged with an equal one: two equal adds in a body are two adds
        self._effects = getattr(self, "_effects", 0) + 1
        return self._node("store_at" if op == "store" else "atomic_" + op, args, val=(int(k), int(component), self._effects))

    def random(self, seed, draw: int) -> Node:
        """A uniform number in [0, 1) for this pixel, from seed (a per-pixel value holding an
        integer below 2^24) and the draw index (distinct draws give unrelated numbers)."""
        return self._node("random", (seed if isinstance(seed, Node) else self.const(seed),), val=int(draw))

    def state(self, name: str) -> Node:
        return self._node("state", val=name)

    def count(self) -> Node:
        return self._node("count")

    def trip(self) -> Node:
        """The loop's trip (updates made before it, as a float): the same on every lane still in
        the loop; the test and the body may read it."""
        return self._node("trip")

    def op(self, kind: str, *args) -> Node:
        args = tuple(a if isinstance(a, Node) else self.const(a) for a in args)
        if kind in UNARY:
            assert len(args) == 1, kind
        elif kind in BINARY:
            assert len(args) == 2, kind
        elif kind in TERNARY:
            assert len(args) == 3, kind
        else:
            raise ProgramError(f"unknown operation {kind!r}")
        return self._node(kind, args)


def _invariant(n: Node) -> bool:
    return not n.deps


class _Emitter:
    """Emits instructions into one section with a linear-scan register allocation over the
    registers not pinned by the program (state and hoisted values)."""

    def __init__(self, code, pinned: dict, reserved: set):
        self.code = code            # shared instruction list
        self.pinned = pinned        # Node -> register held for the whole program
        self.reserved = set(reserved)

    def emit(self, roots):
        """Computes every root; returns {root: register}.  Registers of non-root temporaries are
        freed after their last use."""
        order, seen = [], set()

        def visit(n):
            if id(n) in seen or n in self.pinned:
                return
            seen.add(id(n))
            skip = self._imm_arg(n)
            for k, a in enumerate(n.args):
                if k != skip:
                    visit(a)
            order.append(n)

        for r in roots:
            visit(r)
        last = {}
        for pos, n in enumerate(order):
            skip = self._imm_arg(n)
            for k, a in enumerate(n.args):
                if k != skip:
                    last[id(a)] = pos
        root_ids = {id(r) for r in roots}
        free = [r for r in range(MAX_REGS) if r not in self.reserved]
        reg = {}
        for pos, n in enumerate(order):
            skip = self._imm_arg(n)
            srcs = [None if k == skip else (self.pinned[a] if a in self.pinned else reg[id(a)]) for k, a in enumerate(n.args)]
            # operands whose last use is here free their registers before the result is placed
            for k, a in enumerate(n.args):
                if k == skip:
                    continue
                if a not in self.pinned and id(a) not in root_ids and last.get(id(a)) == pos and reg.get(id(a)) is not None:
                    free.append(reg[id(a)])
                    reg[id(a)] = None
            if n.kind in SCATTERS:  # an effect: reads its operands, writes no register
                self._instr(n, None, srcs)
                continue
            if not free:
                raise ProgramError(f"the program needs more than {MAX_REGS} registers")
            dst = min(free)
            free.remove(dst)
            reg[id(n)] = dst
            self._instr(n, dst, srcs)
        out = {}
        for r in roots:
            out[r] = self.pinned[r] if r in self.pinned else reg.get(id(r))
        return out

    def _imm_arg(self, n):
        """Index of the constant operand an add / mul / sub of n takes as an immediate, or None."""
        if n.kind in ("add", "mul"):
            if n.args[1].kind == "const" and n.args[1] not in self.pinned:
                return 1
            if n.args[0].kind == "const" and n.args[0] not in self.pinned:
                return 0
        if n.kind == "sub" and n.args[1].kind == "const" and n.args[1] not in self.pinned:
            return 1
        return None

    def _instr(self, n, dst, srcs):
        k, imm, a, b, c = n.kind, 0.0, 0, 0, 0
        if k == "const":
            op, imm = OP["const"], float(n.val)
        elif k == "index":
            op, a = OP["index"], n.val
        elif k == "load":
            op, a, c = OP["load"], n.val[0], n.val[1]
        elif k == "load_at":
            op, a, b, c, imm = OP["load_at"], n.val[0], srcs[0], srcs[1], float(n.val[1])
        elif k in SCATTERS:  # dst names the register of the value added (or compared)
            op, dst, a, b, c, imm = OP[k], srcs[2], n.val[0], srcs[0], srcs[1], float(n.val[1])
        elif k == "random":
            op, a, imm = OP["random"], srcs[0], float(n.val)
        elif k == "count":
            op = OP["count"]
        elif k == "trip":
            op = OP["trip"]
        elif k == "state":
            raise ProgramError(f"state {n.val!r} read outside the loop's registers")
        elif k in ("add", "mul") and n.args[1].kind == "const" and n.args[1] not in self.pinned:
            op, a, imm = OP[k + "_imm"], srcs[0], float(n.args[1].val)
        elif k in ("add", "mul") and n.args[0].kind == "const" and n.args[0] not in self.pinned:
            op, a, imm = OP[k + "_imm"], srcs[1], float(n.args[0].val)
        elif k == "sub" and n.args[1].kind == "const" and n.args[1] not in self.pinned:
            op, a, imm = OP["add_imm"], srcs[0], float(-n.args[1].val)  # a - c == a + (-c) exactly
        elif k in UNARY:
            op, a = OP[k], srcs[0]
        elif k in BINARY:
            op, a, b = OP[k], srcs[0], srcs[1]
        elif k in TERNARY:
            op, a, b, c = OP[k], srcs[0], srcs[1], srcs[2]
        else:
            raise ProgramError(f"cannot emit {k!r}")
        if len(self.code) >= MAX_INSTR:
            raise ProgramError(f"the program needs more than {MAX_INSTR} instructions")
        ins = _lib.MapInstr()
        ins.op, ins.dst, ins.a, ins.b, ins.c, ins.imm = op, dst, a, b, c, np.float32(imm)
        self.code.append(ins)


def _node_of(b: Builder, v) -> Node:
    return v if isinstance(v, Node) else b.const(v)


def compile_program(b: Builder, init: dict | None = None, test=None, body: dict | None = None, max_iter: int = 0,
                    out=None, loop: bool | None = None, in_widths=(), in_dtypes=(), out_i32: bool = False,
                    in_extents=(), effects=()) -> PixelProgram:
    """init: {state name: initial Node or number}; test: (op, lhs, rhs) with op in lt/le/gt/ge (None:
    no test), both sides per-pixel values; body: {state name: new value} (the parallel update of
    one loop trip; names not listed keep their value); max_iter: most updates; out: the stored
    value (a Node using states, count() and invariants; a list or tuple of 1-4 of them for a
    field of vectors) or COUNT.  loop defaults to whether a body or test is given.  in_widths:
    components per pixel of each input field (default 1); in_dtypes: F32 or I32 per input (an
    int32 field of one component, read as float); out_i32: store the (single) value into an int32
    field, truncating as a Taichi int field assignment does.  in_extents: (rows, cols) per input of
    another shape than the grid (read only by load_at, clamped to those extents), or None.
    effects: Builder.scatter_add nodes, run after the loop (their order is that of the list);
    out may then be None (a program that stores nothing per pixel)."""
    init = dict(init or {})
    body = dict(body or {})
    effects = list(effects)
    loop = bool(body or test) if loop is None else bool(loop)
    if out is None and not effects:
        raise ProgramError("no output")
    for e in effects:
        if not isinstance(e, Node) or e.kind not in SCATTERS:
            raise ProgramError("effects are scatter_add nodes")
        if "trip" in e.deps:
            raise ProgramError("a scatter-add inside a runtime loop is not supported (only before or after it)")
        if not loop and "count" in e.deps:
            raise ProgramError("the count needs a loop")
    for name in body:
        if name not in init:
            raise ProgramError(f"loop state {name!r} has no initial value")
    state_names = list(init)
    nodes_test = [] if test is None else [_node_of(b, v) for v in test[1:]]
    nodes_body = [_node_of(b, body[nm]) for nm in body]
    outs = [] if out is COUNT or out is None else [_node_of(b, v) for v in (out if isinstance(out, (list, tuple)) else [out])]
    if out is not COUNT and out is not None and not 1 <= len(outs) <= 4:
        raise ProgramError("a pixel stores 1 to 4 components")
    out_node = outs[0] if outs else None
    init_nodes = [_node_of(b, init[nm]) for nm in state_names]
    for n in nodes_test + nodes_body:
        if "count" in n.deps:
            raise ProgramError("the loop count can only be read after the loop")
    for n in init_nodes:
        if n.deps:
            raise ProgramError("an initial value reads loop state, the trip or the count")
    if any("trip" in n.deps for n in outs):
        raise ProgramError("the trip can only be read inside the loop")
    if not loop and (out is COUNT or any("count" in n.deps for n in outs)):
        raise ProgramError("the count needs a loop")
    # Registers pinned for the whole program: one per state, then each maximal loop-invariant
    # subexpression the loop reads (computed once, in pre) and each constant the test compares.
    pinned, reg_next = {}, 0
    for nm in state_names:
        pinned[b.state(nm)] = reg_next
        reg_next += 1
    hoist = []

    def collect(n):
        if n in pinned or n.kind == "const":
            return
        if _invariant(n):
            pinned[n] = None
            hoist.append(n)
            return
        for a in n.args:
            collect(a)

    for n in nodes_test + nodes_body:
        collect(n)
    for n in nodes_test:
        if n.kind == "const" and n not in pinned:
            pinned[n] = None
            hoist.append(n)
    for n in hoist:
        pinned[n] = reg_next
        reg_next += 1
    if reg_next > MAX_REGS:
        raise ProgramError(f"the program needs more than {MAX_REGS} registers")
    reserved = set(pinned.values())
    code = []
    # pre: each hoisted value, then each initial state, computed in turn and moved to its register
    # (values computed earlier are reused by later ones)
    avail = {}
    for n in hoist:
        r = _Emitter(code, avail, reserved).emit([n])[n]
        _move(code, r, pinned[n])
        avail[n] = pinned[n]
    for nm, n in zip(state_names, init_nodes):
        r = _Emitter(code, avail, reserved).emit([n])[n]
        _move(code, r, pinned[b.state(nm)])
    n_pre = len(code)
    test_kind, ta, tb = TESTS["none"], 0, 0
    n_test = n_body = 0
    if loop:
        if test is not None:
            if test[0] not in ("lt", "le", "gt", "ge"):
                raise ProgramError(f"unknown test {test[0]!r}")
            tr = _Emitter(code, pinned, reserved).emit(nodes_test)
            test_kind, ta, tb = TESTS[test[0]], tr[nodes_test[0]], tr[nodes_test[1]]
            n_test = len(code) - n_pre
        br = _Emitter(code, pinned, reserved).emit(nodes_body) if nodes_body else {}
        # Parallel update: a new value held in another state's register is copied to a free
        # temporary first, so no state is overwritten before every new value has been read.
        state_regs = {pinned[b.state(s)] for s in state_names}
        free = [r for r in range(MAX_REGS) if r not in reserved and r not in br.values()]
        staged = {}
        for nm, n in zip(body, nodes_body):
            r = br[n]
            if r in state_regs and r != pinned[b.state(nm)]:
                if not free:
                    raise ProgramError(f"the program needs more than {MAX_REGS} registers")
                t = free.pop(0)
                _move(code, r, t)
                r = t
            staged[nm] = r
        for nm, r in staged.items():
            _move(code, r, pinned[b.state(nm)])
        n_body = len(code) - n_pre - n_test
    out_kind, out_regs = OUT_REG, [0]
    # the post section: the stored value(s), and the effects (whose operands stay live only
    # until their add; the stored registers are held to the end)
    regs = _Emitter(code, pinned, reserved).emit(outs + effects)
    if out is COUNT:
        out_kind = OUT_COUNT
    elif out is None:
        out_kind = OUT_NONE
    else:
        out_regs = [regs[n] for n in outs]
        if out_i32:
            if len(outs) != 1:
                raise ProgramError("an int32 field stores one value per pixel")
            out_kind = OUT_I32
    n_post = len(code) - n_pre - n_test - n_body
    p = PixelProgram()
    p.n_pre, p.n_test, p.n_body, p.n_post = n_pre, n_test, n_body, n_post
    p.loop, p.max_iter = int(loop), int(max_iter)
    p.test, p.test_a, p.test_b = test_kind, ta, tb
    p.out_kind, p.out_width = out_kind, len(out_regs)
    for k, r in enumerate(out_regs):
        p.out_regs[k] = r
    widths = list(in_widths) + [1] * (MAX_INPUTS - len(in_widths))
    dtypes = list(in_dtypes) + [F32] * (MAX_INPUTS - len(in_dtypes))
    for k in range(MAX_INPUTS):
        if not 1 <= widths[k] <= 4:
            raise ProgramError("an input field has 1 to 4 components")
        if dtypes[k] not in (F32, I32) or (dtypes[k] == I32 and widths[k] != 1):
            raise ProgramError("an input field is f32, or int32 of one component")
        p.in_widths[k] = widths[k]
        p.in_dtypes[k] = dtypes[k]
    for k, ext in enumerate(in_extents):
        if ext is not None:
            p.in_rows[k], p.in_cols[k] = int(ext[0]), int(ext[1])
    for k, ins in enumerate(code):
        p.code[k] = ins
    return p


def _move(code, src, dst):
    if src == dst:
        return
    if len(code) >= MAX_INSTR:
        raise ProgramError(f"the program needs more than {MAX_INSTR} instructions")
    ins = _lib.MapInstr()
    ins.op, ins.dst, ins.a = OP["mov"], dst, src
    code.append(ins)


def describe(p: PixelProgram) -> str:
    """The program as text, one instruction per line (for error messages and tests)."""
    names = {v: k for k, v in OP.items()}
    lines = []
    total = p.n_pre + p.n_test + p.n_body + p.n_post
    for k in range(total):
        s = p.code[k]
        sec = "pre" if k < p.n_pre else "test" if k < p.n_pre + p.n_test else "body" if k < p.n_pre + p.n_test + p.n_body else "post"
        if s.op in (OP["atomic_add"], OP["atomic_max"], OP["atomic_min"], OP["store_at"]):
            sym = {OP["atomic_add"]: "+=", OP["atomic_max"]: "max=", OP["atomic_min"]: "min=", OP["store_at"]: "="}[s.op]
            lines.append(f"{sec:4s} input{s.a}[r{s.b}][r{s.c}].{int(s.imm)} {sym} r{s.dst}")
            continue
        lines.append(f"{sec:4s} r{s.dst} = {names.get(s.op, s.op)} a={s.a} b={s.b} c={s.c} imm={s.imm:g}")
    return "\n".join(lines)
