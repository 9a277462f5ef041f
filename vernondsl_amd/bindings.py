"""Binding-model reader for `vernon.semantic` function signatures, without MLIR.

The reference's only lowering pass walks the arguments of `vertex_main`, reads each
`vernon.semantic` string attribute and maps it to a SPIR-V storage class
(VernonToSpirv.cpp:34-58); its test input declares such signatures (color.mlir:4-9, 43-45).
This module reads the same textual form,

    func.func @name(%pos: tensor<3xf32> {vernon.semantic = "input"}, ...)
                    -> (tensor<4xf32> {vernon.semantic="output"}, ...)

and returns one Binding per argument and result: name, shape, element type and the RHI binding
kind (vdsl_binding) the semantic maps to.  Unlike the pass it reports a missing function or an
unknown semantic as an error instead of crashing (VernonToSpirv.cpp:34-36) or reading an
uninitialised storage class (:43,57).  `allocate()` turns the bindings into device buffers.
"""
from __future__ import annotations

import re
from dataclasses import dataclass

from . import _lib

_ELEM = {"f32": "f32", "bf16": "bf16", "i8": "i8", "i32": "i32"}


class BindingError(ValueError):
    pass


@dataclass
class Binding:
    name: str           # "%pos" for arguments, "result0".. for results
    shape: tuple
    dtype: str
    semantic: str
    binding: int        # vdsl_binding
    is_result: bool


def _split_top(s: str, sep: str = ","):
    """Splits on `sep` outside <...>, (...), {...} and quotes."""
    out, depth, cur, q = [], 0, [], False
    for ch in s:
        if ch == '"':
            q = not q
        elif not q and ch in "<({":
            depth += 1
        elif not q and ch in ">)}":
            depth -= 1
        if ch == sep and depth == 0 and not q:
            out.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    tail = "".join(cur).strip()
    if tail:
        out.append(tail)
    return out


def _parse_type(t: str):
    m = re.fullmatch(r"tensor<((?:\d+x)*)(\w+)>", t.strip())
    if not m:
        raise BindingError(f"type {t!r}: only ranked static tensors tensor<AxBx..xT> are supported")
    dims = tuple(int(d) for d in m.group(1).split("x") if d)
    if m.group(2) not in _ELEM:
        raise BindingError(f"element type {m.group(2)!r} is not supported")
    return dims, _ELEM[m.group(2)]


def _semantic(attrs: str):
    m = re.search(r'vernon\.semantic\s*=\s*"([^"]*)"', attrs or "")
    return m.group(1) if m else None


def _binding(sem: str) -> int:
    if sem not in _lib.SEMANTIC_TO_BINDING:
        raise BindingError(f"unknown vernon.semantic {sem!r} (known: {sorted(_lib.SEMANTIC_TO_BINDING)})")
    return _lib.SEMANTIC_TO_BINDING[sem]


def _find_signature(text: str, func: str):
    m = re.search(r"func\.func\s+@" + re.escape(func) + r"\s*\(", text)
    if not m:
        raise BindingError(f"no func.func @{func} in the module")
    i, depth = m.end(), 1
    start = i
    while depth:
        if i >= len(text):
            raise BindingError(f"unbalanced argument list of @{func}")
        depth += {"(": 1, ")": -1}.get(text[i], 0)
        i += 1
    args = text[start:i - 1]
    rest = text[i:]
    results = ""
    r = re.match(r"\s*->\s*", rest)
    if r:
        rest = rest[r.end():]
        if rest.startswith("("):
            j, depth = 1, 1
            while depth:
                depth += {"(": 1, ")": -1}.get(rest[j], 0)
                j += 1
            results = rest[1:j - 1]
        else:
            results = rest.split("{", 1)[0]
    return args, results


def read_bindings(text: str, func: str) -> list:
    """Bindings of @func's arguments and results.  Arguments without a semantic are skipped, as the
    pass skips them (VernonToSpirv.cpp:40-42)."""
    args, results = _find_signature(text, func)
    out = []
    for a in _split_top(args):
        m = re.fullmatch(r"(%[\w.$-]+)\s*:\s*(tensor<[^>]*>)\s*(\{.*\})?", a, flags=re.S)
        if not m:
            raise BindingError(f"argument {a!r} is not `%name: tensor<...> {{attrs}}`")
        sem = _semantic(m.group(3))
        if sem is None:
            continue
        shape, dt = _parse_type(m.group(2))
        out.append(Binding(m.group(1), shape, dt, sem, _binding(sem), False))
    for k, r in enumerate(_split_top(results)):
        m = re.fullmatch(r"(tensor<[^>]*>)\s*(\{.*\})?", r, flags=re.S)
        if not m:
            raise BindingError(f"result {r!r} is not `tensor<...> {{attrs}}`")
        sem = _semantic(m.group(2))
        if sem is None:
            continue
        shape, dt = _parse_type(m.group(1))
        out.append(Binding(f"result{k}", shape, dt, sem, _binding(sem), True))
    return out


def allocate(device, bindings) -> dict:
    """One device tensor per binding, tagged with its binding kind."""
    from .rhi import Tensor
    return {b.name: Tensor(device, b.shape, b.dtype, binding=b.binding) for b in bindings}
