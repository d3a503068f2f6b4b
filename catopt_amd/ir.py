"""Term model of the delivered forms: the duck-typed surface of catopt's IR.

The executors in this package read terms the way the reference's lowering
code does, through the field names of ``catopt_core.ir`` (luisfuturist/catopt,
``packages/catopt-core/src/catopt_core/ir.py``):

* ``Var(name, typ)`` — a program input (ir.py:74-83);
* ``Param(name, typ)`` — a weight or buffer, bound to a tensor by name
  (ir.py:125-134);
* ``Const(value)`` — a scalar literal, equal by spelling (ir.py:86-122);
* ``Op(op, args, attrs)`` — an operation node, hash-consed through
  ``Op.make`` so equal subterms are one object (ir.py:161-256);
* ``IR(root, inputs, ...)`` — the program (ir.py:666-704).

Terms built by the reference (or decoded from its JSON wire format with
:func:`term_from_data`, ir.py:392-445) are read through exactly these
attributes, so any object with the same fields drops in.  No law, e-graph
or validation machinery lives here: the search stays on the CPU side of
catopt, unchanged.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass, field
from typing import Any, Iterator

__all__ = [
    "TensorType",
    "Var",
    "Param",
    "Const",
    "Op",
    "IR",
    "is_op",
    "postorder",
    "term_to_data",
    "term_from_data",
    "metavariables",
    "ir_from_record",
    "record_from_ir",
]


@dataclass(frozen=True)
class TensorType:
    """A tensor type: its shape (``None`` for an unknown extent)."""

    shape: tuple

    @property
    def size(self) -> int | None:
        if any(d is None for d in self.shape):
            return None
        n = 1
        for d in self.shape:
            n *= int(d)
        return n


@dataclass(frozen=True)
class Var:
    """A program input."""

    name: str
    typ: TensorType = TensorType(())

    def __repr__(self) -> str:
        return self.name


@dataclass(frozen=True)
class Param:
    """A weight or buffer, resolved by name against the parameter values."""

    name: str
    typ: TensorType = TensorType(())

    def __repr__(self) -> str:
        return self.name


@dataclass(frozen=True, eq=False)
class Const:
    """A scalar literal.  Equality is by spelling: ``Const(8) != Const(8.0)``."""

    value: Any

    def __repr__(self) -> str:
        return str(self.value)

    def __eq__(self, other: Any) -> bool:
        if not isinstance(other, Const):
            return NotImplemented
        return repr(self.value) == repr(other.value)

    def __hash__(self) -> int:
        return hash(repr(self.value))


def _key(v: Any) -> Any:
    """Spelling-strict hashable form of an attr value (0 and 0.0 differ)."""
    if isinstance(v, (list, tuple)):
        return (type(v).__name__, tuple(_key(x) for x in v))
    if isinstance(v, dict):
        return ("dict", tuple(sorted((k, _key(x)) for k, x in v.items())))
    return (type(v).__name__, repr(v))


def _attr_key(attrs: dict) -> tuple:
    return tuple(sorted((k, _key(v)) for k, v in attrs.items()))


@dataclass(frozen=True, eq=False)
class Op:
    """An operation node.  Build with :meth:`make`, which interns by structure."""

    op: str
    args: tuple
    attrs: dict = field(default_factory=dict)
    _h: int = field(init=False, repr=False, compare=False, hash=False)
    _ak: tuple = field(init=False, repr=False, compare=False, hash=False)

    _INTERN = weakref.WeakValueDictionary()

    def __post_init__(self) -> None:
        ak = _attr_key(self.attrs)
        object.__setattr__(self, "_ak", ak)
        object.__setattr__(self, "_h", hash((self.op, self.args, ak)))

    @staticmethod
    def make(op: str, *args: Any, **attrs: Any) -> "Op":
        key = (op, tuple(args), _attr_key(attrs))
        hit = Op._INTERN.get(key)
        if hit is not None:
            return hit
        t = Op(op, tuple(args), dict(attrs))
        Op._INTERN[key] = t
        return t

    def __eq__(self, other: Any) -> bool:
        if not isinstance(other, Op):
            return NotImplemented
        if self is other:
            return True
        return self._h == other._h and self.op == other.op and self.args == other.args and self._ak == other._ak

    def __hash__(self) -> int:
        return self._h

    def __repr__(self) -> str:
        parts = [repr(a) for a in self.args]
        if self.attrs:
            parts.append(", ".join(f"{k}={v}" for k, v in self.attrs.items()))
        return f"{self.op}({', '.join(parts)})"


@dataclass
class IR:
    """A program: the root term plus its ordered inputs."""

    root: Any
    inputs: list = field(default_factory=list)
    input_names: set = field(default_factory=set)
    params: dict = field(default_factory=dict)

    def __post_init__(self) -> None:
        if not self.input_names:
            self.input_names = {v.name for v in self.inputs}
        if not self.params:
            self.params = {p.name: p for p in iter_leaves(self.root) if isinstance(p, Param)}

    @property
    def roots(self) -> tuple:
        r = self.root
        if getattr(r, "op", None) == "pack":
            return tuple(r.args)
        return (r,)


def is_op(t: Any, name: str | None = None, nargs: int | None = None) -> bool:
    """``t`` is an Op node (named ``name``, with ``nargs`` operands)."""
    if not isinstance(t, Op) and not (hasattr(t, "op") and hasattr(t, "args") and hasattr(t, "attrs")):
        return False
    if name is not None and t.op != name:
        return False
    return nargs is None or len(t.args) == nargs


def postorder(root: Any) -> list:
    """Distinct Op nodes of the DAG under ``root``, operands before users.

    Iterative, so chains deeper than the interpreter's recursion limit (an
    unrolled scan over thousands of steps) are fine.
    """
    out: list = []
    seen: set = set()
    stack: list = [(root, False)]
    while stack:
        t, expanded = stack.pop()
        if not is_op(t):
            continue
        if expanded:
            out.append(t)
            continue
        if t in seen:
            continue
        seen.add(t)
        stack.append((t, True))
        for a in reversed(t.args):
            if is_op(a) and a not in seen:
                stack.append((a, False))
    return out


def iter_leaves(root: Any) -> Iterator:
    """Distinct non-Op leaves (Var / Param / Const) of ``root``."""
    seen: set = set()
    if not is_op(root):
        yield root
        return
    for t in postorder(root):
        for a in t.args:
            if not is_op(a):
                k = (type(a).__name__, repr(a))
                if k not in seen:
                    seen.add(k)
                    yield a


# ------------------------------------------------------------- wire format
# JSON-safe encoding of terms, the scheme of catopt_core/ir.py:366-445
# (term_to_data / term_from_data), kept alike so terms written by catopt's
# own tools (rule caches, lemma certificates, the intake census) load here:
#   {"mvar": name}                       a pattern metavariable (a bare str leaf)
#   {"const": v}                          Const, v raw (json writes ±inf as ±Infinity)
#   {"var" | "param": name, "shape": [..]} typed leaves
#   {"op": name, "args": [...], "attrs": {k: attr}}
# with tuple / list attrs as {"__tuple__": [...]} / {"__list__": [...]}.


def _attr_to_data(v: Any) -> Any:
    if isinstance(v, tuple):
        return {"__tuple__": [_attr_to_data(x) for x in v]}
    if isinstance(v, list):
        return {"__list__": [_attr_to_data(x) for x in v]}
    if isinstance(v, (str, int, float, bool)) or v is None:
        return v
    raise TypeError(f"unserializable attribute value: {v!r}")


def _attr_from_data(v: Any) -> Any:
    if isinstance(v, dict):
        if "__tuple__" in v:
            return tuple(_attr_from_data(x) for x in v["__tuple__"])
        if "__list__" in v:
            return [_attr_from_data(x) for x in v["__list__"]]
        raise ValueError(f"bad attr encoding: {v!r}")
    return v


def term_to_data(t: Any) -> Any:
    """Encode a term as JSON-safe data (DAG sharing is not preserved)."""
    if isinstance(t, str):
        return {"mvar": t}
    if isinstance(t, Const):
        return {"const": t.value}
    if isinstance(t, Var):
        return {"var": t.name, "shape": list(t.typ.shape)}
    if isinstance(t, Param):
        return {"param": t.name, "shape": list(t.typ.shape)}
    if is_op(t):
        return {
            "op": t.op,
            "args": [term_to_data(a) for a in t.args],
            "attrs": {k: _attr_to_data(v) for k, v in t.attrs.items()},
        }
    raise TypeError(f"unserializable term: {t!r}")


def term_from_data(d: Any) -> Any:
    """Decode :func:`term_to_data` output (interning shared subterms again).
    A metavariable decodes to its bare name, as a pattern leaf."""
    if not isinstance(d, dict) or not d:
        raise ValueError(f"bad term encoding: {d!r}")
    if "mvar" in d:
        return d["mvar"]
    if "const" in d:
        return Const(d["const"])
    if "var" in d:
        return Var(d["var"], TensorType(tuple(d["shape"])))
    if "param" in d:
        return Param(d["param"], TensorType(tuple(d["shape"])))
    if "op" in d:
        return Op.make(d["op"], *[term_from_data(a) for a in d["args"]],
                       **{k: _attr_from_data(v) for k, v in d.get("attrs", {}).items()})
    raise ValueError(f"bad term encoding: {d!r}")


def metavariables(t: Any) -> list:
    """Names of the pattern metavariables (bare str leaves) under ``t``."""
    if isinstance(t, str):
        return [t]
    found: list = []
    seen: set = set()
    for n in postorder(t):
        for a in n.args:
            if isinstance(a, str) and a not in seen:
                seen.add(a)
                found.append(a)
    return found


def ir_from_record(rec: dict) -> IR:
    """The program of one term record ``{"term": ..., "inputs": [{"name",
    "shape"}, ...]}`` (the intake census layout, ``intake/ledger.py:127-138``).
    A term holding pattern metavariables is a law's side, not a program:
    it is rejected with the names it holds."""
    term = term_from_data(rec["term"])
    mv = metavariables(term)
    if mv:
        raise ValueError(f"term {rec.get('name', '?')!r} holds pattern metavariables {mv}: "
                         "a rewrite pattern cannot be lowered")
    inputs = [Var(i["name"], TensorType(tuple(i["shape"]))) for i in rec.get("inputs", [])]
    return IR(term, inputs)


def record_from_ir(name: str, ir: IR) -> dict:
    """The term record of a program (the layout :func:`ir_from_record` reads)."""
    return {
        "name": name,
        "ops": sorted({n.op for n in postorder(ir.root)}),
        "term": term_to_data(ir.root),
        "inputs": [{"name": v.name, "shape": list(v.typ.shape)} for v in ir.inputs],
    }
