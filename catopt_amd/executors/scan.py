"""Affine scan executor (diagonal and dense monoids) on the HIP scan kernels.

The counterpart of ``BatchedScanModule`` (luisfuturist/catopt
``packages/catopt-carriers/src/catopt_carriers/scan_lower.py:427-807``,
``build_scan_plan`` :339-424) and of the fused level bodies
``fused_diag_levels`` / ``fused_dense_levels`` (``scan_fused.py:100-143``)
for both affine carriers:

* diagonal — ``aff_diag`` / ``affd_compose`` / ``applyd``
  (``torch_bridge.py:1895-1900``): ``compose(f, g) = (f.a·g.a, f.a·g.b + f.b)``;
* dense — ``aff`` / ``aff_compose`` / ``apply`` (``torch_bridge.py:1873-1881``):
  ``compose(f, g) = (f.A @ g.A, f.A @ g.b + f.b)``, ``apply(f, h) = f.A @ h + f.b``;

``g`` is applied first.  Two roots are planned per carrier:

* **final state** — ``apply[d](F, h)`` with ``F`` a compose tree over the
  carrier's leaves.  Leaves are read in product order (leaf 0 is the
  outermost map, applied last; ``tests/test_scan_fused.py:105-107``), so time
  runs over the reversed leaf list;
* **every prefix state** — the stacked-map form of ``gather_applyd_stack`` /
  ``gather_apply_stack`` (``xcarrier.py:2252-2293``):
  ``apply[d](pack(stack(proj_a f_0 … f_n), stack(proj_b f_0 … f_n)), h)``
  where each ``f_i = compose(leaf_i, f_{i-1})`` extends the previous prefix by
  one step (checked structurally, not assumed).

A third root extends the reference's (which routes it to the generic
executor): a read-out ``sum(mul(S, c), dim)`` of either root ``S``, the
selective SSM's ``y_t = Σ_n c_t[n]·h_t[…, n]``.  It is planned as the inner
scan followed by ``mul`` / ``sum``; when the leaf offsets are the outer
product ``x_t ⊗ bx_t`` of two gathered step reads and the states stack along
axis 1 of a ``(B, D, N)`` state, scan and read-out run as one SSM kernel
launch and the ``(B, T, D, N)`` states are never written.

As in the reference's plan builder, nested applications are folded into the
compose spine first (``apply(f, apply(g, h)) → apply(compose(f, g), h)``,
``scan_lower.py:131-165``) and pure view wrappers around the root are peeled
off and re-applied to the result (``scan_lower.py:74-118``).

Instead of ``log₂ T`` levels of gathers and batched products
(``scan_lower.py:640-698``), the leaf operands are laid out as step-major
arrays and one kernel walks the steps:

* diagonal: lane-parallel over the state, serial over time in registers, or
  chunk-parallel (local chunk maps, a carry fold over the chunk table, a
  re-scan) when the state is too small to fill the GPU;
* dense: the state columns are batched into fp32 MFMA tiles; a map shared by
  every slot (the LTI ``LinearRecurrence`` case) makes each step one product
  over all ``P·k`` columns, per-slot maps stream from HBM.  The same
  chunk-parallel schedule composes dense chunk maps from the identity.

The chunk table is the reference's blocked all-prefix plan
(``omd_lower.py:771-824``: ``blk = ⌈√T⌉``, starts ``c·blk``) as an int64
array.  When every leaf reads a step of one shared array (``select(X, dim,
t)`` / ``getitem(X, t)``), that array is used in place (or gathered once with
``index_select``) instead of stacking ``T`` slices, and a linear part that is
the same term in every leaf is evaluated once.

The kernels compute in fp32: bf16/fp32 operands run on them (results cast
back to the promoted operand dtype); fp64 and host operands, dense maps with
``d > 64`` and operand shapes outside the two supported dense layouts (vector
state ``h (d,)`` with ``b (d,)``; column state ``h (…, d, k)`` with
``b (…, d, 1)``) run the embedded generic module, counted in ``fallbacks``.
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import nn

from .. import _lib as L
from .. import kernels as K
from ..bindings import attr_of
from ..evaluator import HipIRModule
from ..ir import IR, Op, is_op
from .base import HipExecutorBase

__all__ = [
    "HipScanModule",
    "build_scan_plan",
    "is_scan_apply_term",
    "is_scan_term",
    "to_batched_scan_module",
    "prefix_chunk_table",
    "affd_leaves",
    "map_leaves",
    "fold_nested_apply",
    "strip_output_views",
]

#: per root op: (leaf op, compose op, linear-part projection, offset projection, domain)
_CARRIERS = {
    "applyd": ("aff_diag", "affd_compose", "affd_a", "affd_b", "diag"),
    "apply": ("aff", "aff_compose", "aff_A", "aff_b", "dense"),
}

#: Single-argument view / bookkeeping ops the plan is transparent to around
#: the root (the set of ``scan_lower.py:74-104``): the executor re-applies
#: them, innermost first, to the scan result.
VIEW_OPS = frozenset({
    "reshape", "view", "flatten", "unflatten", "squeeze", "unsqueeze", "expand", "broadcast_to",
    "contiguous", "clone", "detach", "to", "alias", "transpose", "permute", "movedim", "t",
    "select", "getitem", "slice", "chunk", "split", "unbind",
})

#: widest dense state the MFMA kernel holds in registers
DENSE_MAX_D = 64


def prefix_chunk_table(T: int) -> list[int]:
    """Chunk starts of the blocked all-prefix plan plus the end ``T``
    (``omd_lower.py:786-788``: ``blk = ⌈√T⌉``, ``C = ⌈T/blk⌉``)."""
    if T < 1:
        raise ValueError("T must be positive")
    blk = math.isqrt(T - 1) + 1 if T > 1 else 1  # ⌈√T⌉ without float rounding
    C = (T + blk - 1) // blk
    return [c * blk for c in range(C)] + [T]


def map_leaves(F: Any, leaf_op: str, compose_op: str) -> list | None:
    """Leaves of a ``compose_op`` tree in product order, with multiplicity
    (a DAG-shared subtree contributes once per occurrence)."""
    out: list = []
    stack = [F]
    while stack:
        n = stack.pop()
        if is_op(n, compose_op, 2):
            stack.append(n.args[1])
            stack.append(n.args[0])
        elif is_op(n, leaf_op, 2):
            out.append(n)
        else:
            return None
    return out


def affd_leaves(F: Any) -> list | None:
    """``aff_diag`` leaves of an ``affd_compose`` tree in product order."""
    return map_leaves(F, "aff_diag", "affd_compose")


def fold_nested_apply(term: Any) -> Any:
    """``apply(f, apply(g, h)) → apply(compose(f, g), h)`` (and the diagonal
    pair), bottom-up and memoised: one compose tree per application chain
    (``scan_lower.py:131-165``).  Composition is sequential application, so
    the value is unchanged."""
    memo: dict[int, Any] = {}

    def go(t: Any) -> Any:
        if not isinstance(t, Op):
            return t
        key = id(t)
        if key in memo:
            return memo[key]
        args = [go(a) for a in t.args]
        r = t if all(a is b for a, b in zip(args, t.args)) else Op.make(t.op, *args, **dict(t.attrs))
        if r.op in _CARRIERS and len(r.args) == 2:
            comp = _CARRIERS[r.op][1]
            f, h = r.args
            folded = False
            while is_op(h, r.op, 2):
                f = Op.make(comp, f, h.args[0])
                h = h.args[1]
                folded = True
            if folded:
                r = Op.make(r.op, f, h)
        memo[key] = r
        return r

    return go(term)


def strip_output_views(root: Any) -> tuple[Any, list]:
    """Peel single-argument view ops off the root: ``(inner, post)`` with
    ``post`` the ``(op, attrs)`` wrappers outermost first."""
    post: list = []
    while isinstance(root, Op) and root.op in VIEW_OPS and len(root.args) == 1:
        post.append((root.op, dict(root.attrs)))
        root = root.args[0]
    return root, post


def _prefix_chain(fs: list, leaf_op: str, compose_op: str) -> list | None:
    """Time-ordered leaves when ``fs[i] = compose(leaf_i, fs[i-1])``."""
    if not fs or not is_op(fs[0], leaf_op, 2):
        return None
    leaves = [fs[0]]
    for i in range(1, len(fs)):
        f = fs[i]
        if not is_op(f, compose_op, 2) or f.args[1] is not fs[i - 1] and f.args[1] != fs[i - 1]:
            return None
        if not is_op(f.args[0], leaf_op, 2):
            return None
        leaves.append(f.args[0])
    return leaves


def _proj_list(t: Any, proj: str) -> tuple | None:
    """``([f_0 … f_n], dim)`` of ``stack(proj(f_0), …, proj(f_n), dim)``."""
    if not is_op(t, "stack") or not t.args:
        return None
    fs = []
    for a in t.args:
        if not is_op(a, proj, 1):
            return None
        fs.append(a.args[0])
    return fs, int(attr_of(t.attrs, "dim", default=0))


def _compose_levels(F: Any, compose_op: str) -> int:
    """Depth of the compose tree: the number of dependent compose levels
    (``levels`` of the reference plan, ``scan_lower.py:376-385``)."""
    memo: dict[int, int] = {}

    def depth(t: Any) -> int:
        if not is_op(t, compose_op, 2):
            return 0
        key = id(t)
        if key not in memo:
            memo[key] = 1 + max(depth(t.args[0]), depth(t.args[1]))
        return memo[key]

    return depth(F)


def _same_term(x: Any, y: Any) -> bool:
    return x is y or x == y


def build_scan_plan(root: Any) -> dict | None:
    root = fold_nested_apply(root)
    root, post = strip_output_views(root)
    ro = _readout(root)
    if ro is not None:
        # a read-out contraction of the states: planned as the inner scan plus
        # ``mul`` / ``sum`` after its own view wrappers
        inner = build_scan_plan(ro[0])
        if inner is None:
            return None
        factors = _offset_factors(inner["leaves"]) if inner["domain"] == "diag" else None
        return {**inner, "post": post, "inner_post": inner["post"], "factors": factors,
                "readout": {"c": ro[1], "dim": ro[2]}}
    if not isinstance(root, Op) or root.op not in _CARRIERS or len(root.args) != 2:
        return None
    leaf_op, comp_op, proj_a, proj_b, domain = _CARRIERS[root.op]
    F, h = root.args
    base = {"domain": domain, "h": h, "post": post, "inner_post": [], "readout": None, "factors": None}
    if is_op(F, leaf_op, 2):
        pa, pb = _proj_list(F.args[0], proj_a), _proj_list(F.args[1], proj_b)
        if pa is not None and pb is not None:
            fs_a, dim_a = pa
            fs_b, dim_b = pb
            if dim_a != dim_b or len(fs_a) != len(fs_b) or any(not _same_term(x, y) for x, y in zip(fs_a, fs_b)):
                return None
            leaves = _prefix_chain(fs_a, leaf_op, comp_op)
            if leaves is None:
                return None
            return {**base, "mode": "prefix", "leaves": leaves, "dim": dim_a, "levels": 0,
                    "gather": _shared_gather(leaves), "a_shared": _a_shared(leaves),
                    "table": K.ChunkTable(prefix_chunk_table(len(leaves)), len(leaves))}
    leaves = map_leaves(F, leaf_op, comp_op)
    if leaves is None:
        return None
    leaves = leaves[::-1]  # time order: the innermost map runs first
    return {**base, "mode": "final", "leaves": leaves, "levels": _compose_levels(F, comp_op),
            "gather": _shared_gather(leaves), "a_shared": _a_shared(leaves),
            "table": K.ChunkTable(prefix_chunk_table(len(leaves)), len(leaves))}


def _a_shared(leaves: list) -> bool:
    """Every leaf's linear part is the same term (an LTI system)."""
    a0 = leaves[0].args[0]
    return all(_same_term(lf.args[0], a0) for lf in leaves)


def _step_index(t: Any) -> tuple | None:
    """``(base, dim, index)`` of ``select(base, dim, index)`` / ``getitem(base, int)``."""
    if is_op(t, "select", 1):
        return t.args[0], int(attr_of(t.attrs, "dim", default=0)), int(attr_of(t.attrs, "index", default=0))
    if is_op(t, "getitem", 1):
        ix = t.attrs.get("index")
        if isinstance(ix, int) and not isinstance(ix, bool):
            return t.args[0], 0, ix
    return None


def _step_view(t: Any) -> tuple | None:
    """``(base, dim, index, unsqueezes)`` of a step read wrapped in
    ``unsqueeze`` ops (``unsqueezes`` innermost first)."""
    unsq: list = []
    while is_op(t, "unsqueeze", 1):
        unsq.append(int(attr_of(t.attrs, "dim", default=0)))
        t = t.args[0]
    s = _step_index(t)
    return None if s is None else (*s, tuple(reversed(unsq)))


def _gather_spec(terms: list) -> tuple | None:
    """``(base, dim, indices, unsqueezes)`` when every term reads one step of
    one shared base along one axis, with the same view wrappers."""
    views = [_step_view(t) for t in terms]
    if not views or any(v is None for v in views):
        return None
    base, dim, _, unsq = views[0]
    if any(not _same_term(v[0], base) or v[1] != dim or v[3] != unsq for v in views):
        return None
    return base, dim, [v[2] for v in views], unsq


def _shared_gather(leaves: list) -> dict:
    """Per leaf slot (0: linear part, 1: offset) whose operands all index one
    base term along one axis: ``(base, dim, indices, unsqueezes)`` in time
    order (``_leaf_b_gather``, scan_lower.py:308-337, extended to the linear
    part and to ``unsqueeze``-wrapped reads)."""
    out = {}
    for slot in (0, 1):
        g = _gather_spec([lf.args[slot] for lf in leaves])
        if g is not None:
            out[slot] = g
    return out


def _offset_factors(leaves: list) -> list | None:
    """When every leaf offset is ``mul(f_t, g_t)`` of two gathered step
    reads (the input term ``x_t ⊗ bx_t`` of a selective SSM): the two gather
    specs, else None."""
    if not all(is_op(lf.args[1], "mul", 2) for lf in leaves):
        return None
    out = [_gather_spec([lf.args[1].args[k] for lf in leaves]) for k in (0, 1)]
    return None if any(g is None for g in out) else out


def _readout(t: Any) -> tuple | None:
    """``(states, c, dim)`` of ``sum(mul(states, c), dim)`` (either operand
    order) whose ``states`` operand is an affine-scan root."""
    if not is_op(t, "sum", 1) or bool(attr_of(t.attrs, "keepdim", default=False)):
        return None
    dim = attr_of(t.attrs, "dim", "axis", default=None)
    if isinstance(dim, (list, tuple)):
        dim = dim[0] if len(dim) == 1 else None
    if dim is None or not is_op(t.args[0], "mul", 2):
        return None
    m = t.args[0]
    for s, c in ((m.args[0], m.args[1]), (m.args[1], m.args[0])):
        core, _ = strip_output_views(fold_nested_apply(s))
        if isinstance(core, Op) and core.op in _CARRIERS and len(core.args) == 2:
            return s, c, int(dim)
    return None


def is_scan_term(term: Any) -> bool:
    return build_scan_plan(term) is not None


def _prod(shape) -> int:
    return math.prod(int(s) for s in shape)


class HipScanModule(HipExecutorBase, nn.Module):
    """Planned executor for affine scans, diagonal and dense (module docstring)."""

    def __init__(self, ir: IR, param_values: dict | None = None, *, eval_mod: HipIRModule | None = None,
                 device: Any = None, ops=None, schedule: int | None = None) -> None:
        super().__init__()
        self.eval_mod = eval_mod if eval_mod is not None else HipIRModule(ir, param_values, device=device, ops=ops)
        self._inputs = list(ir.inputs)
        self._const_cache: dict = {}
        self._gather_kinds: dict = {}
        self.fallbacks = 0
        self.fused_readouts = 0  # calls whose read-out ran inside the SSM kernel
        self.schedule = L.SCAN_AUTO if schedule is None else schedule
        self._plan = build_scan_plan(self.eval_mod._root)
        self._init_graph_state()

    @property
    def n_steps(self) -> int:
        return 0 if self._plan is None else len(self._plan["leaves"])

    @property
    def n_levels(self) -> int:
        """Compose levels of the planned tree (0 when not planned, and for the
        stacked prefix form, whose map is one leaf in the reference's plan)."""
        return 0 if self._plan is None else self._plan["levels"]

    def _gathered(self, ev, key: Any, spec: tuple) -> torch.Tensor | None:
        """Step-major stack (a step-0 axis) of the reads ``spec`` describes:
        the base itself when it holds the steps in order along ``dim``,
        else one ``index_select``; the per-step ``unsqueeze`` wrappers are
        re-applied with their axes shifted past the step axis."""
        base_t, dim, idx, unsq = spec
        T = len(idx)
        base = ev(base_t)
        if not isinstance(base, torch.Tensor) or not -base.dim() <= dim < base.dim():
            return None
        # how the steps sit in the base is decided once per read and extent
        # (each test walks the T indices): in order, gathered, or out of range
        kind_key = (id(spec), base.shape[dim])
        kind = self._gather_kinds.get(kind_key)
        if kind is None:
            n = base.shape[dim]
            kind = "ident" if idx == list(range(T)) and n == T else \
                "select" if all(-n <= i < n for i in idx) else "out"
            self._gather_kinds[kind_key] = kind
        if kind == "ident":
            out = base.movedim(dim, 0)
        elif kind == "select":
            ix = self._cached(("idx", key, id(spec)), base,
                              lambda t: torch.tensor(idx, dtype=torch.long, device=t.device),
                              dtype=torch.long)
            out = base.index_select(dim, ix).movedim(dim, 0)
        else:
            return None
        for d in unsq:
            out = out.unsqueeze(d + 1 if d >= 0 else d)
        return out

    def _slot_values(self, ev, slot: int) -> torch.Tensor | None:
        """Step-major stack of leaf operand ``slot`` (a step-0 axis)."""
        p = self._plan
        g = p["gather"].get(slot)
        if g is not None:
            out = self._gathered(ev, slot, g)
            if out is not None:
                return out
        if slot == 1 and p["factors"] is not None:
            f0, f1 = (self._gathered(ev, ("f", k), p["factors"][k]) for k in (0, 1))
            if f0 is not None and f1 is not None:
                try:
                    return torch.mul(f0, f1)
                except RuntimeError:
                    pass
        vals = [torch.as_tensor(ev(lf.args[slot])) for lf in p["leaves"]]
        try:
            tgt = torch.broadcast_shapes(*[v.shape for v in vals])
        except RuntimeError:
            return None
        return torch.stack([v.expand(tgt) for v in vals])

    def _apply_views(self, out: Any, post: list) -> Any:
        tab = self.eval_mod._bindings().torch_bindings
        for op, attrs in reversed(post):
            out = tab[op](out, **attrs)
        return out

    def _apply_post(self, out: Any) -> Any:
        return self._apply_views(out, self._plan["post"])

    def _apply_readout(self, ev, states: Any) -> Any:
        """``sum(mul(states, c), dim)`` through the op table."""
        ro = self._plan["readout"]
        tab = self.eval_mod._bindings().torch_bindings
        return tab["sum"](tab["mul"](states, ev(ro["c"])), dim=ro["dim"])

    def _forward_impl(self, *xs: Any) -> Any:
        p = self._plan
        if p is None:
            return self.eval_mod(*xs)
        x, env = self._input_env(xs)
        ev = self.ev_factory(env, x)
        out = self._forward_ssm(ev) if p["readout"] is not None else None
        if out is not None:
            self.fused_readouts += 1
        else:
            out = self._forward_diag(ev) if p["domain"] == "diag" else self._forward_dense(ev)
            if out is not None and p["readout"] is not None:
                out = self._apply_readout(ev, self._apply_views(out, p["inner_post"]))
        if out is None:
            self.fallbacks += 1
            return self.eval_mod(*xs)
        return self._apply_post(out)

    @staticmethod
    def _kernel_ok(*ts: Any) -> bool:
        return all(isinstance(t, torch.Tensor) and t.device.type == "cuda"
                   and t.dtype in (torch.float32, torch.bfloat16) for t in ts)

    # ------------------------------------------------------------- diagonal

    def _forward_diag(self, ev) -> torch.Tensor | None:
        p = self._plan
        T = len(p["leaves"])
        shared = p["a_shared"] and p["gather"].get(0) is None
        if shared:
            a = torch.as_tensor(ev(p["leaves"][0].args[0]))  # one map for every step: stride 0 over T
        else:
            a = self._slot_values(ev, 0)
        u = self._slot_values(ev, 1)
        h = ev(p["h"])
        if a is None or u is None or not self._kernel_ok(a, u, h) or u.shape[0] != T:
            return None
        if not shared and a.shape[0] != T:
            return None
        out_dtype = torch.promote_types(torch.promote_types(a.dtype, u.dtype), h.dtype)
        sa, su = (a.shape if shared else a.shape[1:]), u.shape[1:]
        if p["mode"] == "prefix":
            # stack(a-prefixes, dim) ⊙ h + stack(b-prefixes, dim): both stacks
            # must line up, and h must be one state for every step
            R = len(su) + 1
            if len(sa) != len(su) or not -R <= p["dim"] < R or h.dim() > R:
                return None
            ax = h.dim() - R + p["dim"] % R  # the axis of h aligned with the stacked one
            if ax >= 0:
                if h.shape[ax] != 1:
                    return None
                h = h.squeeze(ax)
        try:
            sshape = torch.broadcast_shapes(sa, su, h.shape)
        except RuntimeError:
            return None
        if len(sa) < len(sshape):
            a = a.reshape(a.shape[:0 if shared else 1] + (1,) * (len(sshape) - len(sa)) + tuple(sa))
        if len(su) < len(sshape):
            u = u.reshape((T,) + (1,) * (len(sshape) - len(su)) + tuple(su))
        a_ = a.expand(sshape) if shared else a.expand(T, *sshape)
        u_ = u.expand(T, *sshape)
        h_ = h.expand(sshape)
        states, hf = K.affd_scan(a_, u_, h_, p["table"], schedule=self.schedule,
                                 states=p["mode"] == "prefix")
        if p["mode"] == "final":
            return hf.to(out_dtype)
        return states.to(out_dtype).movedim(0, p["dim"] % (len(sshape) + 1))

    def _forward_ssm(self, ev) -> torch.Tensor | None:
        """Every prefix state read out in the kernel: the selective SSM
        ``h_t = a_t ⊙ h_{t-1} + x_t ⊗ bx_t`` over a ``(B, D, N)`` state, stacked
        along axis 1, contracted with ``c (B, T, 1, N)`` over ``N``, so the
        ``(B, T, D, N)`` states never reach HBM.  None when the operands do
        not have that layout (the caller then scans and reads out apart)."""
        p = self._plan
        fac = p["factors"]
        if fac is None or p["mode"] != "prefix" or p["inner_post"] or p["domain"] != "diag":
            return None
        T = len(p["leaves"])
        f0, f1 = (self._gathered(ev, ("f", k), fac[k]) for k in (0, 1))
        if f0 is None or f1 is None or f0.dim() != 4 or f1.dim() != 4 or T == 0:
            return None
        # the input term: one factor (T, B, D, 1), the other (T, B, 1, N)
        xs, bs = (f0, f1) if f0.shape[-1] == 1 and f1.shape[-2] == 1 else (f1, f0)
        if xs.shape[-1] != 1 or bs.shape[-2] != 1 or xs.shape[:2] != (T, bs.shape[1]) or bs.shape[0] != T:
            return None
        B, D, N = xs.shape[1], xs.shape[2], bs.shape[3]
        if N not in (4, 8, 16, 32, 64) or p["dim"] % 4 != 1 or p["readout"]["dim"] % 4 != 3:
            return None
        if p["a_shared"] and p["gather"].get(0) is None:
            a1 = torch.as_tensor(ev(p["leaves"][0].args[0]))
            A = a1.unsqueeze(0).expand(T, *a1.shape) if a1.dim() == 3 else None
        else:
            A = self._slot_values(ev, 0)
        h, c = ev(p["h"]), ev(p["readout"]["c"])
        if A is None or A.dim() != 4 or A.shape[0] != T or not self._kernel_ok(A, xs, bs, h, c):
            return None
        try:
            if torch.broadcast_shapes(A.shape[1:], (B, D, N)) != (B, D, N):
                return None
            if torch.broadcast_shapes(h.shape, (B, 1, D, N)) != (B, 1, D, N):
                return None  # h varies along the stacked axis: not one scan
            if torch.broadcast_shapes(c.shape, (B, T, 1, N)) != (B, T, 1, N):
                return None  # c varies along D: not a read-out over N
        except RuntimeError:
            return None
        # a per channel (…, D, 1) runs the kernel's broadcast-over-N form
        a = A.movedim(0, 1)
        a = a.squeeze(-1).expand(B, T, D) if A.shape[-1] == 1 and N > 1 else a.expand(B, T, D, N)
        out_dtype = A.dtype
        for t in (xs, bs, h, c):
            out_dtype = torch.promote_types(out_dtype, t.dtype)
        y = K.ssm_scan(a, bs[:, :, 0, :].movedim(0, 1), c.expand(B, T, 1, N)[:, :, 0, :],
                       xs[..., 0].movedim(0, 1), h.expand(B, 1, D, N)[:, 0], p["table"],
                       schedule=self.schedule)
        return y.to(out_dtype)

    # ---------------------------------------------------------------- dense

    def _dense_linear(self, ev) -> torch.Tensor | None:
        """Linear parts as ``(TA, *PA, d, d)``, ``TA = 1`` for a shared map."""
        p = self._plan
        if p["a_shared"]:
            A = torch.as_tensor(ev(p["leaves"][0].args[0]))
            return A.unsqueeze(0)
        return self._slot_values(ev, 0)

    def _forward_dense(self, ev) -> torch.Tensor | None:
        p = self._plan
        T = len(p["leaves"])
        A = self._dense_linear(ev)
        b = self._slot_values(ev, 1)
        h = ev(p["h"])
        if A is None or b is None or not self._kernel_ok(A, b, h) or b.shape[0] != T or A.dim() < 3:
            return None
        d = A.shape[-1]
        if A.shape[-2] != d or not 1 <= d <= DENSE_MAX_D or A.shape[0] not in (1, T):
            return None
        out_dtype = torch.promote_types(torch.promote_types(A.dtype, b.dtype), h.dtype)
        TA = A.shape[0]
        if p["mode"] == "prefix" or (b.dim() == 2 and h.dim() == 1):
            # vector state: A (d, d), b (d,), h (d,)
            if A.dim() != 3 or b.shape[1:] != (d,) or h.shape != (d,):
                return None
            if p["mode"] == "prefix" and p["dim"] not in (0, 1):
                return None  # the stacked maps and offsets would not line up
            A4, b3, h3, pshape, k = A.reshape(TA, 1, d, d), b.reshape(T, 1, d), h.reshape(1, d, 1), (), 1
        else:
            # column state: A (…, d, d), b (…, d, 1), h (…, d, k)
            if b.dim() < 3 or b.shape[-2:] != (d, 1) or h.dim() < 2 or h.shape[-2] != d:
                return None
            k = h.shape[-1]
            PA, PB, PH = A.shape[1:-2], b.shape[1:-2], h.shape[:-2]
            try:
                pshape = torch.broadcast_shapes(PA, PB, PH)
            except RuntimeError:
                return None
            Pn = _prod(pshape)
            A4 = A.reshape(TA, 1, d, d) if _prod(PA) == 1 else A.expand(TA, *pshape, d, d).reshape(TA, Pn, d, d)
            b3 = b.reshape(T, 1, d) if _prod(PB) == 1 else b.expand(T, *pshape, d, 1).reshape(T, Pn, d)
            h3 = h.expand(*pshape, d, k).reshape(Pn, d, k)
        if T == 0:
            return None
        states, hf = K.aff_scan(A4, b3, h3, p["table"], schedule=self.schedule, states=p["mode"] == "prefix")
        if p["mode"] == "prefix":
            return states.reshape(T, d).to(out_dtype).movedim(0, p["dim"])
        if h.dim() == 1:
            return hf.reshape(d).to(out_dtype)
        return hf.reshape(*pshape, d, k).to(out_dtype)


#: The reference's probe name (scan_lower.py:200-214).
is_scan_apply_term = is_scan_term


def to_batched_scan_module(ir: IR, param_values: dict | None = None, *, fused: bool | str = False,
                           **kw) -> HipScanModule:
    """Always a :class:`HipScanModule` (check ``is_batched``), ``scan_lower.py:837-870``.
    ``fused`` is accepted for the reference's signature (its shrinking-tensor
    reduction under torch.compile); the scans here are single kernels, so it
    changes nothing."""
    del fused
    return HipScanModule(ir, param_values, **kw)
