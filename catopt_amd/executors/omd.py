"""Deferred-affine attention (omd) executor.

The counterpart of ``BatchedOmdModule`` / ``build_omd_plan`` (luisfuturist/
catopt ``packages/catopt-carriers/src/catopt_carriers/omd_lower.py:213-558,
562-1019``).  The term is softmax attention over values that are affine in
one shared state ``h`` — attention over the states of a scan:

    omd_apply(<omd_compose tree of omd_elem(s_i, a_i, b_i)>, h)      (diagonal)
    omd_applym(<omd_compose tree of omd_elem(s_i, A_i, b_i)>, h)     (dense)

with ``omd_elem(s, a, b) = (m, l, e@a, e@b)``, ``e = exp(s − m)``, and the
readout ``(fa ⊙ h + fb) / l`` (``fa @ h`` for the dense fibre;
``xcarrier.py:380-454``).  The coefficient arrays ``a_i``, ``b_i`` are
usually ``stack(affd_a f_j)`` / ``stack(affd_b f_j)`` over the prefixes
``f_j = affd_compose(leaf_j, f_{j-1})`` of one scan — O(T²) unrolled terms
for a generic evaluator.

Plan (as in the reference): the projections of maps inside the leaves
(``affd_a``/``affd_b``/``aff_A``/``aff_b``, alone or stacked) are collected;
when every projected map is a prefix of ONE leaf sequence of one carrier,
the plan is ``chain`` and all prefix maps come from the HIP scan kernels in
one pass, then answer every projection and stack by gather (seeded into the
evaluator's memo, so the score terms around them evaluate unchanged).  Maps
of any other bracketing, or of both carriers, make a ``forest`` plan: per
carrier, the compose nodes are grouped by depth (leaves at level 0, shared
subterms once) and each level runs as one HIP launch over slot arrays
(``catopt_hip_affd_compose_slots`` / ``catopt_hip_aff_compose_slots``);
the projections are then answered from the slots the same way.

Execution on the device:

* prefix maps — diagonal: one ``catopt_hip_affd_scan`` over ``[a | a]``
  lanes from ``[1 | 0]`` with offsets ``[0 | b]`` gives
  ``[∏a | prefix b]``; dense: two ``catopt_hip_aff_scan`` launches
  (``I`` under the maps alone, ``0`` under the maps and offsets);
* forest maps — the leaf parts stacked into fp32 slot arrays, then one
  compose launch per level (the diagonal products and sums rounded as the
  serial evaluation rounds them);
* leaves — a score ``scale · q kᵀ`` (unmasked) runs the fused fp32 carrier
  kernel ``catopt_hip_attn_carrier_f32`` over the values ``[a | b]``: the
  scores, exponentials and numerators stay on chip; any other score is
  evaluated, then ``m``, ``l`` and one HIP GEMM ``e @ [a | b]`` (the two
  numerator parts share the exponentials);
* the compose tree — left-folded in product order by the HIP ``om_compose``
  kernel over the concatenated numerator ``[fa | fb]`` (the omd combine is
  om's applied to each part, ``xcarrier.py:407-440``; the ``isfinite``
  guard of fully masked blocks is in the kernel);
* the readout on the device; when every leaf's carrier came from one
  carrier launch and the fibre is diagonal, the combine over the leaf axis
  and the readout ``(fa ⊙ h + fb) / l`` are one ``catopt_hip_omd_fold_apply``
  pass (``fused_omd_levels``, om_fused.py:151-164).

Carriers are fp32 (bf16 operands are widened); the result has the promoted
operand dtype.  Other dtypes, host tensors, and shape surprises run the
embedded generic module, counted in ``fallbacks`` (as the reference's
``_forward_impl`` does on any exception); kernel errors raise.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import nn

from .. import _lib as L
from .. import kernels as K
from ..bindings import _om_compose, attr_of
from ..evaluator import HipIRModule
from ..ir import IR, Op, Param, Var, is_op
from .base import HipExecutorBase
from .om import _peel_scale, parse_score
from .scan import prefix_chunk_table

__all__ = ["HipOmdModule", "build_omd_plan", "is_omd_apply_term", "is_omd_term", "to_batched_omd_module"]

#: projection op -> (component, carrier)
_PROJ = {"affd_a": (0, "diag"), "affd_b": (1, "diag"), "aff_A": (0, "dense"), "aff_b": (1, "dense")}
_COMPOSE = {"affd_compose": "diag", "aff_compose": "dense"}
_LEAF = {"aff_diag": "diag", "aff": "dense"}


def _omd_leaves(t: Any) -> list | None:
    """Leaves of an ``omd_compose`` tree in product order (with multiplicity)."""
    out: list = []
    stack = [t]
    while stack:
        n = stack.pop()
        if is_op(n, "omd_compose", 2):
            stack.append(n.args[1])
            stack.append(n.args[0])
        elif is_op(n, "omd_elem", 3) or is_op(n, "omd", 4):
            out.append(n)
        else:
            return None
    return out


def is_omd_term(root: Any) -> bool:
    """``omd_apply`` / ``omd_applym`` over an omd tree (``omd_lower.py:153-164``)."""
    return (isinstance(root, Op) and root.op in ("omd_apply", "omd_applym") and len(root.args) == 2
            and _omd_leaves(root.args[0]) is not None)


def _app_order(mp: Any) -> list:
    """Leaf maps of a compose term in application order (``compose(f, g)``
    applies ``g`` first; ``omd_lower.py:167-186``)."""
    out: list = []
    stack = [mp]
    while stack:
        u = stack.pop()
        if isinstance(u, Op) and u.op in _COMPOSE and len(u.args) == 2:
            stack.append(u.args[0])
            stack.append(u.args[1])
        else:
            out.append(u)
    return out


def _step_index(t: Any) -> tuple | None:
    if is_op(t, "select", 1):
        return t.args[0], int(attr_of(t.attrs, "dim", default=0)), int(attr_of(t.attrs, "index", default=0))
    if is_op(t, "getitem", 1):
        ix = t.attrs.get("index")
        if isinstance(ix, int) and not isinstance(ix, bool):
            return t.args[0], 0, ix
    return None


def _part_gather(leaves: list, slot: int) -> tuple | None:
    """``(base, dim, indices)`` when every leaf's part ``slot`` indexes one base."""
    if not all(isinstance(lf, Op) and lf.op in _LEAF and len(lf.args) == 2 for lf in leaves):
        return None
    idx = [_step_index(lf.args[slot]) for lf in leaves]
    if any(i is None for i in idx):
        return None
    base, dim = idx[0][0], idx[0][1]
    if any(not (i[0] is base or i[0] == base) or i[1] != dim for i in idx):
        return None
    return base, dim, [i[2] for i in idx]


def _spine_positions(maps: dict, leaf_op: str, comp_op: str) -> tuple | None:
    """O(T) recognition of the common chain: every map lies on one spine
    ``f_j = compose(leaf_j, f_{j-1})`` (``f_0`` a leaf).  Returns
    ``(positions, leaves)`` or ``None`` (the general comparison then runs)."""
    depth: dict = {}
    for mp in maps:
        path, u = [], mp
        while u not in depth:
            if is_op(u, leaf_op, 2):
                depth[u] = 0
                break
            if is_op(u, comp_op, 2) and is_op(u.args[0], leaf_op, 2):
                path.append(u)
                u = u.args[1]
                continue
            return None
        dpt = depth[u]
        for n in reversed(path):
            dpt += 1
            depth[n] = dpt
    top = max(maps, key=lambda m: depth[m])
    spine, u = [], top
    while not is_op(u, leaf_op, 2):
        spine.append(u)
        u = u.args[1]
    spine.append(u)
    spine.reverse()  # spine[j] = f_j
    if any(not (spine[depth[m]] is m or spine[depth[m]] == m) for m in maps):
        return None
    leaves = [spine[0]] + [f.args[0] for f in spine[1:]]
    return {m: depth[m] for m in maps}, leaves


def _plain_score(leaf: Any) -> dict | None:
    """``q``, ``k`` and ``scale`` of an unmasked ``scale · q kᵀ`` leaf score.
    A transpose with absolute axes (``transpose(x, 0, 1)``) of a term whose
    rank is not known here is accepted with those axes recorded; the call
    checks them against the evaluated operand's rank."""
    if leaf.op != "omd_elem":
        return None
    sc = parse_score(leaf.args[0])
    if sc is not None:
        return dict(sc, axes=None) if sc["mask"] is None and sc["bias"] is None else None
    s, scale = _peel_scale(leaf.args[0])
    if not is_op(s, "matmul", 2) or not is_op(s.args[1], "transpose", 1):
        return None
    d0, d1 = attr_of(s.args[1].attrs, "dim0", default=None), attr_of(s.args[1].attrs, "dim1", default=None)
    if d0 is None or d1 is None:
        return None
    return {"q": s.args[0], "k": s.args[1].args[0], "scale": scale, "mask": None,
            "axes": frozenset((int(d0), int(d1)))}


def build_omd_plan(root: Any) -> dict | None:
    if not is_omd_term(root):
        return None
    F, h = root.args
    leaves = _omd_leaves(F)
    # ---- projections of maps inside the leaves (and h) -------------------
    projs: list = []   # (node, component, map): projections outside a stack
    stacks: list = []  # (node, component, [maps], dim)
    maps: dict = {}    # map term -> carrier
    loose: list = []   # map terms in a tensor position (evaluated as pairs)
    bad = False
    seen: set = set()

    def register(mp: Any, dom: str) -> None:
        nonlocal bad
        if maps.setdefault(mp, dom) != dom:
            bad = True

    def scan(t: Any) -> None:
        if not isinstance(t, Op) or id(t) in seen:
            return
        seen.add(id(t))
        info = _PROJ.get(t.op)
        if info is not None and len(t.args) == 1:
            projs.append((t, info[0], t.args[0]))
            register(t.args[0], info[1])
            return
        if t.op == "stack" and t.args and all(isinstance(c, Op) and c.op in _PROJ and len(c.args) == 1
                                              for c in t.args):
            infos = {_PROJ[c.op] for c in t.args}
            if len(infos) == 1:
                ci, dom = next(iter(infos))
                for c in t.args:
                    register(c.args[0], dom)
                stacks.append((t, ci, [c.args[0] for c in t.args], int(attr_of(t.attrs, "dim", default=0))))
                return  # its projections are reached only through the stack: one seed covers them
        if t.op in _COMPOSE or t.op in _LEAF:
            loose.append(t)  # a map in a tensor position: seeded as a pair if it is a chain map
            return
        for a in t.args:
            scan(a)

    for lf in leaves:
        for a in lf.args:
            scan(a)
    scan(h)
    if bad:
        return None
    plan: dict = {"apply": root.op, "h": h, "leaves": leaves, "map_mode": None,
                  "proj_seeds": [], "stack_seeds": [], "map_seeds": [],
                  # unmasked scale·q kᵀ scores: the leaf runs the fused carrier kernel
                  "scores": [_plain_score(lf) for lf in leaves], "blocks": None}
    plan["k_chunks"] = _chunk_keys(plan["scores"])
    if not maps:
        return plan
    # ---- chain: every projected map a prefix of one leaf sequence ---------
    doms = set(maps.values())
    if len(doms) == 1:
        dom = next(iter(doms))
        leaf_op, comp_op = ("aff_diag", "affd_compose") if dom == "diag" else ("aff", "aff_compose")
        fast = _spine_positions(maps, leaf_op, comp_op)
        if fast is not None and _sig_uniform(fast[1], dom):
            return _chain_plan(plan, dom, fast[1], fast[0], projs, stacks, [m for m in loose if m in maps])
    seqs = {mp: _app_order(mp) for mp in maps}  # terms are content-keyed (cached hashes)
    base = max(seqs.values(), key=len)
    dom = next(iter(doms))
    # opaque leaves (any term evaluating to a pair) may sit in a chain; a leaf
    # of the other carrier may not
    chain = (len(doms) == 1
             and all(len(s) <= len(base) and all(x is y or x == y for x, y in zip(s, base)) for s in seqs.values())
             and all(_LEAF.get(lf.op, dom) == dom if isinstance(lf, Op) else True for lf in base)
             and _sig_uniform(base, dom))
    if chain:
        pos = {mp: len(s) - 1 for mp, s in seqs.items()}
        return _chain_plan(plan, dom, base, pos, projs, stacks, [m for m in loose if m in maps])
    return _forest_plan(plan, maps, projs, stacks, loose)


def _static_shape(t: Any) -> tuple | None:
    """The shape of a leaf part where the term states it: a variable or
    weight, or an integer ``select`` / ``getitem`` of one; else ``None``."""
    if isinstance(t, (Var, Param)):
        return tuple(t.typ.shape)
    si = _step_index(t)
    if si is not None:
        base = _static_shape(si[0])
        if base is None or not base:
            return None
        dim = si[1] % len(base)
        return base[:dim] + base[dim + 1:]
    return None


def _leaf_sig(leaf: Any, dom: str) -> Any:
    """``(dom, shape)`` of an ``aff_diag`` / ``aff`` leaf whose part shapes are
    known, ``None`` when unknown or opaque, ``False`` when they break the
    carrier's contract (diagonal: ``a`` and ``b`` of one shape; dense: square
    ``A`` with ``b`` its leading shape), as ``omd_lower.py:189-217`` checks."""
    if not isinstance(leaf, Op) or leaf.op not in _LEAF or len(leaf.args) != 2:
        return None
    a, b = _static_shape(leaf.args[0]), _static_shape(leaf.args[1])
    if a is None or b is None:
        return None
    if leaf.op == "aff_diag":
        return (dom, a) if a == b else False
    if len(a) >= 2 and a[-1] == a[-2] and b == a[:-1]:
        return (dom, a)
    return False


def _sig_uniform(leaves: list, dom: str) -> bool:
    sig = None
    for lf in leaves:
        s = _leaf_sig(lf, dom)
        if s is False:
            return False
        if s is not None:
            if sig is None:
                sig = s
            elif s != sig:
                return False
    return True


def _has_projection(t: Any) -> bool:
    stack, seen = [t], set()
    while stack:
        u = stack.pop()
        if not isinstance(u, Op) or id(u) in seen:
            continue
        seen.add(id(u))
        if u.op in _PROJ:
            return True
        stack.extend(u.args)
    return False


def _walk_maps(maps: dict) -> dict | None:
    """Per carrier: the leaves (level 0, first-met order) and the compose
    nodes by level (one more than the deeper operand) of every map, shared
    subterms once; ``None`` when a compose or leaf op belongs to the other
    carrier, or a map leaf's operands project another map
    (``omd_lower.py:361-455``).  Iterative: prefix chains nest O(T) deep."""
    domains: dict = {}
    for root_mp, expected in maps.items():
        stack = [(root_mp, expected, False)]
        while stack:
            mp, exp, done = stack.pop()
            if isinstance(mp, Op) and mp.op in _COMPOSE and len(mp.args) == 2:
                if _COMPOSE[mp.op] != exp:
                    return None
                d = domains.setdefault(exp, {"leaves": [], "levels": [], "level_of": {}})
                if mp in d["level_of"]:
                    continue
                if not done:
                    stack.append((mp, exp, True))
                    stack.append((mp.args[0], exp, False))
                    stack.append((mp.args[1], exp, False))
                    continue
                lv = max(d["level_of"][c] for c in mp.args) + 1
                d["level_of"][mp] = lv
                while len(d["levels"]) < lv:
                    d["levels"].append([])
                d["levels"][lv - 1].append(mp)
                continue
            if isinstance(mp, Op) and mp.op in _LEAF and len(mp.args) == 2 and _LEAF[mp.op] != exp:
                return None
            d = domains.setdefault(exp, {"leaves": [], "levels": [], "level_of": {}})
            if mp in d["level_of"]:
                continue
            d["level_of"][mp] = 0
            d["leaves"].append(mp)
            if isinstance(mp, Op) and any(_has_projection(c) for c in mp.args):
                return None
    return domains


def _forest_plan(plan: dict, maps: dict, projs: list, stacks: list, loose: list) -> dict | None:
    """Level-batched plan for maps of any bracketing (``omd_lower.py:520-558``):
    per carrier, leaf slots ``0..n-1`` and then each level's nodes in order,
    with the operand slots each level's launch reads."""
    domains = _walk_maps(maps)
    if domains is None:
        return None
    for dom, d in domains.items():
        if not _sig_uniform(d["leaves"], dom):
            return None
        slot = {lf: i for i, lf in enumerate(d["leaves"])}
        nxt, gathers = len(d["leaves"]), []
        for nodes in d["levels"]:
            gathers.append(([slot[t.args[0]] for t in nodes], [slot[t.args[1]] for t in nodes]))
            for t in nodes:
                slot[t] = nxt
                nxt += 1
        d.update(slot=slot, gathers=gathers, n_slots=nxt,
                 a_gather=_part_gather(d["leaves"], 0), b_gather=_part_gather(d["leaves"], 1))
        del d["level_of"]
    src = {dom: ("forest", dom) for dom in domains}
    at = lambda mp: domains[maps[mp]]["slot"][mp]  # noqa: E731
    plan.update(map_mode="forest", forest=domains)
    plan["proj_seeds"] = [(node, ci, src[maps[mp]], at(mp)) for node, ci, mp in projs]
    plan["stack_seeds"] = [(node, ci, src[maps[mps[0]]], [at(mp) for mp in mps], dim)
                           for node, ci, mps, dim in stacks]
    plan["map_seeds"] = [(mp, src[maps[mp]], at(mp)) for mp in dict.fromkeys(m for m in loose if m in maps)]
    return plan


def _chain_plan(plan: dict, dom: str, base: list, pos: dict, projs: list, stacks: list, loose: list) -> dict:
    """Seeds for the evaluator's memo: every stack of projections, every
    projection outside a stack, and every chain map met in a tensor position
    (``omd_lower.py:528-547``); and, when every leaf's coefficients are the
    stacks of one contiguous run of prefix positions, those runs."""
    plan.update(map_mode="chain", chain_domain=dom, chain_leaves=base,
                chain_a_gather=_part_gather(base, 0), chain_b_gather=_part_gather(base, 1))
    src = ("chain",)
    plan["proj_seeds"] = [(node, ci, src, pos[mp]) for node, ci, mp in projs]
    plan["stack_seeds"] = [(node, ci, src, [pos[mp] for mp in mps], dim) for node, ci, mps, dim in stacks]
    plan["map_seeds"] = [(mp, src, pos[mp]) for mp in dict.fromkeys(loose)]
    plan["blocks"] = _leaf_blocks(plan)
    return plan


def _leaf_blocks(plan: dict) -> list | None:
    """``[(start, length)]`` per leaf when its ``a`` and ``b`` arguments stack
    the same contiguous prefix positions along axis 0; else ``None``."""
    by_node = {id(node): (ci, idx, dim) for node, ci, _src, idx, dim in plan["stack_seeds"]}
    out = []
    for lf in plan["leaves"]:
        if lf.op != "omd_elem":
            return None
        sa, sb = by_node.get(id(lf.args[1])), by_node.get(id(lf.args[2]))
        if sa is None or sb is None or sa[0] != 0 or sb[0] != 1 or sa[2] != 0 or sb[2] != 0 or sa[1] != sb[1]:
            return None
        idx = sa[1]
        if idx != list(range(idx[0], idx[0] + len(idx))):
            return None
        out.append((idx[0], len(idx)))
    return out


def _chunk_keys(scores: list) -> tuple | None:
    """``(base, dim)`` when leaf ``i``'s key operand is ``chunk(base, chunks=L,
    dim, index=i)`` of one base over the L leaves."""
    if not scores or any(sc is None for sc in scores):
        return None
    L = len(scores)
    base = dim = None
    for i, sc in enumerate(scores):
        kt = sc["k"]
        if not is_op(kt, "chunk", 1) or int(attr_of(kt.attrs, "index", default=-1)) != i or \
                int(attr_of(kt.attrs, "chunks", default=0)) != L:
            return None
        d = int(attr_of(kt.attrs, "dim", default=0))
        if base is None:
            base, dim = kt.args[0], d
        elif not (kt.args[0] is base or kt.args[0] == base) or d != dim:
            return None
    return base, dim


def _kernel_dtype(t: Any) -> bool:
    return isinstance(t, torch.Tensor) and t.device.type == "cuda" and t.dtype in (torch.float32, torch.bfloat16)


class HipOmdModule(HipExecutorBase, nn.Module):
    """Planned executor for ``omd_apply[m](<omd tree>, h)`` (module docstring)."""

    def __init__(self, ir: IR, param_values: dict | None = None, *, eval_mod: HipIRModule | None = None,
                 device: Any = None, ops=None) -> None:
        super().__init__()
        self.eval_mod = eval_mod if eval_mod is not None else HipIRModule(ir, param_values, device=device, ops=ops)
        self._inputs = list(ir.inputs)
        self._const_cache: dict = {}
        self._tables: dict = {}
        self._identity_gathers: dict = {}
        self.fallbacks = 0
        self._plan = build_omd_plan(self.eval_mod._root)
        self.fused_leaves = 0  # leaves run by the fused carrier kernel on the last call
        self._seeded_ids = set() if self._plan is None else \
            {id(node) for node, *_ in self._plan["proj_seeds"] + self._plan["stack_seeds"]}
        self._init_graph_state()

    @property
    def map_mode(self) -> str | None:
        return None if self._plan is None else self._plan["map_mode"]

    # ------------------------------------------------------------ prefix maps

    def _index(self, idx: list, like: torch.Tensor) -> torch.Tensor:
        """The device copy of a plan's index list, keyed by the list itself
        (plan lists live as long as the module; hashing T entries per call
        would cost more than the gather)."""
        return self._cached(("idx", id(idx), len(idx)), like,
                            lambda x: torch.tensor(idx, dtype=torch.long, device=x.device), dtype=torch.long)

    @staticmethod
    def _leaf_part(leaf: Any, i: int, ev) -> Any:
        """Part ``i`` of a map leaf: the ``aff_diag`` / ``aff`` operand, or
        ``value[i]`` of an opaque leaf (a pair or a stacked tensor), as the
        generic projection reads it (``omd_lower.py:698-713``)."""
        if isinstance(leaf, Op) and leaf.op in _LEAF and len(leaf.args) == 2:
            return ev(leaf.args[i])
        return ev(leaf)[i]

    def _leaf_parts(self, leaves: list, gathers: tuple, ev) -> tuple:
        """Leaf ``(a, b)`` parts stacked leaf-major: one ``index_select`` of a
        shared base when every leaf indexes one, else a stack."""
        out = []
        for slot, g in enumerate(gathers):
            if g is not None:
                base, dim, idx = g
                bt = ev(base)
                # whether the gather is the identity, decided once per plan
                # entry and extent (the comparison walks T indices)
                key = (id(g), bt.shape[dim])
                ident = self._identity_gathers.get(key)
                if ident is None:
                    ident = self._identity_gathers[key] = idx == list(range(bt.shape[dim]))
                if ident:
                    t = bt.movedim(dim, 0)
                else:
                    t = bt.index_select(dim, self._index(idx, bt)).movedim(dim, 0)
            else:
                t = torch.stack([torch.as_tensor(self._leaf_part(lf, slot, ev)) for lf in leaves])
            out.append(t)
        return out[0], out[1]

    def _forest_maps(self, ev, dtypes: list) -> dict:
        """Every map of a forest plan, per carrier: the leaf parts in slots
        ``0..n-1`` of fp32 slot arrays, then one compose launch per level."""
        stores = {}
        for dom, d in self._plan["forest"].items():
            A, B = self._leaf_parts(d["leaves"], (d["a_gather"], d["b_gather"]), ev)
            if not (_kernel_dtype(A) and _kernel_dtype(B)):
                raise _Decline()
            dtypes += [A.dtype, B.dtype]
            n0, n = A.shape[0], d["n_slots"]
            SA = torch.empty((n, *A.shape[1:]), dtype=torch.float32, device=A.device)
            SB = torch.empty((n, *B.shape[1:]), dtype=torch.float32, device=B.device)
            SA[:n0].copy_(A)
            SB[:n0].copy_(B)
            out0 = n0
            for fi, gi in d["gathers"]:
                K.compose_slots(SA, SB, self._index(fi, SA), self._index(gi, SA), out0, dom)
                out0 += len(fi)
            stores[("forest", dom)] = (SA, SB)
        return stores

    def _prefix_maps(self, A: torch.Tensor, B: torch.Tensor) -> tuple:
        """Every prefix map ``f_t = leaf_t ∘ … ∘ leaf_0`` of the chain (fp32)."""
        T = A.shape[0]
        # the blocked plan lets the kernels go chunk-parallel when the lanes
        # are few; the table object (and its device copy) lives with the module
        table = self._tables.get(T)
        if table is None:
            table = self._tables[T] = K.ChunkTable(prefix_chunk_table(T), T)
        if self._plan["chain_domain"] == "diag":
            if A.shape != B.shape:
                raise ValueError("diagonal chain parts differ in shape")
            S = A[0].numel()
            a2 = A.reshape(T, S).repeat(1, 2)                           # [a | a]
            u2 = torch.nn.functional.pad(B.reshape(T, S), (S, 0))      # [0 | b]
            hkey = ("h2", S, A.dtype, A.device)
            h2 = self._tables.get(hkey)                                 # [1 | 0], built once
            if h2 is None:
                h2 = self._tables[hkey] = torch.cat([torch.ones(S, dtype=A.dtype, device=A.device),
                                                     torch.zeros(S, dtype=A.dtype, device=A.device)])
            states, _ = K.affd_scan(a2, u2, h2, table, states=True)
            return states[:, :S].reshape(A.shape), states[:, S:].reshape(B.shape)
        # dense: A (T, *P, d, d), B (T, *P, d)
        d = A.shape[-1]
        if A.shape[-2] != d or B.shape != A.shape[:-1]:
            raise ValueError("dense chain parts do not form square maps with matching offsets")
        pshape = A.shape[1:-2]
        Pn = int(torch.Size(pshape).numel())
        A4 = A.reshape(T, Pn, d, d)
        eye = torch.eye(d, dtype=torch.float32, device=A.device).expand(Pn, d, d)
        zero_b = torch.zeros((T, 1, d), dtype=torch.float32, device=A.device)
        M, _ = K.aff_scan(A4, zero_b, eye, table, states=True)                     # X_t = A_t X, X = I
        v, _ = K.aff_scan(A4, B.reshape(T, Pn, d), torch.zeros((Pn, d, 1), dtype=torch.float32, device=A.device),
                          table, states=True)                                       # x_t = A_t x + b_t
        return M.reshape(A.shape), v.reshape(B.shape)

    def _seed(self, memo: dict, stores: dict) -> None:
        """Answer every projection, stack of projections and map seen in a
        tensor position from the computed maps (``omd_lower.py:871-887``)."""
        for node, ci, src, i in self._plan["proj_seeds"]:
            memo[node] = stores[src][ci][i]
        for mp, src, i in self._plan["map_seeds"]:
            memo[mp] = (stores[src][0][i], stores[src][1][i])
        for node, ci, src, idx, dim in self._plan["stack_seeds"]:
            t = stores[src][ci]
            t = t.index_select(0, self._index(idx, t))
            dn = dim % t.dim()
            memo[node] = t.movedim(0, dn) if dn else t

    # ---------------------------------------------------------------- leaves

    @staticmethod
    def _leaf_carrier(s: torch.Tensor, a: torch.Tensor, b: torch.Tensor) -> tuple:
        """``(m, l, e @ [a | b])`` in fp32, the dense ``a`` flattened; returns
        the numerator width of ``fa`` and its trailing shape too."""
        s32 = s.float()
        m = s32.amax(dim=-1, keepdim=True)
        e = torch.exp(s32 - m)
        lv = e.sum(dim=-1, keepdim=True)
        V, wa, tail = HipOmdModule._values(a, b)
        num = K.matmul(e, V) if e.dim() >= 2 and V.dim() >= 2 else e @ V
        return m, lv, num, wa, tail

    @staticmethod
    def _values(a: torch.Tensor, b: torch.Tensor) -> tuple:
        """``[a | b]`` along the value axis (the dense ``a`` flattened), its
        ``fa`` width and trailing shape."""
        if a.dim() >= 3:  # dense fibre (xcarrier.py:393-399)
            d, i = a.shape[-2], a.shape[-1]
            af, tail = a.reshape(*a.shape[:-2], d * i), (d, i)
        else:
            af, tail = a, (a.shape[-1],)
        V = torch.cat([af.float(), b.float().expand(*af.shape[:-1], b.shape[-1])], dim=-1)
        return V, af.shape[-1], tail

    def _fused_leaf(self, sc: dict, a: torch.Tensor, b: torch.Tensor, ev) -> tuple | None:
        """The leaf's carrier from ``catopt_hip_attn_carrier_f32`` when its
        score is ``scale·q kᵀ`` over device fp32/bf16 operands in the kernel's
        envelope; ``None`` otherwise (the unfused path runs)."""
        q, k = ev(sc["q"]), ev(sc["k"])
        if not all(_kernel_dtype(t) for t in (q, k, a, b)) or q.dim() < 2 or k.dim() != q.dim():
            return None
        n = k.dim()
        if sc["axes"] is not None and {x % n for x in sc["axes"]} != {n - 2, n - 1}:
            return None  # not a transpose of the last two axes: the evaluated score is used
        if q.shape[-1] != k.shape[-1] or q.shape[-1] > 128 or tuple(q.shape[:-2]) != tuple(k.shape[:-2]):
            return None
        V, wa, tail = self._values(a, b)
        if V.shape[-1] > 256 or V.shape[-2] != k.shape[-2] or (V.dim() > 2 and tuple(V.shape[:-2]) != tuple(q.shape[:-2])):
            return None
        m, lv, num = K.attn_carrier_f32(q, k, V, float(sc["scale"]))
        return m, lv, num, wa, tail, [q.dtype, k.dtype]

    def _shared_q(self, ev) -> torch.Tensor | None:
        scs = self._plan["scores"]
        if len(scs) < 2 or any(sc is None for sc in scs):
            return None
        if any(not (sc["q"] is scs[0]["q"] or sc["q"] == scs[0]["q"]) or sc["scale"] != scs[0]["scale"]
               for sc in scs):
            return None
        q = ev(scs[0]["q"])
        if not _kernel_dtype(q) or q.dim() != 2 or q.shape[-1] > 128:
            return None
        return q

    @staticmethod
    def _fold(m: torch.Tensor, lv: torch.Tensor, num: torch.Tensor) -> tuple:
        """The om combine of every carrier along axis 0 at once: weights
        ``exp(m_i − M)``, a carrier with no finite score weighing 0."""
        M = m.amax(dim=0)
        fin = torch.isfinite(m)
        w = torch.where(fin, torch.exp(torch.where(fin, m, M) - M), torch.zeros_like(m))
        return M, (lv * w).sum(dim=0), (num * w).sum(dim=0)

    def _batched_blocks(self, ev, Pa: torch.Tensor, Pb: torch.Tensor) -> tuple | None:
        """The chain plan's fast path: every leaf's coefficients are one
        contiguous run of prefix positions, so the value blocks are rows of
        ``[Pa | Pb]`` (built once) and the key blocks chunks of one key array —
        one carrier launch over all leaves, no per-leaf gathers."""
        p = self._plan
        blocks = p["blocks"]
        if not blocks or p["k_chunks"] is None:
            return None
        q = self._shared_q(ev)
        if q is None:
            return None
        L, C = len(blocks), blocks[0][1]
        if any(n != C for _, n in blocks):
            return None
        base, dim = p["k_chunks"]
        kall = ev(base)
        if not _kernel_dtype(kall) or kall.dim() != 2 or dim % 2 != 0 or kall.shape[0] != L * C or \
                kall.shape[1] != q.shape[1]:
            return None
        T = Pa.shape[0]
        tail = tuple(Pa.shape[1:]) if Pa.dim() >= 3 else (Pa.shape[-1],)  # the fibre test of _omd_elem
        wa = Pa[0].numel()
        Vall = _side_by_side(Pa.reshape(T, -1), Pb.reshape(T, -1))
        if Vall.shape[1] > 256:
            return None
        if blocks == [(i * C, C) for i in range(L)]:
            V = Vall[:L * C].view(L, C, -1)
        else:
            V = torch.stack([Vall[s:s + C] for s, _ in blocks])
        carriers = K.attn_carrier_f32(q, kall.reshape(L, C, -1), V, float(p["scores"][0]["scale"]))
        return carriers, wa, tail, [q.dtype, kall.dtype]

    def _batched_leaves(self, ev) -> tuple | None:
        """Every leaf a ``scale · q k_iᵀ`` score over one shared ``q`` with key
        and value blocks of one shape: one carrier launch over (query tiles x
        leaves), then one weighted fold over the leaf axis (the om combine of
        all blocks at once, with the ``isfinite`` guard).  ``None`` when the
        leaves do not line up (each leaf then runs on its own)."""
        p = self._plan
        scs = p["scores"]
        q = self._shared_q(ev)
        if q is None:
            return None
        ks, Vs, shape = [], [], None
        for lf, sc in zip(p["leaves"], scs):
            k, a, b = ev(sc["k"]), ev(lf.args[1]), ev(lf.args[2])
            if not all(_kernel_dtype(t) for t in (k, a, b)) or k.dim() != 2 or k.shape[-1] != q.shape[-1]:
                return None
            if sc["axes"] is not None and set(sc["axes"]) - {0, 1, -1, -2}:
                return None
            V, wa, tail = self._values(a, b)
            if V.dim() != 2 or V.shape[0] != k.shape[0]:
                return None
            if shape is None:
                shape = (k.shape, V.shape, wa, tail)
            elif (k.shape, V.shape, wa, tail) != shape:
                return None
            ks.append(k)
            Vs.append(V)
        if shape[1][-1] > 256:
            return None
        carriers = K.attn_carrier_f32(q, torch.stack(ks), torch.stack(Vs), float(scs[0]["scale"]))
        return carriers, shape[2], shape[3], [q.dtype] + [k.dtype for k in ks[:1]]

    def _forward_impl(self, *xs: Any) -> Any:
        p = self._plan
        if p is None:
            return self.eval_mod(*xs)
        x, env = self._input_env(xs)
        memo: dict = {}
        ev = self.ev_factory(env, x, memo)
        try:
            return self._run(ev, memo)
        except (L.HipKernelError, L.HipExtensionMissing):
            raise
        except (ValueError, IndexError, TypeError, RuntimeError, _Decline):
            self.fallbacks += 1
            return self.eval_mod(*xs)

    def _run(self, ev, memo: dict) -> torch.Tensor:
        p = self._plan
        dtypes = []
        seeded: set = set()
        Pa = Pb = None
        stores: dict = {}
        if p["map_mode"] == "chain":
            A, B = self._leaf_parts(p["chain_leaves"], (p["chain_a_gather"], p["chain_b_gather"]), ev)
            if not (_kernel_dtype(A) and _kernel_dtype(B)):
                raise _Decline()
            Pa, Pb = self._prefix_maps(A, B)
            stores[("chain",)] = (Pa, Pb)
            # the result's dtype follows the chain's operands, not the fp32 prefix maps
            dtypes += [A.dtype, B.dtype]
            seeded = self._seeded_ids
        elif p["map_mode"] == "forest":
            stores = self._forest_maps(ev, dtypes)
            seeded = self._seeded_ids
        state = None
        width = tail = None
        self.fused_leaves = 0
        self.fused_readout = False
        batched = self._batched_blocks(ev, Pa, Pb) if Pa is not None else None
        if batched is None:
            if stores:
                self._seed(memo, stores)  # the leaves read their coefficient stacks through the memo
            batched = self._batched_leaves(ev)
        if batched is not None:
            carriers, width, tail, sdts = batched
            dtypes += sdts
            self.fused_leaves = len(p["leaves"])
            if p["apply"] == "omd_apply" and tail == (width,) and carriers[2].shape[-1] == 2 * width:
                # every leaf's carrier in one stack: the combine over the
                # leaf axis and the diagonal readout run as one kernel
                h = ev(p["h"])
                if _kernel_dtype(h) and h.dim() == 1 and h.shape[0] == width:
                    self.fused_readout = True
                    return K.omd_fold_apply(*carriers, h.float()).to(_promote(h.dtype, dtypes))
            state = self._fold(*carriers)
        for lf, sc in zip(() if batched is not None else p["leaves"], p["scores"]):
            if lf.op == "omd_elem":
                a, b = ev(lf.args[1]), ev(lf.args[2])
                fused = self._fused_leaf(sc, a, b, ev) if sc is not None else None
                if fused is not None:
                    m, lv, num, wa, tl, sdts = fused
                    self.fused_leaves += 1
                else:
                    s = ev(lf.args[0])
                    if not all(_kernel_dtype(t) for t in (s, a, b)):
                        raise _Decline()
                    sdts = [s.dtype]
                    m, lv, num, wa, tl = self._leaf_carrier(s, a, b)
                dtypes += sdts
                dtypes += [t.dtype for t, arg in ((a, lf.args[1]), (b, lf.args[2])) if id(arg) not in seeded]
            else:
                m, lv, fa, fb = (ev(t) for t in lf.args)
                if not all(_kernel_dtype(t) for t in (m, lv, fa, fb)):
                    raise _Decline()
                dtypes += [fa.dtype, fb.dtype]
                lead = m.dim()
                tl = tuple(fa.shape[lead - 1:])
                fa_f = fa.reshape(*fa.shape[:lead - 1], -1).float()
                wa = fa_f.shape[-1]
                num = torch.cat([fa_f, fb.float()], dim=-1)
                m, lv = m.float(), lv.float()
            if width is None:
                width, tail = wa, tl
            elif (wa, tl) != (width, tail):
                raise _Decline()
            e = (m, lv, num)
            if state is not None and (state[0].shape != m.shape or state[2].shape != num.shape):
                # carriers that broadcast against each other (a leaf of one
                # query row beside a leaf of several): compose at the common
                # shape, as the serial _omd_compose broadcasts
                # (omd_lower.py:1006-1011); shapes that do not broadcast raise
                # and the generic module runs
                ms = torch.broadcast_shapes(state[0].shape, m.shape)
                ns = torch.broadcast_shapes(state[2].shape, num.shape)
                state = (state[0].expand(ms).contiguous(), state[1].expand(ms).contiguous(),
                         state[2].expand(ns).contiguous())
                e = (m.expand(ms).contiguous(), lv.expand(ms).contiguous(), num.expand(ns).contiguous())
            state = e if state is None else _om_compose(state, e)
        m, lv, num = state
        fa = num[..., :width].reshape(*num.shape[:-1], *tail)
        fb = num[..., width:]
        h = ev(p["h"])
        if not _kernel_dtype(h):
            raise _Decline()
        out_dtype = _promote(h.dtype, dtypes)
        hf = h.float()
        if p["apply"] == "omd_apply":
            out = (fa * hf + fb) / lv
        else:
            out = (K.matmul(fa, hf) + fb) / lv
        return out.to(out_dtype)


def _side_by_side(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``cat([a, b], dim=1)`` of two ``(T, ·)`` arrays; a view when ``b``'s
    columns already follow ``a``'s in one row-major buffer (the diagonal
    prefix scan writes ``[∏a | prefix b]`` that way)."""
    T, wa = a.shape
    w = wa + b.shape[1]
    if a.dtype == b.dtype and a.stride() == (w, 1) and b.stride() == (w, 1) and \
            b.data_ptr() == a.data_ptr() + wa * a.element_size():
        return a.as_strided((T, w), (w, 1))
    return torch.cat([a, b], dim=1)


def _promote(dt: torch.dtype, dtypes: list) -> torch.dtype:
    """The result dtype: ``h``'s promoted with every operand's."""
    for other in dtypes:
        dt = torch.promote_types(dt, other)
    return dt


class _Decline(Exception):
    """The batched path does not take these operands (the generic module runs)."""


def to_batched_omd_module(ir: IR, param_values: dict | None = None, **kw) -> HipOmdModule:
    """Always a :class:`HipOmdModule` (check ``is_batched``), ``omd_lower.py:1022-1033``."""
    return HipOmdModule(ir, param_values, **kw)


#: The reference's probe name (omd_lower.py:154-170).
is_omd_apply_term = is_omd_term
