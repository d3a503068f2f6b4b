"""Diagonal-affine scan executor on the HIP scan kernels.

The counterpart of ``BatchedScanModule`` (luisfuturist/catopt
``packages/catopt-carriers/src/catopt_carriers/scan_lower.py:427-807``,
``build_scan_plan`` :339-424) and of the fused level bodies
``fused_diag_levels`` (``scan_fused.py:100-120``) for the diagonal-affine
monoid (bindings ``aff_diag`` / ``affd_compose`` / ``applyd``,
``torch_bridge.py:1895-1900``: ``compose(f, g) = (f.a·g.a, f.a·g.b + f.b)``,
``g`` applied first).  Two roots are planned:

* **final state** — ``applyd(F, h)`` with ``F`` an ``affd_compose`` tree over
  ``aff_diag(a_i, u_i)`` leaves.  Leaves are read in product order (leaf 0
  is the outermost map, applied last; ``tests/test_scan_fused.py:105-107``),
  so time runs over the reversed leaf list;
* **every prefix state** — the stacked-map form of ``gather_applyd_stack``
  (``xcarrier.py:2252-2273``):
  ``applyd(aff_diag(stack(affd_a f_0 … f_n), stack(affd_b f_0 … f_n)), h)``
  where each ``f_i = affd_compose(leaf_i, f_{i-1})`` extends the previous
  prefix by one step (checked structurally, not assumed).

Instead of ``log₂ T`` levels of gathers and pointwise launches
(``scan_lower.py:652-674``), the leaf operands are laid out as ``(T, S)``
arrays and one kernel walks the steps: lane-parallel over the state, serial
over time in registers, or chunk-parallel (local chunk maps, a carry fold
over the chunk table, a re-scan) when the state is too small to fill the
GPU.  The chunk table is the reference's blocked all-prefix plan
(``omd_lower.py:771-824``: ``blk = ⌈√T⌉``, starts ``c·blk``) as an int64
array.  When every leaf reads step ``t`` of one shared array
(``select(X, dim, t)`` / ``getitem(X, t)``), that array is used in place
instead of stacking ``T`` slices.

The kernels compute in fp32: bf16/fp32 operands run on them (results cast
back to the operand dtype); fp64 and host operands run the embedded generic
module, counted in ``fallbacks``.
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
from ..ir import IR, is_op
from .base import HipExecutorBase

__all__ = ["HipScanModule", "build_scan_plan", "is_scan_term", "prefix_chunk_table", "affd_leaves"]


def prefix_chunk_table(T: int) -> list[int]:
    """Chunk starts of the blocked all-prefix plan plus the end ``T``
    (``omd_lower.py:786-788``: ``blk = ⌈√T⌉``, ``C = ⌈T/blk⌉``)."""
    if T < 1:
        raise ValueError("T must be positive")
    blk = math.isqrt(T - 1) + 1 if T > 1 else 1  # ⌈√T⌉ without float rounding
    C = (T + blk - 1) // blk
    return [c * blk for c in range(C)] + [T]


def affd_leaves(F: Any) -> list | None:
    """``aff_diag`` leaves of an ``affd_compose`` tree in product order."""
    out: list = []
    stack = [F]
    while stack:
        n = stack.pop()
        if is_op(n, "affd_compose", 2):
            stack.append(n.args[1])
            stack.append(n.args[0])
        elif is_op(n, "aff_diag", 2):
            out.append(n)
        else:
            return None
    return out


def _prefix_chain(fs: list) -> list | None:
    """Time-ordered leaves when ``fs[i] = affd_compose(leaf_i, fs[i-1])``."""
    if not fs or not is_op(fs[0], "aff_diag", 2):
        return None
    leaves = [fs[0]]
    for i in range(1, len(fs)):
        f = fs[i]
        if not is_op(f, "affd_compose", 2) or f.args[1] is not fs[i - 1] and f.args[1] != fs[i - 1]:
            return None
        if not is_op(f.args[0], "aff_diag", 2):
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


def build_scan_plan(root: Any) -> dict | None:
    if not is_op(root, "applyd", 2):
        return None
    F, h = root.args
    if is_op(F, "aff_diag", 2):
        pa, pb = _proj_list(F.args[0], "affd_a"), _proj_list(F.args[1], "affd_b")
        if pa is not None and pb is not None:
            fs_a, dim_a = pa
            fs_b, dim_b = pb
            if dim_a != dim_b or len(fs_a) != len(fs_b) or any(x is not y and x != y for x, y in zip(fs_a, fs_b)):
                return None
            leaves = _prefix_chain(fs_a)
            if leaves is None:
                return None
            return {"mode": "prefix", "leaves": leaves, "h": h, "dim": dim_a,
                    "gather": _shared_gather(leaves), "table": prefix_chunk_table(len(leaves))}
    leaves = affd_leaves(F)
    if leaves is None:
        return None
    leaves = leaves[::-1]  # time order: the innermost map runs first
    return {"mode": "final", "leaves": leaves, "h": h, "gather": _shared_gather(leaves),
            "table": prefix_chunk_table(len(leaves))}


def _step_index(t: Any) -> tuple | None:
    """``(base, dim, index)`` of ``select(base, dim, index)`` / ``getitem(base, int)``."""
    if is_op(t, "select", 1):
        return t.args[0], int(attr_of(t.attrs, "dim", default=0)), int(attr_of(t.attrs, "index", default=0))
    if is_op(t, "getitem", 1):
        ix = t.attrs.get("index")
        if isinstance(ix, int) and not isinstance(ix, bool):
            return t.args[0], 0, ix
    return None


def _shared_gather(leaves: list) -> dict | None:
    """When leaf ``t`` reads step ``t`` of shared ``a`` / ``u`` arrays (same
    base, same axis, indices 0..T-1 in time order), the bases themselves."""
    out = {}
    for slot in (0, 1):
        idx = [_step_index(lf.args[slot]) for lf in leaves]
        if any(i is None for i in idx):
            return None
        base, dim = idx[0][0], idx[0][1]
        if any(i[0] is not base and i[0] != base for i in idx) or any(i[1] != dim for i in idx):
            return None
        if [i[2] for i in idx] != list(range(len(leaves))):
            return None
        out[slot] = (base, dim)
    return out


def is_scan_term(term: Any) -> bool:
    return build_scan_plan(term) is not None


class HipScanModule(HipExecutorBase, nn.Module):
    """Planned executor for diagonal-affine scans (module docstring)."""

    def __init__(self, ir: IR, param_values: dict | None = None, *, eval_mod: HipIRModule | None = None,
                 device: Any = None, ops=None, schedule: int | None = None) -> None:
        super().__init__()
        self.eval_mod = eval_mod if eval_mod is not None else HipIRModule(ir, param_values, device=device, ops=ops)
        self._inputs = list(ir.inputs)
        self._const_cache: dict = {}
        self.fallbacks = 0
        self.schedule = L.SCAN_AUTO if schedule is None else schedule
        self._plan = build_scan_plan(self.eval_mod._root)
        self._init_graph_state()

    @property
    def n_steps(self) -> int:
        return 0 if self._plan is None else len(self._plan["leaves"])

    def _operands(self, ev) -> tuple:
        p = self._plan
        T = len(p["leaves"])
        if p["gather"] is not None:
            a_base, a_dim = p["gather"][0]
            u_base, u_dim = p["gather"][1]
            a = ev(a_base).movedim(a_dim, 0)
            u = ev(u_base).movedim(u_dim, 0)
            if a.shape[0] != T or u.shape[0] != T:
                a = u = None
            if a is not None:
                return a, u
        a = torch.stack([torch.as_tensor(ev(lf.args[0])) for lf in p["leaves"]])
        u = torch.stack([torch.as_tensor(ev(lf.args[1])) for lf in p["leaves"]])
        return a, u

    def _forward_impl(self, *xs: Any) -> Any:
        p = self._plan
        if p is None:
            return self.eval_mod(*xs)
        x, env = self._input_env(xs)
        ev = self.ev_factory(env, x)
        a, u = self._operands(ev)
        h = ev(p["h"])
        ts = (a, u, h)
        if not all(isinstance(t, torch.Tensor) and t.device.type == "cuda"
                   and t.dtype in (torch.float32, torch.bfloat16) for t in ts):
            self.fallbacks += 1
            return self.eval_mod(*xs)
        out_dtype = torch.result_type(torch.empty((), dtype=a.dtype), torch.empty((), dtype=u.dtype))
        out_dtype = torch.promote_types(out_dtype, h.dtype)
        T = a.shape[0]
        sshape = torch.broadcast_shapes(a.shape[1:], u.shape[1:], h.shape)
        a_ = a.expand(T, *sshape)
        u_ = u.expand(T, *sshape)
        h_ = h.expand(sshape)
        states, hf = K.affd_scan(a_, u_, h_, p["table"], schedule=self.schedule,
                                 states=p["mode"] == "prefix")
        if p["mode"] == "final":
            return hf.to(out_dtype)
        return states.to(out_dtype).movedim(0, p["dim"])
