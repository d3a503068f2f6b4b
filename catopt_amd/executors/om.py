"""Online-softmax executor: ``om_apply(<om tree>)`` on the HIP attention kernel.

The counterpart of ``BatchedOMModule`` (luisfuturist/catopt
``packages/catopt-carriers/src/catopt_carriers/om_lower.py:496-835``, plan
builder ``build_om_plan`` :334-437).  The delivered form of the ``OM_LIFT``
law (``om.py:153-193``) is

    om_apply(om_elem(s, v)),   s = masked_fill(scale · q kᵀ, M, -inf)

possibly split over key blocks into ``om_compose`` trees of ``om_elem``
leaves (``om.py:1116-1400``).  The reference materialises every leaf's score
block and reduces the tree level by level (~10 elementwise launches per
level, ``om_lower.py:817-832``).  Here each leaf's score pattern is parsed
once, at construction, into ``(q, k, v, scale, mask)``:

* one leaf: one launch of the fused attention kernel (scores, mask, online
  softmax and ``a / l`` never leave the chip);
* several leaves: one unnormalised kernel launch per leaf (emitting the
  ``(m, l, a)`` carrier), combined pairwise in tree order with the
  ``om_compose`` kernel, read out as ``a / l``.

The masked set ``M`` is classified at construction when it is weight-only:
the causal generator ``cmask(x, off)`` (``om.py:1023-1029``, keep
``j <= i - off``) and any bool Param equal to a shifted lower triangle
(compared bit-exactly) become the kernel's implicit causal mode; any other
bool mask is handed to the kernel as a uint8 keep-mask.  A mask that depends
on the inputs is evaluated per call.  ``-inf`` is the only accepted fill: a
finite fill changes what a fully masked row means.

A root that does not parse leaves ``_plan = None`` and every call runs the
embedded generic module (``om_lower.py:730-731``).  A call outside the
kernel's envelope (dtype other than bf16, head dim other than 64/128) also
runs the generic module and increments ``fallbacks``.
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import nn

from .. import kernels as K
from ..bindings import attr_of, scalar_value
from ..evaluator import HipIRModule
from ..ir import IR, is_op
from .base import HipExecutorBase

__all__ = ["HipOMModule", "build_om_plan", "is_om_term", "mask_kwargs", "om_leaves", "parse_score"]


def is_om_term(term: Any) -> bool:
    """Term-level probe: an ``om_apply`` over an om tree."""
    return is_op(term, "om_apply") and len(term.args) >= 1 and _om_tree_ok(term.args[0])


def _om_tree_ok(t: Any) -> bool:
    return om_leaves(t) is not None


def om_leaves(t: Any) -> list | None:
    """Leaves of an ``om_compose`` tree, left to right; ``None`` if a leaf is
    not an ``om_elem``."""
    out: list = []
    stack = [t]
    while stack:
        n = stack.pop()
        if is_op(n, "om_compose", 2):
            stack.append(n.args[1])
            stack.append(n.args[0])
        elif is_op(n, "om_elem", 2):
            out.append(n)
        else:
            return None
    return out


def _is_neg_inf(t: Any) -> bool:
    v = scalar_value(t)
    return v is not None and v == float("-inf")


def _peel_scale(s: Any) -> tuple[Any, float]:
    scale = 1.0
    while True:
        if is_op(s, "mul", 2):
            a, b = s.args
            cb, ca = scalar_value(b), scalar_value(a)
            if cb is not None and math.isfinite(cb):
                scale *= cb
                s = a
                continue
            if ca is not None and math.isfinite(ca):
                scale *= ca
                s = b
                continue
        if is_op(s, "div", 2) and not s.attrs.get("rounding_mode"):
            c = scalar_value(s.args[1])
            if c is not None and math.isfinite(c) and c != 0.0:
                scale /= c
                s = s.args[0]
                continue
        return s, scale


def _transposed_operand(kt: Any) -> Any | None:
    """``k`` of ``transpose(k, -2, -1)`` (either dim order)."""
    if not is_op(kt, "transpose", 1):
        return None
    d0 = attr_of(kt.attrs, "dim0", default=None)
    d1 = attr_of(kt.attrs, "dim1", default=None)
    if d0 is None and d1 is None:
        return kt.args[0]  # the 2-D .t() spelling
    dims = {int(d0), int(d1)}
    if dims == {-2, -1}:
        return kt.args[0]
    typ = getattr(kt.args[0], "typ", None)  # a leaf of known rank n: dims n-2, n-1
    rank = len(typ.shape) if typ is not None else None
    if rank is not None and rank >= 2 and dims == {rank - 2, rank - 1}:
        return kt.args[0]
    return None


def parse_score(s: Any) -> dict | None:
    """``(q, k, scale, mask)`` of ``masked_fill(scale·q kᵀ, M, -inf)``."""
    mask = None
    if is_op(s, "masked_fill", 3):
        if not _is_neg_inf(s.args[2]):
            return None
        mask = s.args[1]
        s = s.args[0]
    s, scale = _peel_scale(s)
    if not is_op(s, "matmul", 2):
        return None
    k = _transposed_operand(s.args[1])
    if k is None:
        return None
    return {"q": s.args[0], "k": k, "scale": scale, "mask": mask}


def _triangle_offset(masked: torch.Tensor) -> int | None:
    """``off`` when the masked set is exactly ``¬tril(ones(t, k), -off)``
    (shared over any leading axes), compared bit-exactly; else ``None``."""
    if masked.dim() < 2:
        return None
    m3 = masked.reshape(-1, *masked.shape[-2:]).to(torch.bool)
    if m3.shape[0] != 1 and not bool((m3 == m3[:1]).all()):
        return None
    keep = ~m3[0]
    t, k = keep.shape
    n = keep.sum(dim=1)
    mid = ((n > 0) & (n < k)).nonzero()
    if mid.numel():
        i = int(mid[0])
        off = i + 1 - int(n[i])  # row i keeps j <= i - off
    else:
        full = (n == k).nonzero()
        if full.numel() == 0:
            return None  # every row fully masked: not a triangle
        off = int(full[0]) - (k - 1)
    ref = torch.ones(t, k, dtype=torch.bool, device=keep.device).tril(-off)
    return off if torch.equal(ref, keep) else None


class HipOMModule(HipExecutorBase, nn.Module):
    """Planned executor for ``om_apply(<om tree>)`` (module docstring)."""

    def __init__(self, ir: IR, param_values: dict | None = None, *, eval_mod: HipIRModule | None = None,
                 device: Any = None, ops=None) -> None:
        super().__init__()
        self.eval_mod = eval_mod if eval_mod is not None else HipIRModule(ir, param_values, device=device, ops=ops)
        self._inputs = list(ir.inputs)
        self._const_cache: dict = {}
        self.fallbacks = 0
        self._plan = build_om_plan(self.eval_mod._root, self.eval_mod)
        self._init_graph_state()

    @property
    def n_leaves(self) -> int:
        return 0 if self._plan is None else len(self._plan["leaves"])

    def _forward_impl(self, *xs: Any) -> Any:
        if self._plan is None:
            return self.eval_mod(*xs)
        x, env = self._input_env(xs)
        ev = self.ev_factory(env, x)
        carriers = []
        leaves = self._plan["leaves"]
        single = len(leaves) == 1
        for lf in leaves:
            q, k, v = ev(lf["q"]), ev(lf["k"]), ev(lf["v"])
            mask_kw = self._mask_kwargs(lf, ev)
            if mask_kw is None or not _in_envelope(q, k, v):
                self.fallbacks += 1
                return self.eval_mod(*xs)
            q4, k4, v4, lead = _as_bhtd(q, k, v)
            if q4 is None:
                self.fallbacks += 1
                return self.eval_mod(*xs)
            if single:
                o = K.attention(q4, k4, v4, lf["scale"], normalize=True, **mask_kw)
                return o.reshape(*lead, o.shape[-2], o.shape[-1])
            a, m, lsum = K.attention(q4, k4, v4, lf["scale"], normalize=False, return_ml=True, **mask_kw)
            carriers.append((m, lsum, a.float()))
        # pairwise combine in tree order (adjacent pairs, odd tail carried up)
        while len(carriers) > 1:
            nxt = [K.om_compose(carriers[i], carriers[i + 1]) for i in range(0, len(carriers) - 1, 2)]
            if len(carriers) % 2:
                nxt.append(carriers[-1])
            carriers = [(m.reshape(carriers[0][0].shape), lv.reshape(carriers[0][1].shape),
                         acc.reshape(carriers[0][2].shape)) for m, lv, acc in nxt]
        m, lsum, acc = carriers[0]
        out = (acc / lsum).to(ev(leaves[0]["q"]).dtype)
        return out.reshape(*lead, out.shape[-2], out.shape[-1])

    def _mask_kwargs(self, lf: dict, ev) -> dict | None:
        return mask_kwargs(lf, ev)


def mask_kwargs(lf: dict, ev) -> dict | None:
    """Attention-kernel mask arguments of a parsed leaf; ``None`` when a
    runtime mask is not a single ``(Tq, Tk)`` plane shared over (B, H)."""
    kind = lf["mask_kind"]
    if kind == "none":
        return {}
    if kind == "causal":
        return {"causal": True, "causal_off": lf["causal_off"]}
    if kind == "bool_const":
        return {"mask": lf["keep"]}
    masked = ev(lf["mask"])
    if not isinstance(masked, torch.Tensor) or masked.dim() < 2:
        return None
    m2 = masked.reshape(-1, *masked.shape[-2:])
    if m2.shape[0] != 1:
        return None
    return {"mask": torch.logical_not(m2[0].to(torch.bool))}


def _in_envelope(q, k, v) -> bool:
    ts = (q, k, v)
    if not all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in ts):
        return False
    if any(t.dtype != torch.bfloat16 for t in ts):
        return False
    d = q.shape[-1]
    return d in (64, 128) and k.shape[-1] == d and v.shape[-1] == d and 2 <= q.dim() <= 4


def _as_bhtd(q, k, v):
    lead = tuple(q.shape[:-2])
    if k.shape[:-2] != q.shape[:-2] or v.shape[:-2] != q.shape[:-2] or k.shape[-2] != v.shape[-2]:
        return None, None, None, None
    while q.dim() < 4:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    return q, k, v, lead


def build_om_plan(root: Any, eval_mod: HipIRModule) -> dict | None:
    """Parse ``om_apply(<om tree>)`` into per-leaf kernel arguments."""
    if not is_op(root, "om_apply") or not root.args:
        return None
    leaves = om_leaves(root.args[0])
    if not leaves:
        return None
    plan_leaves = []
    for leaf in leaves:
        s, v = leaf.args
        sc = parse_score(s)
        if sc is None:
            return None
        if not (math.isfinite(sc["scale"]) and sc["scale"] > 0):
            # the kernel tracks the row max of q·k and scales it, which is the
            # max of the scaled scores only for a positive scale
            return None
        lf = {"q": sc["q"], "k": sc["k"], "v": v, "scale": sc["scale"], "mask": sc["mask"]}
        if not _classify_mask(lf, eval_mod):
            return None
        plan_leaves.append(lf)
    return {"leaves": plan_leaves}


def _classify_mask(lf: dict, eval_mod: HipIRModule) -> bool:
    m = lf["mask"]
    if m is None:
        lf["mask_kind"] = "none"
        return True
    if is_op(m, "cmask", 1):
        lf["mask_kind"] = "causal"
        lf["causal_off"] = -int(m.attrs.get("off", 0) or 0)
        return True
    pv = eval_mod._pv(m)
    if pv is not None:  # weight-only mask (folded into a Param)
        if pv.dtype != torch.bool:
            return False
        off = _triangle_offset(pv)
        if off is not None:
            lf["mask_kind"] = "causal"
            lf["causal_off"] = -off
            return True
        m2 = pv.reshape(-1, *pv.shape[-2:])
        if m2.shape[0] != 1:
            return False
        lf["mask_kind"] = "bool_const"
        lf["keep"] = torch.logical_not(m2[0]).contiguous()
        return True
    lf["mask_kind"] = "runtime"
    return True
