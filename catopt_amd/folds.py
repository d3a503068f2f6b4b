"""The causal-mask const fold behind ``HipSink.specialize_causal``.

The counterpart of luisfuturist/catopt
``packages/catopt-torch/src/catopt_torch/folds.py:28-118`` (exposed by the
torch sink as ``specialize_causal``, ``adapters.py:102-113``): a
parameter-only ``sdpa`` mask that is exactly the causal lower triangle is
dropped and ``is_causal`` (attr ``arg5``) set, so the attention kernel runs
its implicit causal mode instead of reading a ``T × T`` mask.  The
orchestrator calls ``sink.specialize_causal(term, params, memo) -> term``
and reads ``memo["_hit"]``.

The mask is folded on the sink's device through the HIP op table (the
backend's own runtime): a bare ``Param`` is taken as bound, any other
parameter-only subtree is evaluated with its parameter values moved to the
device.  Anything that cannot be evaluated — a ``Var``, an unbound
``Param``, a missing or raising binding, a non-tensor result — leaves the
term as it is.
"""

from __future__ import annotations

from typing import Any

import torch

from .evaluator import _is_param, _is_var, eval_term
from .ir import Op, postorder

__all__ = ["eval_const", "is_causal_keep_mask", "specialize_causal"]


def _term_shape(t: Any) -> tuple | None:
    shape = getattr(getattr(t, "typ", None), "shape", None)
    if shape is None or any(d is None for d in shape):
        return None
    return tuple(int(d) for d in shape)


def eval_const(term: Any, params: dict, ops: Any, device: Any = None) -> torch.Tensor | None:
    """The value of a parameter-only subtree, or ``None`` when it has none
    (``folds.py:28-48``)."""
    try:
        if _is_param(term):
            val = params.get(term.name)
            return val if isinstance(val, torch.Tensor) else None
        if not isinstance(term, Op):
            return None
        names = set()
        for node in postorder(term):
            for a in node.args:
                if _is_var(a):
                    return None
                if _is_param(a):
                    if not isinstance(params.get(a.name), torch.Tensor):
                        return None
                    names.add(a.name)
        env = {n: params[n].to(device) if device is not None else params[n] for n in names}
        out = eval_term(term, {}, env, ops)
    except Exception:  # a raising binding is "not foldable", as in the reference
        return None
    return out if isinstance(out, torch.Tensor) else None


def is_causal_keep_mask(mask: torch.Tensor, q_shape: tuple | None) -> bool:
    """``mask`` is exactly ``tril(ones(T, T))`` as a keep-set (a bool keep
    or an additive mask whose kept entries are above -1e30) with ``T`` q's
    sequence extent (``folds.py:51-77``).  With ``q``'s shape unknown a
    square mask of ``T > 1`` still fixes ``Tq = Tk = T``: no other score
    shape broadcasts with it."""
    if mask.dim() < 2 or mask.shape[-1] != mask.shape[-2]:
        return False
    t = mask.shape[-1]
    if q_shape is None:
        if t < 2:
            return False
    elif not isinstance(q_shape, tuple) or len(q_shape) < 2 or q_shape[-2] != t:
        return False
    keep = mask.to(torch.bool) if mask.dtype == torch.bool else mask > -1e30
    tril = torch.ones(t, t, dtype=torch.bool, device=mask.device).tril()
    return bool((keep == tril).all())


def specialize_causal(term: Any, params: dict, memo: dict | None = None, *, ops: Any,
                      device: Any = None) -> Any:
    """``sdpa(q, k, v, mask) → sdpa(q, k, v, arg5=True)`` wherever the
    parameter-only mask is the causal keep-mask; ``memo`` is content-keyed
    and ``memo["_hit"]`` records that a rewrite fired
    (``folds.py:81-118``)."""
    if memo is None:
        memo = {}
    if not isinstance(term, Op):
        return term
    if term in memo:
        return memo[term]
    done: dict = {}
    for node in postorder(term):
        if node in memo:
            done[node] = memo[node]
            continue
        args = tuple(done.get(a, a) if isinstance(a, Op) else a for a in node.args)
        attrs = dict(node.attrs)
        if node.op == "sdpa" and len(args) >= 4 and not attrs.get("arg5"):
            mv = eval_const(args[3], params, ops, device)
            if mv is not None and is_causal_keep_mask(mv, _term_shape(args[0])):
                args = args[:3]
                attrs["arg5"] = True
                memo["_hit"] = True
        out = Op.make(node.op, *args, **attrs)
        memo[node] = out
        done[node] = out
    return memo[term]
