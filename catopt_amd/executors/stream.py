"""Streaming (bounded working set) om attention and the incremental decode API.

The counterpart of ``StreamingOMModule`` and of the module-level helpers
``om_empty_state`` / ``om_step`` / ``om_step_qk`` / ``om_apply_state``
(luisfuturist/catopt
``packages/catopt-carriers/src/catopt_carriers/om_lower.py:871-1040``).

The term is the same as the batched om executor's, ``om_apply(<om_compose
tree>)``, but it is run as a left fold: each leaf's carrier ``(m, l, a)`` is
produced, composed into a running state and released, so peak memory is one
block plus the carrier, never the full q × T_kv score matrix.

Leaves:

* ``om_elem(s, v)`` whose score parses as a positively scaled ``q kᵀ`` with
  a mask the attention kernel takes (the spellings of the batched om
  executor: ``masked_fill(…, M, -inf)``, ``add(…, attnbias(m))``, key-axis
  ``concat`` scores) with bf16 operands and head dims up to 128: one launch
  of the HIP attention kernel in carrier mode (scores, mask and
  exponentials stay on chip; the carrier is fp32); fp32 operands with
  ``dk <= 128``, ``dv <= 256``: one launch of the fp32 carrier kernel, with
  the same mask modes (fp16 operands widened to fp32 for it);
* any other ``om_elem(s, v)``: the score and value operands are evaluated and
  folded with ``om_elem`` (``torch_bridge.py:1974-1981``; on device fp32 /
  bf16 operands the ``catopt_hip_om_rows`` row kernel and the HIP GEMM);
* a packaged carrier ``om(m, l, a)``: used as is.

States compose with the HIP ``om_compose`` kernel when both carriers are
fp32 device tensors of matching shape (the ``isfinite`` guard of
``torch_bridge.py:1984-2006`` is in the kernel), else with the same formula in
device tensor ops.  A DAG-shared leaf contributes once per occurrence, the
fold order is the tree's left-to-right leaf order, and every leaf is
evaluated with a fresh memo (block intermediates die with the iteration),
as in the reference.

The decode helpers are plain device work on torch's current stream (no host
synchronisation, no allocation inside the kernels), so a decode step can be
recorded into a hipGraph by the caller.
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import nn

from .. import kernels as K
from ..bindings import _matmul, _om_compose, om_elem_dense
from ..evaluator import HipIRModule
from ..ir import IR, is_op
from .om import _as_bhtd, _classify_mask, _f32_envelope, _in_envelope, mask_kwargs, parse_score

__all__ = [
    "HipStreamingOMModule",
    "build_stream_plan",
    "om_apply_state",
    "om_empty_state",
    "om_step",
    "om_step_qk",
    "to_streaming_om_module",
]


def om_empty_state(shape: tuple, dv: int, device: Any = None, dtype: torch.dtype | None = None):
    """The ⊕ identity ``(m, l, a) = (-inf, 0, 0)`` (``om_lower.py:871-889``):
    ``m, l`` shaped ``(*shape, 1)``, ``a`` shaped ``(*shape, dv)``."""
    m = torch.full((*shape, 1), float("-inf"), device=device, dtype=dtype)
    lv = torch.zeros(*shape, 1, device=device, dtype=dtype)
    a = torch.zeros(*shape, dv, device=device, dtype=dtype)
    return (m, lv, a)


def _compose(state: tuple | None, e: tuple) -> tuple:
    return e if state is None else _om_compose(state, e)


def om_step(state: tuple | None, s: torch.Tensor, v: torch.Tensor):
    """``state ⊕ om_elem(s, v)`` for one score block ``s (…, Tq, K_blk)`` and
    value block ``v (…, K_blk, dv)`` (``om_lower.py:892-907``)."""
    return _compose(state, om_elem_dense(s, v))


def _carrier_qk(q, k, v, scale: float = 1.0, **mask_kw) -> tuple | None:
    """``om_elem(scale · q kᵀ, v)`` by the attention kernel in carrier mode
    (bf16) or the fp32 carrier kernel (fp32, or fp16 widened), or ``None``
    outside their envelopes."""
    if not _in_envelope(q, k, v):
        if not _f32_envelope(q, k, v):
            return None
        return K.attn_carrier_f32(q, k, v, float(scale), **mask_kw)
    q4, k4, v4, lead = _as_bhtd(q, k, v)
    if q4 is None or not K.attention_grid_ok(q4):
        return None
    a, m, lv = K.attention(q4, k4, v4, scale, normalize=False, return_ml=True, **mask_kw)
    tq, dv = a.shape[-2], a.shape[-1]
    return (m.reshape(*lead, tq, 1), lv.reshape(*lead, tq, 1), a.float().reshape(*lead, tq, dv))


def om_step_qk(state: tuple | None, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """:func:`om_step` for the canonical score ``s = q @ kᵀ`` (no scale),
    ``om_lower.py:910-917``.  bf16 operands with head dims up to 128 (fp32:
    ``dk <= 128``, ``dv <= 256``) never materialise ``s``: an attention
    kernel emits the block's carrier."""
    e = _carrier_qk(q, k, v, 1.0)
    if e is None:
        return om_step(state, _matmul(q, k.transpose(-2, -1)), v)
    return _compose(state, e)


def om_apply_state(state: tuple) -> torch.Tensor:
    """The ``om_apply`` readout ``a / l``, unclamped (a fully masked row
    gives 0/0 = NaN, as dense softmax), ``om_lower.py:920-922``."""
    return state[2] / state[1]


def _stream_leaves(t: Any) -> list | None:
    out: list = []
    stack = [t]
    while stack:
        n = stack.pop()
        if is_op(n, "om_compose", 2):
            stack.append(n.args[1])
            stack.append(n.args[0])
        elif is_op(n, "om_elem", 2) or is_op(n, "om", 3):
            out.append(n)
        else:
            return None
    return out


def build_stream_plan(root: Any, eval_mod: HipIRModule) -> dict | None:
    """Leaves of ``om_apply(<om tree>)`` in fold order, each classified as
    ``qk`` (kernel-eligible score pattern), ``elem`` or ``om``; ``None`` when
    the root is not an om_apply over an om tree."""
    if not is_op(root, "om_apply") or not root.args:
        return None
    leaves = _stream_leaves(root.args[0])
    if not leaves:
        return None
    plan = []
    for leaf in leaves:
        if is_op(leaf, "om", 3):
            plan.append({"kind": "om", "m": leaf.args[0], "l": leaf.args[1], "a": leaf.args[2]})
            continue
        s, v = leaf.args
        lf: dict = {"kind": "elem", "s": s, "v": v}
        sc = parse_score(s)
        # the kernel scales the row max of q·k: the scaled scores' max only
        # for a positive scale
        if sc is not None and math.isfinite(sc["scale"]) and sc["scale"] > 0:
            lq = {"q": sc["q"], "k": sc["k"], "v": v, "scale": sc["scale"], "mask": sc["mask"],
                  "bias": sc["bias"]}
            if _classify_mask(lq, eval_mod) and lq["mask_kind"] != "scores":
                lf.update(lq)
                lf["kind"] = "qk"
        plan.append(lf)
    return {"leaves": plan}


class HipStreamingOMModule(nn.Module):
    """``om_apply(<om tree>)`` as a bounded left fold (module docstring).

    A planned executor (``forward`` + ``_plan``, ``eval_mod`` the generic
    fallback) whose discriminator is ``is_streaming``, as in the reference; a
    root that is not an om tree runs the embedded generic module.
    """

    step = staticmethod(om_step)
    step_qk = staticmethod(om_step_qk)
    apply = staticmethod(om_apply_state)
    empty_state = staticmethod(om_empty_state)

    def __init__(self, ir: IR, param_values: dict | None = None, *, eval_mod: HipIRModule | None = None,
                 device: Any = None, ops=None) -> None:
        super().__init__()
        self.eval_mod = eval_mod if eval_mod is not None else HipIRModule(ir, param_values, device=device, ops=ops)
        self._inputs = list(ir.inputs)
        self._plan = build_stream_plan(self.eval_mod._root, self.eval_mod)
        self.kernel_leaves = 0  # leaves folded by the attention kernel on the last call

    @property
    def is_streaming(self) -> bool:
        return self._plan is not None

    @property
    def n_blocks(self) -> int:
        return 0 if self._plan is None else len(self._plan["leaves"])

    def forward(self, *xs: Any) -> Any:
        if self._plan is None:
            return self.eval_mod(*xs)
        state, dtype = self._fold(xs)
        out = om_apply_state(state)
        return out if dtype is None else out.to(dtype)

    def forward_state(self, *xs: Any) -> Any:
        """The raw ``(m, l, a)`` carrier of the fold: the state a decode loop
        keeps, extends with :func:`om_step` / :func:`om_step_qk` and reads out
        with :func:`om_apply_state`."""
        if self._plan is None:
            return self.eval_mod(*xs)
        return self._fold(xs)[0]

    def _fold(self, xs: tuple) -> tuple[tuple, torch.dtype | None]:
        x = xs[0] if xs else None
        env: dict = {"self": x}
        for i, inp in enumerate(self._inputs):
            env[inp.name] = xs[i] if i < len(xs) else x
        state: tuple | None = None
        out_dtype: torch.dtype | None = None
        n_kernel = 0
        for lf in self._plan["leaves"]:
            memo: dict = {}  # fresh per leaf: block intermediates die with the iteration

            def ev(t: Any) -> Any:
                if is_op(t) and t in memo:
                    return memo[t]
                return self.eval_mod._eval(t, env, x, memo)

            if lf["kind"] == "om":
                e = (ev(lf["m"]), ev(lf["l"]), ev(lf["a"]))
            else:
                e = None
                if lf["kind"] == "qk":
                    q, k, v = ev(lf["q"]), ev(lf["k"]), ev(lf["v"])
                    mkw = mask_kwargs(lf, ev, q.shape[-2], k.shape[-2])
                    if mkw is not None:
                        e = _carrier_qk(q, k, v, lf["scale"], **mkw)
                    if e is not None:
                        n_kernel += 1
                        out_dtype = out_dtype or v.dtype
                if e is None:
                    s, v = ev(lf["s"]), ev(lf["v"])
                    e = om_elem_dense(s, v)
            state = _compose(state, e)
        self.kernel_leaves = n_kernel
        return state, out_dtype


def to_streaming_om_module(ir: IR, param_values: dict | None = None, **kw) -> HipStreamingOMModule:
    """Always a :class:`HipStreamingOMModule` (check ``is_streaming``),
    ``om_lower.py:1043-1054``."""
    return HipStreamingOMModule(ir, param_values, **kw)
