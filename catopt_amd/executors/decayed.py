"""Chunked decayed-retention executor on the HIP retention kernel.

The counterpart of ``ChunkedDecayModule`` (luisfuturist/catopt
``packages/catopt-carriers/src/catopt_carriers/decayed_lower.py:381-724``,
plan parse ``build_decayed_plan`` :329-368).  It accepts the delivered form
of the K-way law ``om_decayed_kway_blocks(K)`` (``om.py:3040-3210``)::

    concat_i( om_decayed(s_ii, decay(γ, t=C), v_i)
              + Σ_{j<i} unsqueeze(decay_vec(γ, t=C, offset=OFF_i_j), -1)
                        ⊙ ((s_ij ⊙ unsqueeze(decay_vec(γ, t=C, sign=-1), -2)) @ v_j) ,  dim=-2)

with ``s_ij = split(split(s, SZ, -2, i), SZ, -1, j)``, ``v_j = split(v, SZ,
-2, j)``, ``SZ = (C,)*K``, ``OFF_i_j = (i-j)·C`` — and its single-block
source ``om_decayed(s, decay(γ, t=T), v)`` — where
``s = scale · q kᵀ`` (a ``div``/``mul`` by a constant is peeled, inside a
summand or around the score).  Every integer of the plan (``K``, ``C``,
``SZ``, each ``OFF_i_j``, the gate signs) is checked exactly against the law's
derive (``om.py:3064-3075``); any mismatch leaves ``_plan = None`` and the
embedded generic module runs the term as written.

All K-way forms of one ``(q, k, v, γ, scale)`` denote the same function
``o[t] = scale · Σ_{s≤t} γ^{t-s} (q_t·k_s) v_s``, so the plan keeps only those
five operands: the kernel picks its own chunk length and carries the
inter-chunk state on chip (``S_{i+1} = γ^C S_i + K̃_iᵀ V_i``) instead of the
reference's O(K²) pair products (``decayed_lower.py:671-700``).  γ is held in
fp32 and every decay factor is formed in fp32 inside the kernel.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import nn

from .. import kernels as K
from ..bindings import attr_of
from ..evaluator import HipIRModule
from ..ir import IR, is_op
from .base import HipExecutorBase
from .om import _peel_scale, _transposed_operand

__all__ = ["HipChunkedDecayModule", "build_decayed_plan", "is_decayed_term"]


def _flat(t: Any, op: str, dim: int | None = None) -> list:
    out, stack = [], [t]
    while stack:
        n = stack.pop()
        if is_op(n, op) and len(n.args) >= 2 and (dim is None or n.attrs.get("dim") == dim):
            stack.extend(reversed(n.args))
        else:
            out.append(n)
    return out


def _split_of(t: Any, dim: int) -> tuple | None:
    """``(base, sizes, index)`` of ``split(base, sizes=SZ, dim=dim, index=i)``."""
    if not is_op(t, "split", 1) or int(attr_of(t.attrs, "dim", default=-1)) != dim:
        return None
    sz = attr_of(t.attrs, "sizes", "split_size", default=None)
    if not isinstance(sz, (list, tuple)):
        return None
    return t.args[0], tuple(int(z) for z in sz), int(attr_of(t.attrs, "index", default=0))


def _score_block(t: Any) -> tuple | None:
    """``(s, SZ, i, j)`` of ``split(split(s, SZ, -2, i), SZ, -1, j)``."""
    outer = _split_of(t, -1)
    if outer is None:
        return None
    inner = _split_of(outer[0], -2)
    if inner is None or inner[1] != outer[1]:
        return None
    return inner[0], outer[1], inner[2], outer[2]


def _gate(t: Any, dim: int) -> tuple | None:
    """``(γ, t, offset, sign)`` of ``unsqueeze(decay_vec(γ, …), dim)``."""
    if not is_op(t, "unsqueeze", 1) or int(attr_of(t.attrs, "dim", default=-1)) != dim:
        return None
    dv = t.args[0]
    if not is_op(dv, "decay_vec", 1):
        return None
    sign = int(dv.attrs["sign"]) if "sign" in dv.attrs else 1
    return dv.args[0], int(dv.attrs.get("t", 0) or 0), int(dv.attrs.get("offset", 0) or 0), sign


def _peel_summand(t: Any) -> tuple[Any, float]:
    return _peel_scale(t)


def _parse_qk(s: Any) -> tuple | None:
    s, scale = _peel_scale(s)
    if not is_op(s, "matmul", 2):
        return None
    k = _transposed_operand(s.args[1])
    if k is None:
        return None
    return s.args[0], k, scale


def is_decayed_term(term: Any) -> bool:
    """Term-level probe: the K-way concat or the single ``om_decayed`` block."""
    return _parse(term) is not None


def _parse(root: Any) -> dict | None:
    body, outer_scale = _peel_scale(root)
    if is_op(body, "om_decayed", 3):
        s, d, v = body.args
        if not is_op(d, "decay", 1):
            return None
        return {"s": s, "v": v, "g": d.args[0], "K": 1, "C": int(d.attrs.get("t", 0) or 0),
                "scale": outer_scale}
    arms = _flat(body, "concat", -2)
    if len(arms) < 2:
        return None
    K_ = len(arms)
    common: dict = {}
    scale_seen = None
    for i, arm in enumerate(arms):
        intra_seen = False
        crosses = set()
        for summand in _flat(arm, "add"):
            t, sc = _peel_summand(summand)
            sc *= outer_scale
            if scale_seen is None:
                scale_seen = sc
            elif abs(sc - scale_seen) > 1e-12 * max(1.0, abs(sc)):
                return None
            if is_op(t, "om_decayed", 3):
                if intra_seen:
                    return None
                intra_seen = True
                blk, d, v_i = t.args
                sb = _score_block(blk)
                vs = _split_of(v_i, -2)
                if sb is None or vs is None or not is_op(d, "decay", 1):
                    return None
                s, SZ, bi, bj = sb
                if (bi, bj) != (i, i) or vs[2] != i or vs[1] != SZ:
                    return None
                C = int(d.attrs.get("t", 0) or 0)
                if not _agree(common, s=s, v=vs[0], g=d.args[0], SZ=SZ, C=C):
                    return None
                continue
            # cross term: mul(row_gate, matmul(mul(s_ij, col_gate), v_j)), either mul order
            if not is_op(t, "mul", 2):
                return None
            row = next((a for a in t.args if _gate(a, -1) is not None), None)
            body_ = next((a for a in t.args if a is not row), None)
            if row is None or not is_op(body_, "matmul", 2):
                return None
            g_r, t_r, off_r, sign_r = _gate(row, -1)
            inner, v_j = body_.args
            if not is_op(inner, "mul", 2):
                return None
            col = next((a for a in inner.args if _gate(a, -2) is not None), None)
            blk = next((a for a in inner.args if a is not col), None)
            if col is None:
                return None
            g_c, t_c, off_c, sign_c = _gate(col, -2)
            sb = _score_block(blk)
            vs = _split_of(v_j, -2)
            if sb is None or vs is None:
                return None
            s, SZ, bi, bj = sb
            if bi != i or bj >= i or vs[2] != bj or vs[1] != SZ or bj in crosses:
                return None
            crosses.add(bj)
            C = t_r
            if not (sign_r == 1 and sign_c == -1 and off_c == 0 and t_c == C and off_r == (i - bj) * C):
                return None
            if not _agree(common, s=s, v=vs[0], g=g_r, SZ=SZ, C=C) or g_c != common["g"]:
                return None
        if not intra_seen or crosses != set(range(i)):
            return None
    if common.get("SZ") != (common.get("C"),) * K_:
        return None
    return {"s": common["s"], "v": common["v"], "g": common["g"], "K": K_, "C": common["C"],
            "scale": scale_seen if scale_seen is not None else 1.0}


def _agree(common: dict, **kv) -> bool:
    for k, v in kv.items():
        if k in common:
            if common[k] != v:
                return False
        else:
            common[k] = v
    return True


def build_decayed_plan(root: Any) -> dict | None:
    """The plan: ``(q, k, v, γ)`` terms, the score scale and the integer
    partition ``(K, C)``; ``None`` when the root is not the delivered form."""
    p = _parse(root)
    if p is None:
        return None
    qk = _parse_qk(p["s"])
    if qk is None:
        return None
    q, k, sscale = qk
    p.update(q=q, k=k, scale=p["scale"] * sscale)
    return p


class HipChunkedDecayModule(HipExecutorBase, nn.Module):
    """Planned executor for the chunked decayed form (module docstring)."""

    def __init__(self, ir: IR, param_values: dict | None = None, *, eval_mod: HipIRModule | None = None,
                 device: Any = None, ops=None) -> None:
        super().__init__()
        self.eval_mod = eval_mod if eval_mod is not None else HipIRModule(ir, param_values, device=device, ops=ops)
        self._inputs = list(ir.inputs)
        self._const_cache: dict = {}
        self.fallbacks = 0
        self._plan = build_decayed_plan(self.eval_mod._root)
        self._init_graph_state()

    @property
    def n_chunks(self) -> int:
        return 0 if self._plan is None else self._plan["K"]

    def _forward_impl(self, *xs: Any) -> Any:
        p = self._plan
        if p is None:
            return self.eval_mod(*xs)
        x, env = self._input_env(xs)
        ev = self.ev_factory(env, x)
        q, k, v, g = ev(p["q"]), ev(p["k"]), ev(p["v"]), ev(p["g"])
        args = _kernel_args(q, k, v, g, p)
        if args is None:
            self.fallbacks += 1
            return self.eval_mod(*xs)
        q4, k4, v4, g32, lead = args
        o = K.retention(q4, k4, v4, g32, p["scale"])
        return o.reshape(*lead, o.shape[-2], o.shape[-1])


def _kernel_args(q, k, v, g, p):
    ts = (q, k, v)
    if not all(isinstance(t, torch.Tensor) and t.device.type == "cuda" and t.dtype == torch.bfloat16 for t in ts):
        return None
    if q.shape != k.shape or v.shape[:-1] != q.shape[:-1] or not 2 <= q.dim() <= 4:
        return None
    if max(q.shape[-1], v.shape[-1]) > K.RETENTION_HEAD_DIM:  # narrower heads run zero-padded
        return None
    T = q.shape[-2]
    if T % K.RETENTION_CHUNK or T != p["K"] * p["C"]:
        return None
    lead = tuple(q.shape[:-2])
    while q.dim() < 4:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    H = q.shape[1]
    g = torch.as_tensor(g, device=q.device)
    if g.dim() == 0:
        g = g.reshape(1).expand(H)
    g = g.reshape(-1)
    if g.numel() != H:
        return None
    return q, k, v, g.to(torch.float32).contiguous(), lead
