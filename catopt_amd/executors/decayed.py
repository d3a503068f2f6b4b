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
summand or around the score).  It accepts equally the spelling that
extraction delivers after the split/matmul bridges (decayed_lower.py:1-10,
``_classify_body`` :154-170)::

    concat_i( om_decayed(q_i @ k_iᵀ, decay(γ, t=C), v_i) / S
              + Σ_{j<i} row_ij ⊙ (q_i @ ((k_j ⊙ unsqueeze(decay_vec(γ, t=C, sign=-1), -1))ᵀ @ v_j)) / S )

with ``q_i = split(q, SZ, -2, i)``, ``k_iᵀ`` either ``split(transpose(k),
SZ, -1, i)`` or ``transpose(split(k, SZ, -2, i))``, the row gate inside or
outside the ``div`` and on either side of its ``mul``, the pair product in
either association, and the two spellings mixed freely across summands.
Every integer of the plan (``K``, ``C``, ``SZ``, each ``OFF_i_j``, the gate
signs) is checked exactly against the law's derive (``om.py:3064-3075``); any
mismatch — or a summand that denotes another function (no row gate, a second
decay base, a gated intra element, a score that is not one ``q kᵀ``) — leaves
``_plan = None`` and the embedded generic module runs the term as written.

All K-way forms of one ``(q, k, v, γ, scale)`` denote the same function
``o[t] = scale · Σ_{s≤t} γ^{t-s} (q_t·k_s) v_s``, so the plan keeps only those
five operands: the kernel picks its own chunk length and carries the
inter-chunk state on chip (``S_{i+1} = γ^C S_i + K̃_iᵀ V_i``) instead of the
reference's O(K²) pair products (``decayed_lower.py:671-700``).  γ is held in
fp32 and every decay factor is formed in fp32 inside the kernel.  bf16
operands run the bf16 kernel (MFMA in bf16, state and accumulation in fp32);
fp32 operands run the fp32 kernel, whose operands, products and state all
stay fp32; fp16 operands run it widened to fp32, the output rounded to fp16.
Other dtypes take the generic module (counted in ``fallbacks``).
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
from .om import _peel_scale, _qk_product, _transposed_operand

__all__ = ["HipChunkedDecayModule", "build_decayed_plan", "is_decayed_chunked_term", "is_decayed_term",
           "to_chunked_decayed_module"]


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


def _gate(t: Any, dim: int) -> tuple | None:
    """``(γ, t, offset, sign)`` of ``unsqueeze(decay_vec(γ, …), dim)``."""
    if not is_op(t, "unsqueeze", 1) or int(attr_of(t.attrs, "dim", default=-1)) != dim:
        return None
    dv = t.args[0]
    if not is_op(dv, "decay_vec", 1):
        return None
    sign = int(dv.attrs["sign"]) if "sign" in dv.attrs else 1
    return dv.args[0], int(dv.attrs.get("t", 0) or 0), int(dv.attrs.get("offset", 0) or 0), sign


def _gated(t: Any, dim: int) -> tuple | None:
    """``(gate, other)`` of a two-operand ``mul`` with exactly one
    ``unsqueeze(decay_vec, dim)`` operand, either order
    (``_gated_factor``, decayed_lower.py:104-115)."""
    if not is_op(t, "mul", 2):
        return None
    g0, g1 = (_gate(a, dim) for a in t.args)
    if (g0 is None) == (g1 is None):
        return None
    return (g0, t.args[1]) if g0 is not None else (g1, t.args[0])


def _key_block_t(t: Any) -> tuple | None:
    """``(k, SZ, j)`` of the transposed key block ``k_jᵀ``, spelled
    ``split(transpose(k), SZ, -1, j)`` or ``transpose(split(k, SZ, -2, j))``."""
    sp = _split_of(t, -1)
    if sp is not None:
        k = _transposed_operand(sp[0])
        return None if k is None else (k, sp[1], sp[2])
    inner = _transposed_operand(t)
    return None if inner is None else _split_of(inner, -2)


def _score_block(t: Any) -> tuple | None:
    """``(q, k, c, SZ, i, j)`` with ``t = c · q_i k_jᵀ``: a block of the
    score, ``split(split(s, SZ, -2, i), SZ, -1, j)`` with ``s = c · q kᵀ``
    (the law's spelling, om.py:3076-3085; either split order), or the product
    of the operand blocks ``matmul(split(q, SZ, -2, i), k_jᵀ)`` (the
    extracted spelling after the split/matmul bridges)."""
    t, c = _peel_scale(t)
    for rows_first in (True, False):
        outer = _split_of(t, -1 if rows_first else -2)
        inner = None if outer is None else _split_of(outer[0], -2 if rows_first else -1)
        if inner is None or inner[1] != outer[1]:
            continue
        qk = _qk_product(inner[0])
        if qk is None:
            return None
        i, j = (inner[2], outer[2]) if rows_first else (outer[2], inner[2])
        return qk[0], qk[1], c * qk[2], outer[1], i, j
    if is_op(t, "matmul", 2):
        qi, qc = _peel_scale(t.args[0])
        qs, kb = _split_of(qi, -2), _key_block_t(t.args[1])
        if qs is not None and kb is not None and qs[1] == kb[1]:
            return qs[0], kb[0], c * qc, qs[1], qs[2], kb[2]
    return None


def _gated_keys(t: Any) -> tuple | None:
    """``(k, SZ, j, gate)`` of ``(k_j ⊙ η)ᵀ``: ``transpose(mul(k_j,
    unsqueeze(η, -1)))`` (the state half ``_state_half`` parses,
    decayed_lower.py:260-288) or ``mul(k_jᵀ, unsqueeze(η, -2))``."""
    inner = _transposed_operand(t)
    if inner is not None:
        gk = _gated(inner, -1)
        sp = None if gk is None else _split_of(gk[1], -2)
        if sp is not None:
            return (*sp, gk[0])
    gk = _gated(t, -2)
    kb = None if gk is None else _key_block_t(gk[1])
    return None if kb is None else (*kb, gk[0])


def _cross_body(t: Any) -> tuple | None:
    """``(q, k, v, c, SZ, i, j, col)`` of the decayed pair product
    ``c · (q_i k_jᵀ ⊙ col) v_j`` in either association: ``(s_ij ⊙ col) @ v_j``
    or ``(q_i @ (k_j ⊙ col)ᵀ) @ v_j`` (left), or ``q_i @ ((k_j ⊙ col)ᵀ @ v_j)``
    (right: the extracted cross term, ``_classify_body``,
    decayed_lower.py:154-170)."""
    t, c = _peel_scale(t)
    if not is_op(t, "matmul", 2):
        return None
    a, b = t.args
    vs = _split_of(b, -2)
    if vs is not None:
        a, ac = _peel_scale(a)
        gs = _gated(a, -2)
        sb = None if gs is None else _score_block(gs[1])
        if sb is not None:
            q, k, sc, SZ, i, j = sb
            col = gs[0]
        elif is_op(a, "matmul", 2):
            qi, qc = _peel_scale(a.args[0])
            qs, gk = _split_of(qi, -2), _gated_keys(a.args[1])
            if qs is None or gk is None or qs[1] != gk[1]:
                return None
            q, k, sc, SZ, i, j, col = qs[0], gk[0], qc, qs[1], qs[2], gk[2], gk[3]
        else:
            return None
        if vs[1] != SZ or vs[2] != j:
            return None
        return q, k, vs[0], c * ac * sc, SZ, i, j, col
    qi, qc = _peel_scale(a)
    qs = _split_of(qi, -2)
    b, bc = _peel_scale(b)
    if qs is None or not is_op(b, "matmul", 2):
        return None
    gk, vs = _gated_keys(b.args[0]), _split_of(b.args[1], -2)
    if gk is None or vs is None or not qs[1] == gk[1] == vs[1] or gk[2] != vs[2]:
        return None
    return qs[0], gk[0], vs[0], c * qc * bc, qs[1], qs[2], gk[2], gk[3]


def _intra(summand: Any) -> dict | None:
    """The intra-chunk element ``c · om_decayed(s_ii, decay(γ, t=C), v_i)``."""
    t, c = _peel_scale(summand)
    if not is_op(t, "om_decayed", 3):
        return None
    blk, d, v_i = t.args
    sb, vs = _score_block(blk), _split_of(v_i, -2)
    if sb is None or vs is None or not is_op(d, "decay", 1):
        return None
    q, k, sc, SZ, i, j = sb
    if i != j or vs[2] != i or vs[1] != SZ:
        return None
    return {"q": q, "k": k, "v": vs[0], "g": d.args[0], "SZ": SZ, "C": int(d.attrs.get("t", 0) or 0),
            "i": i, "scale": c * sc}


def _cross(summand: Any) -> dict | None:
    """A decay-gated pair product ``row ⊙ body`` (the row gate inside or
    outside the scale, either ``mul`` order: ``_peel_summand``,
    decayed_lower.py:118-151)."""
    t, c = _peel_scale(summand)
    gb = _gated(t, -1)
    if gb is None:
        return None
    row, body = gb
    cb = _cross_body(body)
    if cb is None:
        return None
    q, k, v, sc, SZ, i, j, col = cb
    return {"q": q, "k": k, "v": v, "SZ": SZ, "i": i, "j": j, "row": row, "col": col, "scale": c * sc}


def is_decayed_term(term: Any) -> bool:
    """Term-level probe: the K-way concat or the single ``om_decayed`` block."""
    return build_decayed_plan(term) is not None


def _parse(root: Any) -> dict | None:
    body, outer_scale = _peel_scale(root)
    if is_op(body, "om_decayed", 3):
        s, d, v = body.args
        qk = _qk_product(s)
        if qk is None or not is_op(d, "decay", 1):
            return None
        return {"q": qk[0], "k": qk[1], "v": v, "g": d.args[0], "K": 1, "C": int(d.attrs.get("t", 0) or 0),
                "scale": outer_scale * qk[2]}
    arms = _flat(body, "concat", -2)
    if len(arms) < 2:
        return None
    K_ = len(arms)
    common: dict = {}
    scales: list[float] = []
    for i, arm in enumerate(arms):
        intra_seen = False
        crosses = set()
        for summand in _flat(arm, "add"):
            p = _intra(summand)
            if p is not None:
                if intra_seen or p["i"] != i:
                    return None
                intra_seen = True
                if not _agree(common, q=p["q"], k=p["k"], v=p["v"], g=p["g"], SZ=p["SZ"], C=p["C"]):
                    return None
                scales.append(p["scale"])
                continue
            p = _cross(summand)
            if p is None or p["i"] != i or not 0 <= p["j"] < i or p["j"] in crosses:
                return None
            j = p["j"]
            crosses.add(j)
            g_r, C, off_r, sign_r = p["row"]
            g_c, t_c, off_c, sign_c = p["col"]
            # the law's derive (om.py:3064-3075): OFF_i_j = (i-j)·C on the row
            # gate, γ^(-c) on the key axis
            if not (sign_r == 1 and sign_c == -1 and off_c == 0 and t_c == C and off_r == (i - j) * C):
                return None
            if not _agree(common, q=p["q"], k=p["k"], v=p["v"], g=g_r, SZ=p["SZ"], C=C) or g_c != common["g"]:
                return None
            scales.append(p["scale"])
        if not intra_seen or crosses != set(range(i)):
            return None
    if common.get("SZ") != (common.get("C"),) * K_:
        return None
    sc = outer_scale * scales[0]
    if any(abs(x - scales[0]) > 1e-12 * max(1.0, abs(scales[0])) for x in scales):
        return None
    return {"q": common["q"], "k": common["k"], "v": common["v"], "g": common["g"], "K": K_,
            "C": common["C"], "scale": sc}


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
    return _parse(root)


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

    @property
    def n_blocks(self) -> int:
        """Output chunks of the delivered form, 0 when not batched (the
        reference's name, decayed_lower.py:423-426)."""
        return self.n_chunks

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
    if not all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in ts):
        return None
    if q.dtype not in (torch.bfloat16, torch.float32, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return None
    if q.shape != k.shape or v.shape[:-1] != q.shape[:-1] or not 2 <= q.dim() <= 4:
        return None
    if max(q.shape[-1], v.shape[-1]) > K.RETENTION_HEAD_DIM:  # narrower heads run zero-padded
        return None
    T = q.shape[-2]
    if T != p["K"] * p["C"]:
        return None
    lead = tuple(q.shape[:-2])
    while q.dim() < 4:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    H = q.shape[1]
    g = torch.as_tensor(g, device=q.device)
    if g.dim() > 1:  # a rate per (batch, head) or a broadcast axis of its own
        return None
    if g.dim() == 0:
        g = g.reshape(1).expand(H)
    g = g.reshape(-1)
    if g.numel() != H:
        return None
    return q, k, v, g.to(torch.float32).contiguous(), lead


#: The reference's probe name (decayed_lower.py:371-373).
is_decayed_chunked_term = is_decayed_term


def to_chunked_decayed_module(ir: IR, param_values: dict | None = None, **kw) -> HipChunkedDecayModule:
    """Always a :class:`HipChunkedDecayModule` (check ``is_batched``),
    ``decayed_lower.py:727-731``."""
    return HipChunkedDecayModule(ir, param_values, **kw)
