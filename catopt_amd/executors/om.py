"""Online-softmax executor: ``om_apply(<om tree>)`` on the HIP kernels.

The counterpart of ``BatchedOMModule`` (luisfuturist/catopt
``packages/catopt-carriers/src/catopt_carriers/om_lower.py:496-835``, plan
builder ``build_om_plan`` :334-437, score modes ``_analyze_elem_group``
:271-331).  The tree's leaves are ``om_elem(s, v)`` blocks and packaged
carriers ``om(m, l, a)``, combined by ``om_compose``; every om tree plans,
as in the reference, and each leaf is classified once, at construction:

* ``attn`` — the score is a scaled ``q kᵀ`` with an optional mask, in the
  spellings catopt's laws deliver:

  - the scale as ``mul``/``div`` by a constant around the product, or on
    ``q`` as ``mul(q, fill(q, value=SC))`` (the sdpa-cat right-hand sides,
    ``om.py:1195-1230``);
  - one ``matmul(q, transpose(k))``, or a key-axis ``concat`` of such
    products sharing ``q`` (``concat(q kᵢᵀ) = q · concat(kᵢ)ᵀ``);
  - ``masked_fill(·, M, -inf)`` with ``M`` the causal generator
    ``cmask(x, off)`` (also under ``split`` / ``slice`` along either of the
    last two axes: the block's offset is folded into the causal bound), a
    weight-only bool (a shifted lower triangle, compared bit-exactly, is the
    causal mode; any other plane a keep-mask) or an input-dependent mask;
  - ``add(·, attnbias(m))`` or ``add(·, B)`` (the attn_mask right-hand side,
    ``om.py:1315-1340``, and its ``split`` blocks): a bool ``m`` is a
    keep-mask, a float one an additive bias; a weight-only bias holding only
    0 and -inf is a keep-mask.

  bf16 operands with head dims up to 128 (other widths than 64 / 128
  zero-padded) and a mask that is one ``(Tq, Tk)`` plane shared over the
  leading axes run one launch of the fused attention kernel (scores, mask, exponentials and ``e @ v`` stay on chip; a single
  leaf is normalised in the kernel).  fp32 operands (``dk <= 128``,
  ``dv <= 256``) run the fp32 carrier kernel with the same mask modes; fp16
  operands run it widened to fp32 (the output is rounded to fp16).  Any
  other call — another head dim, a per-batch mask — takes the score path
  below for that leaf.
* ``scores`` — any other score (the reference's ``slice`` / ``stack``
  modes): the score block is evaluated, its row statistics and
  ``exp(s - m)`` come from ``catopt_hip_om_rows`` and ``e @ v`` from the HIP
  GEMM.
* ``om`` — a packaged carrier, used as evaluated.

Leaf carriers are sanitised as ``om_lower.py:792-798`` does (a row whose max
is not finite contributes ``l = a = 0``), combined by the canonical
adjacent-pair reduction with the ``om_compose`` kernel (the ``isfinite``
guards of ``torch_bridge.py:1984-2006``, NaN-propagating max), and read out
as ``a / l`` unclamped: a fully masked row is NaN, as dense softmax.  A
DAG-shared leaf contributes once per occurrence.  A root that is not an om
tree leaves ``_plan = None`` and every call runs the embedded generic module
(``om_lower.py:730-731``).  A call with host inputs runs the generic
module, and a leaf whose operands are not fp32 / bf16 runs the module's own
``om_elem`` / ``om_compose`` bindings; both count in ``fallbacks``.
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import nn

from .. import kernels as K
from ..bindings import attr_of, scalar_value
from ..evaluator import HipIRModule, _is_param, _is_var, eval_term
from ..ir import IR, Op, is_op, postorder
from ..planes import fit_plane, shared_plane
from .base import HipExecutorBase

__all__ = ["HipOMModule", "build_om_plan", "is_om_apply_term", "is_om_term", "mask_kwargs", "om_leaves",
           "parse_score", "to_batched_om_module"]


def is_om_term(term: Any) -> bool:
    """Term-level probe: an ``om_apply`` over an om tree."""
    return is_op(term, "om_apply") and len(term.args) >= 1 and om_leaves(term.args[0]) is not None


def om_leaves(t: Any) -> list | None:
    """Leaves (``om_elem`` blocks and packaged ``om`` carriers) of an
    ``om_compose`` tree, left to right and once per occurrence; ``None`` if
    another node appears."""
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


def _is_neg_inf(t: Any) -> bool:
    v = scalar_value(t)
    return v is not None and v == float("-inf")


def _scale_factor(t: Any) -> float | None:
    """The multiplier a factor term stands for: a finite constant, or the
    constant map ``fill(x, value=c)`` (``full_like(x, c)``)."""
    c = scalar_value(t)
    if c is not None:
        return c if math.isfinite(c) else None
    if is_op(t, "fill", 1):
        try:
            v = float(attr_of(t.attrs, "value", default=None))
        except (TypeError, ValueError):
            return None
        return v if math.isfinite(v) else None
    return None


def _peel_scale(s: Any) -> tuple[Any, float]:
    """``(x, c)`` with ``s = c · x`` through ``mul`` / ``div`` by constants."""
    scale = 1.0
    while True:
        if is_op(s, "mul", 2):
            a, b = s.args
            cb, ca = _scale_factor(b), _scale_factor(a)
            if cb is not None:
                scale *= cb
                s = a
                continue
            if ca is not None:
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


_SAME_RANK = frozenset({"concat", "split", "slice", "chunk", "transpose", "contiguous", "fill", "cmask",
                        "attnbias", "masked_fill", "neg", "exp", "to", "clone"})


def _rank(t: Any) -> int | None:
    """Rank of a term: a typed leaf's, carried through rank-preserving ops
    and ``matmul`` of two operands of rank >= 2."""
    for _ in range(64):
        shape = getattr(getattr(t, "typ", None), "shape", None)
        if shape is not None:
            return len(shape)
        if not is_op(t) or not t.args:
            return None
        if t.op == "matmul" and len(t.args) == 2:
            ra, rb = _rank(t.args[0]), _rank(t.args[1])
            return max(ra, rb) if ra is not None and rb is not None and min(ra, rb) >= 2 else None
        if t.op in ("mul", "div", "add", "sub") and len(t.args) == 2:
            ra, rb = _rank(t.args[0]), _rank(t.args[1])
            known = [r for r in (ra, rb) if r is not None]
            return max(known) if known else None
        if t.op not in _SAME_RANK:
            return None
        t = t.args[0]
    return None


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
    rank = _rank(kt.args[0])  # a leaf of known rank n: dims n-2, n-1
    if rank is not None and rank >= 2 and dims == {rank - 2, rank - 1}:
        return kt.args[0]
    return None


def _qk_product(s: Any) -> tuple[Any, Any, float] | None:
    """``(q, k, c)`` of ``c · matmul(c' · q, transpose(k))``, ``c`` the
    product of both scales."""
    s, scale = _peel_scale(s)
    if not is_op(s, "matmul", 2):
        return None
    k = _transposed_operand(s.args[1])
    if k is None:
        return None
    q, qs = _peel_scale(s.args[0])
    return q, k, scale * qs


def _last_axis(t: Any, dim: Any) -> bool:
    if dim is None:
        return False
    d = int(dim)
    rank = _rank(t)
    return d == -1 or (rank is not None and d == rank - 1)


def _qk_parts(s: Any) -> dict | None:
    """``q``, ``k`` and scale of a score product: one ``q kᵀ``; a key-axis
    ``concat`` of products sharing ``q`` and scale, whose ``k`` is the
    key-axis concat of the blocks' keys; or a ``split`` / ``slice`` block of
    either along the key or query axis, taken of ``k`` or ``q`` instead
    (the reference's ``slice`` score mode)."""
    one = _qk_product(s)
    if one is not None:
        return {"q": one[0], "k": one[1], "scale": one[2]}
    body, outer = _peel_scale(s)
    if (is_op(body, "split", 1) or is_op(body, "slice", 1)) and _block_start(body) is not None:
        inner = _qk_parts(body.args[0])
        if inner is None:
            return None
        side = "k" if _block_axis(body) == -1 else "q"
        pushed = _push_block(body, inner[side])
        if pushed is None:
            return None
        return dict(inner, **{side: pushed, "scale": inner["scale"] * outer})
    if not is_op(body, "concat") or len(body.args) < 2:
        return None
    if not _last_axis(body, attr_of(body.attrs, "dim", "axis", default=None)):
        return None
    parts = [_qk_product(p) for p in body.args]
    if any(p is None for p in parts):
        return None
    q0, _, c0 = parts[0]
    if any(p[0] is not q0 or p[2] != c0 for p in parts):
        return None
    k = Op.make("concat", *[p[1] for p in parts], dim=-2)
    return {"q": q0, "k": k, "scale": c0 * outer}


def parse_score(s: Any) -> dict | None:
    """``q``, ``k``, ``scale`` and the mask of a scaled-``q kᵀ`` score:
    ``mask`` the masked set ``M`` of ``masked_fill(·, M, -inf)``, ``bias``
    the addend ``B`` of ``add(·, B)``; ``None`` for any other score."""
    if is_op(s, "masked_fill", 3):
        if not _is_neg_inf(s.args[2]):
            return None  # a finite fill changes what a fully masked row means
        p = _qk_parts(s.args[0])
        return None if p is None else dict(p, mask=s.args[1], bias=None)
    if is_op(s, "add", 2):
        a, b = s.args
        for prod, addend in ((a, b), (b, a)):
            p = _qk_parts(prod)
            if p is not None:
                return dict(p, mask=None, bias=addend)
        return None
    p = _qk_parts(s)
    return None if p is None else dict(p, mask=None, bias=None)


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


def _block_axis(t: Any) -> int | None:
    """The axis, counted from the end (-1 keys, -2 queries), along which a
    ``split`` / ``slice`` takes its block; ``None`` for another axis or an
    unknown rank.  A negative ``slice`` dim counts as axis 0, as the slice
    binding indexes (``torch_bridge.py:1347-1350``)."""
    dim = attr_of(t.attrs, "dim", "axis", default=None)
    if dim is None:
        return None
    d = int(dim)
    rank = _rank(t.args[0])
    if is_op(t, "slice", 1) and d < 0:
        d = 0
    if d >= 0:
        if rank is None:
            return None
        d -= rank
    return d if d in (-1, -2) else None


def _block_start(t: Any) -> tuple[Any, int, int] | None:
    """``(base, axis, start)`` of a ``split`` / ``slice`` taking a block of
    ``base`` along one of its last two axes."""
    d = _block_axis(t)
    if d is None:
        return None
    base = t.args[0]
    if is_op(t, "split", 1):
        idx = attr_of(t.attrs, "index", default=None)
        sizes = attr_of(t.attrs, "sizes", "split_size", default=None)
        if idx is None or sizes is None:
            return None
        idx = int(idx)
        if isinstance(sizes, (list, tuple)):
            return base, d, sum(int(x) for x in sizes[:idx])
        return base, d, idx * int(sizes)
    if not is_op(t, "slice", 1):
        return None
    start = attr_of(t.attrs, "start", default=0) or 0
    step = attr_of(t.attrs, "step", default=1) or 1
    if int(step) != 1 or int(start) < 0:
        return None
    return base, d, int(start)


def _push_block(t: Any, operand: Any) -> Any | None:
    """The block ``t`` takes of a score, taken instead of ``operand``'s
    sequence axis (-2 of ``q`` for query blocks, of ``k`` for key blocks)."""
    attrs = dict(t.attrs)
    attrs.pop("axis", None)
    if is_op(t, "split", 1):
        attrs["dim"] = -2
        return Op.make("split", operand, **attrs)
    rank = _rank(operand)
    if rank is None or rank < 2:
        return None
    attrs["dim"] = rank - 2
    return Op.make("slice", operand, **attrs)


def _cmask_causal_off(M: Any) -> int | None:
    """Causal bound of a ``cmask(x, off)`` masked set or a block of it: keep
    key ``j`` for query ``i`` iff ``j <= i + result`` in the block's own
    coordinates (``cmask`` masks ``j + off > i``, ``om.py:1023-1029``)."""
    qstart = kstart = 0
    t = M
    while is_op(t, "split", 1) or is_op(t, "slice", 1):
        st = _block_start(t)
        if st is None:
            return None
        t, axis, start = st
        if axis == -1:
            kstart += start
        else:
            qstart += start
    if not is_op(t, "cmask", 1):
        return None
    return qstart - kstart - int(t.attrs.get("off", 0) or 0)


def _const_value(t: Any, eval_mod: HipIRModule) -> torch.Tensor | None:
    """The value of a weight-only mask term at construction: a (folded)
    Param, or any other parameter-only subtree (``split`` / ``slice`` /
    ``attnbias`` of a Param, which the weight fold leaves in place)
    evaluated once on the device; ``None`` for a term that reads an
    input."""
    pv = eval_mod._pv(t)
    if pv is not None or not isinstance(t, Op):
        return pv
    for node in postorder(t):
        for a in node.args:
            if _is_var(a) or (_is_param(a) and eval_mod._pv(a) is None):
                return None
    try:
        out = eval_term(t, {}, eval_mod._param_map, eval_mod.ops)
    except Exception:
        return None  # not foldable: the mask is evaluated per call
    return out if isinstance(out, torch.Tensor) else None


def _keep_const(lf: dict, keep: torch.Tensor) -> None:
    """A weight-only keep-mask: its one plane over the leading axes, marked
    ``causal`` when that plane is a triangle.  The plane keeps its own shape
    (``(1, Tk)`` for a key-padding mask): :func:`mask_kwargs` fits it to the
    score at call time, and a triangle counts as one only when it spans the
    score's ``(Tq, Tk)``."""
    plane = shared_plane(keep)
    if plane is None:
        lf["mask_kind"] = "scores"  # a per-batch mask
        return
    plane = plane.contiguous()
    off = _triangle_offset(~plane)
    if off is not None:
        lf["mask_kind"], lf["causal_off"], lf["keep"] = "causal", -off, plane
    else:
        lf["mask_kind"], lf["keep"] = "bool_const", plane


def _bias_const(lf: dict, bias: torch.Tensor) -> None:
    vals = bias.float()
    if bool(((vals == 0) | (vals == float("-inf"))).all()):
        _keep_const(lf, vals == 0)  # a 0 / -inf bias is a keep-mask
        return
    plane = shared_plane(vals)
    if plane is None:
        lf["mask_kind"] = "scores"
    else:
        lf["mask_kind"], lf["bias_plane"] = "bias_const", plane.contiguous()


def _classify_mask(lf: dict, eval_mod: HipIRModule) -> bool:
    """Fix the kernel mask mode of a parsed leaf (keys ``mask`` / ``bias``)
    where the mask is known at construction; ``False`` when it cannot be a
    kernel mode at all.  ``mask_kind`` "scores" marks a weight-only mask
    that differs over the leading axes."""
    M, B = lf.get("mask"), lf.get("bias")
    if M is None and B is None:
        lf["mask_kind"] = "none"
        return True
    if M is not None:
        off = _cmask_causal_off(M)
        if off is not None:
            lf["mask_kind"], lf["causal_off"] = "causal", off
            return True
        pv = _const_value(M, eval_mod)
        if pv is None:
            lf["mask_kind"] = "runtime"
            return True
        if not isinstance(pv, torch.Tensor) or pv.dtype != torch.bool:
            return False
        _keep_const(lf, ~pv)
        return True
    coerce = is_op(B, "attnbias", 1)  # attnbias(m): torch's attn_mask coercion
    src = B.args[0] if coerce else B
    pv = _const_value(src, eval_mod)
    if pv is None:
        lf["mask_kind"], lf["bias_term"], lf["attnbias"] = "bias_runtime", src, coerce
        return True
    if not isinstance(pv, torch.Tensor) or pv.dim() < 2:
        return False
    if pv.dtype == torch.bool:
        if not coerce:
            return False  # adding a bool is not a mask
        _keep_const(lf, pv)
    else:
        _bias_const(lf, pv)
    return True


def _const_fit(lf: dict, key: str, arg: str, tq: int, tk: int) -> dict | None:
    """``{arg: plane}`` for a weight-only plane fitted to ``(tq, tk)``,
    cached per score shape; ``None`` when it does not broadcast to it."""
    cache = lf.setdefault("_fit", {})
    ck = (key, tq, tk)
    if ck not in cache:
        cache[ck] = fit_plane(lf[key], tq, tk)
    plane = cache[ck]
    return None if plane is None else {arg: plane}


def mask_kwargs(lf: dict, ev, tq: int, tk: int) -> dict | None:
    """Attention-kernel mask arguments of an ``attn`` leaf whose score is
    ``(…, tq, tk)``; ``None`` when the call's mask is not one plane shared
    over the leading axes that broadcasts to ``(tq, tk)`` (the leaf then
    takes the score path)."""
    kind = lf["mask_kind"]
    if kind == "none":
        return {}
    if kind == "causal":
        keep = lf.get("keep")
        if keep is None or tuple(keep.shape) == (tq, tk):
            return {"causal": True, "causal_off": lf["causal_off"]}
        return _const_fit(lf, "keep", "mask", tq, tk)  # a triangle of another shape broadcasts
    if kind == "bool_const":
        return _const_fit(lf, "keep", "mask", tq, tk)
    if kind == "bias_const":
        return _const_fit(lf, "bias_plane", "bias", tq, tk)
    if kind == "runtime":
        masked = ev(lf["mask"])
        if not isinstance(masked, torch.Tensor) or masked.dtype != torch.bool:
            return None
        plane = shared_plane(masked)
        plane = None if plane is None else fit_plane(torch.logical_not(plane), tq, tk)
        return None if plane is None else {"mask": plane}
    if kind == "bias_runtime":
        b = ev(lf["bias_term"])
        if not isinstance(b, torch.Tensor):
            return None
        if b.dtype == torch.bool:
            if not lf["attnbias"]:
                return None
        elif not b.dtype.is_floating_point:
            return None
        plane = shared_plane(b)
        plane = None if plane is None else fit_plane(plane, tq, tk)
        if plane is None:
            return None
        return {"mask": plane} if b.dtype == torch.bool else {"bias": plane}
    return None


def _in_envelope(q, k, v) -> bool:
    ts = (q, k, v)
    if not all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in ts):
        return False
    if any(t.dtype != torch.bfloat16 for t in ts):
        return False
    d, dv = q.shape[-1], v.shape[-1]
    return (0 < d <= K.ATTENTION_MAX_HEAD_DIM and 0 < dv <= K.ATTENTION_MAX_HEAD_DIM and k.shape[-1] == d
            and 2 <= q.dim() <= 4)


def _f32_envelope(q, k, v) -> bool:
    """Operands of the fp32 carrier kernel: ``dk <= 128``, ``dv <= 256``, one
    leading shape (or a 2-D ``q`` / ``v`` shared over it); all fp32, or all
    fp16 (widened to fp32 on the device; the result is rounded back)."""
    ts = (q, k, v)
    if not all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in ts):
        return False
    if q.dtype not in (torch.float32, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    if q.dim() < 2 or k.dim() < 2 or v.dim() < 2:
        return False
    lead = tuple(k.shape[:-2])
    return (0 < q.shape[-1] <= 128 and k.shape[-1] == q.shape[-1] and 0 < v.shape[-1] <= 256
            and v.shape[-2] == k.shape[-2] > 0
            and (q.dim() == 2 or tuple(q.shape[:-2]) == lead)
            and (v.dim() == 2 or tuple(v.shape[:-2]) == lead))


def _as_bhtd(q, k, v):
    lead = tuple(q.shape[:-2])
    if k.shape[:-2] != q.shape[:-2] or v.shape[:-2] != q.shape[:-2] or k.shape[-2] != v.shape[-2]:
        return None, None, None, None
    # a 3-D operand's leading axis is the batch (the kernel splits a batch
    # past one launch's grid; its head extent must fit one launch)
    if q.dim() == 3:
        q, k, v = q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1)
    while q.dim() < 4:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
    return q, k, v, lead


def build_om_plan(root: Any, eval_mod: HipIRModule) -> dict | None:
    """Classify the leaves of ``om_apply(<om tree>)``; ``None`` for any other
    root."""
    if not is_op(root, "om_apply") or not root.args:
        return None
    leaves = om_leaves(root.args[0])
    if not leaves:
        return None
    plan_leaves = []
    for leaf in leaves:
        if is_op(leaf, "om", 3):
            plan_leaves.append({"kind": "om", "term": leaf, "m": leaf.args[0], "l": leaf.args[1],
                                "a": leaf.args[2]})
            continue
        s, v = leaf.args
        lf: dict = {"kind": "scores", "term": leaf, "s": s, "v": v}
        sc = parse_score(s)
        # the kernels track the row max of q·k and scale it, which is the max
        # of the scaled scores only for a positive scale
        if sc is not None and math.isfinite(sc["scale"]) and sc["scale"] > 0:
            la = dict(lf, q=sc["q"], k=sc["k"], scale=sc["scale"], mask=sc["mask"], bias=sc["bias"])
            if _classify_mask(la, eval_mod) and la["mask_kind"] != "scores":
                la["kind"] = "attn"
                lf = la
        plan_leaves.append(lf)
    return {"leaves": plan_leaves}


def _device_float(*ts) -> bool:
    return all(isinstance(t, torch.Tensor) and t.device.type == "cuda"
               and t.dtype in (torch.float32, torch.bfloat16) for t in ts)


def _identity_like(f: tuple) -> tuple:
    m, lv, a = f
    return torch.full_like(m, float("-inf")), torch.zeros_like(lv), torch.zeros_like(a)


def _broadcast_carriers(carriers: list) -> list:
    """Expand every carrier component to the common broadcast shape of that
    component, as the reference's stacked reduction does
    (``om_lower.py:806-826``)."""
    shapes = [torch.broadcast_shapes(*[c[i].shape for c in carriers]) for i in range(3)]
    return [tuple(t if t.shape == sh else t.expand(sh).contiguous() for t, sh in zip(c, shapes))
            for c in carriers]


class HipOMModule(HipExecutorBase, nn.Module):
    """Planned executor for ``om_apply(<om tree>)`` (module docstring)."""

    def __init__(self, ir: IR, param_values: dict | None = None, *, eval_mod: HipIRModule | None = None,
                 device: Any = None, ops=None) -> None:
        super().__init__()
        self.eval_mod = eval_mod if eval_mod is not None else HipIRModule(ir, param_values, device=device, ops=ops)
        self._inputs = list(ir.inputs)
        self._const_cache: dict = {}
        self.fallbacks = 0       # leaves (or whole calls) run on the generic tensor ops
        self.kernel_leaves = 0   # leaves of the last call on an attention kernel
        self._plan = build_om_plan(self.eval_mod._root, self.eval_mod)
        self._init_graph_state()

    @property
    def n_leaves(self) -> int:
        return 0 if self._plan is None else len(self._plan["leaves"])

    @property
    def n_blocks(self) -> int:
        """om carrier leaves, 0 when not batched (om_lower.py:596-599)."""
        return self.n_leaves

    @property
    def n_levels(self) -> int:
        """Compose levels of the pairwise reduction (⌈log2 leaves⌉), 0 when
        not batched or for one leaf (om_lower.py:591-594)."""
        n = self.n_leaves
        return 0 if n <= 1 else (n - 1).bit_length()

    @property
    def leaf_kinds(self) -> list[str]:
        """Plan class of each leaf ("attn", "scores" or "om")."""
        return [] if self._plan is None else [lf["kind"] for lf in self._plan["leaves"]]

    def _attn(self, lf: dict, ev, normalize: bool):
        """An ``attn`` leaf on the attention kernels: the normalised output
        when ``normalize`` (bf16 kernel only; fp32 leaves return ``None`` and
        are read out from their carrier), else ``((m, l, a), dtype)``;
        ``None`` outside the kernels' envelopes."""
        q, k, v = ev(lf["q"]), ev(lf["k"]), ev(lf["v"])
        if not _in_envelope(q, k, v):
            if normalize or not _f32_envelope(q, k, v):
                return None
            mask_kw = mask_kwargs(lf, ev, q.shape[-2], k.shape[-2])
            if mask_kw is None:
                return None
            self.kernel_leaves += 1
            return K.attn_carrier_f32(q, k, v, float(lf["scale"]), **mask_kw), v.dtype
        mask_kw = mask_kwargs(lf, ev, q.shape[-2], k.shape[-2])
        if mask_kw is None:
            return None
        q4, k4, v4, lead = _as_bhtd(q, k, v)
        if q4 is None or not K.attention_grid_ok(q4):
            return None
        self.kernel_leaves += 1
        if normalize:
            o = K.attention(q4, k4, v4, lf["scale"], normalize=True, **mask_kw)
            return o.reshape(*lead, o.shape[-2], o.shape[-1])
        a, m, lsum = K.attention(q4, k4, v4, lf["scale"], normalize=False, return_ml=True, **mask_kw)
        tq, dv = a.shape[-2], a.shape[-1]
        return (m.reshape(*lead, tq, 1), lsum.reshape(*lead, tq, 1), a.float().reshape(*lead, tq, dv)), v.dtype

    def _carrier(self, lf: dict, ev):
        """``((m, l, a), value dtype)`` of one leaf, sanitised.  Operands
        outside the kernels' dtypes run the module's own ``om_elem`` /
        ``om_compose`` bindings (counted in ``fallbacks``)."""
        if lf["kind"] == "attn":
            r = self._attn(lf, ev, normalize=False)
            if r is not None:
                return r
        if lf["kind"] == "om":
            f = (ev(lf["m"]), ev(lf["l"]), ev(lf["a"]))
            if _device_float(*f):
                f = tuple(t.float() for t in f)
                # composing with the ⊕ identity applies the isfinite guard
                return self._compose(_identity_like(f), f), f[2].dtype
            self.fallbacks += 1
            return self.eval_mod.ops["om_compose"](_identity_like(f), f), f[2].dtype
        s, v = ev(lf["s"]), ev(lf["v"])
        if _device_float(s, v) and s.dim() and v.dim() and s.numel() and v.numel():
            return K.om_elem_scores(s, v, sanitize=True), torch.promote_types(s.dtype, v.dtype)
        self.fallbacks += 1
        m, lv, a = self.eval_mod.ops["om_elem"](s, v)
        fin = torch.isfinite(m)
        return (m, torch.where(fin, lv, 0.0), torch.where(fin, a, 0.0)), a.dtype

    def _compose(self, f: tuple, g: tuple) -> tuple:
        if all(isinstance(t, torch.Tensor) and t.device.type == "cuda" and t.dtype == torch.float32
               for t in (*f, *g)):
            m, lv, acc = K.om_compose(f, g)
            return m.reshape(f[0].shape), lv.reshape(f[1].shape), acc.reshape(f[2].shape)
        self.fallbacks += 1
        return self.eval_mod.ops["om_compose"](f, g)

    def _forward_impl(self, *xs: Any) -> Any:
        if self._plan is None:
            return self.eval_mod(*xs)
        if any(isinstance(t, torch.Tensor) and t.device.type != "cuda" for t in xs):
            self.fallbacks += 1  # host inputs: the generic module (which raises on the product table)
            return self.eval_mod(*xs)
        x, env = self._input_env(xs)
        ev = self.ev_factory(env, x)
        self.kernel_leaves = 0
        leaves = self._plan["leaves"]
        if len(leaves) == 1 and leaves[0]["kind"] == "attn":
            o = self._attn(leaves[0], ev, normalize=True)
            if o is not None:
                return o
        carriers, out_dtype = [], None
        # a leaf shared in the DAG runs once and enters the reduction once per
        # occurrence (the multiplicity repeat of om_lower.py:642-655)
        done: dict = {}
        for lf in leaves:
            if lf["term"] not in done:
                done[lf["term"]] = self._carrier(lf, ev)
            f, dt = done[lf["term"]]
            carriers.append(f)
            out_dtype = dt if out_dtype is None else torch.promote_types(out_dtype, dt)
        carriers = _broadcast_carriers(carriers)
        # canonical adjacent-pair reduction, odd tail carried up (om_lower.py:800-832)
        while len(carriers) > 1:
            nxt = [self._compose(carriers[i], carriers[i + 1]) for i in range(0, len(carriers) - 1, 2)]
            if len(carriers) % 2:
                nxt.append(carriers[-1])
            carriers = nxt
        _, lsum, acc = carriers[0]
        return (acc / lsum).to(out_dtype)


#: The reference's probe name (om_lower.py:106-113).
is_om_apply_term = is_om_term


def to_batched_om_module(ir: IR, param_values: dict | None = None, fused: bool | str = False,
                         **kw) -> HipOMModule:
    """Always a :class:`HipOMModule` (check ``is_batched``), ``om_lower.py:838-868``.
    ``fused`` is accepted for the reference's signature: it selects a
    torch.compile'd reduction there, and here every leaf and combine already
    runs on the HIP kernels, so it changes nothing."""
    del fused
    return HipOMModule(ir, param_values, **kw)
