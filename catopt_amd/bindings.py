"""The HIP op table: ``op name -> fn(*operand_values, **attrs)``.

This is the ``Binding`` table (luisfuturist/catopt ``ports.py:189-207``)
the generic evaluator and the executors resolve ops through, restated for
the MI355X path:

* the arithmetic ops of the delivered forms run on this package's HIP
  kernels: ``linear`` and ``matmul`` (MFMA GEMMs), ``rms_norm``, ``silu``,
  ``glu`` on a linear, ``om_compose``, ``decay`` / ``decay_vec``, and the
  diagonal-affine scan ops when they arrive stacked;
* layout and glue ops (``split``, ``chunk``, ``concat``, ``unsqueeze``,
  ``transpose``, ``masked_fill`` …) are views or small device ops through
  torch, which here is only the owner of device memory and streams;
* the rest of the reference's core table (norms, clamps, comparisons,
  cumulative and indexed ops, creators, casts) are torch device ops from
  :mod:`catopt_amd.device_ops`, so terms whose leaf operands use them stay
  deliverable.

Argument meaning follows the reference's core table
(``packages/catopt-torch/src/catopt_torch/torch_bridge.py:1146-1902``) and
the carrier tables (``catopt_carriers/om.py:1023-1106``,
``xcarrier.py:460-472``): attrs arrive by their canonical names (``dim``,
``keepdim``, ``chunks``, ``index``, ``sizes``, ``dim0``/``dim1``, ``eps``,
``off``, ``t``, ``offset``, ``sign`` …).  A missing binding is a loud
``ValueError`` at evaluation time, as in ``_EvalPlan``
(torch_bridge.py:2241-2244).
"""

from __future__ import annotations

import math
from typing import Any, Callable

import torch
import torch.nn.functional as F

from . import kernels as K
from .device_ops import DEVICE_OPS
from .planes import fit_plane, shared_plane

__all__ = ["HIP_BINDINGS", "HipOpTable", "attr_of", "om_elem_dense", "torch_fallback_count"]


def attr_of(kw: dict, *names: str, default: Any = None) -> Any:
    """First present attr among ``names`` (canonical name first)."""
    for n in names:
        if n in kw and kw[n] is not None:
            return kw[n]
    return default


def _dims(kw: dict) -> tuple:
    d = attr_of(kw, "dim", "axis", default=None)
    keep = bool(attr_of(kw, "keepdim", default=False))
    if d is None:
        return ()
    if isinstance(d, (list, tuple)):
        d = tuple(int(x) for x in d)
    else:
        d = int(d)
    return (d, keep)


def _on_device(*ts: Any) -> bool:
    """Every tensor operand lives on the ROCm device; a host tensor raises.

    The HIP bindings have no CPU path: a host operand is a usage error, not a
    reason to compute elsewhere."""
    for t in ts:
        if isinstance(t, torch.Tensor) and t.device.type != "cuda" and t.dim() > 0:
            raise ValueError(f"HIP bindings run on the ROCm device; got an operand on {t.device}")
    return True


def _kernel_dtype(*ts: Any) -> bool:
    """All operands share one kernel dtype (fp32 or bf16)."""
    dts = {t.dtype for t in ts if isinstance(t, torch.Tensor)}
    return len(dts) == 1 and dts <= {torch.float32, torch.bfloat16}


# --------------------------------------------------------------- HIP-backed
# Outside the kernels' dtype envelope (fp64, fp16, int) these bindings run
# the same op as a torch device op, counted by torch_fallback_count(); on a
# host tensor they raise.

_torch_fallbacks = 0


def _fell_back() -> None:
    global _torch_fallbacks
    _torch_fallbacks += 1


def torch_fallback_count() -> int:
    """Calls of a HIP-backed binding that ran its torch device op instead."""
    return _torch_fallbacks


def _linear(x, w, *a, **kw):
    bias = a[0] if a else kw.get("bias")
    _on_device(x, w, bias)
    if _kernel_dtype(x, w, bias) and x.dim() >= 1 and w.dim() == 2:
        return K.linear(x, w, bias)
    _fell_back()
    return F.linear(x, w, bias)


def _matmul(a, b, *args, **kw):
    _on_device(a, b)
    if _kernel_dtype(a, b) and a.dim() >= 1 and b.dim() >= 1 and not (a.dim() == 1 and b.dim() == 1):
        return K.matmul(a, b)
    _fell_back()
    return torch.matmul(a, b)


def _rms_norm(x, w=None, *a, **kw):
    _on_device(x, w)
    shape = attr_of(kw, "dim", "normalized_shape", default=None)
    eps = float(attr_of(kw, "eps", default=1e-6))
    if isinstance(shape, (list, tuple)):
        nshape = tuple(int(d) for d in shape)
    else:
        nshape = (int(shape),) if shape is not None else (x.shape[-1],)
    if len(nshape) == 1 and nshape[0] == x.shape[-1] and _kernel_dtype(x, w):
        return K.rmsnorm(x, w, eps)
    _fell_back()
    return F.rms_norm(x, nshape, weight=w, eps=eps)


def _silu(x, *a, **kw):
    _on_device(x)
    if _kernel_dtype(x):
        return K.silu(x)
    _fell_back()
    return F.silu(x)


def _om_compose(f, g, *a, **kw):
    """``_om_compose`` (torch_bridge.py:1984-2006) on the HIP kernel when the
    carriers are device fp32 with matching shapes."""
    m1, l1, a1 = f
    m2, l2, a2 = g
    ts = (m1, l1, a1, m2, l2, a2)
    _on_device(*ts)
    if all(isinstance(t, torch.Tensor) and t.dtype == torch.float32 for t in ts) \
            and m1.shape == m2.shape and a1.shape == a2.shape and l1.shape == m1.shape:
        m, lv, acc = K.om_compose(f, g)
        return m.reshape(m1.shape), lv.reshape(l1.shape), acc.reshape(a1.shape)
    _fell_back()
    return _om_compose_torch(f, g)


def _om_compose_torch(f, g):
    m1, l1, a1 = f
    m2, l2, a2 = g
    mx = torch.maximum(m1, m2)
    fin1, fin2 = torch.isfinite(m1), torch.isfinite(m2)
    e1 = torch.where(fin1, torch.exp(m1 - mx), torch.zeros_like(mx))
    e2 = torch.where(fin2, torch.exp(m2 - mx), torch.zeros_like(mx))
    lv = torch.where(fin1, l1 * e1, torch.zeros_like(l1)) + torch.where(fin2, l2 * e2, torch.zeros_like(l2))
    acc = torch.where(fin1, a1 * e1, torch.zeros_like(a1)) + torch.where(fin2, a2 * e2, torch.zeros_like(a2))
    return mx, lv, acc


def om_elem_dense(s, v, *a, **kw):
    """``_om_elem`` (torch_bridge.py:1974-1981) over a materialised score:
    ``(rowmax s, Σ exp(s - m), exp(s - m) @ v)``, raw (a fully masked row
    gives NaN ``l`` and ``a``).  Device fp32 / bf16 operands run the
    ``catopt_hip_om_rows`` row kernel and the HIP GEMM in fp32; the carrier
    comes back in the operands' promoted dtype, as the tensor formula gives
    it."""
    _on_device(s, v)
    if isinstance(s, torch.Tensor) and isinstance(v, torch.Tensor) and s.dim() and v.dim() \
            and s.numel() and v.numel() \
            and {s.dtype, v.dtype} <= {torch.float32, torch.bfloat16} and s.device.type == "cuda":
        dt = torch.promote_types(s.dtype, v.dtype)
        m, lv, acc = K.om_elem_scores(s, v)
        return m.to(dt), lv.to(dt), acc.to(dt)
    _fell_back()
    m = s.amax(dim=-1, keepdim=True)
    e = torch.exp(s - m)
    return m, e.sum(dim=-1, keepdim=True), _matmul(e, v)


def _omd_elem(s, a, b, *x, **kw):
    """``_omd_elem`` (xcarrier.py:380-400): ``(m, l, e@a, e@b)``; a coefficient
    ``a`` of 3 or more axes is the dense fibre ``(…,K,d,i)`` (key axis
    contracted through a ``(d·i)``-flattened view).  The row statistics of a
    device fp32 / bf16 score come from the ``catopt_hip_om_rows`` kernel."""
    _on_device(s, a, b)
    if isinstance(s, torch.Tensor) and s.dim() and s.numel() and s.device.type == "cuda" \
            and s.dtype in (torch.float32, torch.bfloat16):
        m, lv, e = (t.to(s.dtype) for t in K.om_rows(s))
    else:
        _fell_back()
        m = s.amax(dim=-1, keepdim=True)
        e = torch.exp(s - m)
        lv = e.sum(dim=-1, keepdim=True)
    if a.dim() >= 3:
        d, i = a.shape[-2], a.shape[-1]
        ea = _matmul(e, a.reshape(*a.shape[:-2], d * i))
        return m, lv, ea.reshape(*ea.shape[:-1], d, i), _matmul(e, b)
    return m, lv, _matmul(e, a), _matmul(e, b)


def _omd_compose(f, g, *a, **kw):
    """``_omd_compose`` (xcarrier.py:407-440): the om combine applied to both
    numerator parts; run as one om combine over the concatenated numerator."""
    m1, l1, fa1, fb1 = f
    m2, l2, fa2, fb2 = g
    lead = m1.dim()
    shape_a = fa1.shape
    fl = lambda fa: fa.reshape(*fa.shape[:lead - 1], -1)  # noqa: E731  (…,Tq,d[,i]) -> (…,Tq,·)
    n1 = torch.cat([fl(fa1), fb1], dim=-1)
    n2 = torch.cat([fl(fa2), fb2], dim=-1)
    m, lv, acc = _om_compose((m1, l1, n1), (m2, l2, n2))
    wa = n1.shape[-1] - fb1.shape[-1]
    return m, lv, acc[..., :wa].reshape(shape_a), acc[..., wa:]


def _om_elem_affd(s, a, b, h, *x, **kw):
    """``_om_elem_affd`` (xcarrier.py:348-359): ``(m, l, (e@a)⊙h + e@b)``."""
    m, lv, ea, eb = _omd_elem(s, a, b)
    return m, lv, ea * h + eb


def _om_elem_aff(s, A, b, h, *x, **kw):
    """``_om_elem_aff`` (xcarrier.py:362-377): ``(m, l, (e@A)@h + e@b)``."""
    m, lv, ea, eb = _omd_elem(s, A, b)
    return m, lv, _matmul(ea, h) + eb


def _decay(g, *a, **kw):
    t = int(attr_of(kw, "t", default=0) or 0)
    g = torch.as_tensor(g)
    _on_device(g)
    if g.dtype == torch.float32 and g.dim() <= 1 and g.device.type == "cuda":
        return K.decay(g, t)
    _fell_back()
    pos = torch.arange(t, dtype=g.dtype, device=g.device)
    diff = pos.unsqueeze(-1) - pos.unsqueeze(-2)
    return torch.tril(g[..., None, None] ** diff.clamp_min(0))


def _decay_vec(g, *a, **kw):
    t = int(attr_of(kw, "t", default=0) or 0)
    off = int(attr_of(kw, "offset", default=0) or 0)
    sign = int(kw["sign"]) if "sign" in kw else 1  # sign = 0 is legal (om.py:1082-1083)
    g = torch.as_tensor(g)
    _on_device(g)
    if g.dtype == torch.float32 and g.dim() <= 1 and g.device.type == "cuda":
        return K.decay_vec(g, t, off, sign)
    _fell_back()
    pos = torch.arange(t, dtype=g.dtype, device=g.device)
    return g[..., None] ** (pos * sign + off)


def _om_decayed(s, d, v, *a, **kw):
    """``om_decayed(s, d, v) = (s ⊙ d) @ v`` (om.py:1053-1057); the product
    is taken in the score dtype (the generated decay is cast to it)."""
    p = s * (d.to(s.dtype) if isinstance(d, torch.Tensor) else d)
    return _matmul(p, v.to(p.dtype) if v.dtype != p.dtype else v)


def _cmask(x, *a, **kw):
    """Masked set of the causal generator (om.py:1023-1029):
    ``¬tril(ones(t, k), -off)`` broadcast to ``x``'s shape."""
    off = int(kw.get("off", 0) or 0)
    t, k = x.shape[-2], x.shape[-1]
    keep = torch.ones(t, k, dtype=torch.bool, device=x.device).tril(-off)
    return keep.logical_not().expand(x.shape)


def _attnbias(m, *a, **kw):
    if m.dtype == torch.bool:
        return torch.where(m, torch.zeros((), device=m.device), torch.full((), float("-inf"), device=m.device))
    return m


def _sdpa(q, k, v, *a, **kw):
    """``scaled_dot_product_attention`` (torch_bridge.py:1225-1245: a
    positional mask, attrs ``arg3``..``arg6`` = attn_mask, dropout_p,
    is_causal, scale).  bf16 ``(…, T, d)`` operands with one leading shape,
    head dims up to 128, no dropout, a positive scale, a head extent
    within one launch (a larger batch runs as several), and at most one of ``is_causal`` / a mask
    that is one plane shared over the leading axes and broadcasting to
    ``(Tq, Tk)`` run the fused attention kernel (a bool mask keeps, a float
    one adds; ``is_causal`` keeps ``j <= i``; a fully masked row is 0, as
    torch gives it); any other call runs torch's op."""
    mask = a[0] if a else attr_of(kw, "attn_mask", "arg3", default=None)
    dropout = float(attr_of(kw, "dropout_p", "arg4", default=0.0) or 0.0)
    causal = bool(attr_of(kw, "is_causal", "arg5", default=False))
    scale = attr_of(kw, "scale", "arg6", default=None)
    _on_device(q, k, v, mask)
    kw_mask = _sdpa_kernel_mask(q, k, v, mask, causal, dropout)
    if kw_mask is not None:
        sc = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
        if math.isfinite(sc) and sc > 0:
            lead = q.shape[:-2]
            # (B, H) of a 4-D call; a 3-D call's leading axis is the batch
            q4, k4, v4 = (t if t.dim() == 4 else t.unsqueeze(1) if t.dim() == 3 else t[None, None]
                          for t in (q, k, v))
            if K.attention_grid_ok(q4):
                o = K.attention(q4, k4, v4, sc, empty_rows="zero", **kw_mask)
                return o.reshape(*lead, o.shape[-2], o.shape[-1])
    _fell_back()
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, dropout_p=dropout, is_causal=causal,
                                          scale=None if scale is None else float(scale))


def _sdpa_kernel_mask(q, k, v, mask, causal, dropout) -> dict | None:
    """Mask arguments of the attention kernel for an sdpa call, or ``None``
    when the call is outside the kernel's envelope."""
    ts = (q, k, v)
    if dropout != 0.0 or not all(isinstance(t, torch.Tensor) and t.dtype == torch.bfloat16
                                 and t.device.type == "cuda" for t in ts):
        return None
    if not 2 <= q.dim() <= 4 or k.shape[:-2] != q.shape[:-2] or v.shape[:-2] != q.shape[:-2]:
        return None
    d, dv = q.shape[-1], v.shape[-1]
    if max(d, dv) > K.ATTENTION_MAX_HEAD_DIM or k.shape[-1] != d or v.shape[-2] != k.shape[-2]:
        return None
    if mask is None:
        return {"causal": True, "causal_off": 0} if causal else {}
    if causal or not isinstance(mask, torch.Tensor) or mask.dim() < 2:
        return None
    if mask.dtype != torch.bool and not mask.dtype.is_floating_point:
        return None
    plane = shared_plane(mask)
    plane = None if plane is None else fit_plane(plane, q.shape[-2], k.shape[-2])
    if plane is None:
        return None
    return {"mask": plane} if mask.dtype == torch.bool else {"bias": plane}


def _split_sizes(t, kw):
    sizes = attr_of(kw, "sizes", "split_size", default=None)
    if isinstance(sizes, (list, tuple)):
        return [int(s) for s in sizes]
    return int(sizes)


def _transpose(x, *a, **kw):
    if x.dim() == 2 and "dim0" not in kw and "dim1" not in kw:
        return x.t()
    return x.transpose(int(attr_of(kw, "dim0", default=-2)), int(attr_of(kw, "dim1", default=-1)))


def _scalar_like(v):
    return v.item() if isinstance(v, torch.Tensor) and v.dim() == 0 and v.device.type == "cpu" else v


HIP_BINDINGS: dict[str, Callable] = {
    # ---- the device ops around the delivered forms (norms, clamps, gathers,
    #      creators, casts …); the entries below take precedence
    **DEVICE_OPS,
    # ---- GEMM family and norms (HIP kernels)
    "linear": _linear,
    "matmul": _matmul,
    "rms_norm": _rms_norm,
    "silu": _silu,
    "glu": lambda t, *a, **kw: F.glu(t, dim=int(attr_of(kw, "dim", default=-1))),
    # ---- online-softmax monoid (torch_bridge.py:1885-1890)
    "om": lambda m, lv, acc, *x, **kw: (m, lv, acc),
    "om_elem": om_elem_dense,
    "om_compose": _om_compose,
    "om_apply": lambda f, *a, **kw: f[2] / f[1],
    # ---- decayed attention carrier (om.py:1053-1106)
    "om_decayed": _om_decayed,
    "decay": _decay,
    "decay_vec": _decay_vec,
    "cmask": _cmask,
    "attnbias": _attnbias,
    "fill": lambda x, *a, **kw: torch.full_like(x, float(kw.get("value", 0))),
    # ---- diagonal affine monoid (torch_bridge.py:1895-1900, xcarrier.py:460-472)
    "aff_diag": lambda a_, b_, *x, **kw: (a_, b_),
    "affd_compose": lambda f, g, *a, **kw: (f[0] * g[0], f[0] * g[1] + f[1]),
    "applyd": lambda f, h, *a, **kw: f[0] * h + f[1],
    "affd_a": lambda f, *a, **kw: f[0],
    "affd_b": lambda f, *a, **kw: f[1],
    # ---- deferred-affine om carrier (xcarrier.py:380-472)
    "omd_elem": _omd_elem,
    "omd": lambda m, lv, fa, fb, *a, **kw: (m, lv, fa, fb),
    "omd_compose": _omd_compose,
    "omd_apply": lambda f, h, *a, **kw: (f[2] * h + f[3]) / f[1],
    "omd_applym": lambda f, h, *a, **kw: (_matmul(f[2], h) + f[3]) / f[1],
    "om_elem_affd": _om_elem_affd,
    "om_elem_aff": _om_elem_aff,
    # ---- dense affine monoid (torch_bridge.py:1873-1881, xcarrier.py:460-472)
    "aff": lambda A, b_, *x, **kw: (A, b_),
    "aff_compose": lambda f, g, *a, **kw: (_matmul(f[0], g[0]), _matmul(f[0], g[1]) + f[1]),
    "apply": lambda f, h, *a, **kw: _matmul(f[0], h) + f[1],
    "aff_A": lambda f, *a, **kw: f[0],
    "aff_b": lambda f, *a, **kw: f[1],
    # ---- elementwise / reductions (device ops)
    "add": lambda x, y, *a, **kw: torch.add(x, y),
    "sub": lambda x, y, *a, **kw: torch.sub(x, y),
    "rsub": lambda x, s, *a, **kw: torch.sub(s, x),
    "mul": lambda x, y, *a, **kw: torch.mul(x, y),
    "div": lambda x, y, *a, **kw: torch.div(x, y, rounding_mode=kw.get("rounding_mode")),
    "neg": lambda x, *a, **kw: torch.neg(x),
    "exp": lambda x, *a, **kw: torch.exp(x),
    "sigmoid": lambda x, *a, **kw: torch.sigmoid(x),
    "tanh": lambda x, *a, **kw: torch.tanh(x),
    "relu": lambda x, *a, **kw: F.relu(x),
    "gelu": lambda x, *a, **kw: F.gelu(x),
    "pow": lambda x, y, *a, **kw: torch.pow(x, _scalar_like(y)),
    "square": lambda x, *a, **kw: torch.square(x),
    "sqrt": lambda x, *a, **kw: torch.sqrt(x),
    "rsqrt": lambda x, *a, **kw: torch.rsqrt(x),
    "sum": lambda x, *a, **kw: x.sum(*_dims(kw)),
    "mean": lambda x, *a, **kw: x.mean(*_dims(kw)),
    "amax": lambda x, *a, **kw: x.amax(*_dims(kw)),
    "softmax": lambda x, *a, **kw: F.softmax(x, dim=int(attr_of(kw, "dim", default=-1))),
    "sdpa": _sdpa,
    "masked_fill": lambda x, m, v, *a, **kw: x.masked_fill(m, _scalar_like(v)),
    "where": lambda c, x, y, *a, **kw: torch.where(c, x, y),
    "eq": lambda x, y, *a, **kw: x == y,
    "ne": lambda x, y, *a, **kw: x != y,
    "logical_not": lambda x, *a, **kw: torch.logical_not(x),
    "tril": lambda t, *a, **kw: torch.tril(t, int(attr_of(kw, "diagonal", default=0))),
    # ---- layout (views)
    "transpose": _transpose,
    "reshape": lambda x, *a, **kw: x.reshape(tuple(kw["shape"]) if "shape" in kw else (-1,)),
    "view": lambda x, *a, **kw: x.reshape(tuple(kw["shape"]) if "shape" in kw else (-1,)),
    "contiguous": lambda x, *a, **kw: x.contiguous(),
    "unsqueeze": lambda t, *a, **kw: t.unsqueeze(int(attr_of(kw, "dim", default=-1))),
    "squeeze": lambda t, *a, **kw: t.squeeze() if attr_of(kw, "dim") is None else t.squeeze(int(kw["dim"])),
    "flatten": lambda x, *a, **kw: x.flatten(int(attr_of(kw, "start_dim", default=0)),
                                             int(attr_of(kw, "end_dim", default=-1))),
    "expand": lambda x, *a, **kw: x.expand(*attr_of(kw, "shape", "size", default=())),
    "concat": lambda *ts, **kw: torch.cat(list(ts), dim=int(attr_of(kw, "dim", default=0))),
    "stack": lambda *ts, **kw: torch.stack(list(ts), dim=int(attr_of(kw, "dim", default=0))),
    "chunk": lambda t, *a, **kw: torch.chunk(t, int(attr_of(kw, "chunks", default=2)),
                                             dim=int(attr_of(kw, "dim", default=-1)))[int(attr_of(kw, "index", default=0))],
    "split": lambda t, *a, **kw: torch.split(t, _split_sizes(t, kw), dim=int(attr_of(kw, "dim", default=-1)))[
        int(attr_of(kw, "index", default=0))],
    "slice": lambda t, *a, **kw: t[(slice(None),) * int(attr_of(kw, "dim", default=0))
                                   + (slice(kw.get("start"), kw.get("end"), kw.get("step")),)],
    "select": lambda t, *a, **kw: t.select(int(attr_of(kw, "dim", default=0)), int(attr_of(kw, "index", default=0))),
    "getitem": lambda t, *a, **kw: t[attr_of(kw, "index", default=0)],
    "to": lambda x, *a, **kw: x.to(dtype=getattr(torch, kw["dtype"])) if isinstance(kw.get("dtype"), str) else x,
    "alias": lambda x, *a, **kw: x,
    "clone": lambda x, *a, **kw: x.clone(),
    "dropout": lambda x, *a, **kw: x,
    "broadcast": lambda x, *a, **kw: x,
    "pack": lambda *ts, **kw: tuple(ts),
}


class HipOpTable:
    """The op registry of the HIP sink (the ``OpRegistry`` port,
    ports.py:314-344, and ``OpTable.register``, ops.py:338-389).

    ``torch_bindings`` is the lowering table (the name is the port's
    historical one); ``register`` composes more bindings in and returns
    ``self``.  A module exporting ``TORCH_BINDINGS`` registers as a whole.
    """

    def __init__(self, bindings: dict | None = None) -> None:
        self.torch_bindings: dict[str, Callable] = dict(HIP_BINDINGS if bindings is None else bindings)
        self.shape_rules: dict = {}
        self.attr_schemas: dict = {}

    def register(self, source: Any = None, *, torch_bindings: dict | None = None,
                 shape_rules: dict | None = None, attr_schema: dict | None = None) -> "HipOpTable":
        if source is not None:
            tb = getattr(source, "TORCH_BINDINGS", source)
            if not isinstance(tb, dict):
                raise TypeError("register() takes a bindings dict or a module exporting TORCH_BINDINGS")
            self.torch_bindings.update(tb)
        if torch_bindings:
            self.torch_bindings.update(torch_bindings)
        if shape_rules:
            self.shape_rules.update(shape_rules)
        if attr_schema:
            self.attr_schemas.update(attr_schema)
        return self

    def copy(self) -> "HipOpTable":
        t = HipOpTable(self.torch_bindings)
        t.shape_rules = dict(self.shape_rules)
        t.attr_schemas = dict(self.attr_schemas)
        return t

    def __contains__(self, op: str) -> bool:
        return op in self.torch_bindings

    def __getitem__(self, op: str) -> Callable:
        try:
            return self.torch_bindings[op]
        except KeyError:
            raise ValueError(f"No HIP binding for op {op!r}") from None


def scalar_value(t: Any) -> float | None:
    """The Python number of a ``Const`` leaf (``None`` for anything else)."""
    from .ir import Const

    if isinstance(t, Const) and isinstance(t.value, (int, float)) and not isinstance(t.value, bool):
        return float(t.value)
    return None


def finite_scale(v: float | None) -> bool:
    return v is not None and math.isfinite(v) and v != 0.0

