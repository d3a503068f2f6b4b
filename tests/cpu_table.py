"""A host-only op table for testing the executors' host logic on the CPU.

The product's bindings run on the ROCm device and raise on host tensors.
These tests swap in plain torch functions for the HIP-backed ops — through
the same ``HipOpTable`` seam a caller uses to register bindings — so fold,
fusion, planning, routing and fallback logic can be exercised here.  Nothing
in ``catopt_amd`` imports this module.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from catopt_amd.bindings import HIP_BINDINGS, HipOpTable, attr_of


def _linear(x, w, *a, **kw):
    return F.linear(x, w, a[0] if a else kw.get("bias"))


def _rms(x, w=None, *a, **kw):
    shape = attr_of(kw, "dim", default=(x.shape[-1],))
    return F.rms_norm(x, tuple(shape), weight=w, eps=float(attr_of(kw, "eps", default=1e-6)))


def _swiglu(x, w, **kw):
    y = F.linear(x, w)
    g, u = y.chunk(2, dim=-1)
    return F.silu(g) * u


def _glu(x, w, **kw):
    return F.glu(F.linear(x, w), dim=-1)


def _decay(g, *a, **kw):
    t = int(kw.get("t", 0))
    g = torch.as_tensor(g)
    pos = torch.arange(t, dtype=g.dtype)
    return torch.tril(g[..., None, None] ** (pos[:, None] - pos[None, :]).clamp_min(0))


def _decay_vec(g, *a, **kw):
    t = int(kw.get("t", 0))
    off = int(kw.get("offset", 0) or 0)
    sign = int(kw["sign"]) if "sign" in kw else 1
    g = torch.as_tensor(g)
    pos = torch.arange(t, dtype=g.dtype)
    return g[..., None] ** (pos * sign + off)


def _om_compose(f, g, *a, **kw):
    m1, l1, a1 = f
    m2, l2, a2 = g
    mx = torch.maximum(m1, m2)
    f1, f2 = torch.isfinite(m1), torch.isfinite(m2)
    e1 = torch.where(f1, torch.exp(m1 - mx), torch.zeros_like(mx))
    e2 = torch.where(f2, torch.exp(m2 - mx), torch.zeros_like(mx))
    # a block whose max is not finite contributes nothing, NaN l / a included
    lv = torch.where(f1, l1 * e1, 0.0) + torch.where(f2, l2 * e2, 0.0)
    return mx, lv, torch.where(f1, a1 * e1, 0.0) + torch.where(f2, a2 * e2, 0.0)


def _om_elem(s, v, *a, **kw):
    m = s.amax(dim=-1, keepdim=True)
    e = torch.exp(s - m)
    return m, e.sum(dim=-1, keepdim=True), e @ v


def _omd_elem(s, a, b, *x, **kw):
    m = s.amax(dim=-1, keepdim=True)
    e = torch.exp(s - m)
    if a.dim() >= 3:
        d, i = a.shape[-2], a.shape[-1]
        ea = (e @ a.reshape(*a.shape[:-2], d * i)).reshape(*e.shape[:-1], d, i)
        return m, e.sum(dim=-1, keepdim=True), ea, e @ b
    return m, e.sum(dim=-1, keepdim=True), e @ a, e @ b


def _omd_compose(f, g, *a, **kw):
    m1, l1, fa1, fb1 = f
    m2, l2, fa2, fb2 = g
    lead = m1.dim()
    n1 = torch.cat([fa1.reshape(*fa1.shape[:lead - 1], -1), fb1], -1)
    n2 = torch.cat([fa2.reshape(*fa2.shape[:lead - 1], -1), fb2], -1)
    m, lv, acc = _om_compose((m1, l1, n1), (m2, l2, n2))
    wa = n1.shape[-1] - fb1.shape[-1]
    return m, lv, acc[..., :wa].reshape(fa1.shape), acc[..., wa:]


def cpu_table() -> HipOpTable:
    t = HipOpTable(HIP_BINDINGS)
    t.register(torch_bindings={
        "linear": _linear,
        "matmul": lambda a, b, *x, **kw: torch.matmul(a, b),
        "rms_norm": _rms,
        "silu": lambda x, *a, **kw: F.silu(x),
        "decay": _decay,
        "decay_vec": _decay_vec,
        "om_compose": _om_compose,
        "om_decayed": lambda s, d, v, *a, **kw: (s * d) @ v,
        "om_elem": _om_elem,
        "hip_linear": lambda x, w, b=None, **kw: F.linear(x, w, b),
        "hip_swiglu": _swiglu,
        "hip_glu": _glu,
        "aff_compose": lambda f, g, *a, **kw: (f[0] @ g[0], f[0] @ g[1] + f[1]),
        "apply": lambda f, h, *a, **kw: f[0] @ h + f[1],
        "omd_elem": _omd_elem,
        "omd_compose": _omd_compose,
        "omd_applym": lambda f, h, *a, **kw: (f[2] @ h + f[3]) / f[1],
    })
    return t
