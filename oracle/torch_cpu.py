"""The delivered forms' arithmetic as eager torch ops on the host CPU.

Test infrastructure, like the rest of ``oracle/``: the CPU baseline that
``bench.py`` times beside the GPU (its ``cpu_baseline`` leg), never part of the
product path.  The reference runs a delivered term on the CPU as eager torch
ops through its executors (catopt-torch: ``torch_bridge.py``'s bindings and
the batched modules), in the operands' dtype with torch's own promotion; these
functions restate those op sequences per form, batched over the independent
axes so that torch spreads them over every host core.  ``tests/test_oracle.py``
pins each one against the numpy oracle (float64) on small inputs.

* ``weight_chain``       the folded C1 form: one ``linear`` with the folded
                         weight and bias (``torch_bridge.py:2456-2686`` fold,
                         ``:1147`` linear);
* ``swiglu_block``       C2: ``rms_norm`` (``:1404-1411``), ``linear`` of the
                         fused gate/up weight, ``chunk``/``silu``/``mul``,
                         ``linear`` (``laws/tensor.py:1485-1519``);
* ``causal_attention``   C3: the explicit ``matmul`` / ``masked_fill`` /
                         ``softmax`` / ``matmul`` spelling the term starts from;
* ``retention_chunked``  C4: the chunked decayed form's blocks
                         (``decayed_lower.py:609-724``): intra-chunk
                         ``(q kᵀ ⊙ decay) v`` and the carried cross-chunk state;
* ``ssm_scan``           C5: the diagonal recurrence ``h_t = a_t h_{t-1} +
                         x_t ⊗ b_t``, ``y_t = h_t · c_t``, one step at a time
                         over all lanes (``scan_lower.py:427-807``'s serial
                         meaning);
* ``dense_scan``         the dense affine recurrence ``h_t = A h_{t-1} + b_t``;
* ``omd_attention``      softmax attention over the states of a diagonal scan
                         (``omd_lower.py:562-1019``'s meaning).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["causal_attention", "dense_scan", "omd_attention", "retention_chunked", "ssm_scan",
           "swiglu_block", "weight_chain"]


def weight_chain(x: torch.Tensor, W_eff: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    return F.linear(x, W_eff, c)


def swiglu_block(x: torch.Tensor, gamma: torch.Tensor, W_gate: torch.Tensor, W_up: torch.Tensor,
                 W_down: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    h = F.rms_norm(x, (x.shape[-1],), gamma, eps)
    gu = F.linear(h, torch.cat([W_gate, W_up], 0))
    g, u = gu.chunk(2, dim=-1)
    return F.linear(F.silu(g) * u, W_down)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    T, Tk = q.shape[-2], k.shape[-2]
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    keep = torch.ones(T, Tk, dtype=torch.bool).tril()
    return torch.matmul(torch.softmax(s.masked_fill(~keep, float("-inf")), dim=-1), v)


def retention_chunked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma: torch.Tensor, C: int,
                      scale: float = 1.0) -> torch.Tensor:
    """``q, k, v (B, H, T, d)``, ``gamma (H,)``; ``T`` a multiple of ``C``.
    bf16 operands meet the fp32 decay tensors and compute in fp32 (torch's
    promotion); the result is cast back to the operands' dtype."""
    B, H, T, d = q.shape
    dv = v.shape[-1]
    g = gamma.to(torch.float32).reshape(1, H, 1, 1)
    pos = torch.arange(C, dtype=torch.float32)
    diff = pos[:, None] - pos[None, :]
    lg = torch.log(g)
    D = torch.where(diff >= 0, torch.exp(diff * lg), torch.zeros(()))  # (1, H, C, C)
    row = torch.exp(pos.reshape(1, 1, C, 1) * lg)          # γ^a
    col = torch.exp((C - pos).reshape(1, 1, C, 1) * lg)    # γ^(C - c)
    gC = torch.exp(C * lg)
    S = torch.zeros(B, H, d, dv)
    out = torch.empty(B, H, T, dv)
    for i in range(T // C):
        sl = slice(i * C, (i + 1) * C)
        qi, ki, vi = q[:, :, sl].float(), k[:, :, sl].float(), v[:, :, sl].float()
        out[:, :, sl] = scale * (torch.matmul(torch.matmul(qi, ki.transpose(-1, -2)) * D, vi)
                                 + row * torch.matmul(qi, S))
        S = gC * S + torch.matmul(ki.transpose(-1, -2), col * vi)
    return out.to(q.dtype)


def ssm_scan(a: torch.Tensor, bx: torch.Tensor, c: torch.Tensor, x: torch.Tensor,
             h0: torch.Tensor | None = None) -> torch.Tensor:
    """``a (B,T,D,N)``, ``bx, c (B,T,N)``, ``x (B,T,D)``: all ``y (B,T,D)``."""
    B, T, D, N = a.shape
    h = torch.zeros(B, D, N, dtype=a.dtype) if h0 is None else h0.clone()
    y = torch.empty(B, T, D, dtype=x.dtype)
    for t in range(T):
        h = a[:, t] * h + x[:, t, :, None] * bx[:, t, None, :]
        y[:, t] = (h * c[:, t, None, :]).sum(-1)
    return y


def dense_scan(A: torch.Tensor, b: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """``A (d, d)`` shared, ``b (T, B, d)``, ``h (B, d)``: the final states."""
    for t in range(b.shape[0]):
        h = h @ A.T + b[t]
    return h


def omd_attention(q: torch.Tensor, k: torch.Tensor, a: torch.Tensor, x: torch.Tensor,
                  h: torch.Tensor) -> torch.Tensor:
    """Softmax attention of ``q (Tq, dk)`` over keys ``k (T, dk)`` whose
    values are the states ``h_t = a_t ⊙ h_{t-1} + x_t`` of a diagonal scan
    from ``h``."""
    T = a.shape[0]
    states = torch.empty(T, a.shape[1], dtype=a.dtype)
    s = h
    for t in range(T):
        s = a[t] * s + x[t]
        states[t] = s
    w = torch.softmax(q @ k.T, dim=-1)
    return w @ states

