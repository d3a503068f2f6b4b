"""Torch-facing wrappers over the C ABI: device memory and streams in, kernels out.

Every function here takes ``torch.Tensor`` operands that already live on a
ROCm device, allocates its outputs (and any workspace) with torch's caching
allocator, and enqueues the kernel on torch's current stream.  Shapes,
dtypes and layouts are checked on the host before any launch, so a kernel
only ever sees operands that match what its grid assumes.  There is no CPU
path: a host tensor or a missing library raises.
"""

from __future__ import annotations

import math
from typing import Sequence

import torch

from . import _lib as L

_DT = {torch.float32: L.F32, torch.bfloat16: L.BF16}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# torch's current-stream handle of a device, by index: the raw accessor
# costs ~0.1 us where current_stream(dev).cuda_stream costs ~2 us, which is
# most of a small kernel's launch path
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _need_device(*ts: torch.Tensor | None) -> int:
    """The device index all tensor operands share; raises on a host tensor
    (there is no CPU path), a non-tensor or operands on different devices."""
    dev = -1
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a tensor, got {type(t).__name__}")
        if not t.is_cuda:
            raise ValueError(
                "catopt_amd kernels run on a ROCm device only; got a tensor on "
                f"{t.device} (there is no CPU fallback)"
            )
        d = t.get_device()
        if dev < 0:
            dev = d
        elif d != dev:
            raise ValueError(f"operands on different devices: cuda:{dev} vs cuda:{d}")
    if dev < 0:
        raise ValueError("no tensor operands")
    return dev


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise NotImplementedError(
            f"dtype {t.dtype} is not supported by the HIP kernels (fp32, bf16)"
        ) from None


def _rows_view(x: torch.Tensor) -> tuple[torch.Tensor, int]:
    """(M, K) view with a contiguous last axis and a uniform row stride."""
    if x.dim() == 2 and x.is_contiguous():
        return x, x.shape[1]
    if x.dim() == 0:
        raise ValueError("expected at least a vector")
    x2 = x.reshape(-1, x.shape[-1]) if x.dim() != 2 else x
    if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < x2.shape[1]):
        x2 = x2.contiguous()
    ld = x2.stride(0) if x2.shape[0] > 1 else x2.shape[1]
    return x2, max(ld, x2.shape[1])


# --------------------------------------------------------------------- norms


def rmsnorm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """``x * rsqrt(mean(x², -1) + eps) * weight`` over the last axis."""
    _need_device(x, weight)
    lib = L.load()
    dt = _dtype_code(x)
    if weight is not None:
        if weight.dtype != x.dtype or weight.numel() != x.shape[-1]:
            raise ValueError("rms_norm weight must match x's last axis and dtype")
        weight = weight.contiguous()
    x2, ldx = _rows_view(x)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    rows, cols = x2.shape
    st = lib.catopt_hip_rmsnorm(dt, rows, cols, _ptr(x2), ldx, _ptr(weight), float(eps),
                                _ptr(y), cols, _stream(x))
    L.check("catopt_hip_rmsnorm", st)
    return y


# ---------------------------------------------------------------------- GEMM


def linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor | None = None,
    bias2: torch.Tensor | None = None,
    epilogue: int | None = None,
) -> torch.Tensor:
    """``epi(x @ weightᵀ)`` with nn.Linear weight layout ``(out, in)``.

    ``epilogue`` defaults to NONE / BIAS / BIAS_ADD2 by which biases are
    given.  For ``EPI_SILU_MUL`` / ``EPI_GLU`` the weight holds both
    projections stacked along its rows and the output width is half of them.
    """
    _need_device(x, weight, bias, bias2)
    lib = L.load()
    dt = _dtype_code(x)
    if weight.dtype != x.dtype or weight.dim() != 2:
        raise ValueError("linear weight must be 2-D and share x's dtype")
    if epilogue is None:
        epilogue = L.EPI_NONE if bias is None else (L.EPI_BIAS if bias2 is None else L.EPI_BIAS_ADD2)
    K = x.shape[-1]
    if weight.shape[1] != K:
        raise ValueError(f"linear: x has {K} features, weight expects {weight.shape[1]}")
    paired = epilogue in (L.EPI_SILU_MUL, L.EPI_GLU)
    n_rows = weight.shape[0]
    if paired and n_rows % 2:
        raise ValueError("paired epilogue needs an even number of weight rows")
    N = n_rows // 2 if paired else n_rows
    for b in (bias, bias2):
        if b is not None and (b.numel() != N or b.dtype != x.dtype):
            raise ValueError("bias must be an [N] vector of x's dtype")
    bias = bias.contiguous() if bias is not None else None
    bias2 = bias2.contiguous() if bias2 is not None else None
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    x2, ldx = _rows_view(x)
    M = x2.shape[0]
    y = x.new_empty((*x.shape[:-1], N))
    if M == 0 or N == 0:
        return y
    if K == 0:
        y.zero_()
        if bias is not None:
            y += bias
        if bias2 is not None:
            y += bias2
        if paired:
            raise NotImplementedError("paired epilogue over an empty contraction")
        return y
    st = lib.catopt_hip_linear(dt, M, N, K, _ptr(x2), ldx, _ptr(weight), weight.stride(0),
                               _ptr(bias), _ptr(bias2), int(epilogue), _ptr(y), N, _stream(x))
    L.check("catopt_hip_linear", st)
    return y


def _mat_layout(t: torch.Tensor) -> tuple[torch.Tensor, bool, int, int]:
    """(tensor, transposed, ld, batch_stride) for a (batch, r, c) operand."""
    s_b, s_r, s_c = t.stride()
    r, c = t.shape[1], t.shape[2]
    if s_c == 1 and (r == 1 or s_r >= c):
        return t, False, max(s_r, c), s_b
    if s_r == 1 and (c == 1 or s_c >= r):
        return t, True, max(s_c, r), s_b
    t = t.contiguous()
    return t, False, c, t.stride(0)


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``torch.matmul`` semantics for 2-D and batched 3-D+ operands (fp32/bf16)."""
    _need_device(a, b)
    lib = L.load()
    dt = _dtype_code(a)
    if a.dtype != b.dtype:
        raise ValueError(f"matmul operands must share a dtype: {a.dtype} vs {b.dtype}")
    if a.dim() < 2 or b.dim() < 2:
        if a.dim() == 1 and b.dim() >= 2:
            return matmul(a.unsqueeze(0), b).squeeze(-2)
        if b.dim() == 1 and a.dim() >= 2:
            return matmul(a, b.unsqueeze(-1)).squeeze(-1)
        raise NotImplementedError("matmul of two vectors")
    M, K = a.shape[-2], a.shape[-1]
    K2, N = b.shape[-2], b.shape[-1]
    if K != K2:
        raise ValueError(f"matmul shape mismatch {tuple(a.shape)} @ {tuple(b.shape)}")
    batch_shape = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    nb = math.prod(batch_shape) if batch_shape else 1
    # A single matrix broadcast over the batch keeps batch stride 0 (no copy).
    a3 = a.unsqueeze(0).expand(nb, M, K) if a.dim() == 2 else a.expand(*batch_shape, M, K).reshape(nb, M, K)
    b3 = b.unsqueeze(0).expand(nb, K, N) if b.dim() == 2 else b.expand(*batch_shape, K, N).reshape(nb, K, N)
    a3, ta, lda, sa = _mat_layout(a3)
    b3, tb, ldb, sb = _mat_layout(b3)
    out = torch.empty((nb, M, N), dtype=a.dtype, device=a.device)
    if nb and M and N:
        if K == 0:
            out.zero_()
        else:
            st = lib.catopt_hip_matmul(dt, nb, M, N, K, _ptr(a3), lda, sa, int(ta), _ptr(b3), ldb,
                                       sb, int(tb), _ptr(out), N, M * N, _stream(a))
            L.check("catopt_hip_matmul", st)
    return out.reshape(*batch_shape, M, N)


# ----------------------------------------------------------------- attention


def _bhtd(t: torch.Tensor) -> tuple[torch.Tensor, list[int]]:
    if t.dim() != 4:
        raise ValueError("attention operands are (B, H, T, d)")
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:3]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t, [t.stride(0), t.stride(1), t.stride(2)]


ATTENTION_MAX_HEAD_DIM = 128


#: Largest batch and head extents of one ``catopt_hip_attn_fwd`` launch
#: (CATOPT_E_UNSUPPORTED beyond them).  :func:`attention` splits a larger
#: batch into several launches; the head extent must fit one.
ATTENTION_MAX_GRID_AXIS = 65535


def attention_grid_ok(q4: torch.Tensor) -> bool:
    """Whether :func:`attention` takes a ``(B, H, T, d)`` operand: any batch
    extent, a head extent within one launch."""
    return q4.dim() == 4 and q4.shape[1] <= ATTENTION_MAX_GRID_AXIS


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    *,
    causal: bool = False,
    causal_off: int = 0,
    mask: torch.Tensor | None = None,
    bias: torch.Tensor | None = None,
    normalize: bool = True,
    return_ml: bool = False,
    empty_rows: str = "nan",
):
    """Online-softmax attention ``(B,H,T,d)`` bf16, head dims up to 128
    (other widths than 64 / 128 run zero-padded to the next of them).

    ``causal`` keeps key ``j`` for query ``i`` iff ``j <= i + causal_off``;
    ``mask`` is a bool keep-mask ``(Tq, Tk)`` shared over (B, H); ``bias``
    an additive float ``(Tq, Tk)`` plane added to ``scale·q kᵀ`` (``-inf``
    entries mask).  With
    ``normalize=False`` the raw numerator ``a`` is returned; ``return_ml``
    adds the fp32 ``(m, l)`` om carriers, shaped ``(B, H, Tq, 1)``.  A fully
    masked row normalises to NaN (``empty_rows="nan"``, om_apply's 0/0) or
    to 0 (``"zero"``, torch's scaled_dot_product_attention).
    """
    if empty_rows not in ("nan", "zero"):
        raise ValueError(f"empty_rows is 'nan' or 'zero', got {empty_rows!r}")
    _need_device(q, k, v, mask)
    lib = L.load()
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        raise NotImplementedError("HIP attention runs on bf16 operands")
    B, H, Tq, d = q.shape
    Bk, Hk, Tk, dk = k.shape
    if (Bk, Hk, dk) != (B, H, d) or v.shape[:3] != k.shape[:3]:
        raise ValueError(f"attention shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    dv = v.shape[3]
    if max(d, dv) > ATTENTION_MAX_HEAD_DIM or min(d, dv) < 1:
        raise NotImplementedError(f"HIP attention supports head dims up to {ATTENTION_MAX_HEAD_DIM}, got {d}, {dv}")
    width = 64 if max(d, dv) <= 64 else 128
    if d != width or dv != width:
        # the kernel's widths are 64 and 128 with d = dv: zero columns leave
        # every score unchanged and add zero output columns, dropped below
        q, k = (torch.nn.functional.pad(t, (0, width - d)) if d < width else t for t in (q, k))
        v = torch.nn.functional.pad(v, (0, width - dv)) if dv < width else v
        r = attention(q, k, v, scale, causal=causal, causal_off=causal_off, mask=mask, bias=bias,
                      normalize=normalize, return_ml=return_ml, empty_rows=empty_rows)
        if return_ml:
            return r[0][..., :dv], r[1], r[2]
        return r[..., :dv]
    q, qs = _bhtd(q)
    k, ks = _bhtd(k)
    v, vs = _bhtd(v)
    o = torch.empty((B, H, Tq, dv), dtype=q.dtype, device=q.device)
    m = l = None
    if return_ml:
        m = torch.empty((B, H, Tq), dtype=torch.float32, device=q.device)
        l = torch.empty((B, H, Tq), dtype=torch.float32, device=q.device)
    mode = L.MASK_NONE
    mask_u8 = None
    mask_ld = 0
    if (mask is not None) + (bias is not None) + bool(causal) > 1:
        raise ValueError("pass at most one of causal=True, mask, bias")
    if mask is not None:
        if mask.shape[-2:] != (Tq, Tk) or mask.numel() != Tq * Tk:
            raise NotImplementedError("mask must be a (Tq, Tk) keep-mask shared over (B, H)")
        mask_u8 = mask.reshape(Tq, Tk).to(torch.uint8).contiguous()
        mask_ld = Tk
        mode = L.MASK_BOOL
    elif bias is not None:
        _need_device(bias)
        if bias.shape[-2:] != (Tq, Tk) or bias.numel() != Tq * Tk:
            raise NotImplementedError("bias must be a (Tq, Tk) plane shared over (B, H)")
        mask_u8 = bias.reshape(Tq, Tk).to(torch.float32).contiguous()
        mask_ld = Tk
        mode = L.MASK_BIAS
    elif causal:
        mode = L.MASK_CAUSAL
    os_ = L.i64_array([o.stride(0), o.stride(1), o.stride(2)])
    qs, ks, vs = L.i64_array(qs), L.i64_array(ks), L.i64_array(vs)
    norm = (2 if empty_rows == "zero" else 1) if normalize else 0
    # one launch per run of at most ATTENTION_MAX_GRID_AXIS batch entries:
    # every operand, and the (B, H, Tq) statistics, advance by whole batches
    for b0 in range(0, B, ATTENTION_MAX_GRID_AXIS):
        nb = min(B - b0, ATTENTION_MAX_GRID_AXIS)
        st = lib.catopt_hip_attn_fwd(
            L.BF16, nb, H, Tq, Tk, d, dv, _ptr(q[b0:]), qs, _ptr(k[b0:]), ks, _ptr(v[b0:]), vs,
            float(scale), mode, int(causal_off), _ptr(mask_u8), mask_ld, norm, _ptr(o[b0:]), os_,
            _ptr(m[b0:] if m is not None else None), _ptr(l[b0:] if l is not None else None), _stream(q))
        L.check("catopt_hip_attn_fwd", st)
    if return_ml:
        return o, m.unsqueeze(-1), l.unsqueeze(-1)
    return o


def om_rows(s: torch.Tensor, sanitize: bool = False) -> tuple:
    """Row statistics of a score block ``s (…, cols)``: ``m = rowmax``,
    ``e = exp(s - m)``, ``l = Σ e`` in fp32 (``m``, ``l`` shaped ``(…, 1)``).
    ``sanitize`` zeroes ``l`` and ``e`` on rows whose max is not finite."""
    _need_device(s)
    lib = L.load()
    dt = _dtype_code(s)
    cols = s.shape[-1]
    s2, lds = _rows_view(s) if s.dim() else (s.reshape(1, 1), 1)
    rows = s2.shape[0]
    m = torch.empty(s.shape[:-1] + (1,), dtype=torch.float32, device=s.device)
    lv = torch.empty_like(m)
    e = torch.empty(s.shape, dtype=torch.float32, device=s.device)
    st = lib.catopt_hip_om_rows(dt, rows, cols, _ptr(s2), lds, int(bool(sanitize)), _ptr(m), _ptr(lv),
                                _ptr(e), cols, _stream(s))
    L.check("catopt_hip_om_rows", st)
    return m, lv, e


def om_elem_scores(s: torch.Tensor, v: torch.Tensor, sanitize: bool = False) -> tuple:
    """The om element of an explicit score block: ``(rowmax s, Σ exp(s - m),
    exp(s - m) @ v)`` in fp32, ``v`` broadcasting like ``matmul``."""
    m, lv, e = om_rows(s, sanitize)
    return m, lv, matmul(e, v.to(torch.float32))


def om_compose(f, g):
    """FlashAttention combine of two fp32 om carriers ``(m, l, a)``."""
    m1, l1, a1 = f
    m2, l2, a2 = g
    _need_device(m1, l1, a1, m2, l2, a2)
    lib = L.load()
    ts = [t.float().contiguous() for t in (m1, l1, a1, m2, l2, a2)]
    m1, l1, a1, m2, l2, a2 = ts
    rows = m1.numel()
    if l1.numel() != rows or m2.numel() != rows or l2.numel() != rows:
        raise ValueError("om carriers disagree on their row count")
    dv = a1.numel() // max(rows, 1)
    if a1.shape != a2.shape or dv * rows != a1.numel():
        raise ValueError("om numerators disagree")
    m, l, a = torch.empty_like(m1), torch.empty_like(l1), torch.empty_like(a1)
    st = lib.catopt_hip_om_compose(rows, dv, _ptr(m1), _ptr(l1), _ptr(a1), _ptr(m2), _ptr(l2),
                                   _ptr(a2), _ptr(m), _ptr(l), _ptr(a), _stream(m1))
    L.check("catopt_hip_om_compose", st)
    return m, l, a


# ----------------------------------------------------------------- retention

RETENTION_CHUNK = 64
RETENTION_HEAD_DIM = 128


def retention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, gamma: torch.Tensor,
              scale: float = 1.0) -> torch.Tensor:
    """``scale * Σ_{s<=t} γ_h^(t-s) (q_t·k_s) v_s`` for ``q, k (B,H,T,dk)``,
    ``v (B,H,T,dv)``, all bf16, fp32 or fp16 (widened to fp32), ``dk, dv <=
    128``.  The kernels
    read a head dim ``d`` (a multiple of 8 for bf16, of 4 for fp32) and any
    ``T`` in place: columns past ``d`` and rows past ``T`` of the 64-step
    chunks load as zeros and are never stored.  When ``dk`` and ``dv``
    differ, or are not such multiples, the narrower operands run zero-padded
    to the common width (zero columns leave q·k unchanged and add zero output
    columns, dropped).  fp32 operands compute in fp32 throughout."""
    _need_device(q, k, v, gamma)
    lib = L.load()
    if q.dtype == torch.float16 and k.dtype == q.dtype and v.dtype == q.dtype:
        # fp16: the fp32 kernel on widened operands, the output rounded back
        return retention(q.float(), k.float(), v.float(), gamma, scale).to(torch.float16)
    if q.dtype not in (torch.bfloat16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise NotImplementedError("HIP retention runs on bf16, fp32 or fp16 operands")
    if q.dim() != 4 or q.shape != k.shape or v.dim() != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError("retention operands must be q, k (B, H, T, dk) and v (B, H, T, dv)")
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    if max(dk, dv) > RETENTION_HEAD_DIM:
        raise NotImplementedError(f"HIP retention needs dk, dv <= {RETENTION_HEAD_DIM}")
    if T == 0 or B * H == 0:
        return torch.zeros_like(v)
    step = 4 if q.dtype == torch.float32 else 8
    d = -(-max(dk, dv, step) // step) * step
    if dk != d or dv != d:
        pad = torch.nn.functional.pad
        q, k = (pad(t, (0, d - dk)) for t in (q, k))
        v = pad(v, (0, d - dv))
        return retention(q, k, v, gamma, scale)[..., :dv]
    g = gamma.to(torch.float32).reshape(-1).contiguous()
    if g.numel() != H:
        raise ValueError("gamma must hold one rate per head")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    o = torch.empty_like(v)
    dt = L.F32 if q.dtype == torch.float32 else L.BF16
    wsb = 0  # the fp32 kernel keeps its state in registers and takes no workspace
    if dt == L.BF16:
        wsb = lib.catopt_hip_retention_workspace_bytes(B, H, T, d, RETENTION_CHUNK)
        if wsb < 0:
            raise ValueError("retention workspace query rejected the shape")
    ws = _workspace(wsb, q.device)
    st = lib.catopt_hip_retention_fwd(dt, B, H, T, d, RETENTION_CHUNK, _ptr(q), _ptr(k),
                                      _ptr(v), _ptr(g), float(scale), _ptr(o), _ptr(ws), wsb,
                                      _stream(q))
    L.check("catopt_hip_retention_fwd", st)
    return o


def decay(gamma: torch.Tensor, t: int) -> torch.Tensor:
    """``decay(γ, t)`` on device, fp32, shape ``(*γ.shape, t, t)``."""
    _need_device(gamma)
    lib = L.load()
    g = gamma.to(torch.float32).reshape(-1).contiguous()
    out = torch.empty((g.numel(), t, t), dtype=torch.float32, device=g.device)
    L.check("catopt_hip_decay", lib.catopt_hip_decay(g.numel(), t, _ptr(g), _ptr(out), _stream(g)))
    return out.reshape(*gamma.shape, t, t)


def decay_vec(gamma: torch.Tensor, t: int, offset: int = 0, sign: int = 1) -> torch.Tensor:
    """``decay_vec(γ, t, offset, sign)`` on device, fp32, shape ``(*γ.shape, t)``."""
    _need_device(gamma)
    lib = L.load()
    g = gamma.to(torch.float32).reshape(-1).contiguous()
    out = torch.empty((g.numel(), t), dtype=torch.float32, device=g.device)
    L.check("catopt_hip_decay_vec",
            lib.catopt_hip_decay_vec(g.numel(), t, int(offset), int(sign), _ptr(g), _ptr(out), _stream(g)))
    return out.reshape(*gamma.shape, t)


# ---------------------------------------------------------------------- scans


def _validate_starts(chunk_starts, T: int) -> tuple[int, ...]:
    if isinstance(chunk_starts, torch.Tensor):
        chunk_starts = chunk_starts.detach().cpu().tolist()
    vals = tuple(int(c) for c in chunk_starts)
    if len(vals) < 2:
        raise ValueError("chunk table needs at least [0, T]")
    if vals[0] != 0 or vals[-1] != T or (T > 0 and any(b <= a for a, b in zip(vals, vals[1:]))):
        raise ValueError(f"chunk table must rise strictly from 0 to T={T}")
    return vals


class ChunkTable:
    """A chunk table validated once, holding one int64 device copy per device.

    The kernels index the steps with it, so it is checked on the host when
    built.  The device copies live as long as this object: an executor keeps
    its table in its plan, so a hipGraph that recorded a launch reading a
    copy can never outlive it."""

    __slots__ = ("starts", "T", "_dev")

    def __init__(self, chunk_starts, T: int) -> None:
        self.starts = _validate_starts(chunk_starts, T)
        self.T = int(T)
        self._dev: dict = {}

    @property
    def n_chunks(self) -> int:
        return len(self.starts) - 1

    def on(self, device) -> torch.Tensor:
        key = str(device)
        cs = self._dev.get(key)
        if cs is None:
            cs = torch.tensor(self.starts, dtype=torch.int64).to(device)
            self._dev[key] = cs
        return cs


# Tables passed as plain sequences: cached per (table, device) and never
# evicted, since a graph recorded around such a call holds the device
# pointer.  Past the cap, a new table is uploaded per call (and a graph
# capture of that call fails loudly on the host-to-device copy instead of
# replaying a freed table).
_TABLES: dict = {}
_TABLES_CAP = 4096


def _chunk_table(chunk_starts, T: int, device) -> tuple[torch.Tensor, int]:
    """The validated int64 chunk table on ``device`` and its chunk count."""
    if isinstance(chunk_starts, ChunkTable):
        if chunk_starts.T != T:
            raise ValueError(f"chunk table spans {chunk_starts.T} steps, the scan has {T}")
        return chunk_starts.on(device), chunk_starts.n_chunks
    key_vals = _validate_starts(chunk_starts, T)
    key = (key_vals, str(device))
    cs = _TABLES.get(key)
    if cs is None:
        cs = torch.tensor(key_vals, dtype=torch.int64).to(device)
        if len(_TABLES) < _TABLES_CAP:
            _TABLES[key] = cs
    return cs, len(key_vals) - 1


def _workspace(nbytes: int, device) -> torch.Tensor | None:
    """Caller workspace for a launch that reads ``nbytes`` (none when 0)."""
    if nbytes == 0:
        return None
    return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=device)


def affd_scan(a: torch.Tensor, u: torch.Tensor, h0: torch.Tensor | None,
              chunk_starts, *, schedule: int = L.SCAN_AUTO, states: bool = True):
    """Diagonal affine scan over the leading axis: ``h_t = a_t h_{t-1} + u_t``.

    ``a`` is ``(T, *S)`` or ``(*S)`` (shared over steps), ``u`` is ``(T, *S)``.
    Returns ``(states (T, *S) or None, h_final (*S))`` in fp32.
    """
    _need_device(a, u, h0)
    lib = L.load()
    T = u.shape[0]
    sshape = u.shape[1:]
    S = math.prod(sshape)
    u2 = u.to(torch.float32).reshape(T, S).contiguous()
    if a.shape == sshape:
        a2, lda = a.to(torch.float32).reshape(1, S).contiguous(), 0
    elif a.shape == u.shape:
        a2, lda = a.to(torch.float32).reshape(T, S).contiguous(), S
    else:
        raise ValueError(f"scan a{tuple(a.shape)} does not fit u{tuple(u.shape)}")
    h = h0.to(torch.float32).reshape(S).contiguous() if h0 is not None else None
    cs, nc = _chunk_table(chunk_starts, T, u.device)
    out = torch.empty((T, S), dtype=torch.float32, device=u.device) if states else None
    hf = torch.empty((S,), dtype=torch.float32, device=u.device)
    wsb = lib.catopt_hip_affd_scan_workspace_bytes(T, S, nc, int(schedule))
    if wsb < 0:
        raise ValueError("affd scan workspace query rejected the call")
    ws = _workspace(wsb, u.device)
    st = lib.catopt_hip_affd_scan(T, S, _ptr(a2), lda, _ptr(u2), S, _ptr(h), _ptr(cs), nc,
                                  int(schedule), _ptr(out), _ptr(hf), _ptr(ws), wsb, _stream(u))
    L.check("catopt_hip_affd_scan", st)
    return (out.reshape(T, *sshape) if out is not None else None), hf.reshape(sshape)


def _rows3(t: torch.Tensor, nb: int, rows: int, cols: int) -> tuple:
    """``t`` as fp32 ``(nb, rows, cols)`` with unit column stride — a view
    when the leading axes collapse to one stride, else a contiguous copy —
    and its batch and row strides (elements, both non-negative, the row
    stride at least ``cols``)."""
    t3 = t.to(torch.float32).reshape(nb, rows, cols)
    sb, ld = t3.stride(0), t3.stride(1)
    if rows <= 1:
        ld = cols  # the row stride is never applied
    if nb <= 1:
        sb = 0
    if t3.stride(2) != 1 or sb < 0 or ld < cols:
        t3 = t3.contiguous()
        sb, ld = (rows * cols if nb > 1 else 0), cols
    return t3, sb, ld


def attn_carrier_f32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float = 1.0, *,
                     causal: bool = False, causal_off: int = 0, mask: torch.Tensor | None = None,
                     bias: torch.Tensor | None = None) -> tuple:
    """The om element of ``s = scale · q kᵀ`` over values ``v`` in fp32:
    ``(m (…,Tq,1), l (…,Tq,1), a (…,Tq,dv))``, ``dk ≤ 128``, ``dv ≤ 256``.
    ``k (…,Tk,dk)``; ``q (…,Tq,dk)`` or ``(Tq,dk)`` and ``v (…,Tk,dv)`` or
    ``(Tk,dv)``, a 2-D operand shared over the leading axes.

    The mask keywords are :func:`attention`'s: ``causal`` keeps key ``j``
    for query ``i`` iff ``j <= i + causal_off``; ``mask`` is a bool keep
    plane and ``bias`` an additive float plane (added to the scaled score),
    each ``(Tq, Tk)`` and shared over the leading axes.  Rows with every key
    masked get the empty carrier ``(-inf, 0, 0)``."""
    _need_device(q, k, v, mask, bias)
    lib = L.load()
    lead = tuple(k.shape[:-2])
    Tq, dk = q.shape[-2], q.shape[-1]
    Tk, dv = k.shape[-2], v.shape[-1]
    if k.shape[-1] != dk or v.shape[-2] != Tk or (q.dim() > 2 and tuple(q.shape[:-2]) != lead) or \
            (v.dim() > 2 and tuple(v.shape[:-2]) != lead):
        raise ValueError(f"attn_carrier_f32: q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)} do not fit")
    nb = math.prod(lead) if lead else 1
    # operands are read in place through (batch, row) strides: a key block cut
    # from a longer sequence is not copied
    q3, q_sb, ldq = _rows3(q, 1 if q.dim() == 2 else nb, Tq, dk)
    k3, k_sb, ldk = _rows3(k, nb, Tk, dk)
    v3, v_sb, ldv = _rows3(v, 1 if v.dim() == 2 else nb, Tk, dv)
    if q.dim() == 2:  # one query block shared by every key block
        q_sb = 0
    if v.dim() == 2:
        v_sb = 0
    if (mask is not None) + (bias is not None) + bool(causal) > 1:
        raise ValueError("pass at most one of causal=True, mask, bias")
    mode, plane, mask_ld = L.MASK_NONE, None, 0
    if mask is not None or bias is not None:
        t = mask if mask is not None else bias
        if t.shape[-2:] != (Tq, Tk) or t.numel() != Tq * Tk:
            raise NotImplementedError(f"the mask plane must be ({Tq}, {Tk}) shared over the leading axes, "
                                      f"got {tuple(t.shape)}")
        if mask is not None:
            plane, mode = mask.reshape(Tq, Tk).to(torch.uint8).contiguous(), L.MASK_BOOL
        else:
            plane, mode = bias.reshape(Tq, Tk).to(torch.float32).contiguous(), L.MASK_BIAS
        mask_ld = Tk
    elif causal:
        mode = L.MASK_CAUSAL
    m = torch.empty((nb, Tq), dtype=torch.float32, device=q.device)
    lv = torch.empty((nb, Tq), dtype=torch.float32, device=q.device)
    a = torch.empty((nb, Tq, dv), dtype=torch.float32, device=q.device)
    st = lib.catopt_hip_attn_carrier_f32_masked(nb, Tq, Tk, dk, dv, _ptr(q3), q_sb, ldq, _ptr(k3), k_sb, ldk,
                                                _ptr(v3), v_sb, ldv, float(scale), mode, int(causal_off),
                                                _ptr(plane), mask_ld, _ptr(m), _ptr(lv), _ptr(a), Tq * dv, dv,
                                                _stream(q))
    L.check("catopt_hip_attn_carrier_f32_masked", st)
    return m.reshape(*lead, Tq, 1), lv.reshape(*lead, Tq, 1), a.reshape(*lead, Tq, dv)


def omd_fold_apply(m: torch.Tensor, lv: torch.Tensor, num: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    """The om combine of ``L`` carriers over axis 0 followed by the diagonal
    readout ``(fa ⊙ h + fb) / l`` (``fused_omd_levels``, om_fused.py:151-164),
    one pass: ``m, lv (L, Tq[, 1])``, ``num (L, Tq, 2d)`` = ``[fa | fb]``,
    ``h (d,)``, all fp32 on the device; returns ``(Tq, d)`` fp32."""
    _need_device(m, lv, num, h)
    lib = L.load()
    Lc, Tq, W = num.shape
    d = h.shape[-1]
    if h.dim() != 1 or W != 2 * d or m.numel() != Lc * Tq or lv.numel() != Lc * Tq or \
            any(t.dtype != torch.float32 for t in (m, lv, num, h)):
        raise ValueError(f"omd_fold_apply: m{tuple(m.shape)} l{tuple(lv.shape)} num{tuple(num.shape)} "
                         f"h{tuple(h.shape)} do not fit")
    m2, l2, h1, num = m.reshape(Lc, Tq).contiguous(), lv.reshape(Lc, Tq).contiguous(), h.contiguous(), \
        num.contiguous()
    out = torch.empty((Tq, d), dtype=torch.float32, device=num.device)
    st = lib.catopt_hip_omd_fold_apply(Lc, Tq, d, _ptr(m2), _ptr(l2), _ptr(num), num.stride(1), num.stride(0),
                                       _ptr(h1), _ptr(out), _stream(num))
    L.check("catopt_hip_omd_fold_apply", st)
    return out


def aff_scan(A: torch.Tensor, b: torch.Tensor, h0: torch.Tensor, chunk_starts, *,
             schedule: int = L.SCAN_AUTO, states: bool = True):
    """Dense affine scan over the leading axis: ``X_t = A_t X_{t-1} + b_t 1ᵀ``.

    ``A`` is ``(TA, PA, d, d)`` with ``TA`` in {1, T} (1: one map for every
    step) and ``PA`` in {1, P} (1: one map for every slot); ``b`` is
    ``(T, PB, d)`` with ``PB`` in {1, P}; ``h0`` is the ``(P, d, k)`` initial
    state.  Returns ``(states (T, P, d, k) or None, h_final (P, d, k))`` in
    fp32.
    """
    _need_device(A, b, h0)
    lib = L.load()
    if A.dim() != 4 or b.dim() != 3 or h0.dim() != 3:
        raise ValueError("aff_scan wants A (TA, PA, d, d), b (T, PB, d), h0 (P, d, k)")
    T, PB, d = b.shape
    P, dh, k = h0.shape
    TA, PA = A.shape[0], A.shape[1]
    if A.shape[2:] != (d, d) or dh != d or TA not in (1, T) or PA not in (1, P) or PB not in (1, P):
        raise ValueError(f"aff_scan shapes do not fit: A{tuple(A.shape)} b{tuple(b.shape)} h0{tuple(h0.shape)}")
    f = lambda t: t.to(torch.float32).contiguous()  # noqa: E731
    A2, b2, h2 = f(A), f(b), f(h0)
    lda_t = d * d * PA if TA > 1 else 0
    lda_p = d * d if PA > 1 else 0
    ldb_t = d * PB
    ldb_p = d if PB > 1 else 0
    cs, nc = _chunk_table(chunk_starts, T, b.device)
    out = torch.empty((T, P, d, k), dtype=torch.float32, device=b.device) if states else None
    hf = torch.empty((P, d, k), dtype=torch.float32, device=b.device)
    wsb = lib.catopt_hip_aff_scan_workspace_bytes(P, d, k, int(lda_p == 0), nc)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=b.device)
    st = lib.catopt_hip_aff_scan(T, P, d, k, _ptr(A2), lda_t, lda_p, _ptr(b2), ldb_t, ldb_p, _ptr(h2),
                                 _ptr(cs), nc, int(schedule), _ptr(out), _ptr(hf), _ptr(ws), wsb, _stream(b))
    L.check("catopt_hip_aff_scan", st)
    return out, hf


def compose_slots(A: torch.Tensor, B: torch.Tensor, f: torch.Tensor, g: torch.Tensor, out0: int,
                  domain: str) -> None:
    """One level of a compose forest, in place: slot ``out0 + j`` of the
    contiguous fp32 slot arrays becomes ``compose(slot f[j], slot g[j])``
    (``g`` applied first).  ``domain`` "diag": ``A`` and ``B`` are
    ``(n_slots, *shape)`` of one shape; "dense": ``A`` is
    ``(n_slots, *P, d, d)`` and ``B`` is ``(n_slots, *P, d)``.  ``f`` and
    ``g`` are device int64 slot indices, each below ``out0``."""
    _need_device(A, B, f, g)
    lib = L.load()
    if A.dtype != torch.float32 or B.dtype != torch.float32 or not (A.is_contiguous() and B.is_contiguous()):
        raise ValueError("compose_slots wants contiguous fp32 slot arrays")
    if f.dtype != torch.long or g.dtype != torch.long or f.shape != g.shape or f.dim() != 1:
        raise ValueError("compose_slots wants two int64 index vectors of one length")
    n, Lv = A.shape[0], f.shape[0]
    if B.shape[0] != n or not 1 <= out0 <= n or out0 + Lv > n:
        raise ValueError(f"compose_slots: {Lv} outputs from slot {out0} do not fit {n} slots")
    if domain == "diag":
        if A.shape != B.shape:
            raise ValueError("diagonal slot arrays differ in shape")
        st = lib.catopt_hip_affd_compose_slots(n, A[0].numel(), _ptr(A), _ptr(B), _ptr(f), _ptr(g), Lv, out0,
                                               _stream(A))
        L.check("catopt_hip_affd_compose_slots", st)
        return
    d = A.shape[-1]
    if A.dim() < 3 or A.shape[-2] != d or B.shape != A.shape[:-1]:
        raise ValueError("dense slot arrays are not square maps with matching offsets")
    P = int(torch.Size(A.shape[1:-2]).numel())
    st = lib.catopt_hip_aff_compose_slots(n, P, d, _ptr(A), _ptr(B), _ptr(f), _ptr(g), Lv, out0, _stream(A))
    L.check("catopt_hip_aff_compose_slots", st)


def ssm_scan(a: torch.Tensor, bx: torch.Tensor, c: torch.Tensor, x: torch.Tensor,
             h0: torch.Tensor | None, chunk_starts, *, schedule: int = L.SCAN_AUTO,
             return_state: bool = False):
    """Selective diagonal SSM with fused input/readout, fp32.

    ``a`` (B,T,D,N) or (B,T,D); ``bx``, ``c`` (B,T,N); ``x`` (B,T,D);
    ``h0`` (B,D,N) or None.  Returns ``y`` (B,T,D) [and ``h_T`` (B,D,N)].
    """
    _need_device(a, bx, c, x, h0)
    lib = L.load()
    B, T, D = x.shape
    N = bx.shape[-1]
    if bx.shape != (B, T, N) or c.shape != (B, T, N):
        raise ValueError("bx and c must be (B, T, N)")
    if a.shape == (B, T, D, N):
        aps = 1
    elif a.shape == (B, T, D):
        aps = 0
    else:
        raise ValueError(f"a must be (B,T,D,N) or (B,T,D), got {tuple(a.shape)}")
    if N not in (4, 8, 16, 32, 64):
        raise NotImplementedError(f"HIP SSM scan supports N in (4, 8, 16, 32, 64), got {N}")
    f = lambda t: None if t is None else t.to(torch.float32).contiguous()  # noqa: E731
    a, bx, c, x, h0 = f(a), f(bx), f(c), f(x), f(h0)
    if h0 is not None and h0.shape != (B, D, N):
        raise ValueError("h0 must be (B, D, N)")
    cs, nc = _chunk_table(chunk_starts, T, x.device)
    y = torch.empty((B, T, D), dtype=torch.float32, device=x.device)
    hf = torch.empty((B, D, N), dtype=torch.float32, device=x.device) if return_state else None
    wsb = lib.catopt_hip_ssm_scan_workspace_bytes(B, T, D, N, nc, int(schedule))
    if wsb < 0:
        raise ValueError("SSM scan workspace query rejected the call")
    ws = _workspace(wsb, x.device)
    st = lib.catopt_hip_ssm_scan(B, T, D, N, _ptr(a), aps, _ptr(bx), _ptr(c), _ptr(x), _ptr(h0),
                                 _ptr(cs), nc, int(schedule), _ptr(y), _ptr(hf), _ptr(ws), wsb,
                                 _stream(x))
    L.check("catopt_hip_ssm_scan", st)
    return (y, hf) if return_state else y


# --------------------------------------------------------------- elementwise


def silu(x: torch.Tensor) -> torch.Tensor:
    _need_device(x)
    lib = L.load()
    xc = x.contiguous()
    y = torch.empty_like(xc)
    L.check("catopt_hip_silu", lib.catopt_hip_silu(_dtype_code(x), xc.numel(), _ptr(xc), _ptr(y), _stream(x)))
    return y


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    _need_device(g, u)
    lib = L.load()
    if g.shape != u.shape or g.dtype != u.dtype:
        g, u = torch.broadcast_tensors(g, u)
    gc, uc = g.contiguous(), u.contiguous()
    y = torch.empty_like(gc)
    L.check("catopt_hip_silu_mul",
            lib.catopt_hip_silu_mul(_dtype_code(gc), gc.numel(), _ptr(gc), _ptr(uc), _ptr(y), _stream(g)))
    return y


def hbm_read(buf: torch.Tensor, sink: torch.Tensor) -> None:
    """Read every byte of a contiguous device buffer once (the read-only HBM
    stream; ``sink`` is a 4-byte device scratch)."""
    _need_device(buf, sink)
    lib = L.load()
    if not buf.is_contiguous() or sink.numel() * sink.element_size() < 4:
        raise ValueError("hbm_read takes a contiguous buffer and a 4-byte sink")
    nbytes = buf.numel() * buf.element_size()
    st = lib.catopt_hip_hbm_read(_ptr(buf), nbytes - nbytes % 16, _ptr(sink), _stream(buf))
    L.check("catopt_hip_hbm_read", st)
