"""numpy restatement of the reference's delivered-form arithmetic (test oracle).

Reference paths are relative to luisfuturist/catopt.  Arrays are numpy; the
caller chooses the precision by the dtype it passes (tests use float64 for
law-level checks and float32 for parity against bf16/fp32 kernels).
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "verify_equiv",
    "rms_norm",
    "linear",
    "linear_chain",
    "fold_linear_chain",
    "folded_chain_forward",
    "silu",
    "swiglu_fused",
    "swiglu_unfused",
    "cmask_keep",
    "om_elem",
    "om_compose",
    "om_apply",
    "fused_om_levels",
    "attention_om",
    "attention_dense",
    "decay",
    "decay_vec",
    "kway_plan",
    "kway_pair_tables",
    "retention_kway",
    "retention_quadratic",
    "affd_compose",
    "fused_diag_levels",
    "prefix_plan",
    "prefix_chunk_table",
    "prefix_scan",
    "serial_affd_scan",
    "ssm_serial",
    "ssm_chunked",
    "aff_compose",
    "aff_apply",
    "aff_homogeneous",
    "fused_dense_levels",
    "serial_aff_scan",
    "aff_chunked_scan",
    "omd_elem",
    "omd_compose",
    "omd_apply",
    "omd_applym",
]

_REL_FLOOR = 1e-8


# ---------------------------------------------------------------- verify gate


def verify_equiv(ref, out, rtol: float = 1e-4, atol: float | None = None) -> dict:
    """The verify gate: ``max|ref-out| / (max|ref| + 1e-8) < rtol``.

    Follows report.py:128-140 (``_verify_pair``) — a *global* relative error,
    NaN anywhere makes ``max_abs`` NaN and the gate fail.
    """
    ref = np.asarray(ref, dtype=np.float64)
    out = np.asarray(out, dtype=np.float64)
    diff = np.abs(ref - out)
    max_abs = float(np.max(diff)) if diff.size else 0.0
    if diff.size and np.isnan(diff).any():
        max_abs = float("nan")
    denom = float(np.max(np.abs(ref))) if ref.size else 0.0
    max_rel = max_abs / (denom + _REL_FLOOR)
    passed = bool(max_rel < rtol) and (atol is None or bool(max_abs <= atol))
    return {"max_abs": max_abs, "max_rel": max_rel, "passed": passed}


# ---------------------------------------------------------------- norms / GEMM


def rms_norm(x, w=None, eps: float = 1e-6):
    """``x · rsqrt(mean(x², -1) + eps) · w`` — the "rms_norm" binding
    (torch_bridge.py:1404-1411 → F.rms_norm) that RMS_NORM_FOLD's RHS
    (laws/tensor.py:734-741) delivers for the RMSNorm model
    (models/__init__.py:41-55)."""
    x = np.asarray(x)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    y = x * r
    return y * w if w is not None else y


def linear(x, W, b=None):
    """``x @ Wᵀ + b`` — the "linear" binding (torch_bridge.py:1251-1253)."""
    y = np.asarray(x) @ np.asarray(W).T
    return y + b if b is not None else y


def linear_chain(x, Ws, bs):
    """The un-optimised weight chain: ``linear(…linear(x, W1, b1)…, WL, bL)``
    (8 stacked nn.Linear: the C1 weight-chain workload)."""
    h = x
    for W, b in zip(Ws, bs):
        h = linear(h, W, b)
    return h


def fold_linear_chain(Ws, bs):
    """Fold the chain by repeated ASSOC_LINEAR_BIAS (laws/tensor.py:1374-1394):
    ``linear(linear(x,A,b1),B,b2) → add(linear(x, B@A, B@b1), b2)``.

    Innermost pair first: after step i the delivered form is
    ``add(…add(linear(x, W_eff, c_0), c_1)…, c_i)`` where every ``matmul``
    of Params is folded at construction (IRModule._fold_weight_chains,
    torch_bridge.py:2451-2476).  Returns ``(W_eff, [c_0, c_1, …])`` — the
    fused weight and the ordered bias addends of the delivered form.
    """
    W = np.asarray(Ws[0])
    adds = [np.asarray(bs[0])]
    for B, b2 in zip(Ws[1:], bs[1:]):
        B = np.asarray(B)
        W = B @ W
        # every earlier addend is pushed through the new layer: B·c
        adds = [B @ c for c in adds]
        adds.append(np.asarray(b2))
    return W, adds


def folded_chain_forward(x, W_eff, adds):
    """Delivered form of the folded chain: one GEMM, then the bias adds
    in term order (the add spine of the ASSOC_LINEAR_BIAS RHS)."""
    y = linear(x, W_eff, adds[0])
    for c in adds[1:]:
        y = y + c
    return y


def silu(x):
    """``x · σ(x)`` — the "silu" binding (torch_bridge.py:1159)."""
    return x / (1.0 + np.exp(-x))


def swiglu_fused(x, W_gate, W_up, W_down):
    """SWIGLU_FUSE's RHS (laws/tensor.py:1485-1519) then the down projection:
    ``y = linear(x, concat(A, B, dim=0))``;
    ``h = mul(silu(chunk(y, 2, -1, 0)), chunk(y, 2, -1, 1))``;
    ``out = linear(h, W_down)`` (chunk binding torch_bridge.py:1310-1314)."""
    Wcat = np.concatenate([W_gate, W_up], axis=0)
    y = linear(x, Wcat)
    d = y.shape[-1] // 2
    g, u = y[..., :d], y[..., d:]
    return linear(silu(g) * u, W_down)


def swiglu_unfused(x, W_gate, W_up, W_down):
    """The source module: ``down(silu(gate(x)) * up(x))`` (models/__init__.py:22-38)."""
    return linear(silu(linear(x, W_gate)) * linear(x, W_up), W_down)


# ---------------------------------------------------------------- online softmax


def cmask_keep(t: int, k: int, off: int = 0):
    """Keep-mask of the causal ``cmask`` generator (om.py:1023-1029):
    ``keep = ones(t, k).tril(-off)`` — key ``j`` kept for row ``i`` iff
    ``j <= i - off`` (the binding's ``off`` is the masked set's shift)."""
    i = np.arange(t)[:, None]
    j = np.arange(k)[None, :]
    return j <= i - off


def om_elem(s, v):
    """``_om_elem`` (torch_bridge.py:1974-1981): ``(rowmax s, Σ exp(s-m), exp(s-m) @ v)``."""
    with np.errstate(invalid="ignore"):
        m = np.max(s, axis=-1, keepdims=True)
        e = np.exp(s - m)
    return m, e.sum(axis=-1, keepdims=True), e @ v


def om_compose(f, g):
    """``_om_compose`` (torch_bridge.py:1984-2006): the FlashAttention merge with
    the ``isfinite`` guards (a fully masked block contributes 0, not NaN)."""
    m1, l1, a1 = f
    m2, l2, a2 = g
    mx = np.maximum(m1, m2)
    fin1, fin2 = np.isfinite(m1), np.isfinite(m2)
    with np.errstate(invalid="ignore"):
        e1 = np.where(fin1, np.exp(m1 - mx), 0.0)
        e2 = np.where(fin2, np.exp(m2 - mx), 0.0)
        lv = np.where(fin1, l1 * e1, 0.0) + np.where(fin2, l2 * e2, 0.0)
        a = np.where(fin1, a1 * e1, 0.0) + np.where(fin2, a2 * e2, 0.0)
    return mx, lv, a


def om_apply(f):
    """"om_apply" binding (torch_bridge.py:1890): ``a / l`` UNCLAMPED — a fully
    masked row gives 0/0 = NaN, as dense softmax does."""
    with np.errstate(invalid="ignore", divide="ignore"):
        return f[2] / f[1]


def _pad_pow2(t, fill):
    """``_pad_to_pow2`` (scan_fused.py:85-97): identity rows up to a power of 2."""
    n = t.shape[0]
    pad = (1 << max(n - 1, 0).bit_length()) - n
    if not pad:
        return t
    return np.concatenate([t, np.full((pad, *t.shape[1:]), fill, dtype=t.dtype)])


def fused_om_levels(m_seq, l_seq, a_seq):
    """``fused_om_levels`` (om_fused.py:65-96): identity-pad to a power of two,
    sanitise leaves once (non-finite m ⇒ l = a = 0), then adjacent-pair
    combine levels, reading out ``a/l``."""
    m = _pad_pow2(np.asarray(m_seq), -np.inf)
    lv = _pad_pow2(np.asarray(l_seq), 0.0)
    a = _pad_pow2(np.asarray(a_seq), 0.0)
    fin = np.isfinite(m)
    lv = np.where(fin, lv, 0.0)
    a = np.where(fin, a, 0.0)
    while m.shape[0] > 1:
        m1, m2 = m[0::2], m[1::2]
        mx = np.maximum(m1, m2)
        with np.errstate(invalid="ignore"):
            e1 = np.where(np.isfinite(m1), np.exp(m1 - mx), 0.0)
            e2 = np.where(np.isfinite(m2), np.exp(m2 - mx), 0.0)
        lv = lv[0::2] * e1 + lv[1::2] * e2
        a = a[0::2] * e1 + a[1::2] * e2
        m = mx
    with np.errstate(invalid="ignore", divide="ignore"):
        return a[0] / lv[0]


def attention_om(q, k, v, scale: float, *, causal: bool = True, causal_off: int = 0,
                 mask=None, block: int | None = None, return_ml: bool = False):
    """The OM_LIFT delivered form (om.py:153-193) over key blocks:

    ``s = masked_fill(scale · q kᵀ, ¬keep, -inf)`` (masked_fill binding
    torch_bridge.py:1864; causal keep ``j <= i + causal_off``, i.e. the
    cmask of om.py:1023-1029 with ``off = -causal_off``), split along keys
    into blocks (OM_SPLIT), one ``om_elem`` per block, combined by
    ``fused_om_levels`` (om_fused.py:65-96), read out by ``om_apply``.
    ``block=None`` is the single-leaf form.  Shapes ``(..., T, d)``.
    """
    q, k, v = (np.asarray(t) for t in (q, k, v))
    Tq, Tk = q.shape[-2], k.shape[-2]
    s = scale * (q @ np.swapaxes(k, -1, -2))
    if causal:
        keep = cmask_keep(Tq, Tk, -causal_off)
    elif mask is not None:
        keep = np.asarray(mask, dtype=bool)
    else:
        keep = np.ones((Tq, Tk), dtype=bool)
    s = np.where(keep, s, -np.inf)
    blk = Tk if block is None else block
    leaves = [om_elem(s[..., j:j + blk], v[..., j:j + blk, :]) for j in range(0, Tk, blk)]
    m_seq = np.stack([lf[0] for lf in leaves])
    l_seq = np.stack([lf[1] for lf in leaves])
    a_seq = np.stack([lf[2] for lf in leaves])
    out = fused_om_levels(m_seq, l_seq, a_seq)
    if not return_ml:
        return out
    f = leaves[0]
    for g in leaves[1:]:
        f = om_compose(f, g)
    return out, f[0], f[1]


def attention_dense(q, k, v, scale: float, keep):
    """Source-module attention ``softmax(masked_fill(scale q kᵀ)) @ v``
    (models/__init__.py:952-981 TrilCausalAttention's arithmetic)."""
    s = scale * (np.asarray(q) @ np.swapaxes(np.asarray(k), -1, -2))
    s = np.where(keep, s, -np.inf)
    with np.errstate(invalid="ignore"):
        m = np.max(s, axis=-1, keepdims=True)
        e = np.exp(s - m)
        return (e / e.sum(axis=-1, keepdims=True)) @ np.asarray(v)


# ---------------------------------------------------------------- retention


def decay(g, t: int):
    """``_decay_torch`` (om.py:1060-1072): ``tril(γ^(i-j))`` on the last two
    axes, γ's dims leading; ``diff.clamp_min(0)`` before the power."""
    g = np.asarray(g)
    pos = np.arange(t, dtype=g.dtype)
    diff = np.maximum(pos[:, None] - pos[None, :], 0)
    return np.tril(g[..., None, None] ** diff)


def decay_vec(g, t: int, offset: int = 0, sign: int = 1):
    """``_decay_vec_torch`` (om.py:1075-1089): ``γ^(sign·k + offset)``, k in [0,t)
    (``sign = 0`` is legal: the constant γ^offset)."""
    g = np.asarray(g)
    pos = np.arange(t, dtype=g.dtype)
    return g[..., None] ** (pos * sign + offset)


def kway_plan(T: int, K: int) -> dict:
    """Integer plan of ``om_decayed_kway_blocks(K)`` (om.py:3040-3075):
    ``C = T // K``, ``SZ = (C,)*K``, ``OFF_i_j = (i-j)·C`` for ``j < i``.
    ``None`` when the check rejects the shape (``T < K`` or ``T % K``)."""
    if not isinstance(T, int) or T < K or T % K:
        return None
    C = T // K
    off = {(i, j): (i - j) * C for i in range(K) for j in range(i)}
    return {"C": C, "SZ": (C,) * K, "OFF": off}


def kway_pair_tables(K: int) -> dict:
    """The pair schedule ChunkedDecayModule builds from the K-way term
    (decayed_lower.py:304-368 ``_cross_tables``/``_assemble_plan``): pairs in
    arm order (target chunk i ascending, source j ascending), with the
    deduplicated q / state-half indices and per-chunk pair counts."""
    q_idx, m_idx = [], []
    qseen, mseen = {}, {}
    counts = []
    for i in range(K):
        counts.append(i)
        for j in range(i):
            qi = qseen.setdefault(i, len(qseen))  # q_i first seen at its first cross
            mj = mseen.setdefault(j, len(mseen))
            q_idx.append(qi)
            m_idx.append(mj)
    return {
        "q_idx": np.asarray(q_idx, dtype=np.int64),
        "m_idx": np.asarray(m_idx, dtype=np.int64),
        "pair_counts": np.asarray(counts, dtype=np.int64),
        "n_pairs": K * (K - 1) // 2,
    }


def retention_kway(q, k, v, g, K: int, scale: float = 1.0):
    """The K-way delivered form, evaluated block by block as its RHS spells it
    (om.py:3100-3160, bindings om.py:1053-1089):

    ``out_i = om_decayed(s_ii, decay(γ, C), v_i)
             + Σ_{j<i} unsq(decay_vec(γ,C,offset=OFF_i_j),-1) ⊙ ((s_ij ⊙ unsq(decay_vec(γ,C,sign=-1),-2)) @ v_j)``

    with ``s = q kᵀ`` split into ``(C,)*K`` blocks, scaled by ``scale`` (the
    ``/S`` divisor of ChunkedDecayModule, decayed_lower.py:609-639), and the
    row blocks concatenated.  Shapes: q, k, v ``(..., H, T, d)``, γ ``(H,)``.
    """
    q, k, v = (np.asarray(t) for t in (q, k, v))
    T = q.shape[-2]
    plan = kway_plan(T, K)
    if plan is None:
        raise ValueError(f"T={T} is not a uniform {K}-way partition")
    C = plan["C"]
    g = np.asarray(g)
    d_intra = decay(g, C)                                 # (H, C, C)
    eta = decay_vec(g, C, 0, -1)[..., None, :]            # unsq(-2): (H, 1, C)
    outs = []
    for i in range(K):
        qi = q[..., i * C:(i + 1) * C, :]
        s_ii = qi @ np.swapaxes(k[..., i * C:(i + 1) * C, :], -1, -2)
        acc = (s_ii * d_intra) @ v[..., i * C:(i + 1) * C, :]
        for j in range(i):
            s_ij = qi @ np.swapaxes(k[..., j * C:(j + 1) * C, :], -1, -2)
            xi = decay_vec(g, C, plan["OFF"][(i, j)], 1)[..., :, None]  # unsq(-1): (H, C, 1)
            acc = acc + xi * ((s_ij * eta) @ v[..., j * C:(j + 1) * C, :])
        outs.append(acc * scale)
    return np.concatenate(outs, axis=-2)


def retention_quadratic(q, k, v, g, scale: float = 1.0):
    """The source form: ``((q kᵀ) ⊙ decay(γ, T)) v · scale`` — the decayed
    quadratic retention (discovery/zoo.py:452-484, om_decayed binding
    om.py:1053-1057 over the full ``decay(γ, T)``)."""
    q, k, v = (np.asarray(t) for t in (q, k, v))
    T = q.shape[-2]
    s = q @ np.swapaxes(k, -1, -2)
    return ((s * decay(g, T)) @ v) * scale


# ---------------------------------------------------------------- diagonal scans


def affd_compose(f, g):
    """"affd_compose" binding (torch_bridge.py:1897-1900): ``f ∘ g`` with g
    applied first: ``(f.a ⊙ g.a, f.a ⊙ g.b + f.b)``."""
    return f[0] * g[0], f[0] * g[1] + f[1]


def fused_diag_levels(a_seq, b_seq, h):
    """``fused_diag_levels`` (scan_fused.py:100-120): leaves in product order
    (leaf 0 is the OUTERMOST map, applied last), identity-padded to a power
    of two with ``(1, 0)``, adjacent-pair levels ``a = fa·ga``,
    ``b = fa·gb + fb``, read out ``a·h + b``."""
    a = _pad_pow2(np.asarray(a_seq), 1.0)
    b = _pad_pow2(np.asarray(b_seq), 0.0)
    while a.shape[0] > 1:
        fa, ga = a[0::2], a[1::2]
        fb, gb = b[0::2], b[1::2]
        a = fa * ga
        b = fa * gb + fb
    return a[0] * h + b[0]


def prefix_plan(T: int) -> dict:
    """Integer plan of ``BatchedOmdModule._prefix_scan`` (omd_lower.py:771-790):
    ``blk = ⌈√T⌉``, ``C = ⌈T/blk⌉``, ``pad = C·blk − T``, block starts ``c·blk``."""
    if T < 1:
        raise ValueError("T must be positive")
    blk = math.ceil(math.sqrt(T))
    C = (T + blk - 1) // blk
    return {"blk": blk, "C": C, "pad": C * blk - T,
            "starts": np.arange(C, dtype=np.int64) * blk}


def prefix_chunk_table(T: int) -> np.ndarray:
    """The chunk table handed to the HIP scans: the plan's block starts plus
    the end ``T`` (the padded tail block ends at T — padding lanes carry the
    exact identity in the reference, so cutting them off changes nothing)."""
    p = prefix_plan(T)
    return np.concatenate([p["starts"], np.asarray([T], dtype=np.int64)])


def prefix_scan(A, B):
    """``_prefix_scan`` (omd_lower.py:771-824) for the diagonal domain: all
    prefix maps of the leaf sequence ``(A_t, B_t)`` (leaf 0 first in time).
    Local prefixes within blocks of ⌈√T⌉, a carry fold over block totals,
    then one compose of locals onto carries; identity-padded tail."""
    A, B = np.asarray(A), np.asarray(B)
    T = A.shape[0]
    if T == 1:
        return A, B
    p = prefix_plan(T)
    blk, C, pad = p["blk"], p["C"], p["pad"]
    sa, sb = A.shape[1:], B.shape[1:]
    if pad:
        A = np.concatenate([A, np.ones((pad, *sa), dtype=A.dtype)])
        B = np.concatenate([B, np.zeros((pad, *sb), dtype=B.dtype)])
    A = A.reshape(C, blk, *sa)
    B = B.reshape(C, blk, *sb)
    las, lbs = [A[:, 0]], [B[:, 0]]
    for kk in range(1, blk):
        na, nb = affd_compose((A[:, kk], B[:, kk]), (las[-1], lbs[-1]))
        las.append(na)
        lbs.append(nb)
    La, Lb = np.stack(las, axis=1), np.stack(lbs, axis=1)
    cpa, cpb = [np.ones(sa, dtype=A.dtype)], [np.zeros(sb, dtype=B.dtype)]
    for c in range(1, C):
        na, nb = affd_compose((La[c - 1, -1], Lb[c - 1, -1]), (cpa[-1], cpb[-1]))
        cpa.append(na)
        cpb.append(nb)
    CPa = np.stack(cpa)[:, None]
    CPb = np.stack(cpb)[:, None]
    Pa, Pb = affd_compose((La, Lb), (CPa, CPb))
    n = C * blk
    return Pa.reshape(n, *sa)[:T], Pb.reshape(n, *sb)[:T]


def serial_affd_scan(a, u, h0=None):
    """The serial recurrence ``h_t = a_t ⊙ h_{t-1} + u_t`` (the "applyd" chain
    evaluated one step at a time, torch_bridge.py:1895-1900); all states."""
    a, u = np.asarray(a), np.asarray(u)
    T = u.shape[0]
    h = np.zeros(u.shape[1:], dtype=u.dtype) if h0 is None else np.asarray(h0).copy()
    out = np.empty_like(u)
    for t in range(T):
        at = a if a.shape == u.shape[1:] else a[t]
        h = at * h + u[t]
        out[t] = h
    return out


def ssm_serial(a, bx, c, x, h0=None):
    """The selective diagonal SSM of the C5 workload, serially:
    ``h[b,t,d,n] = a[b,t,d,n]·h[b,t-1,d,n] + bx[b,t,n]·x[b,t,d]``,
    ``y[b,t,d] = Σ_n c[b,t,n]·h[b,t,d,n]`` (DiagonalSSM's step,
    models/ssm.py:121-160, with the stacked read-out of all prefix states,
    xcarrier.py:2252-2273).  ``a`` may be ``(B,T,D)`` (broadcast over n)."""
    a, bx, c, x = (np.asarray(t) for t in (a, bx, c, x))
    B, T, D = x.shape
    N = bx.shape[-1]
    h = np.zeros((B, D, N), dtype=x.dtype) if h0 is None else np.asarray(h0).copy()
    y = np.empty((B, T, D), dtype=x.dtype)
    for t in range(T):
        at = a[:, t] if a.ndim == 4 else a[:, t][..., None]
        h = at * h + bx[:, t][:, None, :] * x[:, t][..., None]
        y[:, t] = np.einsum("bn,bdn->bd", c[:, t], h)
    return y, h


def ssm_chunked(a, bx, c, x, h0, table):
    """The SSM through the blocked all-prefix scan: every prefix state from
    ``prefix_scan``-style chunking driven by ``table`` (chunk starts + T),
    then the read-out.  Same function as ``ssm_serial``; exists to pin the
    chunk-carry algebra the HIP chunk-parallel schedule uses."""
    a, bx, c, x = (np.asarray(t) for t in (a, bx, c, x))
    B, T, D = x.shape
    N = bx.shape[-1]
    A = a if a.ndim == 4 else np.broadcast_to(a[..., None], (B, T, D, N))
    U = bx[:, :, None, :] * x[..., None]
    h = np.zeros((B, D, N), dtype=x.dtype) if h0 is None else np.asarray(h0)
    # phase 1: chunk-local maps
    locs = []
    for s, e in zip(table[:-1], table[1:]):
        P = np.ones((B, D, N), dtype=x.dtype)
        H = np.zeros((B, D, N), dtype=x.dtype)
        for t in range(s, e):
            P, H = affd_compose((A[:, t], U[:, t]), (P, H))
        locs.append((P, H))
    # phase 2: carries in table order
    carries = []
    h_final = h
    for P, H in locs:
        carries.append(h_final)
        h_final = P * h_final + H
    # phase 3: re-run each chunk from its carry
    y = np.empty((B, T, D), dtype=x.dtype)
    for (s, e), carry in zip(zip(table[:-1], table[1:]), carries):
        hh = carry
        for t in range(s, e):
            hh = A[:, t] * hh + U[:, t]
            y[:, t] = np.einsum("bn,bdn->bd", c[:, t], hh)
    return y, h_final


# ---------------------------------------------------------------- dense scans


def aff_compose(f, g):
    """"aff_compose" binding (torch_bridge.py:1877-1880): ``f ∘ g`` with g
    applied first: ``(f.A @ g.A, f.A @ g.b + f.b)``."""
    return f[0] @ g[0], f[0] @ g[1] + f[1]


def aff_apply(f, h):
    """"apply" binding (torch_bridge.py:1881): ``f.A @ h + f.b``."""
    return f[0] @ h + f[1]


def aff_homogeneous(A, b):
    """Leaf packing of ``BatchedScanModule._leaf_homogeneous``
    (scan_lower.py:716-741): ``[[A, b], [0 … 0, 1]]``, ``(n, d+1, d+1)`` from
    ``A (n, d, d)`` and a vector ``b (n, d)``."""
    A, b = np.asarray(A), np.asarray(b)
    n, d = A.shape[0], A.shape[-1]
    M = np.zeros((n, d + 1, d + 1), dtype=np.result_type(A, b))
    M[:, :d, :d] = A
    M[:, :d, d] = b
    M[:, d, d] = 1
    return M


def fused_dense_levels(m_seq, h):
    """``fused_dense_levels`` (scan_fused.py:123-143): leaf homogeneous
    matrices in product order (leaf 0 is the OUTERMOST map), identity-padded
    to a power of two, adjacent-pair levels ``m = m[0::2] @ m[1::2]``, read
    out ``A_root h + b_root``."""
    m = np.asarray(m_seq)
    n, d1 = m.shape[0], m.shape[-1]
    pad = (1 << max(n - 1, 0).bit_length()) - n
    if pad:
        m = np.concatenate([m, np.broadcast_to(np.eye(d1, dtype=m.dtype), (pad, d1, d1))])
    while m.shape[0] > 1:
        m = m[0::2] @ m[1::2]
    r = m[0]
    d = d1 - 1
    return r[:d, :d] @ h + r[:d, d]


def serial_aff_scan(A, b, h0):
    """The dense recurrence one step at a time, every state (the "apply"
    chain of LinearRecurrence, models/__init__.py:593-598, with batched
    columns): ``X_t = A_t X_{t-1} + b_t 1ᵀ``.  ``A`` is ``(d, d)`` (one map),
    ``(T, d, d)`` or ``(T, P, d, d)``; ``b`` is ``(T, d)`` or ``(T, P, d)``;
    ``h0`` is ``(d, k)`` or ``(P, d, k)``.  Returns ``(T, *h0.shape)``."""
    A, b, h = np.asarray(A), np.asarray(b), np.asarray(h0).copy()
    T = b.shape[0]
    out = np.empty((T, *h.shape), dtype=np.result_type(A, b, h))
    for t in range(T):
        At = A if A.ndim == 2 else A[t]
        h = At @ h + b[t][..., None]
        out[t] = h
    return out


def aff_chunked_scan(A, b, h0, table):
    """The dense scan through the chunk-carry algebra of the HIP chunk-parallel
    schedule (the blocked all-prefix plan, omd_lower.py:771-824, in the dense
    domain): (1) each chunk's map ``(M_c, v_c)`` composed from the identity,
    (2) carries folded over the chunks in table order, (3) each chunk re-run
    from its carry.  Same function as ``serial_aff_scan``; shapes as there."""
    A, b, h0 = np.asarray(A), np.asarray(b), np.asarray(h0)
    T = b.shape[0]
    d = b.shape[-1]
    At = (lambda t: A) if A.ndim == 2 else (lambda t: A[t])
    eye = np.broadcast_to(np.eye(d, dtype=A.dtype), (*b.shape[1:-1], d, d))
    locs = []
    for s, e in zip(table[:-1], table[1:]):
        M, v = eye, np.zeros((*b.shape[1:], 1), dtype=b.dtype)  # v as a column: batched @ stays per slot
        for t in range(s, e):
            M, v = aff_compose((At(t), b[t][..., None]), (M, v))
        locs.append((M, v))
    carries, h = [], h0
    for M, v in locs:
        carries.append(h)
        h = M @ h + v
    out = np.empty((T, *h0.shape), dtype=np.result_type(A, b, h0))
    for (s, e), carry in zip(zip(table[:-1], table[1:]), carries):
        hh = carry
        for t in range(s, e):
            hh = At(t) @ hh + b[t][..., None]
            out[t] = hh
    return out, h


# ---------------------------------------------------------------- deferred-affine om (omd)


def omd_elem(s, a, b):
    """``_omd_elem`` (xcarrier.py:380-400): the om triple of the scores ``s``
    over values affine in a symbolic state, ``v_k = a_k ⊙ h + b_k`` (diagonal
    fibre, ``a (K,d)``) or ``v_k = A_k @ h + b_k`` (dense fibre, any ``a`` of
    3 or more axes, ``(…,K,d,i)``): ``(m, l, e@a, e@b)`` with
    ``e = exp(s − m)``; the dense ``e@A`` contracts the key axis of ``A``."""
    s, a, b = np.asarray(s), np.asarray(a), np.asarray(b)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l_ = e.sum(axis=-1, keepdims=True)
    if a.ndim >= 3:  # the reference's fibre test: a 3-D+ coefficient is dense
        d, i = a.shape[-2], a.shape[-1]
        ea = (e @ a.reshape(*a.shape[:-2], d * i)).reshape(*e.shape[:-1], d, i)
        return m, l_, ea, e @ b
    return m, l_, e @ a, e @ b


def omd_compose(f, g):
    """``_omd_compose`` (xcarrier.py:407-440): both numerator parts rescale
    like om's ``a``, with the same ``isfinite`` guard (a block whose max is
    −inf contributes nothing)."""
    m1, l1, fa1, fb1 = (np.asarray(t) for t in f)
    m2, l2, fa2, fb2 = (np.asarray(t) for t in g)
    mx = np.maximum(m1, m2)
    fin1, fin2 = np.isfinite(m1), np.isfinite(m2)
    with np.errstate(invalid="ignore", over="ignore"):
        e1 = np.where(fin1, np.exp(np.where(fin1, m1 - mx, 0.0)), 0.0)
        e2 = np.where(fin2, np.exp(np.where(fin2, m2 - mx, 0.0)), 0.0)

    def lift(e, x):  # row weight (…,Tq,1) onto a numerator with trailing axes
        return e.reshape(*e.shape, *([1] * (x.ndim - e.ndim)))

    l_ = np.where(fin1, l1 * e1, 0.0) + np.where(fin2, l2 * e2, 0.0)
    fa = np.where(lift(fin1, fa1), fa1 * lift(e1, fa1), 0.0) + np.where(lift(fin2, fa2), fa2 * lift(e2, fa2), 0.0)
    fb = np.where(fin1, fb1 * e1, 0.0) + np.where(fin2, fb2 * e2, 0.0)
    return mx, l_, fa, fb


def omd_apply(f, h):
    """``_omd_apply`` (xcarrier.py:443-445): ``(fa ⊙ h + fb) / l``."""
    return (np.asarray(f[2]) * h + f[3]) / f[1]


def omd_applym(f, h):
    """``_omd_applym`` (xcarrier.py:448-454): ``(fa @ h + fb) / l``, the
    dense fibre's map input axis contracted with ``h``."""
    return (np.asarray(f[2]) @ h + f[3]) / f[1]
