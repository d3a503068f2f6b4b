"""Constructors of the delivered terms for the five benchmark configurations.

catopt's search extracts these terms on the CPU; the constructors spell them
from the law right-hand sides that produce them, so tests and the benchmark
can feed this package's sink exactly what the orchestrator would route:

* :func:`weight_chain_form` — ``L`` stacked ``linear`` layers folded by
  repeated ``ASSOC_LINEAR_BIAS`` (luisfuturist/catopt
  ``packages/catopt-core/src/catopt_core/laws/tensor.py:1374-1394``):
  ``linear(linear(x,A,b1),B,b2) → add(linear(x, matmul(B,A), matmul(B,b1)), b2)``,
  applied from the innermost pair out;
* :func:`swiglu_block_form` — ``RMS_NORM_FOLD`` (``tensor.py:712-741``) then
  the ``SWIGLU_FUSE`` RHS (``tensor.py:1485-1519``) and the down projection;
* :func:`causal_attention_form` — the ``OM_LIFT`` RHS (``om.py:153-193``)
  over ``masked_fill(q kᵀ / √d, ¬mask, -inf)`` with a bool lower-triangular
  mask Param (or the ``cmask`` generator);
* :func:`retention_kway_form` — ``om_decayed_kway_blocks(K)``
  (``om.py:3040-3210``), built arm by arm as ``_kway_rhs`` spells it;
* :func:`scan_final_form` / :func:`scan_prefix_form` — the diagonal-affine
  chain ``applyd(affd_compose(…), h)`` and its stacked all-prefix form
  (``xcarrier.py:2252-2273``), with leaves reading step ``t`` of shared
  ``a`` / ``u`` arrays;
* :func:`linear_recurrence_form` / :func:`dense_scan_form` /
  :func:`dense_scan_prefix_form` — the dense affine monoid: ``apply`` over a
  balanced ``aff_compose`` tree (the depth-extracted ``LinearRecurrence``
  term) and the stacked all-prefix form (``xcarrier.py:2276-2293``);
* :func:`omd_scan_attention_form` — softmax attention over a scan's states
  as the deferred-affine ``omd_apply`` term (``omd_lower.py:1-12``);
  :func:`omd_block_restart_form` — the same over states that restart at
  every key block (maps of several leaf sequences: a forest plan).

Each returns ``(IR, param_shapes)``; parameter values come from the caller.
"""

from __future__ import annotations

import math

from .ir import IR, Const, Op, Param, TensorType, Var

__all__ = [
    "weight_chain_form",
    "swiglu_block_form",
    "causal_attention_form",
    "retention_kway_form",
    "retention_block_form",
    "scan_final_form",
    "scan_prefix_form",
    "linear_recurrence_form",
    "dense_scan_form",
    "dense_scan_prefix_form",
    "diag_ssm_form",
    "omd_scan_attention_form",
    "omd_block_restart_form",
]

mk = Op.make


def weight_chain_form(L: int = 8, d: int = 512, rows: int = 64) -> tuple[IR, dict]:
    """``add(…add(linear(x, W_eff, c_0), c_1)…, c_{L-1})`` with ``W_eff`` and
    every ``c_i`` spelled as ``matmul`` chains of the layer Params."""
    x = Var("x", TensorType((rows, d)))
    Ws = [Param(f"W{i + 1}", TensorType((d, d))) for i in range(L)]
    bs = [Param(f"b{i + 1}", TensorType((d,))) for i in range(L)]
    W = Ws[0]
    adds: list = [bs[0]]
    for Wl, bl in zip(Ws[1:], bs[1:]):
        W = mk("matmul", Wl, W)
        adds = [mk("matmul", Wl, c) for c in adds] + [bl]
    y = mk("linear", x, W, adds[0])
    for c in adds[1:]:
        y = mk("add", y, c)
    shapes = {p.name: p.typ.shape for p in Ws + bs}
    return IR(y, [x]), shapes


def swiglu_block_form(rows_shape=(8, 2048), D: int = 4096, F: int = 11008,
                      eps: float = 1e-6) -> tuple[IR, dict]:
    """``linear(mul(silu(chunk(Y, 2, -1, 0)), chunk(Y, 2, -1, 1)), W_down)``,
    ``Y = linear(rms_norm(x, γ), concat(W_gate, W_up, dim=0))``."""
    x = Var("x", TensorType((*rows_shape, D)))
    g = Param("gamma", TensorType((D,)))
    wg, wu = Param("W_gate", TensorType((F, D))), Param("W_up", TensorType((F, D)))
    wd = Param("W_down", TensorType((D, F)))
    h = mk("rms_norm", x, g, dim=(D,), eps=eps)
    y = mk("linear", h, mk("concat", wg, wu, dim=0))
    gate = mk("chunk", y, chunks=2, dim=-1, index=0)
    up = mk("chunk", y, chunks=2, dim=-1, index=1)
    out = mk("linear", mk("mul", mk("silu", gate), up), wd)
    return IR(out, [x]), {"gamma": (D,), "W_gate": (F, D), "W_up": (F, D), "W_down": (D, F)}


def causal_attention_form(B: int = 4, H: int = 32, T: int = 4096, d: int = 128,
                          mask: str = "param") -> tuple[IR, dict]:
    """``om_apply(om_elem(masked_fill(q kᵀ / √d, ¬mask, -inf), v))``.

    ``mask="param"``: a bool keep-mask Param ``mask (T, T)`` (lower
    triangle); ``mask="cmask"``: the causal generator ``cmask(s, off=0)``."""
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    s = mk("div", mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1)), Const(math.sqrt(d)))
    shapes = {}
    if mask == "param":
        m = Param("mask", TensorType((T, T)))
        masked = mk("logical_not", m)
        shapes["mask"] = (T, T)
    elif mask == "cmask":
        masked = mk("cmask", s, off=0)
    else:
        raise ValueError(mask)
    sm = mk("masked_fill", s, masked, Const(float("-inf")))
    return IR(mk("om_apply", mk("om_elem", sm, v)), [q, k, v]), shapes


def _kway_rhs(s, v, g, K: int, C: int):
    SZ = (C,) * K

    def score(i, j):
        return mk("split", mk("split", s, sizes=SZ, dim=-2, index=i), sizes=SZ, dim=-1, index=j)

    def value(j):
        return mk("split", v, sizes=SZ, dim=-2, index=j)

    blocks = []
    for i in range(K):
        acc = mk("om_decayed", score(i, i), mk("decay", g, t=C), value(i))
        for j in range(i):
            row = mk("unsqueeze", mk("decay_vec", g, t=C, offset=(i - j) * C), dim=-1)
            col = mk("unsqueeze", mk("decay_vec", g, t=C, sign=-1), dim=-2)
            acc = mk("add", acc, mk("mul", row, mk("matmul", mk("mul", score(i, j), col), value(j))))
        blocks.append(acc)
    out = blocks[-1]
    for blk in reversed(blocks[:-1]):
        out = mk("concat", blk, out, dim=-2)
    return out


def retention_kway_form(B: int = 4, H: int = 16, T: int = 8192, d: int = 128, C: int = 64,
                        scale: float | None = None) -> tuple[IR, dict]:
    """The K-way chunked form (``K = T / C``) of
    ``om_decayed(s, decay(γ, T), v)`` with ``s = q kᵀ`` (``/ 1/scale`` when
    ``scale`` is given, spelled as a ``div`` by the constant)."""
    if T % C:
        raise ValueError("T must be a multiple of C")
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    g = Param("gamma", TensorType((H,)))
    s = mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))
    if scale is not None:
        s = mk("div", s, Const(1.0 / scale))
    return IR(_kway_rhs(s, v, g, T // C, C), [q, k, v]), {"gamma": (H,)}


def retention_block_form(B: int, H: int, T: int, d: int = 128) -> tuple[IR, dict]:
    """The un-chunked source ``om_decayed(q kᵀ, decay(γ, T), v)``."""
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    g = Param("gamma", TensorType((H,)))
    s = mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))
    return IR(mk("om_decayed", s, mk("decay", g, t=T), v), [q, k, v]), {"gamma": (H,)}


def _leaf(a, u, t: int):
    return mk("aff_diag", mk("select", a, dim=0, index=t), mk("select", u, dim=0, index=t))


def scan_final_form(T: int, state_shape: tuple) -> tuple[IR, dict]:
    """``applyd(f_{T-1} ∘ … ∘ f_0, h)``, ``f_t = aff_diag(a[t], u[t])``, as a
    left-leaning compose chain (leaf 0 of the product is the last step)."""
    a = Var("a", TensorType((T, *state_shape)))
    u = Var("u", TensorType((T, *state_shape)))
    h = Var("h", TensorType(tuple(state_shape)))
    F = _leaf(a, u, 0)
    for t in range(1, T):
        F = mk("affd_compose", _leaf(a, u, t), F)
    return IR(mk("applyd", F, h), [a, u, h]), {}


def scan_prefix_form(T: int, state_shape: tuple) -> tuple[IR, dict]:
    """``applyd(aff_diag(stack(affd_a f_t), stack(affd_b f_t)), h)`` over the
    prefixes ``f_t = f_{t-1} ∘ leaf_t``: every state ``h_0 … h_{T-1}``."""
    a = Var("a", TensorType((T, *state_shape)))
    u = Var("u", TensorType((T, *state_shape)))
    h = Var("h", TensorType(tuple(state_shape)))
    fs = [_leaf(a, u, 0)]
    for t in range(1, T):
        fs.append(mk("affd_compose", _leaf(a, u, t), fs[-1]))
    A = mk("stack", *[mk("affd_a", f) for f in fs], dim=0)
    Bm = mk("stack", *[mk("affd_b", f) for f in fs], dim=0)
    return IR(mk("applyd", mk("aff_diag", A, Bm), h), [a, u, h]), {}


def _balanced(leaves: list, compose: str):
    """Balanced compose tree over ``leaves`` in product order."""
    if len(leaves) == 1:
        return leaves[0]
    mid = len(leaves) // 2
    return mk(compose, _balanced(leaves[:mid], compose), _balanced(leaves[mid:], compose))


def linear_recurrence_form(T: int, d: int) -> tuple[IR, dict]:
    """``LinearRecurrence`` (models/__init__.py:576-598, ``h_t = A h_{t-1} +
    x_t``) as the depth-extracted scan term: ``apply(<balanced aff_compose
    tree>, p_h0)`` over leaves ``aff(p_a, select(x, 0, t))``, later steps on
    the left (the shape of ``_balanced_scan_ir``, tests/test_scan_batched.py:
    56-88)."""
    x = Var("x", TensorType((T, d)))
    A = Param("p_a", TensorType((d, d)))
    h0 = Param("p_h0", TensorType((d,)))
    leaves = [mk("aff", A, mk("select", x, dim=0, index=t)) for t in reversed(range(T))]
    return IR(mk("apply", _balanced(leaves, "aff_compose"), h0), [x]), {"p_a": (d, d), "p_h0": (d,)}


def dense_scan_form(T: int, d: int, batch: tuple = (), k: int = 1, *, time_varying: bool = False,
                    per_slot: bool = False) -> tuple[IR, dict]:
    """Batched dense scan with column states: ``apply(<balanced tree>, h)``
    over leaves ``aff(A_t, select(b, 0, t))`` with ``b (T, *batch, d, 1)``,
    ``h (*batch, d, k)``; ``A_t`` is ``select(A, 0, t)`` of ``A (T, [*batch,]
    d, d)`` when time-varying, else the shared ``A ([*batch,] d, d)``
    (``per_slot`` adds the batch dims to the map)."""
    mshape = (*batch, d, d) if per_slot else (d, d)
    A = Var("A", TensorType((T, *mshape) if time_varying else mshape))
    b = Var("b", TensorType((T, *batch, d, 1)))
    h = Var("h", TensorType((*batch, d, k)))

    def leaf(t):
        At = mk("select", A, dim=0, index=t) if time_varying else A
        return mk("aff", At, mk("select", b, dim=0, index=t))

    leaves = [leaf(t) for t in reversed(range(T))]
    return IR(mk("apply", _balanced(leaves, "aff_compose"), h), [A, b, h]), {}


def dense_scan_prefix_form(T: int, d: int, *, time_varying: bool = True, dim: int = 0) -> tuple[IR, dict]:
    """The stacked all-prefix form ``apply(aff(stack(aff_A f_t), stack(aff_b
    f_t)), h)`` (gather_apply_stack, xcarrier.py:2276-2293) over the prefixes
    ``f_t = aff_compose(leaf_t, f_{t-1})``: every state ``h_0 … h_{T-1}``,
    stacked along ``dim``; vector state ``h (d,)``, ``b (T, d)``."""
    A = Var("A", TensorType((T, d, d) if time_varying else (d, d)))
    b = Var("b", TensorType((T, d)))
    h = Var("h", TensorType((d,)))

    def leaf(t):
        At = mk("select", A, dim=0, index=t) if time_varying else A
        return mk("aff", At, mk("select", b, dim=0, index=t))

    fs = [leaf(0)]
    for t in range(1, T):
        fs.append(mk("aff_compose", leaf(t), fs[-1]))
    SA = mk("stack", *[mk("aff_A", f) for f in fs], dim=dim)
    SB = mk("stack", *[mk("aff_b", f) for f in fs], dim=dim)
    return IR(mk("apply", mk("aff", SA, SB), h), [A, b, h]), {}


def diag_ssm_form(B: int, T: int, D: int, N: int, *, a_per_state: bool = True) -> tuple[IR, dict]:
    """The selective diagonal SSM with every output: the ``DiagonalSSM`` step
    (models/ssm.py:121-160) over a ``(B, D, N)`` state,
    ``h_t = a_t ⊙ h_{t-1} + x_t ⊗ bx_t``, read out as
    ``y_t = Σ_n c_t[n]·h_t[…, n]``.  Delivered as the stacked all-prefix form
    (xcarrier.py:2252-2273) inside the contraction:
    ``sum(mul(applyd(aff_diag(stack(affd_a f_t, dim=1), stack(affd_b f_t,
    dim=1)), unsqueeze(h, 1)), unsqueeze(c, 2)), dim=-1)`` with
    ``f_t = affd_compose(aff_diag(a_t, x_t ⊗ bx_t), f_{t-1})``.
    ``a_per_state=False`` takes ``a (B, T, D)``, broadcast over ``N``."""
    a = Var("a", TensorType((B, T, D, N) if a_per_state else (B, T, D)))
    bx, c = Var("bx", TensorType((B, T, N))), Var("c", TensorType((B, T, N)))
    x, h = Var("x", TensorType((B, T, D))), Var("h", TensorType((B, D, N)))
    fs = []
    for t in range(T):
        at = mk("select", a, dim=1, index=t)
        if not a_per_state:
            at = mk("unsqueeze", at, dim=-1)
        ut = mk("mul", mk("unsqueeze", mk("select", x, dim=1, index=t), dim=-1),
                mk("unsqueeze", mk("select", bx, dim=1, index=t), dim=-2))
        leaf = mk("aff_diag", at, ut)
        fs.append(leaf if t == 0 else mk("affd_compose", leaf, fs[-1]))
    states = mk("applyd", mk("aff_diag", mk("stack", *[mk("affd_a", f) for f in fs], dim=1),
                             mk("stack", *[mk("affd_b", f) for f in fs], dim=1)),
                mk("unsqueeze", h, dim=1))
    y = mk("sum", mk("mul", states, mk("unsqueeze", c, dim=2)), dim=-1)
    return IR(y, [a, bx, c, x, h]), {}


def omd_scan_attention_form(T: int, d: int, Tq: int, blocks: int, dk: int = 16, *,
                            dense: bool = False) -> tuple[IR, dict]:
    """Softmax attention over the states of a scan, as the cross-carrier lift
    delivers it (omd_lower.py:1-12, the ``_ScanAttn`` model of
    tests/test_omd_lower.py:72-124): ``omd_apply(<balanced omd_compose tree
    of omd_elem(s_i, stack(affd_a f_j), stack(affd_b f_j))>, h)`` over key
    blocks ``i``, with ``s_i = q · chunk(k, i)ᵀ`` and the prefix chain
    ``f_j = affd_compose(aff_diag(a[j], x[j]), f_{j-1})``.  ``dense`` uses
    ``aff`` maps ``A (T, d, d)`` and ``omd_applym``."""
    if T % blocks:
        raise ValueError("blocks must divide T")
    q = Var("q", TensorType((Tq, dk)))
    k = Var("k", TensorType((T, dk)))
    a = Var("a", TensorType((T, d, d) if dense else (T, d)))
    x = Var("x", TensorType((T, d)))
    h = Var("h", TensorType((d,)))
    leaf_op, comp, pa, pb = ("aff", "aff_compose", "aff_A", "aff_b") if dense else \
        ("aff_diag", "affd_compose", "affd_a", "affd_b")
    fs = []
    for j in range(T):
        leaf = mk(leaf_op, mk("select", a, dim=0, index=j), mk("select", x, dim=0, index=j))
        fs.append(leaf if j == 0 else mk(comp, leaf, fs[-1]))
    C = T // blocks
    elems = []
    for i in range(blocks):
        blk = fs[i * C:(i + 1) * C]
        s = mk("matmul", q, mk("transpose", mk("chunk", k, chunks=blocks, dim=0, index=i), dim0=0, dim1=1))
        elems.append(mk("omd_elem", s, mk("stack", *[mk(pa, f) for f in blk], dim=0),
                        mk("stack", *[mk(pb, f) for f in blk], dim=0)))
    root = mk("omd_applym" if dense else "omd_apply", _balanced(elems, "omd_compose"), h)
    return IR(root, [q, k, a, x, h]), {}


def omd_block_restart_form(T: int, d: int, Tq: int, blocks: int, dk: int = 16, *,
                           dense: bool = False, bracket: str = "chain") -> tuple[IR, dict]:
    """Attention over scan states that restart from ``h`` at every key block:
    the coefficient maps of block ``i`` are the local prefixes
    ``g_j = leaf_j ∘ … ∘ leaf_{iC}`` of that block's own leaves, so no map is
    a prefix of another block's leaf sequence and the plan is a forest
    (level-batched, ``omd_lower.py:520-558``; the disjoint-trees case of
    tests/test_omd_lower.py:184-211 at scale).  ``bracket="chain"`` spells
    ``g_j = compose(leaf_j, g_{j-1})``; ``"tree"`` spells every ``g_j`` as its
    own balanced compose tree (equal subtrees are one term).  Operands as
    :func:`omd_scan_attention_form`."""
    if T % blocks:
        raise ValueError("blocks must divide T")
    q = Var("q", TensorType((Tq, dk)))
    k = Var("k", TensorType((T, dk)))
    a = Var("a", TensorType((T, d, d) if dense else (T, d)))
    x = Var("x", TensorType((T, d)))
    h = Var("h", TensorType((d,)))
    leaf_op, comp, pa, pb = ("aff", "aff_compose", "aff_A", "aff_b") if dense else \
        ("aff_diag", "affd_compose", "affd_a", "affd_b")
    C = T // blocks
    elems = []
    if bracket not in ("chain", "tree"):
        raise ValueError(bracket)
    for i in range(blocks):
        blk, lvs = [], []
        for j in range(i * C, (i + 1) * C):
            leaf = mk(leaf_op, mk("select", a, dim=0, index=j), mk("select", x, dim=0, index=j))
            lvs.append(leaf)
            if bracket == "tree":
                blk.append(_balanced(lvs[::-1], comp))  # product order: latest leaf first
            else:
                blk.append(leaf if j == i * C else mk(comp, leaf, blk[-1]))
        s = mk("matmul", q, mk("transpose", mk("chunk", k, chunks=blocks, dim=0, index=i), dim0=0, dim1=1))
        elems.append(mk("omd_elem", s, mk("stack", *[mk(pa, f) for f in blk], dim=0),
                        mk("stack", *[mk(pb, f) for f in blk], dim=0)))
    root = mk("omd_applym" if dense else "omd_apply", _balanced(elems, "omd_compose"), h)
    return IR(root, [q, k, a, x, h]), {}
