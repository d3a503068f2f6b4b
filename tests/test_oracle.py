"""Pins of the numpy oracle (CPU only).

Each oracle function is checked against something that is not a retyping
of its own formula: a torch library routine (``F.rms_norm``,
``F.scaled_dot_product_attention``, ``F.linear``, ``F.silu``), brute force
over index loops on tiny inputs, a closed form, or an algebraic identity of
the reference's monoids.  ``test_planted_*`` show that a plausible mistake
(a transposed operand, a dropped term, an off-by-one index, a swapped
composition order) fails the corresponding pin.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

rng = np.random.default_rng(1234)


def _close(a, b, tol=1e-12):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    err = np.max(np.abs(a - b)) / (np.max(np.abs(b)) + 1e-300) if a.size else 0.0
    assert err <= tol, err


# ------------------------------------------------------------------ verify gate


def test_verify_equiv_global_metric():
    ref = np.array([1.0, -4.0, 2.0])
    out = np.array([1.0, -4.0, 2.1])
    r = oracle.verify_equiv(ref, out, rtol=0.03)
    assert r["max_abs"] == pytest.approx(0.1)
    assert r["max_rel"] == pytest.approx(0.1 / (4.0 + 1e-8))  # global, not elementwise
    assert r["passed"]
    assert not oracle.verify_equiv(ref, out, rtol=0.02)["passed"]
    assert not oracle.verify_equiv(ref, out, rtol=0.03, atol=0.05)["passed"]
    nan = oracle.verify_equiv(ref, np.array([1.0, np.nan, 2.0]))
    assert math.isnan(nan["max_abs"]) and not nan["passed"]
    assert oracle.verify_equiv(np.zeros(0), np.zeros(0))["passed"]


# ------------------------------------------------------------------ norms / GEMM


@pytest.mark.parametrize("with_w", [True, False])
def test_rms_norm_matches_torch(with_w):
    x = rng.standard_normal((7, 33))
    w = 1 + 0.02 * rng.standard_normal(33) if with_w else None
    ref = F.rms_norm(torch.from_numpy(x), (33,), None if w is None else torch.from_numpy(w), 1e-6)
    _close(oracle.rms_norm(x, w, 1e-6), ref.numpy(), 1e-14)


def test_linear_matches_torch():
    x, W, b = rng.standard_normal((5, 12)), rng.standard_normal((9, 12)), rng.standard_normal(9)
    ref = F.linear(torch.from_numpy(x), torch.from_numpy(W), torch.from_numpy(b)).numpy()
    _close(oracle.linear(x, W, b), ref, 1e-14)


def test_fold_linear_chain_equals_chain():
    d = 16
    Ws = [rng.standard_normal((d, d)) / 4 for _ in range(8)]
    bs = [rng.standard_normal(d) for _ in range(8)]
    x = rng.standard_normal((6, d))
    W, adds = oracle.fold_linear_chain(Ws, bs)
    assert len(adds) == 8
    # closed form: W_eff = W8 … W1, and the chain through torch layers
    _close(W, np.linalg.multi_dot(Ws[::-1]), 1e-12)
    h = torch.from_numpy(x)
    for Wl, bl in zip(Ws, bs):
        h = F.linear(h, torch.from_numpy(Wl), torch.from_numpy(bl))
    _close(oracle.folded_chain_forward(x, W, adds), h.numpy(), 1e-12)
    _close(oracle.linear_chain(x, Ws, bs), h.numpy(), 1e-12)


def test_planted_fold_transpose_fails():
    d = 8
    Ws = [rng.standard_normal((d, d)) for _ in range(3)]
    bs = [rng.standard_normal(d) for _ in range(3)]
    x = rng.standard_normal((4, d))
    W, adds = oracle.fold_linear_chain(Ws, bs)
    good = oracle.linear_chain(x, Ws, bs)
    assert np.max(np.abs(oracle.folded_chain_forward(x, W.T, adds) - good)) > 1e-3
    assert np.max(np.abs(oracle.folded_chain_forward(x, W, adds[:-1]) - good)) > 1e-3


def test_silu_and_swiglu_match_torch():
    x = rng.standard_normal((4, 10))
    _close(oracle.silu(x), F.silu(torch.from_numpy(x)).numpy(), 1e-14)
    wg, wu, wd = rng.standard_normal((6, 10)), rng.standard_normal((6, 10)), rng.standard_normal((10, 6))
    t = torch.from_numpy
    ref = F.linear(F.silu(F.linear(t(x), t(wg))) * F.linear(t(x), t(wu)), t(wd)).numpy()
    _close(oracle.swiglu_fused(x, wg, wu, wd), ref, 1e-13)
    _close(oracle.swiglu_unfused(x, wg, wu, wd), ref, 1e-13)


def test_planted_swiglu_swapped_halves_fails():
    x = rng.standard_normal((4, 10))
    wg, wu, wd = rng.standard_normal((6, 10)), rng.standard_normal((6, 10)), rng.standard_normal((10, 6))
    assert np.max(np.abs(oracle.swiglu_fused(x, wu, wg, wd) - oracle.swiglu_unfused(x, wg, wu, wd))) > 1e-3


# ------------------------------------------------------------------ online softmax


@pytest.mark.parametrize("t,k,off", [(5, 5, 0), (4, 7, 0), (6, 6, 2), (6, 6, -3)])
def test_cmask_keep_brute_force(t, k, off):
    keep = oracle.cmask_keep(t, k, off)
    for i in range(t):
        for j in range(k):
            assert keep[i, j] == (j <= i - off)
    # the reference generator's library spelling: ones(t, k).tril(-off)
    assert np.array_equal(keep, torch.ones(t, k, dtype=torch.bool).tril(-off).numpy())


def _sdpa(q, k, v, scale, keep):
    t = lambda z: torch.from_numpy(np.ascontiguousarray(z))  # noqa: E731
    return F.scaled_dot_product_attention(t(q), t(k), t(v), attn_mask=t(keep), scale=scale).numpy()


@pytest.mark.parametrize("block", [None, 4, 5, 16])
def test_attention_om_matches_sdpa_causal(block):
    q, k, v = (rng.standard_normal((2, 3, 13, 8)) for _ in range(3))
    keep = oracle.cmask_keep(13, 13)
    ref = _sdpa(q, k, v, 0.3, keep)
    _close(oracle.attention_om(q, k, v, 0.3, causal=True, block=block), ref, 1e-12)
    _close(oracle.attention_dense(q, k, v, 0.3, keep), ref, 1e-12)


def test_attention_om_causal_offset_and_bool_mask():
    q = rng.standard_normal((1, 1, 5, 4))
    k, v = rng.standard_normal((1, 1, 9, 4)), rng.standard_normal((1, 1, 9, 4))
    keep = np.array([[j <= i + 4 for j in range(9)] for i in range(5)])
    _close(oracle.attention_om(q, k, v, 0.5, causal=True, causal_off=4, block=2), _sdpa(q, k, v, 0.5, keep), 1e-12)
    m = rng.random((5, 9)) < 0.5
    m[:, 0] = True
    _close(oracle.attention_om(q, k, v, 0.5, causal=False, mask=m, block=3), _sdpa(q, k, v, 0.5, m), 1e-12)


def test_attention_fully_masked_row_is_nan():
    # om_apply is a/l unclamped: a row with no kept key is 0/0 = NaN,
    # exactly where dense softmax gives NaN.
    q, k, v = (rng.standard_normal((1, 1, 4, 3)) for _ in range(3))
    m = np.ones((4, 4), dtype=bool)
    m[2, :] = False
    out = oracle.attention_om(q, k, v, 1.0, causal=False, mask=m, block=2)
    dense = oracle.attention_dense(q, k, v, 1.0, m)
    assert np.array_equal(np.isnan(out), np.isnan(dense))
    assert np.isnan(out[0, 0, 2]).all() and not np.isnan(np.delete(out[0, 0], 2, 0)).any()


def test_om_compose_monoid_laws():
    def leaf(n=3, d=4):
        s = rng.standard_normal((n, 5))
        return oracle.om_elem(s, rng.standard_normal((5, d)))

    f, g, h = leaf(), leaf(), leaf()
    ident = (np.full((3, 1), -np.inf), np.zeros((3, 1)), np.zeros((3, 4)))
    for a, b in zip(oracle.om_compose(f, ident), f):
        _close(a, b, 0)
    lhs = oracle.om_compose(oracle.om_compose(f, g), h)
    rhs = oracle.om_compose(f, oracle.om_compose(g, h))
    for a, b in zip(lhs, rhs):
        _close(a, b, 1e-13)
    # commutativity of the merge, and equality with one elem over the concat
    s1, s2 = rng.standard_normal((3, 5)), rng.standard_normal((3, 6))
    v1, v2 = rng.standard_normal((5, 4)), rng.standard_normal((6, 4))
    both = oracle.om_elem(np.concatenate([s1, s2], -1), np.concatenate([v1, v2], 0))
    merged = oracle.om_compose(oracle.om_elem(s1, v1), oracle.om_elem(s2, v2))
    _close(oracle.om_apply(merged), oracle.om_apply(both), 1e-13)


def test_planted_om_compose_missing_rescale_fails():
    s1, s2 = rng.standard_normal((3, 5)) + 3, rng.standard_normal((3, 6))
    v1, v2 = rng.standard_normal((5, 4)), rng.standard_normal((6, 4))
    f, g = oracle.om_elem(s1, v1), oracle.om_elem(s2, v2)
    wrong = (np.maximum(f[0], g[0]), f[1] + g[1], f[2] + g[2])  # no exp(m_i - mx) rescale
    both = oracle.om_elem(np.concatenate([s1, s2], -1), np.concatenate([v1, v2], 0))
    assert np.max(np.abs(oracle.om_apply(wrong) - oracle.om_apply(both))) > 1e-3


def test_fused_om_levels_equals_serial_fold_and_pads():
    for n in (1, 3, 4, 7):
        leaves = [oracle.om_elem(rng.standard_normal((2, 3)), rng.standard_normal((3, 2))) for _ in range(n)]
        f = leaves[0]
        for g in leaves[1:]:
            f = oracle.om_compose(f, g)
        out = oracle.fused_om_levels(*(np.stack([lf[i] for lf in leaves]) for i in range(3)))
        _close(out, oracle.om_apply(f), 1e-13)


# ------------------------------------------------------------------ retention


def test_decay_brute_force():
    g = np.array([0.5, 0.9, 1.0])
    D = oracle.decay(g, 6)
    assert D.shape == (3, 6, 6)
    for h in range(3):
        for i in range(6):
            for j in range(6):
                assert D[h, i, j] == (g[h] ** (i - j) if i >= j else 0.0)
    assert oracle.decay(np.float64(0.7), 3).shape == (3, 3)


@pytest.mark.parametrize("off,sign", [(0, 1), (0, -1), (12, 1), (5, 0), (3, -1)])
def test_decay_vec_brute_force(off, sign):
    g = np.array([0.5, 0.8])
    vec = oracle.decay_vec(g, 5, off, sign)
    for h in range(2):
        for k in range(5):
            assert vec[h, k] == pytest.approx(g[h] ** (sign * k + off), rel=1e-15)


def test_kway_plan_closed_form():
    p = oracle.kway_plan(512, 8)
    assert p["C"] == 64 and p["SZ"] == (64,) * 8
    assert p["OFF"] == {(i, j): (i - j) * 64 for i in range(8) for j in range(i)}
    assert oracle.kway_plan(100, 8) is None and oracle.kway_plan(4, 8) is None


def test_kway_pair_tables_brute_force():
    for K in (2, 3, 8):
        t = oracle.kway_pair_tables(K)
        pairs = [(i, j) for i in range(K) for j in range(i)]  # arm order
        assert t["n_pairs"] == len(pairs)
        assert t["q_idx"].tolist() == [i - 1 for i, _ in pairs]  # q_i first seen at arm i (arm 0 has no cross)
        assert t["m_idx"].tolist() == [j for _, j in pairs]
        assert t["pair_counts"].tolist() == list(range(K))
        assert t["q_idx"].dtype == np.int64


def _retention_recurrent(q, k, v, g, scale):
    """Textbook recurrent retention: S_t = γ S_{t-1} + k_tᵀ v_t; o_t = q_t S_t."""
    H, T, d = q.shape
    out = np.zeros((H, T, v.shape[-1]))
    for h in range(H):
        S = np.zeros((d, v.shape[-1]))
        for t in range(T):
            S = g[h] * S + np.outer(k[h, t], v[h, t])
            out[h, t] = q[h, t] @ S
    return out * scale


@pytest.mark.parametrize("K", [1, 2, 4, 8])
def test_retention_kway_equals_quadratic_and_recurrence(K):
    H, T, d = 2, 32, 5
    q, k, v = (rng.standard_normal((H, T, d)) for _ in range(3))
    g = np.array([0.9, 0.97])
    rec = _retention_recurrent(q, k, v, g, 0.5)
    _close(oracle.retention_quadratic(q, k, v, g, 0.5), rec, 1e-12)
    if K > 1:
        _close(oracle.retention_kway(q, k, v, g, K, 0.5), rec, 1e-12)


def test_planted_retention_wrong_offset_fails():
    H, T, d = 1, 16, 3
    q, k, v = (rng.standard_normal((H, T, d)) for _ in range(3))
    g = np.array([0.8])
    good = _retention_recurrent(q, k, v, g, 1.0)
    # an off-by-one-chunk decay offset is a plausible mistake
    orig = oracle.kway_plan
    try:
        oracle.ref.kway_plan = lambda T_, K_: {**orig(T_, K_), "OFF": {ij: (ij[0] - ij[1] + 1) * (T_ // K_) for ij in orig(T_, K_)["OFF"]}}
        bad = oracle.ref.retention_kway(q, k, v, g, 4, 1.0)
    finally:
        oracle.ref.kway_plan = orig
    assert np.max(np.abs(bad - good)) > 1e-3


# ------------------------------------------------------------------ diagonal scans


def test_affd_compose_monoid_and_order():
    f = (rng.random(4), rng.standard_normal(4))
    g = (rng.random(4), rng.standard_normal(4))
    h = rng.standard_normal(4)
    a, b = oracle.affd_compose(f, g)
    _close(a * h + b, f[0] * (g[0] * h + g[1]) + f[1], 1e-14)  # g applied first
    swapped = oracle.affd_compose(g, f)
    assert np.max(np.abs(swapped[0] * h + swapped[1] - (a * h + b))) > 1e-6


@pytest.mark.parametrize("n", [1, 2, 5, 8])
def test_fused_diag_levels_reversed_leaf_order(n):
    # leaf 0 is the OUTERMOST map: the serial loop runs leaves in reverse
    a = rng.random((n, 6))
    b = rng.standard_normal((n, 6))
    h0 = rng.standard_normal(6)
    h = h0.copy()
    for t in reversed(range(n)):
        h = a[t] * h + b[t]
    _close(oracle.fused_diag_levels(a, b, h0), h, 1e-13)


@pytest.mark.parametrize("T", [1, 2, 5, 16, 17, 100])
def test_prefix_plan_closed_form_and_scan(T):
    p = oracle.prefix_plan(T)
    blk = math.ceil(math.sqrt(T))
    C = -(-T // blk)
    assert (p["blk"], p["C"], p["pad"]) == (blk, C, C * blk - T)
    assert p["starts"].tolist() == [c * blk for c in range(C)] and p["starts"].dtype == np.int64
    table = oracle.prefix_chunk_table(T)
    assert table[0] == 0 and table[-1] == T and np.all(np.diff(table) > 0)
    A, B = rng.random((T, 3)), rng.standard_normal((T, 3))
    Pa, Pb = oracle.prefix_scan(A, B)
    ca, cb = np.ones(3), np.zeros(3)
    for t in range(T):  # brute-force all prefixes: P_t = leaf_t ∘ … ∘ leaf_0
        ca, cb = A[t] * ca, A[t] * cb + B[t]
        _close(Pa[t], ca, 1e-13)
        _close(Pb[t], cb, 1e-13)


def test_serial_affd_scan_closed_form_lti():
    T, S = 9, 4
    a = rng.random(S)
    u = rng.standard_normal((T, S))
    h0 = rng.standard_normal(S)
    out = oracle.serial_affd_scan(a, u, h0)
    for t in range(T):
        closed = a ** (t + 1) * h0 + sum(a ** (t - s) * u[s] for s in range(t + 1))
        _close(out[t], closed, 1e-12)


@pytest.mark.parametrize("aps", [True, False])
def test_ssm_serial_brute_force_and_chunked(aps):
    B, T, D, N = 2, 11, 3, 4
    a = rng.random((B, T, D, N) if aps else (B, T, D))
    bx, c = rng.standard_normal((B, T, N)), rng.standard_normal((B, T, N))
    x = rng.standard_normal((B, T, D))
    h0 = rng.standard_normal((B, D, N))
    y, hT = oracle.ssm_serial(a, bx, c, x, h0)
    for b in range(B):
        for d in range(D):
            for n in range(N):
                h = h0[b, d, n]
                for t in range(T):
                    at = a[b, t, d, n] if aps else a[b, t, d]
                    h = at * h + bx[b, t, n] * x[b, t, d]
                assert hT[b, d, n] == pytest.approx(h, rel=1e-12, abs=1e-12)
    yb = np.zeros((B, T, D))
    for b in range(B):
        for d in range(D):
            h = h0[b, d].copy()
            for t in range(T):
                at = a[b, t, d] if aps else np.full(N, a[b, t, d])
                h = at * h + bx[b, t] * x[b, t, d]
                yb[b, t, d] = c[b, t] @ h
    _close(y, yb, 1e-12)
    for table in ([0, T], [0, 4, 8, T], list(oracle.prefix_chunk_table(T))):
        yc, hc = oracle.ssm_chunked(a, bx, c, x, h0, np.asarray(table))
        _close(yc, yb, 1e-12)
        _close(hc, hT, 1e-12)


# ------------------------------------------------------------------ dense scans


def test_aff_compose_order_homogeneous_and_associative():
    d = 5
    f = (rng.standard_normal((d, d)), rng.standard_normal(d))
    g = (rng.standard_normal((d, d)), rng.standard_normal(d))
    e = (rng.standard_normal((d, d)), rng.standard_normal(d))
    h = rng.standard_normal(d)
    fg = oracle.aff_compose(f, g)
    _close(oracle.aff_apply(fg, h), oracle.aff_apply(f, oracle.aff_apply(g, h)), 1e-12)  # g applied first
    swapped = oracle.aff_compose(g, f)
    assert np.max(np.abs(oracle.aff_apply(swapped, h) - oracle.aff_apply(fg, h))) > 1e-6
    # the homogeneous-matrix trick: packing is a monoid homomorphism onto matmul
    Mf, Mg = oracle.aff_homogeneous(f[0][None], f[1][None])[0], oracle.aff_homogeneous(g[0][None], g[1][None])[0]
    Mfg = oracle.aff_homogeneous(fg[0][None], fg[1][None])[0]
    _close(Mf @ Mg, Mfg, 1e-12)
    _close((Mf @ np.append(h, 1.0))[:d], oracle.aff_apply(f, h), 1e-12)
    l1 = oracle.aff_compose(oracle.aff_compose(f, g), e)
    l2 = oracle.aff_compose(f, oracle.aff_compose(g, e))
    _close(l1[0], l2[0], 1e-12)
    _close(l1[1], l2[1], 1e-12)


@pytest.mark.parametrize("n", [1, 2, 5, 8])
def test_fused_dense_levels_reversed_leaf_order(n):
    d = 4
    A = rng.standard_normal((n, d, d)) * 0.5
    b = rng.standard_normal((n, d))
    h0 = rng.standard_normal(d)
    h = h0.copy()
    for t in reversed(range(n)):  # leaf 0 is the OUTERMOST map
        h = np.array([sum(A[t, i, j] * h[j] for j in range(d)) for i in range(d)]) + b[t]
    _close(oracle.fused_dense_levels(oracle.aff_homogeneous(A, b), h0), h, 1e-12)


def test_serial_aff_scan_closed_form_lti():
    T, d, k = 9, 4, 3
    A = rng.standard_normal((d, d)) * 0.5
    assert np.max(np.abs(A - A.T)) > 1e-3  # a transposed operand would show
    b = rng.standard_normal((T, d))
    h0 = rng.standard_normal((d, k))
    out = oracle.serial_aff_scan(A, b, h0)
    mp = np.linalg.matrix_power
    for t in range(T):
        closed = mp(A, t + 1) @ h0 + sum(mp(A, t - s) @ b[s] for s in range(t + 1))[:, None]
        _close(out[t], closed, 1e-12)
        wrong = mp(A.T, t + 1) @ h0 + sum(mp(A.T, t - s) @ b[s] for s in range(t + 1))[:, None]
        if t > 0:
            assert np.max(np.abs(out[t] - wrong)) > 1e-6


def test_serial_aff_scan_special_cases():
    T, d = 7, 3
    b = rng.standard_normal((T, d))
    h0 = rng.standard_normal((d, 1))
    # A = I: running sums
    _close(oracle.serial_aff_scan(np.eye(d), b, h0)[..., 0], h0[:, 0] + np.cumsum(b, axis=0), 1e-12)
    # diagonal maps: the diagonal scan (pinned above by its closed form)
    a = rng.random((T, d))
    At = np.stack([np.diag(x) for x in a])
    _close(oracle.serial_aff_scan(At, b, h0)[..., 0], oracle.serial_affd_scan(a, b, h0[:, 0]), 1e-12)
    # per-slot maps: slot p evolves alone
    P = 3
    Ap = rng.standard_normal((T, P, d, d)) * 0.5
    bp = rng.standard_normal((T, P, d))
    hp = rng.standard_normal((P, d, 2))
    out = oracle.serial_aff_scan(Ap, bp, hp)
    for p in range(P):
        _close(out[:, p], oracle.serial_aff_scan(Ap[:, p], bp[:, p], hp[p]), 1e-12)


@pytest.mark.parametrize("T", [1, 7, 50])
@pytest.mark.parametrize("per_slot", [False, True])
def test_aff_chunked_scan_matches_serial(T, per_slot):
    d, P, k = 4, 2, 3
    A = rng.standard_normal((T, P, d, d) if per_slot else (d, d)) * 0.5
    b = rng.standard_normal((T, P, d))
    h0 = rng.standard_normal((P, d, k))
    ser = oracle.serial_aff_scan(A, b, h0)
    tables = [[0, T], list(oracle.prefix_chunk_table(T))] + ([[0, 3, 4, T]] if T > 4 else [])
    for table in tables:
        out, hT = oracle.aff_chunked_scan(A, b, h0, np.asarray(table))
        _close(out, ser, 1e-10)
        _close(hT, ser[-1], 1e-10)


# ------------------------------------------------------------------ deferred-affine om


def test_omd_elem_is_om_elem_of_the_affine_values():
    """The defining identity: applying the deferred carrier to h equals
    softmax attention over the materialised values a⊙h + b (diagonal) or
    A@h + b (dense)."""
    Tq, K, d = 5, 7, 4
    s = rng.standard_normal((2, Tq, K))  # two heads over shared per-key coefficients
    a, b, h = rng.standard_normal((K, d)), rng.standard_normal((K, d)), rng.standard_normal(d)
    f = oracle.omd_elem(s, a, b)
    dense = np.exp(s - s.max(-1, keepdims=True))
    dense = dense / dense.sum(-1, keepdims=True)
    _close(oracle.omd_apply(f, h), dense @ (a * h + b), 1e-12)
    _close(oracle.omd_apply(f, h), oracle.om_apply(oracle.om_elem(s, a * h + b)), 1e-12)
    A = rng.standard_normal((2, K, d, 3))
    hm = rng.standard_normal(3)
    fm = oracle.omd_elem(s, A, b)
    assert fm[2].shape == (2, Tq, d, 3)
    _close(oracle.omd_applym(fm, hm), dense @ (A @ hm + b), 1e-12)
    # a transposed map or a dropped offset would not pass
    Asq = rng.standard_normal((2, K, d, d))
    hs = rng.standard_normal(d)
    fsq = oracle.omd_elem(s, Asq, b)
    assert np.max(np.abs(oracle.omd_applym(fsq, hs) - dense @ (np.swapaxes(Asq, -1, -2) @ hs + b))) > 1e-6
    assert np.max(np.abs(oracle.omd_applym(fsq, hs) - dense @ (Asq @ hs))) > 1e-6


def test_omd_compose_is_om_compose_on_concatenated_numerators():
    Tq, K, d = 4, 6, 3
    s1, s2 = rng.standard_normal((Tq, K)), rng.standard_normal((Tq, K)) + 3.0
    a1, b1, a2, b2 = (rng.standard_normal((K, d)) for _ in range(4))
    f, g = oracle.omd_elem(s1, a1, b1), oracle.omd_elem(s2, a2, b2)
    c = oracle.omd_compose(f, g)
    om = oracle.om_compose((f[0], f[1], np.concatenate([f[2], f[3]], -1)),
                           (g[0], g[1], np.concatenate([g[2], g[3]], -1)))
    _close(c[0], om[0], 1e-12)
    _close(c[1], om[1], 1e-12)
    _close(np.concatenate([c[2], c[3]], -1), om[2], 1e-12)
    # = one leaf over the concatenated keys (the softmax is over all keys)
    whole = oracle.omd_elem(np.concatenate([s1, s2], -1), np.concatenate([a1, a2]), np.concatenate([b1, b2]))
    h = rng.standard_normal(d)
    _close(oracle.omd_apply(c, h), oracle.omd_apply(whole, h), 1e-12)
    # associativity, and order matters only through rounding
    e3 = oracle.omd_elem(rng.standard_normal((Tq, K)), rng.standard_normal((K, d)), rng.standard_normal((K, d)))
    l1 = oracle.omd_compose(oracle.omd_compose(f, g), e3)
    l2 = oracle.omd_compose(f, oracle.omd_compose(g, e3))
    _close(oracle.omd_apply(l1, h), oracle.omd_apply(l2, h), 1e-12)


def test_omd_compose_masked_block_and_dense_fibre():
    Tq, K, d, i = 3, 4, 2, 5
    s = rng.standard_normal((Tq, K))
    s_masked = s.copy()
    s_masked[1] = -np.inf  # row 1 of this block fully masked
    A, b = rng.standard_normal((K, d, i)), rng.standard_normal((K, d))
    f = oracle.omd_elem(s, A, b)
    with np.errstate(invalid="ignore"):
        g = oracle.omd_elem(s_masked, A, b)
    c = oracle.omd_compose(f, g)
    assert np.all(np.isfinite(c[2])) and np.all(np.isfinite(c[3]))
    # row 1: only f contributes
    _close(c[1][1], f[1][1], 1e-12)
    _close(c[2][1], f[2][1], 1e-12)
    # other rows: the two blocks of the same keys weigh equally
    _close(c[2][0] / c[1][0], f[2][0] / f[1][0], 1e-12)
    # both fully masked: the empty carrier (0/0 on apply, as dense softmax)
    with np.errstate(invalid="ignore"):
        z = oracle.omd_compose(g, g)
        out = oracle.omd_applym(z, rng.standard_normal(i))
    assert np.isneginf(z[0][1]).all() and z[1][1] == 0 and np.isnan(out[1]).all()


# ------------------------------------------- the torch CPU restatement
# oracle.torch_cpu (the CPU baseline bench.py times) against the numpy
# functions above, in float64 where the form allows it (fp32 for the
# chunked retention's promoted arithmetic)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def test_torch_cpu_weight_chain_and_swiglu():
    rng = np.random.default_rng(3)
    Ws = [rng.standard_normal((16, 16)) / 4 for _ in range(3)]
    bs = [rng.standard_normal(16) for _ in range(3)]
    x = rng.standard_normal((5, 16))
    W, adds = oracle.fold_linear_chain(Ws, bs)
    c = sum(adds[1:], adds[0]) if len(adds) > 1 else adds[0]
    got = oracle.torch_cpu.weight_chain(_t(x), _t(W), _t(np.asarray(c)))
    _close(oracle.linear_chain(x, Ws, bs), got.numpy(), 1e-12)
    g = 1 + 0.1 * rng.standard_normal(16)
    wg, wu, wd = rng.standard_normal((24, 16)), rng.standard_normal((24, 16)), rng.standard_normal((16, 24))
    got = oracle.torch_cpu.swiglu_block(_t(x), _t(g), _t(wg), _t(wu), _t(wd), 1e-6)
    _close(oracle.swiglu_fused(oracle.rms_norm(x, g, 1e-6), wg, wu, wd), got.numpy(), 1e-12)


def test_torch_cpu_causal_attention():
    rng = np.random.default_rng(4)
    q, k, v = (rng.standard_normal((2, 3, 40, 8)) for _ in range(3))
    got = oracle.torch_cpu.causal_attention(_t(q), _t(k), _t(v), 0.3)
    _close(oracle.attention_om(q, k, v, 0.3, causal=True), got.numpy(), 1e-12)


def test_torch_cpu_retention_chunked_equals_quadratic():
    rng = np.random.default_rng(5)
    q, k, v = (rng.standard_normal((2, 3, 256, 16)).astype(np.float32) / 4 for _ in range(3))
    g = np.array([0.9, 0.97, 0.995], dtype=np.float32)
    got = oracle.torch_cpu.retention_chunked(_t(q), _t(k), _t(v), _t(g), 64, 0.5)
    ref = oracle.retention_quadratic(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                                     g.astype(np.float64), 0.5)
    _close(ref, got.double().numpy(), 1e-5)


def test_torch_cpu_scans():
    rng = np.random.default_rng(6)
    B, T, D, N = 2, 50, 6, 4
    a = rng.random((B, T, D, N)) * 0.9
    bx, c = rng.standard_normal((B, T, N)), rng.standard_normal((B, T, N))
    x = rng.standard_normal((B, T, D))
    ys, _ = oracle.ssm_serial(a, bx, c, x)
    got = oracle.torch_cpu.ssm_scan(_t(a), _t(bx), _t(c), _t(x), torch.zeros(B, D, N, dtype=torch.float64))
    _close(ys, got.numpy(), 1e-12)
    A = rng.standard_normal((5, 5)) * 0.3
    b = rng.standard_normal((30, 7, 5))
    h = rng.standard_normal((7, 5))
    ref = oracle.serial_aff_scan(A, b, h[..., None])[-1][..., 0]
    _close(ref, oracle.torch_cpu.dense_scan(_t(A), _t(b), _t(h)).numpy(), 1e-12)


def test_torch_cpu_omd_attention():
    rng = np.random.default_rng(7)
    T, d, Tq, dk = 40, 6, 9, 5
    q, k = rng.standard_normal((Tq, dk)), rng.standard_normal((T, dk))
    a, x, h = rng.random((T, d)) * 0.5 + 0.5, rng.standard_normal((T, d)), rng.standard_normal(d)
    states = oracle.serial_affd_scan(a, x, h)
    s = q @ k.T
    w = np.exp(s - s.max(-1, keepdims=True))
    ref = (w / w.sum(-1, keepdims=True)) @ states
    _close(ref, oracle.torch_cpu.omd_attention(_t(q), _t(k), _t(a), _t(x), _t(h)).numpy(), 1e-12)
