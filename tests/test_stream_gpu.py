"""Streaming / decode om attention on the GPU (``catopt_amd.executors.stream``).

The counterpart of the reference's ``tests/test_om_stream.py`` and the decode
cases of ``tests/test_om_lower_edges.py:520-560``: the left fold over an om
tree equals dense softmax attention whatever the tree's bracketing, the
chunked-K/V term folds block by block, raw-score and packaged ``om`` leaves
fold in order, and ``om_step_qk`` from ``om_empty_state`` (or from ``None``)
reproduces the dense result one block at a time — also when the decode step
is recorded into a hipGraph and replayed on new blocks.  References: the
numpy oracle's ``om_elem`` / ``om_compose`` / ``om_apply`` fold and the
closed-form softmax, in float64.  Gates: bf16 ≤ 2e-2, fp32 ≤ 1e-5.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.executors import (
    HipStreamingOMModule,
    om_apply_state,
    om_empty_state,
    om_step,
    om_step_qk,
    to_streaming_om_module,
)
from catopt_amd.ir import IR, Const, Op, TensorType, Var

pytestmark = pytest.mark.gpu
mk = Op.make
TOL_BF16 = 2e-2
TOL_F32 = 1e-5


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _gate(ref, out, tol):
    rep = oracle.verify_equiv(ref, _np(out), rtol=tol)
    assert rep["passed"], rep
    return rep


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _dense(q, ks, vs, scale=1.0):
    k = np.concatenate([_np(x) for x in ks], axis=-2)
    v = np.concatenate([_np(x) for x in vs], axis=-2)
    s = _np(q) @ np.swapaxes(k, -1, -2) * scale
    s = s - s.max(-1, keepdims=True)
    e = np.exp(s)
    return (e / e.sum(-1, keepdims=True)) @ v


def _oracle_fold(q, ks, vs, scale=1.0):
    st = None
    for k, v in zip(ks, vs):
        e = oracle.om_elem(_np(q) @ np.swapaxes(_np(k), -1, -2) * scale, _np(v))
        st = e if st is None else oracle.om_compose(st, e)
    return oracle.om_apply(st)


def _balanced(leaves):
    if len(leaves) == 1:
        return leaves[0]
    mid = len(leaves) // 2
    return mk("om_compose", _balanced(leaves[:mid]), _balanced(leaves[mid:]))


def _left(leaves):
    t = leaves[0]
    for lf in leaves[1:]:
        t = mk("om_compose", t, lf)
    return t


def _qk_ir(B, H, T, d, kb, n, tree, scale=None):
    q = Var("q", TensorType((B, H, T, d)))
    ks = [Var(f"k{i}", TensorType((B, H, kb, d))) for i in range(n)]
    vs = [Var(f"v{i}", TensorType((B, H, kb, d))) for i in range(n)]

    def score(k):
        s = mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))
        return s if scale is None else mk("mul", s, Const(scale))

    root = mk("om_apply", tree([mk("om_elem", score(k), v) for k, v in zip(ks, vs)]))
    return IR(root, [q, *ks, *vs])


@pytest.mark.parametrize("tree", [_balanced, _left])
@pytest.mark.parametrize("d", [64, 128])
def test_streaming_matches_dense_and_oracle_fold(dev, tree, d):
    B, H, T, kb, n = 2, 4, 256, 64, 4
    scale = 1.0 / math.sqrt(d)
    ir = _qk_ir(B, H, T, d, kb, n, tree, scale)
    mod = to_streaming_om_module(ir)
    assert isinstance(mod, HipStreamingOMModule) and mod.is_streaming and mod.n_blocks == n
    q = _rand((B, H, T, d), torch.bfloat16, 1)
    ks = [_rand((B, H, kb, d), torch.bfloat16, 10 + i) for i in range(n)]
    vs = [_rand((B, H, kb, d), torch.bfloat16, 20 + i) for i in range(n)]
    out = mod(q.to(dev), *(x.to(dev) for x in ks), *(x.to(dev) for x in vs))
    assert mod.kernel_leaves == n  # every block folded by the attention kernel
    assert out.dtype == torch.bfloat16 and out.shape == (B, H, T, d)
    ref = _dense(q, ks, vs, scale)
    assert np.abs(ref - _oracle_fold(q, ks, vs, scale)).max() < 1e-10  # the fold is softmax
    _gate(ref, out, TOL_BF16)
    # the raw carrier: (m, l) per row, a relative to m
    m, lv, a = mod.forward_state(q.to(dev), *(x.to(dev) for x in ks), *(x.to(dev) for x in vs))
    assert m.dtype == torch.float32 and m.shape == (B, H, T, 1) and a.shape == (B, H, T, d)
    s = _np(q) @ np.swapaxes(np.concatenate([_np(x) for x in ks], -2), -1, -2) * scale
    _gate(s.max(-1, keepdims=True), m, 1e-5)
    _gate(np.exp(s - s.max(-1, keepdims=True)).sum(-1, keepdims=True), lv, TOL_BF16)


def test_streaming_chunked_kv_term(dev):
    """om_apply over om_elem(q @ chunk(K, i)ᵀ, chunk(V, i)): the chunk views
    are evaluated per leaf, never the full score matrix."""
    B, H, Tq, d, n, C = 2, 2, 128, 128, 4, 64
    q = Var("q", TensorType((B, H, Tq, d)))
    Kv = Var("K", TensorType((B, H, n * C, d)))
    Vv = Var("V", TensorType((B, H, n * C, d)))
    leaves = [mk("om_elem", mk("matmul", q, mk("transpose", mk("chunk", Kv, chunks=n, dim=-2, index=i),
                                                dim0=-2, dim1=-1)),
                 mk("chunk", Vv, chunks=n, dim=-2, index=i)) for i in range(n)]
    mod = to_streaming_om_module(IR(mk("om_apply", _balanced(leaves)), [q, Kv, Vv]))
    assert mod.is_streaming and mod.n_blocks == n
    tq = _rand((B, H, Tq, d), torch.bfloat16, 3, 0.3)
    tK = _rand((B, H, n * C, d), torch.bfloat16, 4, 0.3)
    tV = _rand((B, H, n * C, d), torch.bfloat16, 5)
    out = mod(tq.to(dev), tK.to(dev), tV.to(dev))
    assert mod.kernel_leaves == n
    _gate(_dense(tq, [tK], [tV]), out, TOL_BF16)


def test_streaming_score_vars_and_om_leaf_fp32(dev):
    """Raw score leaves and a packaged om(m, l, a) leaf fold in tree order
    (fp32: the elem path; reference test_om_stream.py:214-260)."""
    B, H, T, dv, K = 1, 2, 16, 8, 8
    ss = [Var(f"s{i}", TensorType((B, H, T, K))) for i in range(2)]
    vs = [Var(f"v{i}", TensorType((B, H, K, dv))) for i in range(2)]
    m3, l3, a3 = Var("m3", TensorType((B, H, T, 1))), Var("l3", TensorType((B, H, T, 1))), \
        Var("a3", TensorType((B, H, T, dv)))
    tree = mk("om_compose", mk("om_compose", mk("om_elem", ss[0], vs[0]), mk("om", m3, l3, a3)),
              mk("om_elem", ss[1], vs[1]))
    mod = to_streaming_om_module(IR(mk("om_apply", tree), [*ss, *vs, m3, l3, a3]))
    assert mod.is_streaming and [lf["kind"] for lf in mod._plan["leaves"]] == ["elem", "om", "elem"]
    tss = [_rand((B, H, T, K), torch.float32, 30 + i) for i in range(2)]
    tvs = [_rand((B, H, K, dv), torch.float32, 40 + i) for i in range(2)]
    s3, v3 = _rand((B, H, T, K), torch.float32, 50), _rand((B, H, K, dv), torch.float32, 51)
    e3 = oracle.om_elem(_np(s3), _np(v3))
    st = oracle.om_compose(oracle.om_compose(oracle.om_elem(_np(tss[0]), _np(tvs[0])), e3),
                           oracle.om_elem(_np(tss[1]), _np(tvs[1])))
    carr = [torch.from_numpy(x).float().to(dev) for x in e3]
    out = mod(*(x.to(dev) for x in tss), *(x.to(dev) for x in tvs), *carr)
    assert mod.kernel_leaves == 0
    _gate(oracle.om_apply(st), out, TOL_F32)


def test_decode_steps_from_empty_and_none(dev):
    """om_step_qk over K/V blocks, one at a time (reference
    test_om_lower_edges.py:540-560): the final readout is dense softmax,
    starting from om_empty_state or from None alike, and om_step on the
    materialised score agrees with the fused step."""
    B, H, T, d, kb, n = 2, 4, 32, 128, 64, 5
    q = _rand((B, H, T, d), torch.bfloat16, 60, 0.2)
    ks = [_rand((B, H, kb, d), torch.bfloat16, 61 + i, 0.2) for i in range(n)]
    vs = [_rand((B, H, kb, d), torch.bfloat16, 71 + i) for i in range(n)]
    qd, kd, vd = q.to(dev), [x.to(dev) for x in ks], [x.to(dev) for x in vs]
    st_none, st_empty, st_dense = None, om_empty_state((B, H, T), d, device=dev, dtype=torch.float32), None
    for k, v in zip(kd, vd):
        st_none = om_step_qk(st_none, qd, k, v)
        st_empty = om_step_qk(st_empty, qd, k, v)
        st_dense = om_step(st_dense, (qd.float() @ k.float().transpose(-2, -1)), v.float())
    ref = _dense(q, ks, vs)
    _gate(ref, om_apply_state(st_none), TOL_BF16)
    _gate(ref, om_apply_state(st_empty), TOL_BF16)
    _gate(ref, om_apply_state(st_dense), 1e-4)
    assert torch.equal(st_none[0], st_empty[0])  # the empty state is the identity
    m, lv, a = om_empty_state((3, 4), 6)
    assert m.shape == (3, 4, 1) and torch.isneginf(m).all() and not lv.any() and not a.any()


def test_decode_step_in_a_hip_graph(dev):
    """A decode step recorded into a hipGraph: replays on new K/V blocks,
    with eager work in between, match the eager step every time."""
    B, H, T, d, kb = 1, 4, 16, 64, 64
    q = _rand((B, H, T, d), torch.bfloat16, 80).to(dev)
    k0 = _rand((B, H, kb, d), torch.bfloat16, 81).to(dev)
    v0 = _rand((B, H, kb, d), torch.bfloat16, 82).to(dev)
    st0 = om_step_qk(None, q, k0, v0)
    st_in = tuple(t.clone() for t in st0)
    k_in, v_in = torch.empty_like(k0), torch.empty_like(v0)
    k_in.copy_(k0), v_in.copy_(v0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            om_step_qk(st_in, q, k_in, v_in)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st_out = om_step_qk(st_in, q, k_in, v_in)
    for rep in range(3):
        kn = _rand((B, H, kb, d), torch.bfloat16, 90 + rep).to(dev)
        vn = _rand((B, H, kb, d), torch.bfloat16, 95 + rep).to(dev)
        k_in.copy_(kn), v_in.copy_(vn)
        g.replay()
        eager = om_step_qk(st0, q, kn, vn)
        torch.cuda.synchronize()
        for x, y in zip(st_out, eager):
            assert torch.equal(x, y), rep
        _gate(_dense(q.cpu(), [k0.cpu(), kn.cpu()], [v0.cpu(), vn.cpu()]), om_apply_state(st_out), TOL_BF16)


def _chunked_kv_ir(B, H, Tq, d, dv, Tkv, C):
    n = Tkv // C
    q = Var("q", TensorType((B, H, Tq, d)))
    Kv = Var("K", TensorType((B, H, n * C, d)))
    Vv = Var("V", TensorType((B, H, n * C, dv)))
    leaves = [mk("om_elem", mk("matmul", q, mk("transpose", mk("chunk", Kv, chunks=n, dim=-2, index=i),
                                                dim0=-2, dim1=-1)),
                 mk("chunk", Vv, chunks=n, dim=-2, index=i)) for i in range(n)]
    return IR(mk("om_apply", _balanced(leaves)), [q, Kv, Vv])


def _peak_bytes(fn):
    """Device bytes allocated during ``fn`` beyond what was live before."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    fn()
    torch.cuda.synchronize()
    return torch.cuda.max_memory_allocated() - base


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_streaming_peak_memory_is_flat_in_the_key_count(dev, dtype):
    # the reference's test_om_stream.py:368-401 shapes: the fold's working
    # set tracks the block, not the key count (8 blocks, then 16)
    B, H, Tq, d, dv, C = 1, 8, 32, 64, 64, 2048
    peaks = []
    for Tkv in (16384, 32768):
        mod = to_streaming_om_module(_chunked_kv_ir(B, H, Tq, d, dv, Tkv, C))
        q = torch.randn(B, H, Tq, d, device=dev).to(dtype)
        K = torch.randn(B, H, Tkv, d, device=dev).to(dtype)
        V = torch.randn(B, H, Tkv, dv, device=dev).to(dtype)
        mod(q, K, V)  # first call outside the measurement (library workspaces)
        peaks.append(_peak_bytes(lambda: mod(q, K, V)))
        del q, K, V
    s1, s2 = peaks
    assert s2 < s1 * 1.5 + 4 * 2 ** 20, peaks
    # and far below one block-set of scores over every key
    assert s2 < B * H * Tq * 32768 * 4 // 4, peaks


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_streaming_where_the_full_scores_would_be_half_a_gib(dev, dtype):
    # the reference's test_om_stream.py:404-426: T_kv = 262144, whose full
    # score matrix is 512 MiB in fp32; the fold needs about one block
    B, H, Tq, d, dv, C = 1, 8, 64, 64, 64, 4096
    Tkv = 262144
    mod = to_streaming_om_module(_chunked_kv_ir(B, H, Tq, d, dv, Tkv, C))
    q = (torch.randn(B, H, Tq, d, device=dev) * 0.125).to(dtype)
    K = torch.randn(B, H, Tkv, d, device=dev).to(dtype)
    V = torch.randn(B, H, Tkv, dv, device=dev).to(dtype)
    mod(q, K, V)  # first call outside the measurement (library workspaces)
    out = None

    def run():
        nonlocal out
        out = mod(q, K, V)

    peak = _peak_bytes(run)
    score_bytes = B * H * Tq * Tkv * 4
    assert peak < score_bytes // 8, (peak, score_bytes)
    # the result on a sample of heads and rows against the dense softmax
    for h in (0, 5):
        s = q[0, h, ::16].double() @ K[0, h].double().T
        ref = torch.softmax(s, dim=-1) @ V[0, h].double()
        rep = oracle.verify_equiv(ref.cpu().numpy(), _np(out[0, h, ::16]), rtol=TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)
        assert rep["passed"], rep
