"""Every om leaf spelling on the HIP kernels, against the numpy oracle.

Each test delivers an ``om_apply`` term through ``HipSink`` (routed to the
``om_batched`` executor), then checks the output against the oracle's
``om_elem`` / ``fused_om_levels`` / ``om_apply`` over the same bf16-rounded
(or fp32) inputs, that every leaf ran on a HIP kernel (``kernel_leaves``,
``fallbacks == 0``), and NaN positions exactly where a row has no key.
Spellings: the sdpa-cat right-hand sides (scale as ``mul(q, fill(q, SC))``,
key-axis ``concat`` of products, causal ``cmask``) whole and split into key
blocks; ``add(·, attnbias(m))`` with weight and input masks, bool and float;
explicit score blocks and packaged carriers; fp32 operands; the ``sdpa``
binding; ``specialize_causal`` on the device; the delivery record.
Gates: bf16 ≤ 2e-2, fp32 ≤ 1e-4 (global relative error, the verify metric).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import forms
from catopt_amd.evaluator import HipIRModule
from catopt_amd.executors import HipOMModule
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make
NEG_INF = Const(float("-inf"))
TOL_BF16, TOL_F32 = 2e-2, 1e-4


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _rand(shape, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _gate_nan(ref, out, tol):
    on = _np(out) if isinstance(out, torch.Tensor) else out
    assert on.shape == ref.shape, (on.shape, ref.shape)
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    rep = oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, on, 0), rtol=tol)
    assert rep["passed"], rep


def _oracle_blocks(s, v, cuts):
    """om over key blocks of an explicit score ``s`` (float64): one
    ``om_elem`` per block, reduced by ``fused_om_levels``."""
    edges = [0, *np.cumsum(cuts)]
    leaves = [oracle.om_elem(s[..., a:b], v[..., a:b, :]) for a, b in zip(edges[:-1], edges[1:])]
    return oracle.fused_om_levels(np.stack([f[0] for f in leaves]), np.stack([f[1] for f in leaves]),
                                  np.stack([f[2] for f in leaves]))


def _qkt(q, k):
    return mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))


def _tree(leaves):
    t = leaves[0]
    for lf in leaves[1:]:
        t = mk("om_compose", t, lf)
    return mk("om_apply", t)


def _deliver(sink, ir, params, inputs, n_kernel):
    res = deliver(ir, params, sink, tuple(inputs))
    mod = res.module
    assert isinstance(mod, HipOMModule) and res.stats["executor"] == "om_batched"
    out = mod(*inputs)
    assert mod.fallbacks == 0
    assert mod.kernel_leaves == n_kernel, mod.leaf_kinds
    assert res.stats["hip_kernel"] and res.stats["torch_fallback_ops"] == 0
    return out


# ----------------------------------------------------------- sdpa-cat forms


def _sdpa_cat_ir(B, H, Tq, cuts, d, sc, causal, split):
    q = Var("q", TensorType((B, H, Tq, d)))
    ks = [Var(f"k{i}", TensorType((B, H, c, d))) for i, c in enumerate(cuts)]
    vs = [Var(f"v{i}", TensorType((B, H, c, d))) for i, c in enumerate(cuts)]
    qs = mk("mul", q, mk("fill", q, value=sc))
    S = mk("concat", *[_qkt(qs, k) for k in ks], dim=-1)
    V = mk("concat", *vs, dim=-2)
    M = mk("cmask", S)
    if not split:
        s = mk("masked_fill", S, M, NEG_INF) if causal else S
        root = mk("om_apply", mk("om_elem", s, V))
    else:
        leaves = []
        for i in range(len(cuts)):
            s_i = mk("split", S, sizes=tuple(cuts), dim=-1, index=i)
            if causal:
                s_i = mk("masked_fill", s_i, mk("split", M, sizes=tuple(cuts), dim=-1, index=i), NEG_INF)
            leaves.append(mk("om_elem", s_i, mk("split", V, sizes=tuple(cuts), dim=-2, index=i)))
        root = _tree(leaves)
    return IR(root, [q, *ks, *vs])


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("split", [False, True])
def test_sdpa_cat_forms(sink, dev, d, causal, split):
    B, H, Tq, cuts, sc = 1, 4, 192, (96, 96), d ** -0.5
    ir = _sdpa_cat_ir(B, H, Tq, cuts, d, sc, causal, split)
    q = _rand((B, H, Tq, d), 1)
    ks = [_rand((B, H, c, d), 10 + i) for i, c in enumerate(cuts)]
    vs = [_rand((B, H, c, d), 20 + i) for i, c in enumerate(cuts)]
    out = _deliver(sink, ir, {}, [t.to(dev) for t in (q, *ks, *vs)], 2 if split else 1)
    K = np.concatenate([_np(k) for k in ks], -2)
    V = np.concatenate([_np(v) for v in vs], -2)
    # the scale is applied as q·fill(q, SC) in q's dtype: bf16(SC)
    scq = float(torch.tensor(sc, dtype=torch.bfloat16))
    s = scq * (_np(q) @ np.swapaxes(K, -1, -2))
    if causal:
        s = np.where(oracle.cmask_keep(Tq, sum(cuts)), s, -np.inf)
    _gate_nan(_oracle_blocks(s, V, cuts if split else (sum(cuts),)), out, TOL_BF16)


def test_sdpa_cat_split_blocks_with_uneven_sizes_and_empty_rows(sink, dev):
    # causal blocks of 80 / 176 keys over 96 queries: in the second block
    # rows 0..79 see no key and contribute nothing
    B, H, Tq, cuts, d = 2, 2, 96, (80, 176), 128
    ir = _sdpa_cat_ir(B, H, Tq, cuts, d, 0.088, True, True)
    q = _rand((B, H, Tq, d), 3)
    ks = [_rand((B, H, c, d), 30 + i) for i, c in enumerate(cuts)]
    vs = [_rand((B, H, c, d), 40 + i) for i, c in enumerate(cuts)]
    out = _deliver(sink, ir, {}, [t.to(dev) for t in (q, *ks, *vs)], 2)
    K = np.concatenate([_np(k) for k in ks], -2)
    V = np.concatenate([_np(v) for v in vs], -2)
    scq = float(torch.tensor(0.088, dtype=torch.bfloat16))
    s = np.where(oracle.cmask_keep(Tq, sum(cuts)), scq * (_np(q) @ np.swapaxes(K, -1, -2)), -np.inf)
    _gate_nan(_oracle_blocks(s, V, cuts), out, TOL_BF16)


# ------------------------------------------------------------ attnbias forms


def _bias_ir(B, H, T, d, m_term, cuts=None):
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    S = mk("mul", _qkt(q, k), Const(d ** -0.5))
    bias = mk("attnbias", m_term)
    inputs = [q, k, v] + ([m_term] if isinstance(m_term, Var) else [])
    if cuts is None:
        return IR(mk("om_apply", mk("om_elem", mk("add", S, bias), v)), inputs)
    leaves = [mk("om_elem", mk("add", mk("split", S, sizes=cuts, dim=-1, index=i),
                               mk("split", bias, sizes=cuts, dim=-1, index=i)),
                 mk("split", v, sizes=cuts, dim=-2, index=i)) for i in range(len(cuts))]
    return IR(_tree(leaves), inputs)


def _bias_oracle(q, k, v, d, bias, cuts):
    s = d ** -0.5 * (_np(q) @ np.swapaxes(_np(k), -1, -2)) + bias
    return _oracle_blocks(s, _np(v), cuts)


@pytest.mark.parametrize("kind", ["param_bool", "param_float", "input_bool", "input_float"])
@pytest.mark.parametrize("cuts", [None, (100, 156)])
def test_attnbias_forms(sink, dev, kind, cuts):
    B, H, T, d = 1, 2, 256, 64
    rng = np.random.default_rng(7)
    keep = rng.random((T, T)) < 0.4
    keep[9, :] = False  # a row with no key: NaN, as dense softmax
    fbias = rng.standard_normal((T, T)).astype(np.float32)
    fbias[17, :] = -np.inf
    fbias[30, rng.random(T) < 0.5] = -np.inf
    if kind.endswith("bool"):
        mval, bias_np = torch.from_numpy(keep), np.where(keep, 0.0, -np.inf)
    else:
        mval, bias_np = torch.from_numpy(fbias), fbias.astype(np.float64)
    if kind.startswith("param"):
        m_term, params, extra = Param("m", TensorType((T, T))), {"m": mval}, []
    else:
        m_term, params, extra = Var("m", TensorType((T, T))), {}, [mval.to(dev)]
    ir = _bias_ir(B, H, T, d, m_term, cuts)
    q, k, v = (_rand((B, H, T, d), s) for s in (50, 51, 52))
    out = _deliver(sink, ir, params, [q.to(dev), k.to(dev), v.to(dev), *extra], 1 if cuts is None else 2)
    _gate_nan(_bias_oracle(q, k, v, d, bias_np, cuts or (T,)), out, TOL_BF16)


def test_per_head_bias_takes_the_score_path(sink, dev):
    # a bias that differs over (b, h) is not one plane: the leaf evaluates its
    # score and runs the om_rows kernel and the HIP GEMM
    B, H, T, d = 1, 2, 64, 64
    rng = np.random.default_rng(8)
    bias = rng.standard_normal((B, H, T, T)).astype(np.float32)
    m_term = Var("m", TensorType((B, H, T, T)))
    ir = _bias_ir(B, H, T, d, m_term)
    q, k, v = (_rand((B, H, T, d), s) for s in (60, 61, 62))
    res = deliver(ir, {}, sink, (q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(bias).to(dev)))
    mod = res.module
    out = mod(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(bias).to(dev))
    assert mod.fallbacks == 0 and mod.kernel_leaves == 0 and mod.leaf_kinds == ["attn"]
    _gate_nan(_bias_oracle(q, k, v, d, bias.astype(np.float64), (T,)), out, TOL_BF16)


# ------------------------------------------------ explicit scores, carriers


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_explicit_score_blocks_and_a_packaged_carrier(sink, dev, dtype):
    # the reference's "slice" / "stack" score modes: leaves whose score is
    # an input block; one leaf is a packaged carrier om(m, l, a)
    T, d = 40, 48
    cuts = (24, 70)
    s_vars = [Var(f"s{i}", TensorType((3, T, c))) for i, c in enumerate(cuts)]
    v_vars = [Var(f"v{i}", TensorType((3, c, d))) for i, c in enumerate(cuts)]
    mm, ll, aa = Var("m", TensorType((3, T, 1))), Var("l", TensorType((3, T, 1))), Var("a", TensorType((3, T, d)))
    leaves = [mk("om_elem", s_vars[0], v_vars[0]), mk("om", mm, ll, aa), mk("om_elem", s_vars[1], v_vars[1])]
    ir = IR(_tree(leaves), [*s_vars, *v_vars, mm, ll, aa])
    rng = np.random.default_rng(9)
    ss = [rng.standard_normal((3, T, c)) * 2 for c in cuts]
    ss[0][1, 5, :] = -np.inf  # no key in this block for one row
    ss[0][2, 7, :] = -np.inf
    ss[1][2, 7, :] = -np.inf  # ...and in both blocks: then only the carrier holds the row
    vv = [rng.standard_normal((3, c, d)) for c in cuts]
    f0 = oracle.om_elem(rng.standard_normal((3, T, 5)), rng.standard_normal((3, 5, d)))
    ins = [torch.from_numpy(a).to(dtype) for a in (*ss, *vv)] + [torch.from_numpy(a).float() for a in f0]
    res = deliver(ir, {}, sink, tuple(t.to(dev) for t in ins))
    mod = res.module
    out = mod(*[t.to(dev) for t in ins])
    assert mod.leaf_kinds == ["scores", "om", "scores"] and mod.fallbacks == 0
    r = [_np(t) for t in ins]
    f0r = (r[4], r[5], r[6])
    ref = oracle.om_apply(oracle.om_compose(oracle.om_compose(oracle.om_elem(r[0], r[2]), f0r),
                                            oracle.om_elem(r[1], r[3])))
    # bf16 scores are exact in fp32: the row kernel and the GEMM run in fp32
    _gate_nan(ref, out, TOL_F32)


def test_negative_scale_runs_the_score_path(sink, dev):
    B, H, T, d = 1, 2, 48, 64
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    ir = IR(mk("om_apply", mk("om_elem", mk("mul", _qkt(q, k), Const(-0.3)), v)), [q, k, v])
    xs = [_rand((B, H, T, d), s, torch.float32) for s in (70, 71, 72)]
    res = deliver(ir, {}, sink, tuple(t.to(dev) for t in xs))
    out = res.module(*[t.to(dev) for t in xs])
    assert res.module.leaf_kinds == ["scores"] and res.module.fallbacks == 0
    s = -0.3 * (_np(xs[0]) @ np.swapaxes(_np(xs[1]), -1, -2))
    _gate_nan(_oracle_blocks(s, _np(xs[2]), (T,)), out, TOL_F32)


@pytest.mark.parametrize("d", [40, 96])
def test_bf16_leaves_of_other_head_dims_run_the_attention_kernel(sink, dev, d):
    B, H, Tq, cuts = 1, 2, 128, (64, 64)
    ir = _sdpa_cat_ir(B, H, Tq, cuts, d, d ** -0.5, True, True)
    q = _rand((B, H, Tq, d), 5)
    ks = [_rand((B, H, c, d), 50 + i) for i, c in enumerate(cuts)]
    vs = [_rand((B, H, c, d), 60 + i) for i, c in enumerate(cuts)]
    out = _deliver(sink, ir, {}, [t.to(dev) for t in (q, *ks, *vs)], 2)
    K_ = np.concatenate([_np(k) for k in ks], -2)
    V = np.concatenate([_np(v) for v in vs], -2)
    scq = float(torch.tensor(d ** -0.5, dtype=torch.bfloat16))
    s = np.where(oracle.cmask_keep(Tq, sum(cuts)), scq * (_np(q) @ np.swapaxes(K_, -1, -2)), -np.inf)
    _gate_nan(_oracle_blocks(s, V, cuts), out, TOL_BF16)


@pytest.mark.parametrize("d", [32, 96])
def test_fp32_attention_runs_the_carrier_kernel(sink, dev, d):
    # fp32 operands, a head dim the bf16 kernel does not take: the fp32
    # carrier kernel, two key blocks composed
    B, H, T, cuts = 2, 2, 80, (30, 50)
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    S = mk("div", _qkt(q, k), Const(float(d) ** 0.5))
    leaves = [mk("om_elem", mk("split", S, sizes=cuts, dim=-1, index=i), mk("split", v, sizes=cuts, dim=-2, index=i))
              for i in range(2)]
    ir = IR(_tree(leaves), [q, k, v])
    xs = [_rand((B, H, T, d), s, torch.float32) for s in (80, 81, 82)]
    out = _deliver(sink, ir, {}, [t.to(dev) for t in xs], 2)
    s = (_np(xs[0]) @ np.swapaxes(_np(xs[1]), -1, -2)) / np.sqrt(d)
    _gate_nan(_oracle_blocks(s, _np(xs[2]), cuts), out, TOL_F32)


# ------------------------------------------------------------ sdpa binding


@pytest.mark.parametrize("mode", ["none", "causal", "bool", "float"])
def test_sdpa_binding_runs_the_attention_kernel(dev, mode):
    from catopt_amd import _lib as L
    from catopt_amd.bindings import torch_fallback_count

    B, H, T, d = 2, 3, 160, 128
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    rng = np.random.default_rng(11)
    keep = rng.random((T, T)) < 0.5
    keep[4] = False  # torch's sdpa gives 0 for a row with no key
    fb = rng.standard_normal((T, T)).astype(np.float32)
    args, ins, attrs = [q, k, v], [], {}
    if mode == "causal":
        attrs["arg5"] = True
    elif mode in ("bool", "float"):
        m = Var("m", TensorType((T, T)))
        args.append(m)
        ins.append(torch.from_numpy(keep if mode == "bool" else fb).to(dev))
    ir = IR(mk("sdpa", *args, **attrs), [q, k, v] + args[3:])
    xs = [_rand((B, H, T, d), s) for s in (90, 91, 92)]
    mod = HipIRModule(ir, {}, device=dev)
    n_hip, n_torch = L.call_count(), torch_fallback_count()
    out = mod(*[t.to(dev) for t in xs], *ins)
    assert L.call_count() > n_hip and torch_fallback_count() == n_torch
    s = d ** -0.5 * (_np(xs[0]) @ np.swapaxes(_np(xs[1]), -1, -2))
    if mode == "causal":
        s = np.where(oracle.cmask_keep(T, T), s, -np.inf)
    elif mode == "bool":
        s = np.where(keep, s, -np.inf)
    elif mode == "float":
        s = s + fb
    ref = _oracle_blocks(s, _np(xs[2]), (T,))
    ref = np.nan_to_num(ref, nan=0.0)  # torch's value for a row with no key
    on = _np(out)
    assert np.isfinite(on).all()
    rep = oracle.verify_equiv(ref, on, rtol=TOL_BF16)
    assert rep["passed"], rep


def test_specialize_causal_on_the_device_then_the_causal_kernel(sink, dev):
    B, H, T, d = 1, 2, 128, 64
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    mp = Param("mask", TensorType((T, T)))
    params = {"mask": torch.ones(T, T, dtype=torch.bool).triu(1)}  # the masked set
    term = mk("sdpa", q, k, v, mk("logical_not", mp))
    memo: dict = {}
    out_term = sink.specialize_causal(term, params, memo)
    assert memo.get("_hit") is True and out_term.attrs["arg5"] is True and len(out_term.args) == 3
    xs = [_rand((B, H, T, d), s) for s in (93, 94, 95)]
    out = HipIRModule(IR(out_term, [q, k, v]), {}, device=dev)(*[t.to(dev) for t in xs])
    s = np.where(oracle.cmask_keep(T, T), d ** -0.5 * (_np(xs[0]) @ np.swapaxes(_np(xs[1]), -1, -2)), -np.inf)
    rep = oracle.verify_equiv(_oracle_blocks(s, _np(xs[2]), (T,)), _np(out), rtol=TOL_BF16)
    assert rep["passed"], rep
    # a non-causal weight mask is left in place
    memo2: dict = {}
    params2 = {"mask": torch.zeros(T, T, dtype=torch.bool)}
    assert len(sink.specialize_causal(term, params2, memo2).args) == 4 and "_hit" not in memo2


def test_delivery_record_counts_hip_calls_on_generic_routed_forms(sink, dev):
    # C2's block routes to the generic module; the record shows it ran HIP
    # entry points only
    ir, shapes = forms.swiglu_block_form((64,), 128, 256)
    g = torch.Generator().manual_seed(0)
    vals = {n: (torch.randn(sh, generator=g) * 0.05).to(torch.bfloat16) for n, sh in shapes.items()}
    x = torch.randn(64, 128, generator=g).to(torch.bfloat16).to(dev)
    res = deliver(ir, vals, sink, (x,))
    assert res.stats["executor"] == "generic"
    assert res.stats["hip_calls"] >= 3 and res.stats["torch_fallback_ops"] == 0 and res.stats["hip_kernel"]
