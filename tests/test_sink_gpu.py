"""The drop-in path on the GPU: delivered terms routed through ``HipSink``.

Each test builds a delivered term (``catopt_amd.forms``), lowers it through
the sink's executor table exactly as catopt's orchestrator would (route →
lower → hipGraph runner → verify against the un-optimised program), and
compares the module's output with the numpy oracle on the same inputs.
Gates: fp32 ≤ 1e-5, bf16 ≤ 2e-2 (global relative error, the verify metric);
NaN positions exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import forms
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var
from catopt_amd.runner import HipGraphRunner
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _gate(ref, out, tol):
    rep = oracle.verify_equiv(ref, _np(out), rtol=tol)
    assert rep["passed"], rep
    return rep


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def test_weight_chain_full_config_with_graph_replay(sink, dev):
    torch.manual_seed(0)
    layers = [torch.nn.Linear(512, 512) for _ in range(8)]
    vals = {}
    for i, l in enumerate(layers):
        vals[f"W{i + 1}"], vals[f"b{i + 1}"] = l.weight.detach(), l.bias.detach()
    x = torch.randn(64, 512)
    ir, _ = forms.weight_chain_form(8, 512, 64)
    res = deliver(ir, vals, sink, (x.to(dev),), runner=HipGraphRunner())
    mod = res.module
    assert [s[0] for s in mod._tape.steps] == ["hip_linear"]
    assert res.stats["cuda_graph"] is True
    ref = oracle.linear_chain(x.double().numpy(), [_np(l.weight) for l in layers], [_np(l.bias) for l in layers])
    for _ in range(3):  # replays, with eager work in between
        y = mod(x.to(dev)).clone()
        torch.cuda.synchronize()
        _gate(ref, y, 1e-5)
        _ = torch.ones(8, device=dev).sum().item()
    x2 = torch.randn(64, 512)
    ref2 = oracle.linear_chain(x2.double().numpy(), [_np(l.weight) for l in layers], [_np(l.bias) for l in layers])
    _gate(ref2, mod(x2.to(dev)).clone(), 1e-5)


def _spelled_swiglu(D, F_, rows_shape, eps=1e-6):
    """The un-optimised source: x·rsqrt(mean(x², -1) + eps)·γ, then
    down(silu(gate(h)) · up(h)) (models/__init__.py:22-55)."""
    x = Var("x", TensorType((*rows_shape, D)))
    g = Param("gamma", TensorType((D,)))
    wg, wu = Param("W_gate", TensorType((F_, D))), Param("W_up", TensorType((F_, D)))
    wd = Param("W_down", TensorType((D, F_)))
    ms = mk("mean", mk("pow", x, Const(2)), dim=-1, keepdim=True)
    h = mk("mul", mk("mul", x, mk("rsqrt", mk("add", ms, Const(eps)))), g)
    out = mk("linear", mk("mul", mk("silu", mk("linear", h, wg)), mk("linear", h, wu)), wd)
    return IR(out, [x])


def test_swiglu_block_delivered_and_verified(sink, dev):
    D, F_, rows = 256, 512, (2, 64)
    ir, shapes = forms.swiglu_block_form(rows, D, F_)
    vals = {"gamma": (1 + 0.02 * _rand((D,), torch.float32, 1)).to(torch.bfloat16),
            "W_gate": _rand((F_, D), torch.bfloat16, 2, 0.05),
            "W_up": _rand((F_, D), torch.bfloat16, 3, 0.05),
            "W_down": _rand((D, F_), torch.bfloat16, 4, 0.05)}
    x = _rand((*rows, D), torch.bfloat16, 5)
    res = deliver(ir, vals, sink, (x.to(dev),), verify_ir=_spelled_swiglu(D, F_, rows), rtol=2e-2)
    assert res.verified.passed, res.verified
    assert [s[0] for s in res.module._tape.steps] == ["rms_norm", "hip_swiglu", "hip_linear"]
    h = oracle.rms_norm(_np(x), _np(vals["gamma"]), 1e-6)
    ref = oracle.swiglu_fused(h, _np(vals["W_gate"]), _np(vals["W_up"]), _np(vals["W_down"]))
    _gate(ref, res.module(x.to(dev)), 2e-2)


@pytest.mark.parametrize("mask", ["param", "cmask"])
def test_causal_attention_executor(sink, dev, mask):
    B, H, T, d = 1, 2, 256, 128
    ir, _ = forms.causal_attention_form(B, H, T, d, mask=mask)
    vals = {"mask": torch.ones(T, T, dtype=torch.bool).tril()} if mask == "param" else {}
    q, k, v = (_rand((B, H, T, d), torch.bfloat16, 10 + i) for i in range(3))
    res = deliver(ir, vals, sink, tuple(t.to(dev) for t in (q, k, v)), runner=HipGraphRunner())
    assert res.stats["executor"] == "om_batched" and res.stats["hip_kernel"]
    assert res.stats["cuda_graph"] is True
    out = res.module(*(t.to(dev) for t in (q, k, v))).clone()
    assert res.module.fallbacks == 0
    ref = oracle.attention_om(_np(q), _np(k), _np(v), 1 / math.sqrt(d), causal=True)
    _gate(ref, out, 2e-2)
    q2 = _rand((B, H, T, d), torch.bfloat16, 99)  # replay on new inputs recomputes
    out2 = res.module(q2.to(dev), k.to(dev), v.to(dev)).clone()
    _gate(oracle.attention_om(_np(q2), _np(k), _np(v), 1 / math.sqrt(d), causal=True), out2, 2e-2)


def test_attention_two_key_blocks_compose(sink, dev):
    """om_compose(om_elem(s_1, v_1), om_elem(s_2, v_2)) over key blocks with
    causal offsets: one kernel per leaf + the om_compose kernel."""
    B, H, T, d, T1 = 1, 2, 192, 128, 64
    q = Var("q", TensorType((B, H, T, d)))
    ks = [Var("k1", TensorType((B, H, T1, d))), Var("k2", TensorType((B, H, T - T1, d)))]
    vs = [Var("v1", TensorType((B, H, T1, d))), Var("v2", TensorType((B, H, T - T1, d)))]
    leaves = []
    for kk, vv, off in ((ks[0], vs[0], 0), (ks[1], vs[1], T1)):
        s = mk("mul", mk("matmul", q, mk("transpose", kk, dim0=-2, dim1=-1)), Const(1 / math.sqrt(d)))
        leaves.append(mk("om_elem", mk("masked_fill", s, mk("cmask", s, off=off), Const(float("-inf"))), vv))
    ir = IR(mk("om_apply", mk("om_compose", leaves[0], leaves[1])), [q, ks[0], ks[1], vs[0], vs[1]])
    qq, kk_, vv_ = (_rand((B, H, T, d), torch.bfloat16, 20 + i) for i in range(3))
    ins = (qq, kk_[:, :, :T1], kk_[:, :, T1:], vv_[:, :, :T1], vv_[:, :, T1:])
    res = deliver(ir, {}, sink, tuple(t.contiguous().to(dev) for t in ins))
    assert res.module.n_leaves == 2
    out = res.module(*(t.contiguous().to(dev) for t in ins))
    assert res.module.fallbacks == 0
    ref = oracle.attention_om(_np(qq), _np(kk_), _np(vv_), 1 / math.sqrt(d), causal=True)
    _gate(ref, out, 2e-2)


def test_attention_random_bool_mask_nan_rows(sink, dev):
    B, H, T, d = 1, 2, 128, 64
    ir, _ = forms.causal_attention_form(B, H, T, d, mask="param")
    keep = torch.rand(T, T, generator=torch.Generator().manual_seed(7)) < 0.4
    keep[9] = False  # a fully masked row: a / l = 0 / 0 = NaN there
    q, k, v = (_rand((B, H, T, d), torch.bfloat16, 30 + i) for i in range(3))
    res = deliver(ir, {"mask": keep}, sink, tuple(t.to(dev) for t in (q, k, v)))
    assert res.module._plan["leaves"][0]["mask_kind"] == "bool_const"
    out = _np(res.module(*(t.to(dev) for t in (q, k, v))))
    ref = oracle.attention_om(_np(q), _np(k), _np(v), 1 / math.sqrt(d), causal=False, mask=keep.numpy())
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, out, 0), rtol=2e-2)["passed"]


@pytest.mark.parametrize("C", [64, 128])
def test_retention_kway_executor(sink, dev, C):
    B, H, T = 1, 3, 512
    ir, _ = forms.retention_kway_form(B, H, T, 128, C, scale=0.5)
    gam = torch.tensor([1 - 2.0 ** (-5 - h / 2) for h in range(H)], dtype=torch.float32)
    q, k, v = (_rand((B, H, T, 128), torch.bfloat16, 40 + i, 1 / math.sqrt(128)) for i in range(3))
    res = deliver(ir, {"gamma": gam}, sink, tuple(t.to(dev) for t in (q, k, v)), runner=HipGraphRunner())
    assert res.stats["executor"] == "om_decayed_chunked" and res.stats["hip_kernel"]
    assert res.module.n_chunks == T // C
    out = res.module(*(t.to(dev) for t in (q, k, v))).clone()
    assert res.module.fallbacks == 0
    ref = oracle.retention_kway(_np(q), _np(k), _np(v), gam.double().numpy(), T // C, 0.5)
    _gate(ref, out, 2e-2)
    _gate(oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.double().numpy(), 0.5), out, 2e-2)
    assert res.stats["cuda_graph"] is True
    v2 = _rand((B, H, T, 128), torch.bfloat16, 77, 1 / math.sqrt(128))
    out2 = res.module(q.to(dev), k.to(dev), v2.to(dev)).clone()
    _gate(oracle.retention_quadratic(_np(q), _np(k), _np(v2), gam.double().numpy(), 0.5), out2, 2e-2)


def test_retention_kway_executor_head_dim_64(sink, dev):
    # d = 64 runs the d = 128 kernel on zero-padded operands, still no fallback
    B, H, T, d = 2, 2, 256, 64
    ir, _ = forms.retention_kway_form(B, H, T, d, 64)
    gam = torch.tensor([1 - 2.0 ** (-5 - h / 2) for h in range(H)], dtype=torch.float32)
    q, k, v = (_rand((B, H, T, d), torch.bfloat16, 50 + i, 1 / math.sqrt(d)) for i in range(3))
    res = deliver(ir, {"gamma": gam}, sink, tuple(t.to(dev) for t in (q, k, v)))
    assert res.stats["executor"] == "om_decayed_chunked" and res.stats["hip_kernel"]
    out = res.module(*(t.to(dev) for t in (q, k, v)))
    assert res.module.fallbacks == 0 and out.shape == (B, H, T, d)
    _gate(oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.double().numpy()), out, 2e-2)


def test_retention_verified_against_the_spelled_block_form(sink, dev):
    B, H, T = 1, 2, 256
    ir, _ = forms.retention_kway_form(B, H, T, 128, 64)
    irb, _ = forms.retention_block_form(B, H, T)
    gam = torch.tensor([0.96875, 0.99], dtype=torch.float32)
    ins = tuple(_rand((B, H, T, 128), torch.bfloat16, 50 + i, 1 / math.sqrt(128)).to(dev) for i in range(3))
    res = deliver(ir, {"gamma": gam}, sink, ins, verify_ir=irb, rtol=2e-2)
    assert res.verified.passed, res.verified


@pytest.mark.parametrize("form", ["final", "prefix"])
def test_scan_executor(sink, dev, form):
    T, S = 300, 1000
    rng = np.random.default_rng(6)
    a = rng.uniform(0.5, 1.0, (T, S)).astype(np.float32)
    u = rng.standard_normal((T, S)).astype(np.float32)
    h = rng.standard_normal(S).astype(np.float32)
    ir, _ = (forms.scan_final_form if form == "final" else forms.scan_prefix_form)(T, (S,))
    ins = tuple(torch.from_numpy(z).to(dev) for z in (a, u, h))
    res = deliver(ir, {}, sink, ins, runner=HipGraphRunner())
    assert res.stats["executor"] == "scan" and res.stats["hip_kernel"]
    assert res.stats["cuda_graph"] is True and res.module.is_graph_captured
    out = res.module(*ins).clone()
    assert res.module.fallbacks == 0
    ref = oracle.serial_affd_scan(a.astype(np.float64), u.astype(np.float64), h.astype(np.float64))
    _gate(ref[-1] if form == "final" else ref, out, 1e-5)
    # the replay recomputes from the new inputs (not the captured call's output)
    a2 = rng.uniform(0.2, 0.9, (T, S)).astype(np.float32)
    out2 = res.module(torch.from_numpy(a2).to(dev), ins[1], ins[2]).clone()
    ref2 = oracle.serial_affd_scan(a2.astype(np.float64), u.astype(np.float64), h.astype(np.float64))
    _gate(ref2[-1] if form == "final" else ref2, out2, 1e-5)


@pytest.mark.parametrize("N,per_state,dtype", [(16, True, torch.float32), (8, False, torch.float32),
                                               (3, True, torch.float32), (16, True, torch.bfloat16)])
def test_ssm_readout_executor(sink, dev, N, per_state, dtype):
    """The selective SSM delivered as sum(mul(<stacked prefix states>, c), -1):
    N in the kernel's set runs the fused scan + read-out (the states never
    reach HBM); N = 3 scans every prefix state along the stacked axis and
    reads out through the op table.  Replays follow new inputs."""
    B, T, D = 2, 300, 24
    ir, _ = forms.diag_ssm_form(B, T, D, N, a_per_state=per_state)
    rng = np.random.default_rng(8 + N)

    def inputs():
        z = rng.standard_normal((B, T, D, N) if per_state else (B, T, D))
        vals = (1.0 / (1.0 + np.exp(z)), rng.standard_normal((B, T, N)), rng.standard_normal((B, T, N)),
                rng.standard_normal((B, T, D)), rng.standard_normal((B, D, N)))  # a = exp(-softplus(z))
        return tuple(torch.from_numpy(v.astype(np.float32)).to(dtype).to(dev) for v in vals)

    ins = inputs()
    res = deliver(ir, {}, sink, ins, runner=HipGraphRunner())
    assert res.stats["executor"] == "scan" and res.stats["hip_kernel"] and res.stats["cuda_graph"] is True
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for _ in range(2):
        out = res.module(*ins).clone()
        assert out.dtype == dtype and out.shape == (B, T, D)
        ref, _ = oracle.ssm_serial(*(_np(t) for t in ins))
        _gate(ref, out, tol)
        ins = inputs()
    mod = res.module
    assert mod.fallbacks == 0 and (mod.fused_readouts > 0) == (N != 3)


def test_load_state_dict_reaches_a_captured_graph(sink, dev):
    # parameters load in place, so a graph that baked their addresses
    # replays with the new values: the generic module (C1's fused chain) and
    # a planned executor (the extracted decayed form, its projections inside)
    from tests.decayed_terms import DecayedTerms

    torch.manual_seed(3)
    layers = [torch.nn.Linear(64, 64) for _ in range(3)]
    vals = {}
    for i, lyr in enumerate(layers):
        vals[f"W{i + 1}"], vals[f"b{i + 1}"] = lyr.weight.detach().to(dev), lyr.bias.detach().to(dev)
    ir, _ = forms.weight_chain_form(3, 64, 16)
    x = torch.randn(16, 64, device=dev)
    b = DecayedTerms(B=1, K=4, C=64, D=64, heads=2)
    dvals, dx = b.values(dtype=torch.bfloat16, seed=4, gamma_dtype=torch.float32)
    cases = [(ir, vals, x), (b.ir(b.root()), {n: t.to(dev) for n, t in dvals.items()}, dx.to(dev))]
    for ir_, vals_, x_ in cases:
        res = deliver(ir_, vals_, sink, (x_,), runner=HipGraphRunner())
        mod = res.module
        assert res.stats["cuda_graph"] is True and mod.is_graph_captured
        before = mod(x_).clone()
        sd = mod.state_dict()
        mod.load_state_dict({k: v * 0.5 for k, v in sd.items()})
        replayed = mod(x_).clone()
        mod.drop_cuda_graph()
        eager = mod(x_)
        torch.cuda.synchronize()
        assert not torch.allclose(replayed.float(), before.float())
        _gate(_np(eager), replayed, 1e-6)
