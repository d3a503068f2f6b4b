"""Host logic of the HIP sink on the CPU: term model, weight fold, epilogue
fusion, the three executor plans, routing, verify and the fallback contract.

The HIP-backed ops are swapped for torch functions through the op-table seam
(``tests/cpu_table.py``); every numeric check compares against the numpy
oracle in float64.  Planted mistakes (a wrong offset, a missing cross block,
a flipped sign, a shifted mask) must make the plan decline.
"""

from __future__ import annotations

import json
import math

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import forms
from catopt_amd.evaluator import HipIRModule
from catopt_amd.executors import (
    HipChunkedDecayModule,
    HipOMModule,
    HipScanModule,
    build_decayed_plan,
    build_scan_plan,
    prefix_chunk_table,
)
from catopt_amd.executors.om import _triangle_offset, parse_score
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var, postorder, term_from_data, term_to_data
from catopt_amd.sink import HipSink, route_spec, verify_equiv
from tests.cpu_table import cpu_table

mk = Op.make


def _np(t):
    return t.detach().double().numpy()


# ------------------------------------------------------------------ term model


def test_op_interning_and_spelling_strict_identity():
    x = Var("x", TensorType((2, 3)))
    a = mk("mul", x, Const(2))
    assert mk("mul", x, Const(2)) is a
    assert mk("mul", x, Const(2.0)) is not a  # Const(2) != Const(2.0)
    assert mk("sum", x, dim=0) is not mk("sum", x, dim=0.0)
    assert hash(mk("add", a, a)) == hash(mk("add", a, a))


def test_wire_format_round_trip():
    ir, _ = forms.retention_kway_form(1, 2, 256, 128, 64, scale=0.5)
    data = term_to_data(ir.root)
    back = term_from_data(json.loads(json.dumps(data)))
    assert back is ir.root  # interning gives back the very same object
    ir3, _ = forms.causal_attention_form(1, 1, 64, 64, mask="cmask")
    assert term_from_data(json.loads(json.dumps(term_to_data(ir3.root)))) is ir3.root


def test_postorder_deep_chain_has_no_recursion_limit():
    ir, _ = forms.scan_final_form(5000, (4,))
    nodes = postorder(ir.root)
    assert nodes[-1] is ir.root
    assert len(nodes) == 1 + 3 * 5000 + 4999
    pos = {n: i for i, n in enumerate(nodes)}
    for n in nodes:
        for a in n.args:
            if isinstance(a, Op):
                assert pos[a] < pos[n]


# ------------------------------------------------------------- generic module


def _chain_values(L, d, seed=0):
    torch.manual_seed(seed)
    layers = [torch.nn.Linear(d, d) for _ in range(L)]  # fp32: the GEMM kernels' dtype
    vals = {}
    for i, l in enumerate(layers):
        vals[f"W{i + 1}"] = l.weight.detach()
        vals[f"b{i + 1}"] = l.bias.detach()
    return layers, vals


def test_weight_chain_folds_to_one_gemm_with_bias():
    L, d = 5, 32
    ir, _ = forms.weight_chain_form(L, d, rows=7)
    layers, vals = _chain_values(L, d)
    mod = HipIRModule(ir, vals, ops=cpu_table())
    assert [s[0] for s in mod._tape.steps] == ["hip_linear"]
    assert mod.stats["fused"] == {"linear": 1, "bias_add": L - 1}
    x = torch.randn(7, d)
    ref = oracle.linear_chain(_np(x), [_np(l.weight) for l in layers], [_np(l.bias) for l in layers])
    rep = oracle.verify_equiv(ref, _np(mod(x)), rtol=1e-5)
    assert rep["passed"], rep


def test_weight_chain_fold_pins_the_bias_spine():
    # Planted mistake on the oracle side: dropping one pushed-through addend
    # must be caught by the same comparison.
    L, d = 4, 16
    ir, _ = forms.weight_chain_form(L, d, rows=3)
    layers, vals = _chain_values(L, d, seed=1)
    W, adds = oracle.fold_linear_chain([_np(l.weight) for l in layers], [_np(l.bias) for l in layers])
    x = torch.randn(3, d)
    out = _np(HipIRModule(ir, vals, ops=cpu_table())(x))
    assert oracle.verify_equiv(oracle.folded_chain_forward(_np(x), W, adds), out, rtol=1e-5)["passed"]
    assert not oracle.verify_equiv(oracle.folded_chain_forward(_np(x), W, adds[:-1]), out, rtol=1e-6)["passed"]


def test_swiglu_block_fuses_to_norm_and_two_gemms():
    D, F_ = 16, 24
    ir, shapes = forms.swiglu_block_form((2, 5), D, F_)
    g = torch.Generator().manual_seed(3)
    vals = {n: (torch.randn(s, generator=g) * (0.2 if n != "gamma" else 1)).to(torch.bfloat16)
            for n, s in shapes.items()}
    mod = HipIRModule(ir, vals, ops=cpu_table())
    assert [s[0] for s in mod._tape.steps] == ["rms_norm", "hip_swiglu", "hip_linear"]
    # the concat was folded into one weight; the separate halves are pruned
    assert "W_gate" not in mod._param_map and "W_up" not in mod._param_map
    x = torch.randn(2, 5, D, generator=g).to(torch.bfloat16)
    h = oracle.rms_norm(_np(x), _np(vals["gamma"]), 1e-6)
    ref = oracle.swiglu_fused(h, _np(vals["W_gate"]), _np(vals["W_up"]), _np(vals["W_down"]))
    out = _np(mod(x).float())
    assert oracle.verify_equiv(ref, out, rtol=2e-2)["passed"]
    assert oracle.verify_equiv(oracle.swiglu_unfused(h, _np(vals["W_gate"]), _np(vals["W_up"]),
                                                     _np(vals["W_down"])), out, rtol=2e-2)["passed"]


def test_unfused_swiglu_spelling_takes_the_paired_epilogue_path():
    x = Var("x", TensorType((4, 8)))
    A, B = Param("A", TensorType((6, 8))), Param("B", TensorType((6, 8)))
    root = mk("mul", mk("silu", mk("linear", x, A)), mk("linear", x, B))
    vals = {"A": torch.randn(6, 8, dtype=torch.float64), "B": torch.randn(6, 8, dtype=torch.float64)}
    mod = HipIRModule(IR(root, [x]), vals, ops=cpu_table())
    # fp64 weights are outside the GEMM kernels' dtypes: nothing is fused
    assert [s[0] for s in mod._tape.steps] == ["linear", "silu", "linear", "mul"]
    vals16 = {k: v.to(torch.bfloat16) for k, v in vals.items()}
    mod16 = HipIRModule(IR(root, [x]), vals16, ops=cpu_table())
    assert [s[0] for s in mod16._tape.steps] == ["hip_swiglu"]
    xx = torch.randn(4, 8).to(torch.bfloat16)
    ref = oracle.silu(_np(xx) @ _np(vals16["A"]).T) * (_np(xx) @ _np(vals16["B"]).T)
    assert oracle.verify_equiv(ref, _np(mod16(xx).float()), rtol=2e-2)["passed"]


def test_missing_binding_is_loud():
    x = Var("x", TensorType((2,)))
    mod = HipIRModule(IR(mk("frobnicate", x), [x]), {}, ops=cpu_table())
    with pytest.raises(ValueError, match="No HIP binding"):
        mod(torch.zeros(2))


# ----------------------------------------------------------------- om plan


def test_triangle_offset_brute_force():
    for t, k in [(8, 8), (5, 9), (9, 5), (1, 4)]:
        for off in range(-k - 1, t + 2):
            keep = torch.ones(t, k, dtype=torch.bool).tril(-off)
            got = _triangle_offset(~keep)
            if keep.any():
                ref_keep = torch.ones(t, k, dtype=torch.bool).tril(-got)
                assert torch.equal(ref_keep, keep), (t, k, off, got)
            else:
                assert got is None
    m = torch.ones(6, 6, dtype=torch.bool).tril()
    m[3, 1] = False  # one flipped bit is no longer a triangle
    assert _triangle_offset(~m) is None


def test_om_plan_causal_param_mask_and_cmask():
    ir, shapes = forms.causal_attention_form(1, 2, 16, 64, mask="param")
    vals = {"mask": torch.ones(16, 16, dtype=torch.bool).tril()}
    mod = HipOMModule(ir, vals, ops=cpu_table())
    lf = mod._plan["leaves"][0]
    assert lf["mask_kind"] == "causal" and lf["causal_off"] == 0
    assert math.isclose(lf["scale"], 1 / 8.0)
    ir2, _ = forms.causal_attention_form(1, 2, 16, 64, mask="cmask")
    mod2 = HipOMModule(ir2, {}, ops=cpu_table())
    assert mod2._plan["leaves"][0]["mask_kind"] == "causal"
    # a shifted triangle keeps its offset; a random mask becomes a keep-mask
    vals3 = {"mask": torch.ones(16, 16, dtype=torch.bool).tril(2)}
    assert HipOMModule(ir, vals3, ops=cpu_table())._plan["leaves"][0]["causal_off"] == 2
    vals4 = {"mask": torch.rand(16, 16, generator=torch.Generator().manual_seed(0)) < 0.5}
    lf4 = HipOMModule(ir, vals4, ops=cpu_table())._plan["leaves"][0]
    assert lf4["mask_kind"] == "bool_const" and torch.equal(lf4["keep"], vals4["mask"])


def test_om_parse_declines_a_finite_fill_and_an_untransposed_key():
    q, k = Var("q", TensorType((4, 8))), Var("k", TensorType((4, 8)))
    s = mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))
    m = Param("m", TensorType((4, 4)))
    assert parse_score(mk("masked_fill", s, m, Const(float("-inf")))) is not None
    assert parse_score(mk("masked_fill", s, m, Const(-1e9))) is None
    assert parse_score(mk("matmul", q, k)) is None
    assert parse_score(mk("matmul", q, mk("transpose", k, dim0=0, dim1=1))) is not None  # 2-D dims are free
    sc = parse_score(mk("mul", mk("div", s, Const(4.0)), Const(3.0)))
    assert math.isclose(sc["scale"], 0.75)


@pytest.mark.parametrize("c", [0.0, -2.0])
def test_om_plan_declines_a_non_positive_scale(c):
    # the kernel scales the row max of q·k, which is the max of the scaled
    # scores only for a positive scale: such a leaf takes the score path
    q, k, v = (Var(n, TensorType((1, 2, 16, 64))) for n in "qkv")
    s = mk("mul", mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1)), Const(c))
    root = mk("om_apply", mk("om_elem", s, v))
    mod = HipOMModule(IR(root, [q, k, v]), {}, ops=cpu_table())
    assert mod.leaf_kinds == ["scores"]
    qs, ks, vs = (torch.randn(1, 2, 16, 64, dtype=torch.float64) for _ in range(3))
    out = mod(qs, ks, vs)
    ref = torch.softmax(c * (qs @ ks.transpose(-2, -1)), -1) @ vs
    assert oracle.verify_equiv(_np(ref), _np(out), rtol=1e-12)["passed"]


def test_om_module_falls_back_on_host_inputs():
    ir, _ = forms.causal_attention_form(1, 2, 16, 64, mask="param")
    vals = {"mask": torch.ones(16, 16, dtype=torch.bool).tril()}
    mod = HipOMModule(ir, vals, ops=cpu_table())
    q, k, v = (torch.randn(1, 2, 16, 64, dtype=torch.float64) for _ in range(3))
    out = mod(q, k, v)
    assert mod.fallbacks == 1
    ref = oracle.attention_om(_np(q), _np(k), _np(v), 1 / 8.0, causal=True)
    assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]


# --------------------------------------------------------------- decayed plan


def _kway(K, C, *, off_bump=None, drop=None, sign=-1, swap=None, scale_div=None):
    """The K-way RHS with optional planted mistakes."""
    T = K * C
    q, k, v = (Var(n, TensorType((1, 2, T, 128))) for n in "qkv")
    g = Param("gamma", TensorType((2,)))
    s = mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))
    if scale_div is not None:
        s = mk("div", s, Const(scale_div))
    SZ = (C,) * K

    def score(i, j):
        return mk("split", mk("split", s, sizes=SZ, dim=-2, index=i), sizes=SZ, dim=-1, index=j)

    def value(j):
        return mk("split", v, sizes=SZ, dim=-2, index=j)

    blocks = []
    for i in range(K):
        acc = mk("om_decayed", score(i, i), mk("decay", g, t=C), value(i))
        for j in range(i):
            if drop == (i, j):
                continue
            off = (i - j) * C + (1 if off_bump == (i, j) else 0)
            jj = swap[1] if swap is not None and swap[0] == (i, j) else j
            row = mk("unsqueeze", mk("decay_vec", g, t=C, offset=off), dim=-1)
            col = mk("unsqueeze", mk("decay_vec", g, t=C, sign=sign), dim=-2)
            acc = mk("add", acc, mk("mul", row, mk("matmul", mk("mul", score(i, jj), col), value(jj))))
        blocks.append(acc)
    out = blocks[-1]
    for blk in reversed(blocks[:-1]):
        out = mk("concat", blk, out, dim=-2)
    return IR(out, [q, k, v])


def test_decayed_plan_accepts_the_kway_form_and_pins_its_integers():
    p = build_decayed_plan(_kway(4, 32, scale_div=2.0).root)
    assert (p["K"], p["C"]) == (4, 32) and math.isclose(p["scale"], 0.5)
    assert build_decayed_plan(_kway(4, 32, off_bump=(2, 0)).root) is None
    assert build_decayed_plan(_kway(4, 32, drop=(3, 1)).root) is None
    assert build_decayed_plan(_kway(4, 32, sign=1).root) is None
    assert build_decayed_plan(_kway(4, 32, swap=((3, 1), 2)).root) is None
    ir, _ = forms.retention_kway_form(1, 2, 256, 128, 64)
    assert build_decayed_plan(ir.root)["K"] == 4
    irb, _ = forms.retention_block_form(1, 2, 128)
    assert build_decayed_plan(irb.root)["K"] == 1


def test_kway_form_equals_the_quadratic_form_on_cpu():
    # The plan keeps only (q, k, v, γ, scale): legitimate because every K-way
    # form equals the quadratic one.  Check that through the generic module.
    ir = _kway(4, 8, scale_div=4.0)
    gam = torch.tensor([0.9, 0.75], dtype=torch.float64)
    mod = HipChunkedDecayModule(ir, {"gamma": gam}, ops=cpu_table())
    assert mod.n_chunks == 4
    q, k, v = (torch.randn(1, 2, 32, 128, dtype=torch.float64) * 0.1 for _ in range(3))
    out = mod(q, k, v)  # host inputs: the generic module runs (fallback)
    assert mod.fallbacks == 1
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), _np(gam), 0.25)
    assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]


# ------------------------------------------------------------------ scan plan


def test_prefix_chunk_table_matches_the_blocked_plan():
    for T in list(range(1, 300)) + [16384, 16385, 99991]:
        assert prefix_chunk_table(T) == list(oracle.prefix_chunk_table(T)), T


def test_scan_plans_final_and_prefix():
    ir, _ = forms.scan_final_form(7, (3,))
    p = build_scan_plan(ir.root)
    assert p["mode"] == "final" and len(p["leaves"]) == 7 and p["gather"] is not None
    irp, _ = forms.scan_prefix_form(7, (3,))
    pp = build_scan_plan(irp.root)
    assert pp["mode"] == "prefix" and len(pp["leaves"]) == 7
    # a stacked form whose members are not successive prefixes is declined
    a, u, h = (Var(n, TensorType((3,))) for n in "auh")
    f0 = mk("aff_diag", a, u)
    f1 = mk("affd_compose", mk("aff_diag", u, a), f0)
    bad = mk("applyd", mk("aff_diag", mk("stack", mk("affd_a", f1), mk("affd_a", f0)),
                          mk("stack", mk("affd_b", f1), mk("affd_b", f0))), h)
    assert build_scan_plan(bad) is None


def test_scan_module_fallback_matches_the_serial_recurrence():
    T, S = 9, 5
    ir, _ = forms.scan_final_form(T, (S,))
    mod = HipScanModule(ir, {}, ops=cpu_table())
    a = torch.rand(T, S, dtype=torch.float64)
    u = torch.randn(T, S, dtype=torch.float64)
    h = torch.randn(S, dtype=torch.float64)
    out = mod(a, u, h)
    assert mod.fallbacks == 1
    ref = oracle.serial_affd_scan(_np(a), _np(u), _np(h))[-1]
    assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]
    irp, _ = forms.scan_prefix_form(T, (S,))
    modp = HipScanModule(irp, {}, ops=cpu_table())
    refp = oracle.serial_affd_scan(_np(a), _np(u), _np(h))
    assert oracle.verify_equiv(refp, _np(modp(a, u, h)), rtol=1e-12)["passed"]


def test_ssm_readout_plan_and_fallback():
    """The selective SSM delivered as a read-out of the stacked prefix
    states: planned as a prefix scan with its input factors and read-out
    recognised, routed to the scan executor, and (on host tensors, outside
    the kernels' envelope) run by the generic module to the serial
    recurrence's values."""
    B, T, D, N = 2, 9, 3, 4
    for per_state in (True, False):
        ir, _ = forms.diag_ssm_form(B, T, D, N, a_per_state=per_state)
        p = build_scan_plan(ir.root)
        assert p is not None and p["mode"] == "prefix" and p["dim"] == 1 and p["domain"] == "diag"
        assert p["readout"]["dim"] == -1 and p["inner_post"] == [] and p["post"] == []
        (fx, fb) = p["factors"]
        assert fx[1] == 1 and fx[2] == list(range(T)) and fx[3] == (-1,)
        assert fb[1] == 1 and fb[2] == list(range(T)) and fb[3] == (-2,)
        assert p["gather"][0][2] == list(range(T)) and p["gather"][0][3] == (() if per_state else (-1,))
        assert route_spec(ir.root, HipSink(device="cpu", ops=cpu_table())).name == "scan"
        g = torch.Generator().manual_seed(3)
        a = torch.rand((B, T, D, N) if per_state else (B, T, D), generator=g, dtype=torch.float64)
        bx, c = (torch.randn(B, T, N, generator=g, dtype=torch.float64) for _ in range(2))
        x = torch.randn(B, T, D, generator=g, dtype=torch.float64)
        h = torch.randn(B, D, N, generator=g, dtype=torch.float64)
        mod = HipScanModule(ir, {}, ops=cpu_table())
        out = mod(a, bx, c, x, h)
        assert mod.fallbacks == 1 and out.shape == (B, T, D)
        ref, _ = oracle.ssm_serial(*(_np(t) for t in (a, bx, c, x, h)))
        assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]
    # a contraction whose operand is not a scan root is not a read-out
    v = Var("v", TensorType((3, 4)))
    assert build_scan_plan(mk("sum", mk("mul", v, v), dim=-1)) is None


# ---------------------------------------------------------------------- sink


def test_sink_surface_routing_and_verify():
    sink = HipSink(device="cpu", ops=cpu_table())
    names = list(sink.executors)
    assert names == ["om_decayed_chunked", "scan", "om_batched", "omd_batched", "om_streaming", "generic"]
    assert sink.executors["generic"].carrier is None
    assert {"linear", "matmul", "rms_norm", "om_elem", "om_compose", "om_apply", "om_decayed",
            "decay", "decay_vec", "aff_diag", "affd_compose", "applyd", "aff", "aff_compose",
            "apply", "aff_A", "aff_b"} <= sink.supported_ops
    cases = [
        (forms.retention_kway_form(1, 2, 128, 128, 64)[0], "om_decayed_chunked"),
        (forms.scan_final_form(4, (2,))[0], "scan"),
        (forms.causal_attention_form(1, 1, 8, 64, mask="cmask")[0], "om_batched"),
    ]
    for ir, want in cases:
        assert route_spec(ir.root, sink).name == want
    assert route_spec(forms.weight_chain_form(2, 8, 2)[0].root, sink) is None
    ref = torch.tensor([1.0, -2.0])
    assert verify_equiv(ref, ref + 1e-5, rtol=1e-4).passed
    rep = verify_equiv(ref, torch.tensor([1.0, float("nan")]))
    assert not rep.passed
    assert math.isclose(verify_equiv(ref, torch.tensor([1.0, -2.1])).max_rel, 0.1 / (2 + 1e-8), rel_tol=1e-6)


# ------------------------------------------------------------------ streaming om plan


def test_streaming_plan_leaf_kinds_and_fold_order():
    from catopt_amd.executors import HipStreamingOMModule, om_empty_state

    q = Var("q", TensorType((1, 2, 8, 64)))
    ks = [Var(f"k{i}", TensorType((1, 2, 4, 64))) for i in range(3)]
    vs = [Var(f"v{i}", TensorType((1, 2, 4, 64))) for i in range(3)]
    s_raw = Var("s", TensorType((1, 2, 8, 4)))
    m, lv, a = (Var(n, TensorType((1, 2, 8, d))) for n, d in (("m", 1), ("l", 1), ("a", 64)))

    def qk(i):
        return mk("om_elem", mk("mul", mk("matmul", q, mk("transpose", ks[i], dim0=-2, dim1=-1)), Const(0.125)),
                  vs[i])

    # left-leaning tree mixing all three leaf kinds; a DAG-shared leaf counts twice
    shared = qk(1)
    tree = mk("om_compose", mk("om_compose", mk("om_compose", qk(0), shared),
                               mk("om_elem", s_raw, vs[2])), mk("om_compose", mk("om", m, lv, a), shared))
    ir = IR(mk("om_apply", tree), [q, *ks, *vs, s_raw, m, lv, a])
    mod = HipStreamingOMModule(ir, ops=cpu_table())
    assert mod.is_streaming and mod.n_blocks == 5
    kinds = [lf["kind"] for lf in mod._plan["leaves"]]
    assert kinds == ["qk", "qk", "elem", "om", "qk"]
    assert [lf["scale"] for lf in mod._plan["leaves"] if lf["kind"] == "qk"] == [0.125] * 3
    assert mod._plan["leaves"][1]["k"] is ks[1] and mod._plan["leaves"][4]["k"] is ks[1]
    # a root that is not om_apply over an om tree: not streaming
    assert not HipStreamingOMModule(IR(mk("relu", q), [q]), ops=cpu_table()).is_streaming
    bad = mk("om_apply", mk("om_compose", qk(0), mk("relu", s_raw)))
    assert not HipStreamingOMModule(IR(bad, [q, ks[0], vs[0], s_raw]), ops=cpu_table()).is_streaming
    e_m, e_l, e_a = om_empty_state((2, 3), 5, dtype=torch.float64)
    assert e_m.shape == (2, 3, 1) and e_a.shape == (2, 3, 5) and e_m.dtype == torch.float64
    assert torch.isneginf(e_m).all() and not e_l.any() and not e_a.any()


# ------------------------------------------------------------------ dense scan plan


def test_dense_scan_plans_and_levels():
    ir, _ = forms.linear_recurrence_form(8, 4)
    p = build_scan_plan(ir.root)
    assert p["domain"] == "dense" and p["mode"] == "final" and len(p["leaves"]) == 8
    assert p["levels"] == 3 and p["a_shared"]  # balanced over 8 leaves: 4 + 2 + 1 composes
    # time order: the innermost leaf reads step 0
    assert [lf.args[1].attrs["index"] for lf in p["leaves"]] == list(range(8))
    assert p["gather"][1][2] == list(range(8)) and 0 not in p["gather"]
    irt, _ = forms.dense_scan_form(5, 4, (2,), 3, time_varying=True, per_slot=True)
    pt = build_scan_plan(irt.root)
    assert not pt["a_shared"] and pt["gather"][0][2] == list(range(5))
    irp, _ = forms.dense_scan_prefix_form(6, 4)
    pp = build_scan_plan(irp.root)
    assert pp["domain"] == "dense" and pp["mode"] == "prefix" and len(pp["leaves"]) == 6 and pp["levels"] == 0
    # mixed carriers are not one scan
    A, b, h = Var("A", TensorType((3, 3))), Var("b", TensorType((3,))), Var("h", TensorType((3,)))
    mixed = mk("apply", mk("aff_compose", mk("aff", A, b), mk("aff_diag", b, b)), h)
    assert build_scan_plan(mixed) is None
    assert build_scan_plan(mk("aff_compose", mk("aff", A, b), mk("aff", A, b))) is None  # no apply root


def test_nested_apply_folds_and_output_views_strip():
    A, b, h = Var("A", TensorType((3, 3))), Var("b", TensorType((3,))), Var("h", TensorType((3,)))
    f = mk("aff", A, b)
    g = mk("aff", mk("transpose", A, dim0=0, dim1=1), b)
    nested = mk("reshape", mk("apply", f, mk("apply", g, mk("apply", f, h))), shape=(1, 3))
    p = build_scan_plan(nested)
    assert p is not None and p["mode"] == "final" and p["post"] == [("reshape", {"shape": (1, 3)})]
    assert [lf is g for lf in p["leaves"]] == [False, True, False] and p["h"] is h
    # the diagonal pair folds the same way
    d = mk("applyd", mk("aff_diag", b, b), mk("applyd", mk("aff_diag", h, b), h))
    pd = build_scan_plan(d)
    assert pd["domain"] == "diag" and len(pd["leaves"]) == 2


def test_dense_scan_module_fallback_matches_the_recurrence():
    T, d = 9, 4
    ir, _ = forms.linear_recurrence_form(T, d)
    A = torch.randn(d, d, dtype=torch.float64) * 0.3
    h0 = torch.randn(d, dtype=torch.float64)
    mod = HipScanModule(ir, {"p_a": A, "p_h0": h0}, ops=cpu_table())
    assert mod.is_batched and mod.n_levels == 4
    x = torch.randn(T, d, dtype=torch.float64)
    out = mod(x)  # host / fp64 operands: the generic module runs
    assert mod.fallbacks == 1
    ref = oracle.serial_aff_scan(_np(A), _np(x), _np(h0)[:, None])[-1, :, 0]
    assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]
    irp, _ = forms.dense_scan_prefix_form(T, d)
    modp = HipScanModule(irp, {}, ops=cpu_table())
    At = torch.randn(T, d, d, dtype=torch.float64) * 0.3
    refp = oracle.serial_aff_scan(_np(At), _np(x), _np(h0)[:, None])[..., 0]
    assert oracle.verify_equiv(refp, _np(modp(At, x, h0)), rtol=1e-12)["passed"]


# ------------------------------------------------------------------ omd plan


def test_omd_plan_chain_and_seeds():
    from catopt_amd.executors import build_omd_plan, is_omd_term

    T, d, Tq, nb = 12, 3, 5, 3
    ir, _ = forms.omd_scan_attention_form(T, d, Tq, nb)
    assert is_omd_term(ir.root)
    p = build_omd_plan(ir.root)
    assert p["map_mode"] == "chain" and p["chain_domain"] == "diag" and len(p["chain_leaves"]) == T
    assert p["chain_a_gather"][2] == list(range(T)) and p["chain_b_gather"][2] == list(range(T))
    assert len(p["stack_seeds"]) == 2 * nb and len(p["leaves"]) == nb
    # each block's stack reads prefix positions i·C … i·C + C - 1
    C = T // nb
    assert sorted(tuple(s[3]) for s in p["stack_seeds"]) == sorted(
        [tuple(range(i * C, (i + 1) * C)) for i in range(nb)] * 2)
    pd = build_omd_plan(forms.omd_scan_attention_form(8, 2, 3, 2, dense=True)[0].root)
    assert pd["map_mode"] == "chain" and pd["chain_domain"] == "dense" and pd["apply"] == "omd_applym"
    # two unrelated compose trees: forest (level-batched map evaluation)
    a = [Var(f"a{i}", TensorType((2,))) for i in range(4)]
    t1 = mk("affd_compose", mk("aff_diag", a[1], a[1]), mk("aff_diag", a[0], a[0]))
    t2 = mk("affd_compose", mk("aff_diag", a[3], a[3]), mk("aff_diag", a[2], a[2]))
    s = Var("s", TensorType((2, 2)))
    leaf = mk("omd_elem", s, mk("stack", mk("affd_a", t1), mk("affd_a", t2), dim=0),
              mk("stack", mk("affd_b", t1), mk("affd_b", t2), dim=0))
    pf = build_omd_plan(mk("omd_apply", leaf, a[0]))
    assert pf["map_mode"] == "forest"
    fd = pf["forest"]["diag"]
    assert len(fd["leaves"]) == 4 and fd["n_slots"] == 6 and len(fd["gathers"]) == 1
    # not omd-shaped
    assert build_omd_plan(mk("om_apply", mk("om_elem", s, s))) is None
    assert not is_omd_term(mk("omd_apply", mk("omd_compose", leaf, s), a[0]))


def test_omd_module_fallback_matches_attention_over_states():
    from catopt_amd.executors import HipOmdModule

    T, d, Tq, nb, dk = 12, 3, 5, 3, 4
    ir, _ = forms.omd_scan_attention_form(T, d, Tq, nb, dk)
    mod = HipOmdModule(ir, {}, ops=cpu_table())
    g = torch.Generator().manual_seed(0)
    q, k = torch.randn(Tq, dk, generator=g, dtype=torch.float64), torch.randn(T, dk, generator=g, dtype=torch.float64)
    a, x, h = (torch.rand(T, d, generator=g, dtype=torch.float64), torch.randn(T, d, generator=g, dtype=torch.float64),
               torch.randn(d, generator=g, dtype=torch.float64))
    out = mod(q, k, a, x, h)  # host fp64: the generic module runs
    assert mod.fallbacks == 1
    states = oracle.serial_affd_scan(_np(a), _np(x), _np(h))
    sc = _np(q) @ _np(k).T
    w = np.exp(sc - sc.max(-1, keepdims=True))
    ref = (w / w.sum(-1, keepdims=True)) @ states
    assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]


def test_omd_plan_chain_with_other_bracketing():
    """A prefix bracketed differently (compose(compose(l3, l2), f1)) is still a
    prefix of the same leaf sequence: the general check keeps the chain."""
    from catopt_amd.executors import build_omd_plan

    a = Var("a", TensorType((4, 2)))
    lv = [mk("aff_diag", mk("select", a, dim=0, index=j), mk("select", a, dim=0, index=j)) for j in range(4)]
    f1 = mk("affd_compose", lv[1], lv[0])
    f3 = mk("affd_compose", mk("affd_compose", lv[3], lv[2]), f1)
    s, h = Var("s", TensorType((3, 2))), Var("h", TensorType((2,)))
    leaf = mk("omd_elem", s, mk("stack", mk("affd_a", f1), mk("affd_a", f3), dim=0),
              mk("stack", mk("affd_b", f1), mk("affd_b", f3), dim=0))
    p = build_omd_plan(mk("omd_apply", leaf, h))
    assert p["map_mode"] == "chain" and len(p["chain_leaves"]) == 4
    assert [tuple(x[3]) for x in p["stack_seeds"]] == [(1, 3), (1, 3)]


def _omd_over(amap, bmap, s_shape=(3, 2), h_shape=(2,)):
    s, h = Var("s", TensorType(s_shape)), Var("h", TensorType(h_shape))
    return mk("omd_apply", mk("omd_elem", s, amap, bmap), h)


def test_omd_forest_plan_slots_and_levels():
    """A balanced compose tree over 8 leaves, every internal node projected:
    leaves take slots 0-7 in application order, each level's nodes the next
    slots, and each level's gather names its operands' slots
    (``omd_lower.py:520-558``)."""
    from catopt_amd.executors import build_omd_plan

    a = [Var(f"a{i}", TensorType((2,))) for i in range(8)]
    lv = [mk("aff_diag", x, x) for x in a]
    l1 = [mk("affd_compose", lv[2 * i + 1], lv[2 * i]) for i in range(4)]
    l2 = [mk("affd_compose", l1[2 * i + 1], l1[2 * i]) for i in range(2)]
    top = mk("affd_compose", l2[1], l2[0])
    nodes = l1 + l2 + [top]
    p = build_omd_plan(_omd_over(mk("stack", *[mk("affd_a", n) for n in nodes], dim=0),
                                 mk("stack", *[mk("affd_b", n) for n in nodes], dim=0)))
    assert p["map_mode"] == "forest" and set(p["forest"]) == {"diag"}
    fd = p["forest"]["diag"]
    assert fd["leaves"] == lv and fd["n_slots"] == 15
    assert fd["gathers"] == [([1, 3, 5, 7], [0, 2, 4, 6]), ([9, 11], [8, 10]), ([13], [12])]
    assert [fd["slot"][n] for n in nodes] == list(range(8, 15))
    # both stacks read slots 8..14 in order from the diagonal store
    assert [(ci, src, tuple(ix)) for _, ci, src, ix, _ in p["stack_seeds"]] == [
        (0, ("forest", "diag"), tuple(range(8, 15))), (1, ("forest", "diag"), tuple(range(8, 15)))]
    # a leaf gather: every leaf part is a variable, so none
    assert fd["a_gather"] is None and fd["b_gather"] is None


def test_omd_forest_plan_shares_subterms_and_mixes_carriers():
    from catopt_amd.executors import build_omd_plan

    a = [Var(f"a{i}", TensorType((2,))) for i in range(3)]
    A = [Var(f"A{i}", TensorType((2, 2))) for i in range(2)]
    lv = [mk("aff_diag", x, x) for x in a]
    shared = mk("affd_compose", lv[1], lv[0])
    t1 = mk("affd_compose", lv[2], shared)
    t2 = mk("affd_compose", shared, lv[2])  # not a prefix of t1's sequence
    dense = mk("aff_compose", mk("aff", A[1], a[1]), mk("aff", A[0], a[0]))
    amap = mk("stack", mk("affd_a", t1), mk("affd_a", t2), dim=0)
    p = build_omd_plan(_omd_over(amap, mk("add", mk("aff_b", dense), mk("affd_b", shared))))
    assert p["map_mode"] == "forest" and set(p["forest"]) == {"diag", "dense"}
    fd, fx = p["forest"]["diag"], p["forest"]["dense"]
    # shared once: 3 leaves + shared + t1 + t2
    assert fd["n_slots"] == 6 and fd["slot"][shared] == 3
    assert fd["gathers"] == [([1], [0]), ([2, 3], [3, 2])]
    assert fx["n_slots"] == 3 and fx["gathers"] == [([1], [0])]
    srcs = {src for _, _, src, _ in p["proj_seeds"]}
    assert srcs == {("forest", "diag"), ("forest", "dense")}


def test_omd_forest_plan_declines():
    """Plans the reference declines (``build_omd_plan`` returns None and the
    generic module runs): a compose of the other carrier under a projection,
    leaf shapes that break the carrier's contract or differ between leaves,
    and a map leaf whose operands project another map."""
    from catopt_amd.executors import build_omd_plan

    a2, a3 = Var("a2", TensorType((2,))), Var("a3", TensorType((3,)))
    A = Var("A", TensorType((2, 2)))
    bm = Var("bm", TensorType((2,)))
    dense = mk("aff_compose", mk("aff", A, a2), mk("aff", A, a2))
    assert build_omd_plan(_omd_over(mk("affd_a", dense), bm)) is None
    bad = mk("affd_compose", mk("aff_diag", a2, a3), mk("aff_diag", a2, a2))
    assert build_omd_plan(_omd_over(mk("affd_a", bad), bm)) is None
    mixed = mk("affd_compose", mk("aff_diag", a3, a3), mk("aff_diag", a2, a2))
    assert build_omd_plan(_omd_over(mk("affd_a", mixed), bm)) is None
    inner = mk("affd_compose", mk("aff_diag", a2, a2), mk("aff_diag", a2, a2))
    nested = mk("affd_compose", mk("aff_diag", mk("affd_a", inner), a2), mk("aff_diag", a2, a2))
    other = mk("affd_compose", mk("aff_diag", a2, bm), mk("aff_diag", bm, a2))
    assert build_omd_plan(_omd_over(mk("stack", mk("affd_a", nested), mk("affd_a", other), dim=0), bm)) is None


def test_omd_chain_plan_takes_opaque_leaves():
    """A leaf that is any term evaluating to a pair (here a (2, d) input) may
    sit in a prefix chain (``omd_lower.py:488-497``); its parts are read as
    ``value[0]`` / ``value[1]``."""
    from catopt_amd.executors import build_omd_plan

    a = Var("a", TensorType((3,)))
    M = Var("M", TensorType((2, 3)))
    f1 = mk("affd_compose", mk("aff_diag", a, a), M)
    p = build_omd_plan(_omd_over(mk("stack", mk("affd_a", M), mk("affd_a", f1), dim=0),
                                 mk("stack", mk("affd_b", M), mk("affd_b", f1), dim=0), h_shape=(3,)))
    assert p["map_mode"] == "chain" and p["chain_leaves"][0] is M
    assert p["chain_a_gather"] is None


@pytest.mark.parametrize("dense,bracket", [(False, "chain"), (False, "tree"), (True, "tree")])
def test_omd_block_restart_form_is_attention_over_restarted_states(dense, bracket):
    """The forest-plan form, run by the generic module on host fp64, is
    softmax attention over scan states restarted from h at every key block
    (float64 serial recurrences of the oracle)."""
    from catopt_amd.executors import HipOmdModule

    T, d, Tq, nb, dk = 16, 3, 5, 4, 4
    ir, _ = forms.omd_block_restart_form(T, d, Tq, nb, dk, dense=dense, bracket=bracket)
    mod = HipOmdModule(ir, {}, ops=cpu_table())
    assert mod.map_mode == "forest"
    g = torch.Generator().manual_seed(3)
    q, k = torch.randn(Tq, dk, generator=g, dtype=torch.float64), torch.randn(T, dk, generator=g, dtype=torch.float64)
    a = (torch.randn(T, d, d, generator=g, dtype=torch.float64) * 0.4 if dense
         else torch.rand(T, d, generator=g, dtype=torch.float64))
    x, h = torch.randn(T, d, generator=g, dtype=torch.float64), torch.randn(d, generator=g, dtype=torch.float64)
    out = mod(q, k, a, x, h)
    C = T // nb
    blocks = []
    for i in range(nb):
        sl = slice(i * C, (i + 1) * C)
        if dense:
            blocks.append(oracle.serial_aff_scan(_np(a)[sl], _np(x)[sl], _np(h)[:, None])[..., 0])
        else:
            blocks.append(oracle.serial_affd_scan(_np(a)[sl], _np(x)[sl], _np(h)))
    sc = _np(q) @ _np(k).T
    w = np.exp(sc - sc.max(-1, keepdims=True))
    ref = (w / w.sum(-1, keepdims=True)) @ np.concatenate(blocks)
    assert oracle.verify_equiv(ref, _np(out), rtol=1e-12)["passed"]


def test_attention_q64_asm_is_the_generator_output():
    # attn_q64_loop.inc is committed generated code: it must be exactly what
    # gen_attn_q64.py emits, and its clobbers must cover every register the
    # loop names
    import importlib.util
    import re
    from pathlib import Path

    csrc = Path(__file__).resolve().parents[1] / "catopt_amd" / "csrc"
    spec = importlib.util.spec_from_file_location("gen_attn_q64", csrc / "gen_attn_q64.py")
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    text = gen.render()
    assert (csrc / "attn_q64_loop.inc").read_text() == text
    body = text.split("#define ATTN_Q64_CLOBBERS")[0]
    vregs = {int(x) for x in re.findall(r"\bv(\d+)\b", body)}
    vregs |= {int(b) for a, b in re.findall(r"\bv\[(\d+):(\d+)\]", body)}
    aregs = {int(x) for x in re.findall(r"\ba(\d+)\b", body)} | {int(b) for a, b in re.findall(r"\ba\[(\d+):(\d+)\]", body)}
    assert max(vregs) < gen.NVGPR and max(aregs) < 256
    assert body.count("v_mfma_f32_32x32x16_bf16") == 3 * 64 + 16  # three unrolled tiles and the drain
    assert body.count("s_barrier") == 1 + 3
