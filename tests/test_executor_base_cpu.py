"""Shared machinery of the planned executors (CPU), after catopt's
executor-base tests (tests/test_executor_base.py of luisfuturist/catopt):
the methods come from the one mixin; ``eval_mod`` is a registered
submodule; capture is a no-op without a device and refuses host inputs
with one; a captured slot replays verbatim, drops clean and re-captures;
the input environment and the memoised leaf evaluator; the
device/dtype-keyed constant cache."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from catopt_amd import forms
from catopt_amd.executors import HipChunkedDecayModule, HipOMModule, HipOmdModule, HipScanModule
from catopt_amd.executors.base import HipExecutorBase
from catopt_amd.graphs import signature
from catopt_amd.ir import Op
from tests.cpu_table import cpu_table
from tests.decayed_terms import DecayedTerms

CLASSES = (HipScanModule, HipOMModule, HipOmdModule, HipChunkedDecayModule)


def _cases():
    g = torch.Generator().manual_seed(0)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    ir, _ = forms.scan_final_form(5, (3,))
    scan = HipScanModule(ir, {}, ops=cpu_table())
    scan_args = (r(5, 3).clamp(-0.9, 0.9), r(5, 3), r(3))
    ir, _ = forms.causal_attention_form(1, 2, 8, 16, mask="cmask")
    om = HipOMModule(ir, {}, ops=cpu_table())
    om_args = (r(1, 2, 8, 16), r(1, 2, 8, 16), r(1, 2, 8, 16))
    ir, _ = forms.omd_scan_attention_form(16, 4, 5, 2, 3)
    omd = HipOmdModule(ir, {}, ops=cpu_table())
    omd_args = (r(5, 3), r(16, 3), torch.rand(16, 4, generator=g, dtype=torch.float64), r(16, 4), r(4))
    b = DecayedTerms()
    vals, x = b.values()
    dec = HipChunkedDecayModule(b.ir(b.root()), vals, ops=cpu_table())
    return [(scan, scan_args), (om, om_args), (omd, omd_args), (dec, (x,))]


def test_the_shared_methods_come_from_the_mixin():
    for cls in CLASSES:
        assert issubclass(cls, HipExecutorBase) and issubclass(cls, torch.nn.Module)
        for name in ("capture_cuda_graph", "drop_cuda_graph", "_input_env", "ev_factory", "_cached", "forward"):
            assert getattr(cls, name) is getattr(HipExecutorBase, name), (cls, name)
        assert cls.is_graph_captured.fget is HipExecutorBase.is_graph_captured.fget


def test_every_case_plans_and_registers_its_generic_module():
    for mod, _ in _cases():
        assert mod.is_batched and mod._plan is not None
        assert "eval_mod" in dict(mod.named_modules())


def test_capture_is_a_no_op_without_a_device_and_refuses_host_inputs_with_one(monkeypatch):
    for mod, args in _cases():
        monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
        assert mod.capture_cuda_graph(*args) is mod
        assert mod._graph is None and mod._graph_inputs == [] and mod._graph_out is None
        monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
        with pytest.raises(ValueError, match="device"):
            mod.capture_cuda_graph(*args)
        assert not mod.is_graph_captured


class _FakeGraph:
    def __init__(self):
        self.replays = 0

    def replay(self):
        self.replays += 1


def test_a_captured_slot_replays_drops_and_recaptures():
    for mod, args in _cases():
        sentinel = torch.full((1,), 3.0, dtype=torch.float64)
        static = [torch.zeros_like(a) for a in args]
        mod._graph, mod._graph_inputs, mod._graph_out = _FakeGraph(), static, sentinel
        mod._graph_sig = signature(tuple(args))
        assert mod.is_graph_captured
        assert mod(*[a.clone() for a in args]) is sentinel and mod._graph.replays == 1
        assert all(torch.equal(s, a) for s, a in zip(static, args))  # inputs copied in
        # another shape runs eagerly even while captured
        other = tuple(torch.cat([a, a]) if a.dim() else a for a in args[:1]) + tuple(args[1:])
        assert signature(other) != mod._graph_sig
        mod.drop_cuda_graph()
        assert not mod.is_graph_captured and mod._graph is None
        assert mod._graph_inputs == [] and mod._graph_out is None
        fake = _FakeGraph()
        mod._graph, mod._graph_inputs, mod._graph_out = fake, list(static), sentinel
        mod._graph_sig = signature(tuple(args))
        assert mod(*args) is sentinel and fake.replays == 1
        mod.drop_cuda_graph()
        out, ref = mod(*args), mod.eval_mod(*args)
        torch.testing.assert_close(out, ref, rtol=0, atol=0)


def test_the_input_environment():
    for mod, args in _cases():
        x, env = mod._input_env(args)
        assert x is args[0] and env["self"] is args[0]
        assert set(env) == {"self"} | {inp.name for inp in mod._inputs}
        for i, inp in enumerate(mod._inputs):
            assert env[inp.name] is args[i]
        x, env = mod._input_env(args[:1])
        assert all(env[inp.name] is args[0] for inp in mod._inputs)
        x, env = mod._input_env(())
        assert x is None and env["self"] is None and all(env[inp.name] is None for inp in mod._inputs)


def test_the_leaf_evaluator_memoises():
    for mod, args in _cases():
        x, env = mod._input_env(args)
        memo: dict = {}
        ev = mod.ev_factory(env, x, memo)
        inp = mod._inputs[0]
        assert ev(inp) is args[0]
        t = Op.make("relu", inp)
        out = ev(t)
        torch.testing.assert_close(out, args[0].clamp_min(0))
        assert memo[t] is out and ev(t) is out


def test_the_constant_cache_rekeys_on_dtype():
    for mod, args in _cases():
        made = []

        def make(like):
            made.append(like)
            return torch.tensor([0, 1], device=like.device)

        a = mod._cached(("k",), args[0], make, dtype=torch.long)
        assert mod._cached(("k",), args[0], make, dtype=torch.long) is a and len(made) == 1
        b = mod._cached(("k",), args[0], make, dtype=torch.float64)
        assert b is not a and len(made) == 2 and mod._const_cache[("k",)] is b
        assert np.array_equal(b.numpy(), [0.0, 1.0])


def test_the_reference_constructor_and_probe_names():
    # code written against catopt's executors finds the same entry points:
    # to_batched_*_module / to_chunked_decayed_module always return the
    # executor (check is_batched); the is_*_term probes; n_blocks / n_levels
    from catopt_amd import executors as E
    from catopt_amd.ir import IR, Op, TensorType, Var

    b = DecayedTerms()
    vals, _ = b.values()
    dec = E.to_chunked_decayed_module(b.ir(b.root()), vals, ops=cpu_table())
    assert isinstance(dec, HipChunkedDecayModule) and dec.is_batched and dec.n_blocks == b.K
    assert E.is_decayed_chunked_term(b.root()) and not E.is_decayed_chunked_term(b.q)
    ir, _ = forms.causal_attention_form(1, 2, 8, 16, mask="cmask")
    om = E.to_batched_om_module(ir, {}, fused=True, ops=cpu_table())
    assert isinstance(om, HipOMModule) and om.is_batched and (om.n_blocks, om.n_levels) == (1, 0)
    assert E.is_om_apply_term(ir.root)
    q = Var("q", TensorType((8, 4)))
    ks = [Var(f"k{i}", TensorType((4, 4))) for i in range(5)]
    leaves = [Op.make("om_elem", Op.make("matmul", q, Op.make("transpose", k, dim0=-2, dim1=-1)), k) for k in ks]
    tree = leaves[0]
    for lf in leaves[1:]:
        tree = Op.make("om_compose", tree, lf)
    om5 = E.to_batched_om_module(IR(Op.make("om_apply", tree), [q, *ks]), {}, ops=cpu_table())
    assert (om5.n_blocks, om5.n_levels) == (5, 3)
    ir, _ = forms.scan_final_form(6, (3,))
    sc = E.to_batched_scan_module(ir, {}, fused=True, ops=cpu_table())
    assert isinstance(sc, HipScanModule) and sc.is_batched and sc.n_levels > 0
    assert E.is_scan_apply_term(ir.root)
    ir, _ = forms.omd_scan_attention_form(16, 4, 5, 2, 3)
    assert E.is_omd_apply_term(ir.root) and E.to_batched_omd_module(ir, {}, ops=cpu_table()).is_batched
    x = Var("x", TensorType((4,)))
    relu = IR(Op.make("relu", x), [x])
    for make in (E.to_batched_om_module, E.to_batched_scan_module, E.to_chunked_decayed_module,
                 E.to_batched_omd_module):
        m = make(relu, {}, ops=cpu_table())
        assert not m.is_batched
        assert torch.equal(m(torch.full((4,), -1.0)), torch.zeros(4))
    assert dec.n_blocks == b.K and E.to_chunked_decayed_module(relu, {}, ops=cpu_table()).n_blocks == 0


def test_side_by_side_is_a_view_only_when_the_columns_already_follow():
    from catopt_amd.executors.omd import _side_by_side

    st = torch.randn(6, 10)
    a, b = st[:, :4], st[:, 4:]
    v = _side_by_side(a, b)
    assert torch.equal(v, st) and v.data_ptr() == st.data_ptr()
    for x, y in ((st[:, 4:], st[:, :4]), (torch.randn(6, 3), torch.randn(6, 2)), (st[:, :4], st[:, 5:])):
        assert torch.equal(_side_by_side(x, y), torch.cat([x, y], dim=1))
