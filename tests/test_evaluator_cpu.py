"""The generic executor's contract (CPU), after catopt's eval-plan tests
(tests/test_eval_plan.py of luisfuturist/catopt): leaf kinds and roots,
call-time constants, per-call binding resolution, parameters named by the
IR in the state dict, in-place loads, and random init for a Param given no
value.  The HIP-backed ops are swapped for torch functions through the
op-table seam (``tests/cpu_table.py``)."""

from __future__ import annotations

import pytest
import torch

from catopt_amd.evaluator import HipIRModule
from catopt_amd.executors import HipChunkedDecayModule
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var
from tests.cpu_table import cpu_table
from tests.decayed_terms import DecayedTerms

mk = Op.make


def _mod(root, inputs=(), pv=None, ops=None, **kw):
    return HipIRModule(IR(root, list(inputs)), pv or {}, ops=ops or cpu_table(), **kw)


def test_param_and_const_roots_take_no_arguments():
    assert torch.equal(_mod(Param("W", TensorType((3,))), pv={"W": torch.full((3,), 7.0)})(), torch.full((3,), 7.0))
    assert torch.equal(torch.as_tensor(_mod(Const(5))()), torch.tensor(5))


def test_var_roots_and_missing_positionals_read_the_first_input():
    x, y = Var("x", TensorType((2,))), Var("y", TensorType((2,)))
    xv, yv = torch.randn(2), torch.randn(2)
    assert _mod(x, [x])(xv) is xv
    assert _mod(y, [])(xv) is xv  # not an input: reads x
    both = _mod(mk("add", x, y), [x, y])
    assert torch.equal(both(xv), xv + xv) and torch.equal(both(xv, yv), xv + yv)


def test_constants_follow_the_default_dtype_at_call_time():
    x = Var("x", TensorType((4,)))
    mod = _mod(mk("mul", x, Const(0.5)), [x])
    assert mod(torch.randn(4)).dtype == torch.float32
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    try:
        assert mod(torch.randn(4).double()).dtype == torch.float64
    finally:
        torch.set_default_dtype(prev)


def test_bindings_resolve_per_call():
    x = Var("x", TensorType((4,)))
    table = cpu_table()
    mod = _mod(mk("relu", x), [x], ops=table)
    calls = []
    orig = table.torch_bindings["relu"]
    table.torch_bindings["relu"] = lambda t, *a, **kw: (calls.append(1), orig(t))[1]
    xv = torch.randn(4)
    assert torch.equal(mod(xv), xv.clamp_min(0)) and calls == [1]
    del table.torch_bindings["relu"]
    with pytest.raises(ValueError, match="binding"):
        mod(xv)


def test_a_param_with_no_value_is_randomly_initialised():
    x = Var("x", TensorType((1, 3)))
    mod = _mod(mk("add", x, Param("W", TensorType((None, 3)))), [x])
    w = mod.state_dict()["W"]
    assert w.shape == (1, 3) and 0 < w.abs().max() < 0.2
    assert mod(torch.zeros(1, 3)).shape == (1, 3)


def test_the_state_dict_speaks_ir_names_and_loads_in_place():
    x = Var("x", TensorType((2,)))
    mod = _mod(mk("add", x, Param("W", TensorType((2,)))), [x], {"W": torch.zeros(2)})
    sd = mod.state_dict()
    assert list(sd) == ["W"]
    buf = sd["W"]
    xv = torch.ones(2)
    assert torch.equal(mod(xv), xv)
    mod.load_state_dict({"W": torch.full((2,), 3.0)})
    assert torch.equal(mod(xv), xv + 3.0)
    assert mod.state_dict()["W"].data_ptr() == buf.data_ptr()  # same storage: graphs stay valid
    with pytest.raises(RuntimeError, match="Unexpected"):
        mod.load_state_dict({"W": torch.zeros(2), "V": torch.zeros(2)})
    with pytest.raises(RuntimeError, match="Missing"):
        mod.load_state_dict({})
    with pytest.raises(RuntimeError, match="size mismatch"):
        mod.load_state_dict({"W": torch.zeros(3)})
    res = mod.load_state_dict({"W": torch.zeros(2), "V": torch.zeros(2)}, strict=False)
    assert res.unexpected_keys == ["V"] and res.missing_keys == []


def test_a_folded_chain_lists_its_fused_parameter():
    x = Var("x", TensorType((2, 4)))
    A, B = Param("A", TensorType((4, 4))), Param("B", TensorType((4, 4)))
    mod = _mod(mk("matmul", x, mk("matmul", A, B)), [x], {"A": torch.eye(4), "B": 2 * torch.eye(4)})
    keys = list(mod.state_dict())
    assert "A" not in keys and "B" not in keys and len(keys) == 1
    (k,) = keys
    mod.load_state_dict({k: 3 * torch.eye(4)})
    xv = torch.randn(2, 4)
    assert torch.allclose(mod(xv), 3 * xv)


def test_a_planned_executor_loads_through_its_generic_module():
    b = DecayedTerms()
    vals, x = b.values()
    mod = HipChunkedDecayModule(b.ir(b.root()), vals, ops=cpu_table())
    sd = mod.state_dict()
    assert set(sd) == {f"eval_mod.{n}" for n in vals if n != "g2"}
    before = mod(x)
    mod.load_state_dict({k: (v * 0.5 if k.endswith("bv") else v) for k, v in sd.items()})
    after = mod(x)
    assert not torch.allclose(before, after)
