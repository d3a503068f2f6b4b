"""Operand spellings on the planned executors' edges (GPU), from catopt's
second wave of lowering tests (tests/test_model_blocks_lowering.py:193-985
of luisfuturist/catopt):

* a scan whose leaf offsets are ``select(x, dim=1, t)`` of a ``(d, T)``
  input;
* om leaves whose keys are ``chunk``s of one tensor along the feature axis,
  whose query and keys differ in rank (both ways), or whose values are
  ``select``s of one stacked tensor;
* omd chains whose projection stacks run along axis 1 (under a transpose),
  whose leaf parts are ``select``s along axis 1, or every other step; an
  ``omd`` packaging leaf of Params; two leaves whose carriers broadcast
  against each other.

Each term is delivered through the sink on the GPU and compared with the
same term evaluated as written by the generic module on the CPU in float64
(the torch op table), at fp32 <= 1e-5 and bf16 <= 2e-2 (global relative
error).  The planned executor must engage where it plans the term.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.evaluator import HipIRModule
from catopt_amd.ir import IR, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink, deliver
from tests.cpu_table import cpu_table

pytestmark = pytest.mark.gpu
mk = Op.make
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(99 + seed)
    return torch.randn(tuple(shape), dtype=torch.float64, generator=g) * scale


def _compose(op, leaves):
    if len(leaves) == 1:
        return leaves[0]
    mid = len(leaves) // 2
    return mk(op, _compose(op, leaves[:mid]), _compose(op, leaves[mid:]))


def _check(sink, dev, ir, params, ins, dtype, executor):
    """Deliver on the GPU in ``dtype``; compare with the CPU float64
    evaluation of the term on the same (rounded) values."""
    params = {n: v.to(dtype) for n, v in params.items()}
    ins = [v.to(dtype) for v in ins]
    res = deliver(ir, {n: v.to(dev) for n, v in params.items()}, sink, tuple(v.to(dev) for v in ins))
    mod = res.module
    assert res.stats["executor"] == executor and mod.is_batched, res.stats
    out = mod(*[v.to(dev) for v in ins])
    assert getattr(mod, "fallbacks", 0) == 0
    ref = HipIRModule(ir, {n: v.double() for n, v in params.items()}, ops=cpu_table())(*[v.double() for v in ins])
    rep = oracle.verify_equiv(ref.numpy(), out.detach().float().cpu().double().numpy(), rtol=TOL[dtype])
    assert rep["passed"], rep


def test_scan_offsets_selected_along_axis_1(sink, dev):
    T, d = 8, 3
    x = Var("x", TensorType((d, T)))
    leaves = [mk("aff", Param(f"A{t}", TensorType((d, d))), mk("select", x, dim=1, index=t)) for t in range(T)]
    ir = IR(mk("apply", _compose("aff_compose", leaves), Param("h", TensorType((d,)))), [x])
    params = {f"A{t}": _rand((d, d), t, 0.3) for t in range(T)} | {"h": _rand((d,), 9)}
    _check(sink, dev, ir, params, [_rand((d, T), 5)], torch.float32, "scan")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_om_keys_chunked_along_the_feature_axis(sink, dev, dtype):
    n, T, d, dv = 2, 6, 16, 8
    q, Kb = Var("q", TensorType((T, d))), Var("Kb", TensorType((4, n * d)))
    vs = [Var(f"v{i}", TensorType((4, dv))) for i in range(n)]
    elems = [mk("om_elem", mk("matmul", q, mk("transpose", mk("chunk", Kb, chunks=n, dim=-1, index=i),
                                                dim0=-2, dim1=-1)), vs[i]) for i in range(n)]
    ir = IR(mk("om_apply", _compose("om_compose", elems)), [q, Kb, *vs])
    ins = [_rand((T, d), 1), _rand((4, n * d), 2)] + [_rand((4, dv), 3 + i) for i in range(n)]
    _check(sink, dev, ir, {}, ins, dtype, "om_batched")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("gap", ["q_lower", "k_lower"])
def test_om_query_and_keys_of_different_rank(sink, dev, dtype, gap):
    n, B, H, T, d, dv = 3, 2, 2, 6, 16, 8
    if gap == "q_lower":  # q (T, d) against k_i (B, K, d)
        q = Var("q", TensorType((T, d)))
        ks = [Var(f"k{i}", TensorType((B, 4, d))) for i in range(n)]
        vs = [Var(f"v{i}", TensorType((B, 4, dv))) for i in range(n)]
        ins = [_rand((T, d), 1)] + [_rand((B, 4, d), 2 + i) for i in range(n)] + \
              [_rand((B, 4, dv), 10 + i) for i in range(n)]
    else:  # q (B, H, T, d) against k_i (K, d); v carries the batch axes
        q = Var("q", TensorType((B, H, T, d)))
        ks = [Var(f"k{i}", TensorType((4, d))) for i in range(n)]
        vs = [Var(f"v{i}", TensorType((B, H, 4, dv))) for i in range(n)]
        ins = [_rand((B, H, T, d), 20)] + [_rand((4, d), 30 + i) for i in range(n)] + \
              [_rand((B, H, 4, dv), 40 + i) for i in range(n)]
    elems = [mk("om_elem", mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1)), v) for k, v in zip(ks, vs)]
    ir = IR(mk("om_apply", _compose("om_compose", elems)), [q, *ks, *vs])
    _check(sink, dev, ir, {}, ins, dtype, "om_batched")


def test_om_values_selected_from_one_stack(sink, dev):
    n, B, T, dv = 3, 2, 6, 4
    s, V = Var("s", TensorType((B, T, 4))), Var("V", TensorType((n, B, 4, dv)))
    elems = [mk("om_elem", s, mk("select", V, dim=0, index=i)) for i in range(n)]
    ir = IR(mk("om_apply", _compose("om_compose", elems)), [s, V])
    _check(sink, dev, ir, {}, [_rand((B, T, 4), 1), _rand((n, B, 4, dv), 2)], torch.float32, "om_batched")


def _omd_chain(T, d, gather_dim=0, idxs=None, stack_dim=0):
    idxs = list(range(T)) if idxs is None else idxs
    N = max(idxs) + 1
    shape = (d, N) if gather_dim else (N, d)
    a_p, x_v = Param("p_a", TensorType(shape)), Var("x", TensorType(shape))
    leaves = [mk("aff_diag", mk("select", a_p, dim=gather_dim, index=i), mk("select", x_v, dim=gather_dim, index=i))
              for i in idxs]
    fs = [leaves[0]]
    for t in range(1, len(idxs)):
        fs.append(mk("affd_compose", leaves[t], fs[-1]))

    def stk(proj):
        node = mk("stack", *(mk(proj, f) for f in fs), dim=stack_dim)
        return mk("transpose", node, dim0=0, dim1=1) if stack_dim else node

    term = mk("omd_apply", mk("omd_elem", Param("s", TensorType((3, len(idxs)))), stk("affd_a"), stk("affd_b")),
              Param("h", TensorType((d,))))
    return IR(term, [x_v]), shape


@pytest.mark.parametrize("case", ["stack_dim_1", "gather_dim_1", "every_other_step"])
def test_omd_chains_on_other_axes_and_strides(sink, dev, case):
    T, d = 6, 4
    if case == "stack_dim_1":
        ir, shape = _omd_chain(T, d, stack_dim=1)
        nsteps = T
    elif case == "gather_dim_1":
        ir, shape = _omd_chain(T, d, gather_dim=1)
        nsteps = T
    else:
        idxs = [0, 2, 4, 6, 8, 10]
        ir, shape = _omd_chain(len(idxs), d, idxs=idxs)
        nsteps = len(idxs)
    params = {"p_a": _rand(shape, 1).clamp(-0.9, 0.9), "s": _rand((3, nsteps), 2), "h": _rand((d,), 3)}
    _check(sink, dev, ir, params, [_rand(shape, 4)], torch.float32, "omd_batched")


def test_omd_packaging_leaf_and_broadcasting_leaves(sink, dev):
    Tq, T, d = 3, 6, 4
    P = lambda n, *s: Param(n, TensorType(s))  # noqa: E731
    pkg = mk("omd", P("m", Tq, 1), P("l", Tq, 1), P("fa", Tq, d), P("fb", Tq, d))
    elem = mk("omd_elem", P("s", Tq, T), P("aa", T, d), P("bb", T, d))
    ir = IR(mk("omd_apply", mk("omd_compose", elem, pkg), P("h", d)), [Var("dummy", TensorType((1,)))])
    params = {"s": _rand((Tq, T), 1), "aa": _rand((T, d), 2), "bb": _rand((T, d), 3), "h": _rand((d,), 4),
              "m": _rand((Tq, 1), 5), "l": _rand((Tq, 1), 6).abs() + 0.5, "fa": _rand((Tq, d), 7),
              "fb": _rand((Tq, d), 8)}
    _check(sink, dev, ir, params, [torch.zeros(1, dtype=torch.float64)], torch.float32, "omd_batched")
    # a leaf whose carrier broadcasts against the other's: (3, 4) and (1, 4) scores
    h = Var("h", TensorType((d,)))
    comp = mk("omd_compose", mk("omd_elem", P("s1", 3, 4), P("a1", 4, d), P("b1", 4, d)),
              mk("omd_elem", P("s2", 1, 4), P("a2", 4, d), P("b2", 4, d)))
    ir2 = IR(mk("omd_apply", comp, h), [h])
    params2 = {"s1": _rand((3, 4), 1), "s2": _rand((1, 4), 2), "a1": _rand((4, d), 3), "b1": _rand((4, d), 4),
               "a2": _rand((4, d), 5), "b2": _rand((4, d), 6)}
    _check(sink, dev, ir2, params2, [_rand((d,), 7)], torch.float32, "omd_batched")


def test_a_bare_affine_compose_root_returns_the_map(sink, dev):
    # no apply above the tree (tests/test_scan_batched.py:271-302): not a
    # scan root; the generic module returns the composed (A, b) pair,
    # (A, x1) ∘ (A, x0) = (A A, A x0 + x1)
    d = 8
    A, x = Param("p_a", TensorType((d, d))), Var("x", TensorType((4, d)))
    bare = mk("aff_compose", mk("aff", A, mk("select", x, dim=0, index=1)), mk("aff", A, mk("select", x, dim=0, index=0)))
    Av, xv = _rand((d, d), 1, 0.3), _rand((4, d), 2)
    res = deliver(IR(bare, [x]), {"p_a": Av.float().to(dev)}, sink, (xv.float().to(dev),))
    assert not getattr(res.module, "is_batched", False)
    out = res.module(xv.float().to(dev))
    assert isinstance(out, tuple) and len(out) == 2
    for r, o in zip((Av @ Av, Av @ xv[0] + xv[1]), out):
        rep = oracle.verify_equiv(r.numpy(), o.detach().cpu().double().numpy(), rtol=1e-5)
        assert rep["passed"], rep
