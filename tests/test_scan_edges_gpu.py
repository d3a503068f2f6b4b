"""Edge cases of the scan executor that catopt's lowering tests pin
(tests/test_scan_lower_edges.py of luisfuturist/catopt), on the HIP scans.

The terms are the reference test's own: balanced ``aff_compose`` /
``affd_compose`` trees (``_compose``) over leaves whose map is a shared
Param, one Param per leaf, or one input Var in every leaf, and whose offset
is a ``select`` of an input (contiguous or every other row) or a Param per
leaf; nested applications ``apply(f, apply(g, h))``.  ``compose(f, g)``
applies ``g`` first, so leaf 0 of a tree applies last: the reference output
is the recurrence run over the leaves right to left, in float64.  Each case
runs at the reference test's shape and at a longer one; gate fp32 <= 1e-5
(global relative error).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.executors import HipScanModule
from catopt_amd.ir import IR, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make
TOL = 1e-5


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _compose(op, leaves):
    if len(leaves) == 1:
        return leaves[0]
    mid = len(leaves) // 2
    return mk(op, _compose(op, leaves[:mid]), _compose(op, leaves[mid:]))


def _serial(As, bs, h, diagonal):
    hh = np.array(h, dtype=np.float64)
    for A, b in zip(As[::-1], bs[::-1]):
        hh = (A * hh if diagonal else A @ hh) + b
    return hh


def _gate(ref, out):
    rep = oracle.verify_equiv(ref, out.detach().cpu().double().numpy(), rtol=TOL)
    assert rep["passed"], rep


def _rng(seed):
    return np.random.default_rng(seed)


def _run(sink, ir, params, ins, dev):
    res = deliver(ir, {n: torch.from_numpy(v).float().to(dev) for n, v in params.items()}, sink,
                  tuple(torch.from_numpy(v).float().to(dev) for v in ins))
    mod = res.module
    assert isinstance(mod, HipScanModule) and res.stats["executor"] == "scan" and mod.is_batched
    out = mod(*[torch.from_numpy(v).float().to(dev) for v in ins])
    assert mod.fallbacks == 0
    return out


def _maps(rng, n, d, diagonal):
    if diagonal:
        return [rng.uniform(-0.9, 0.9, d) for _ in range(n)]
    return [rng.standard_normal((d, d)) * (0.3 / np.sqrt(d / 4)) for _ in range(n)]


@pytest.mark.parametrize("diagonal", [False, True])
@pytest.mark.parametrize("T,d", [(6, 4), (300, 16)])
def test_a_shared_map_over_selected_offsets(sink, dev, diagonal, T, d):
    A = Param("A", TensorType((d,) if diagonal else (d, d)))
    h, x = Param("h", TensorType((d,))), Var("x", TensorType((T, d)))
    leaf_op, comp, app = ("aff_diag", "affd_compose", "applyd") if diagonal else ("aff", "aff_compose", "apply")
    leaves = [mk(leaf_op, A, mk("select", x, dim=0, index=t)) for t in range(T)]
    ir = IR(mk(app, _compose(comp, leaves), h), [x])
    rng = _rng(T + d)
    Av, hv, xv = _maps(rng, 1, d, diagonal)[0], rng.standard_normal(d), rng.standard_normal((T, d))
    out = _run(sink, ir, {"A": Av, "h": hv}, [xv], dev)
    _gate(_serial([Av] * T, list(xv), hv, diagonal), out)


@pytest.mark.parametrize("diagonal", [False, True])
@pytest.mark.parametrize("T,d", [(4, 3), (96, 8)])
def test_a_map_per_leaf_over_every_other_row(sink, dev, diagonal, T, d):
    As = [Param(f"A{t}", TensorType((d,) if diagonal else (d, d))) for t in range(T)]
    h, x = Param("h", TensorType((d,))), Var("x", TensorType((2 * T, d)))
    leaf_op, comp, app = ("aff_diag", "affd_compose", "applyd") if diagonal else ("aff", "aff_compose", "apply")
    leaves = [mk(leaf_op, As[t], mk("select", x, dim=0, index=2 * t)) for t in range(T)]
    ir = IR(mk(app, _compose(comp, leaves), h), [x])
    rng = _rng(7 * T + d)
    Avs, hv, xv = _maps(rng, T, d, diagonal), rng.standard_normal(d), rng.standard_normal((2 * T, d))
    params = {f"A{t}": Avs[t] for t in range(T)} | {"h": hv}
    out = _run(sink, ir, params, [xv], dev)
    _gate(_serial(Avs, [xv[2 * t] for t in range(T)], hv, diagonal), out)


@pytest.mark.parametrize("T,d", [(3, 2), (40, 12)])
def test_one_input_map_in_every_leaf_and_offsets_per_leaf(sink, dev, T, d):
    a = Var("a", TensorType((d, d)))
    xs = [Var(f"x{t}", TensorType((d,))) for t in range(T)]
    h = Param("h", TensorType((d,)))
    ir = IR(mk("apply", _compose("aff_compose", [mk("aff", a, xt) for xt in xs]), h), [a, *xs])
    rng = _rng(3 * T + d)
    av, hv = _maps(rng, 1, d, False)[0], rng.standard_normal(d)
    xvs = [rng.standard_normal(d) for _ in range(T)]
    out = _run(sink, ir, {"h": hv}, [av, *xvs], dev)
    _gate(_serial([av] * T, xvs, hv, False), out)


@pytest.mark.parametrize("T,d", [(4, 3), (64, 16)])
def test_offsets_as_parameters(sink, dev, T, d):
    A, h = Param("A", TensorType((d, d))), Param("h", TensorType((d,)))
    bs = [Param(f"b{t}", TensorType((d,))) for t in range(T)]
    ir = IR(mk("apply", _compose("aff_compose", [mk("aff", A, b) for b in bs]), h), [])
    rng = _rng(11 * T + d)
    Av, hv = _maps(rng, 1, d, False)[0], rng.standard_normal(d)
    bvs = [rng.standard_normal(d) for _ in range(T)]
    out = _run(sink, ir, {"A": Av, "h": hv} | {f"b{t}": bvs[t] for t in range(T)}, [], dev)
    _gate(_serial([Av] * T, bvs, hv, False), out)


@pytest.mark.parametrize("diagonal", [False, True])
def test_nested_applications_fold_into_one_scan(sink, dev, diagonal):
    d, n = 5, 3
    leaf_op, app = ("aff_diag", "applyd") if diagonal else ("aff", "apply")
    As = [Var(f"A{i}", TensorType((d,) if diagonal else (d, d))) for i in range(n)]
    bs = [Var(f"b{i}", TensorType((d,))) for i in range(n)]
    h = Var("h", TensorType((d,)))
    t = h
    for i in reversed(range(n)):  # apply(f0, apply(f1, apply(f2, h)))
        t = mk(app, mk(leaf_op, As[i], bs[i]), t)
    ir = IR(t, [*As, *bs, h])
    rng = _rng(5 + diagonal)
    Avs, bvs, hv = _maps(rng, n, d, diagonal), [rng.standard_normal(d) for _ in range(n)], rng.standard_normal(d)
    out = _run(sink, ir, {}, [*Avs, *bvs, hv], dev)
    _gate(_serial(Avs, bvs, hv, diagonal), out)
