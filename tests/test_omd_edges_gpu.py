"""The omd executor on the terms of catopt's own omd lowering tests
(tests/test_omd_lower.py of luisfuturist/catopt), on the GPU.

The terms are spelled as those tests spell them: a diagonal prefix chain
``f_t = affd_compose(aff_diag(a[t], x[t]), f_{t-1})`` (or its dense
``aff`` counterpart) stacked into ``stack(affd_a f_t)`` / ``stack(affd_b
f_t)`` coefficient maps, scores as Params, the state ``h`` a Param, the
scanned input ``x`` the one input.  Cases: two score blocks over one chain
with a row live in one block only and a row masked in both (NaN); the dense
fibre under ``omd_applym``, alone and as a compose of two blocks; a
projection inside an ordinary tensor term (``matmul(E, stack(affd_a
f_t))``); coefficient maps that are plain Params; determinism across calls
and instances; a bare ``omd_compose`` tree (no ``omd_apply``), which is not
an executor root and returns the carrier tuple.

References are computed independently in float64: softmax attention over
the scan's states from the oracle's serial recurrence (the function the
omd term denotes), or the oracle's carrier ops for the terms that are not
attention over states.  Gate fp32 <= 1e-5 (global relative error), NaN
positions exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.executors import HipOmdModule
from catopt_amd.ir import IR, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make
TOL = 1e-5


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _np(t):
    return t.detach().cpu().double().numpy()


def _gate_nan(ref, out):
    on = _np(out)
    assert on.shape == ref.shape, (on.shape, ref.shape)
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    rep = oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, on, 0), rtol=TOL)
    assert rep["passed"], rep


def _rand(rng, *shape, scale=1.0):
    return rng.standard_normal(shape) * scale


def _chain(a_t, x_v, T, dense=False):
    leaf, comp = ("aff", "aff_compose") if dense else ("aff_diag", "affd_compose")
    fs = []
    for t in range(T):
        lf = mk(leaf, mk("select", a_t, dim=0, index=t), mk("select", x_v, dim=0, index=t))
        fs.append(lf if t == 0 else mk(comp, lf, fs[-1]))
    pa, pb = ("aff_A", "aff_b") if dense else ("affd_a", "affd_b")
    return mk("stack", *[mk(pa, f) for f in fs], dim=0), mk("stack", *[mk(pb, f) for f in fs], dim=0)


def _softmax_rows(sc):
    """Row softmax; a row with no finite score is NaN (0 / 0, as om_apply)."""
    m = sc.max(-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        w = np.exp(sc - m)
        return w / w.sum(-1, keepdims=True)


def _deliver(sink, ir, params, x, dev):
    res = deliver(ir, {n: torch.from_numpy(np.asarray(v, dtype=np.float32)).to(dev) for n, v in params.items()},
                  sink, (torch.from_numpy(x.astype(np.float32)).to(dev),))
    return res


def _run(sink, ir, params, x, dev, mode):
    res = _deliver(sink, ir, params, x, dev)
    mod = res.module
    assert isinstance(mod, HipOmdModule) and res.stats["executor"] == "omd_batched"
    assert mod.is_batched and mod.map_mode == mode, mod.map_mode
    out = mod(torch.from_numpy(x.astype(np.float32)).to(dev))
    assert mod.fallbacks == 0
    return out


def _f32(*arrs):
    return [np.asarray(a, dtype=np.float32).astype(np.float64) for a in arrs]


@pytest.mark.parametrize("T,Tq,d", [(6, 3, 4), (96, 20, 16)])
def test_two_score_blocks_with_dead_and_masked_rows(sink, dev, T, Tq, d):
    p_a, p_h = Param("p_a", TensorType((T, d))), Param("p_h", TensorType((d,)))
    s1, s2 = Param("s1", TensorType((Tq, T))), Param("s2", TensorType((Tq, T)))
    x_v = Var("x", TensorType((T, d)))
    am, bm = _chain(p_a, x_v, T)
    ir = IR(mk("omd_apply", mk("omd_compose", mk("omd_elem", s1, am, bm), mk("omd_elem", s2, am, bm)), p_h), [x_v])
    rng = np.random.default_rng(T)
    sv1, sv2 = _rand(rng, Tq, T), _rand(rng, Tq, T)
    sv2[0, :] = -np.inf  # row 0: keys in block 1 only
    sv1[1, :] = -np.inf  # row 1: no key at all -> NaN
    sv2[1, :] = -np.inf
    av, hv, xv = rng.uniform(-0.9, 0.9, (T, d)), _rand(rng, d), _rand(rng, T, d)
    out = _run(sink, ir, {"p_a": av, "p_h": hv, "s1": sv1, "s2": sv2}, xv, dev, "chain")
    av, hv, xv, sv1, sv2 = _f32(av, hv, xv, sv1, sv2)
    states = oracle.serial_affd_scan(av, xv, hv)
    ref = _softmax_rows(np.concatenate([sv1, sv2], -1)) @ np.concatenate([states, states], 0)
    assert np.isnan(ref[1]).all() and not np.isnan(ref[0]).any()
    _gate_nan(ref, out)


@pytest.mark.parametrize("blocks", [1, 2])
@pytest.mark.parametrize("T,Tq,d", [(7, 3, 4), (64, 9, 12)])
def test_dense_fibre_under_omd_applym(sink, dev, blocks, T, Tq, d):
    p_A, p_h = Param("p_A", TensorType((T, d, d))), Param("p_h", TensorType((d,)))
    ss = [Param(f"s{i}", TensorType((Tq, T))) for i in range(blocks)]
    x_v = Var("x", TensorType((T, d)))
    elems = []
    for s in ss:
        Am, bm = _chain(p_A, x_v, T, dense=True)  # interned: the same maps in every block
        elems.append(mk("omd_elem", s, Am, bm))
    tree = elems[0] if blocks == 1 else mk("omd_compose", elems[0], elems[1])
    ir = IR(mk("omd_applym", tree, p_h), [x_v])
    rng = np.random.default_rng(100 + T + blocks)
    Av = _rand(rng, T, d, d, scale=0.6 / np.sqrt(d))
    hv, xv = _rand(rng, d), _rand(rng, T, d)
    svs = [_rand(rng, Tq, T) for _ in ss]
    out = _run(sink, ir, {"p_A": Av, "p_h": hv} | {f"s{i}": svs[i] for i in range(blocks)}, xv, dev, "chain")
    Av, hv, xv, *svs = _f32(Av, hv, xv, *svs)
    states = oracle.serial_aff_scan(Av, xv, hv[:, None])[..., 0]
    ref = _softmax_rows(np.concatenate(svs, -1)) @ np.concatenate([states] * blocks, 0)
    _gate_nan(ref, out)


def test_a_projection_inside_a_tensor_term(sink, dev):
    T, Tq, d = 6, 4, 3
    p_a, p_h = Param("p_a", TensorType((T, d))), Param("p_h", TensorType((d,)))
    p_s, p_E = Param("p_s", TensorType((Tq, T))), Param("p_E", TensorType((T, T)))
    x_v = Var("x", TensorType((T, d)))
    am, bm = _chain(p_a, x_v, T)
    ir = IR(mk("omd_apply", mk("omd_elem", p_s, mk("matmul", p_E, am), bm), p_h), [x_v])
    rng = np.random.default_rng(70)
    av, hv, sv, Ev, xv = _rand(rng, T, d, scale=0.3), _rand(rng, d), _rand(rng, Tq, T), _rand(rng, T, T), \
        _rand(rng, T, d)
    out = _run(sink, ir, {"p_a": av, "p_h": hv, "p_s": sv, "p_E": Ev}, xv, dev, "chain")
    av, hv, sv, Ev, xv = _f32(av, hv, sv, Ev, xv)
    Pa, Pb = np.cumprod(av, axis=0), oracle.serial_affd_scan(av, xv, np.zeros(d))
    ref = oracle.omd_apply(oracle.omd_elem(sv, Ev @ Pa, Pb), hv)
    _gate_nan(ref, out)


def test_coefficients_as_plain_parameters(sink, dev):
    Tq, K, d = 2, 3, 4
    s, a, b, h = (Param(n, TensorType(sh)) for n, sh in (("s", (Tq, K)), ("a", (K, d)), ("b", (K, d)), ("h", (d,))))
    x_v = Var("x", TensorType((1,)))
    ir = IR(mk("omd_apply", mk("omd_elem", s, a, b), h), [x_v])
    rng = np.random.default_rng(100)
    vals = {"s": _rand(rng, Tq, K), "a": _rand(rng, K, d), "b": _rand(rng, K, d), "h": _rand(rng, d)}
    res = _deliver(sink, ir, vals, np.zeros(1), dev)
    assert res.module.is_batched
    out = res.module(torch.zeros(1, device=dev))
    assert res.module.fallbacks == 0
    sv, av, bv, hv = _f32(vals["s"], vals["a"], vals["b"], vals["h"])
    _gate_nan(oracle.omd_apply(oracle.omd_elem(sv, av, bv), hv), out)


def test_determinism_across_calls_and_instances(sink, dev):
    T, Tq, d = 64, 8, 16
    p_a, p_h, p_s = Param("p_a", TensorType((T, d))), Param("p_h", TensorType((d,))), Param("p_s", TensorType((Tq, T)))
    x_v = Var("x", TensorType((T, d)))
    am, bm = _chain(p_a, x_v, T)
    ir = IR(mk("omd_apply", mk("omd_elem", p_s, am, bm), p_h), [x_v])
    rng = np.random.default_rng(90)
    vals = {"p_a": rng.uniform(-0.9, 0.9, (T, d)), "p_h": _rand(rng, d), "p_s": _rand(rng, Tq, T)}
    xd = torch.from_numpy(_rand(rng, T, d).astype(np.float32)).to(dev)
    m1 = _deliver(sink, ir, vals, xd.cpu().numpy(), dev).module
    m2 = _deliver(sink, ir, vals, xd.cpu().numpy(), dev).module
    o1, o2, o3 = m1(xd).clone(), m1(xd).clone(), m2(xd).clone()
    assert torch.equal(o1, o2) and torch.equal(o1, o3)


def test_a_bare_compose_tree_returns_the_carrier(sink, dev):
    Tq, K, d = 3, 4, 5
    s, a, b = Param("s", TensorType((Tq, K))), Param("a", TensorType((K, d))), Param("b", TensorType((K, d)))
    e = mk("omd_elem", s, a, b)
    ir = IR(mk("omd_compose", e, e), [Var("x", TensorType((1,)))])
    rng = np.random.default_rng(80)
    vals = {"s": _rand(rng, Tq, K), "a": _rand(rng, K, d), "b": _rand(rng, K, d)}
    res = _deliver(sink, ir, vals, np.zeros(1), dev)
    assert not getattr(res.module, "is_batched", False)
    out = res.module(torch.zeros(1, device=dev))
    assert isinstance(out, tuple) and len(out) == 4
    sv, av, bv = _f32(vals["s"], vals["a"], vals["b"])
    f = oracle.omd_elem(sv, av, bv)
    for r, o in zip(oracle.omd_compose(f, f), out):
        rep = oracle.verify_equiv(np.broadcast_to(r, tuple(o.shape)), _np(o), rtol=TOL)
        assert rep["passed"], rep
