"""Leaves shared in the DAG, on every planned executor (GPU).

catopt's lowering tests pin that a leaf used twice, ``compose(leaf, leaf)``,
enters the product or the reduction once per occurrence
(tests/test_scan_fused.py:189-245, test_om_stream.py:259-287,
test_om_fused.py:472-502 of luisfuturist/catopt; the occurrence gather of
scan_fused.py:47-82).  Here: the diagonal and dense scans over a shared
leaf (Params only, no input), a shared subtree four levels deep, the
streaming om fold, and the omd reduction; and the reference's bare
``om_compose`` root, which is not a streaming root and returns the carrier.
References are closed forms (``(a,b)∘(a,b)`` applied to ``h``) or the dense
softmax over duplicated keys, in float64.  Gates fp32 <= 1e-5, NaN exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.executors import HipOmdModule, HipScanModule, HipStreamingOMModule
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


def _gate(ref, out):
    on = _np(out)
    assert on.shape == np.shape(ref), (on.shape, np.shape(ref))
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    rep = oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, on, 0), rtol=TOL)
    assert rep["passed"], rep


def _t(a, dev):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dev)


def _f64(a):
    return np.asarray(a, dtype=np.float32).astype(np.float64)


@pytest.mark.parametrize("depth", [1, 2])
@pytest.mark.parametrize("dense", [False, True])
def test_a_shared_scan_leaf(sink, dev, dense, depth):
    d = 6
    rng = np.random.default_rng(10 + dense + depth)
    h = Param("h", TensorType((d,)))
    if dense:
        A, b = Param("A", TensorType((d, d))), Param("b", TensorType((d,)))
        leaf, comp, app = mk("aff", A, b), "aff_compose", "apply"
        vals = {"A": rng.standard_normal((d, d)) * 0.3, "b": rng.standard_normal(d)}
    else:
        A, b = Param("a", TensorType((d,))), Param("b", TensorType((d,)))
        leaf, comp, app = mk("aff_diag", A, b), "affd_compose", "applyd"
        vals = {"a": rng.uniform(0.1, 0.9, d), "b": rng.standard_normal(d)}
    vals["h"] = rng.standard_normal(d)
    t = mk(comp, leaf, leaf)
    if depth == 2:
        t = mk(comp, t, t)  # a shared subtree: the leaf four times
    ir = IR(mk(app, t, h), [])
    res = deliver(ir, {n: _t(v, dev) for n, v in vals.items()}, sink, ())
    mod = res.module
    assert isinstance(mod, HipScanModule) and mod.is_batched
    out = mod()
    assert mod.fallbacks == 0
    Av, bv, hv = (_f64(vals[n]) for n in (("A" if dense else "a"), "b", "h"))
    ref = hv
    for _ in range(2 ** depth):
        ref = (Av @ ref if dense else Av * ref) + bv
    _gate(ref, out)


def test_a_shared_leaf_in_the_streaming_fold(dev):
    B, H, T, dv, K = 1, 2, 16, 8, 8
    s, v = Var("s", TensorType((B, H, T, K))), Var("v", TensorType((B, H, K, dv)))
    leaf = mk("om_elem", s, v)
    mod = HipStreamingOMModule(IR(mk("om_apply", mk("om_compose", leaf, leaf)), [s, v]), {})
    assert mod.is_streaming
    rng = np.random.default_rng(20)
    ts, tv = rng.standard_normal((B, H, T, K)), rng.standard_normal((B, H, K, dv))
    ts[0, 1, 3] = -np.inf  # a row with no key: NaN
    out = mod(_t(ts, dev), _t(tv, dev))
    ts, tv = _f64(ts), _f64(tv)
    ref = oracle.om_apply(oracle.om_elem(np.concatenate([ts, ts], -1), np.concatenate([tv, tv], -2)))
    _gate(ref, out)


def test_a_shared_leaf_in_the_omd_reduction(sink, dev):
    Tq, K, d = 3, 2, 4
    s = Var("s", TensorType((Tq, K)))
    a, b, h = Param("a", TensorType((K, d))), Param("b", TensorType((K, d))), Param("h", TensorType((d,)))
    leaf = mk("omd_elem", s, a, b)
    ir = IR(mk("omd_apply", mk("omd_compose", leaf, leaf), h), [s])
    rng = np.random.default_rng(30)
    vals = {"a": rng.standard_normal((K, d)), "b": rng.standard_normal((K, d)), "h": rng.standard_normal(d)}
    ts = rng.standard_normal((Tq, K))
    res = deliver(ir, {n: _t(v, dev) for n, v in vals.items()}, sink, (_t(ts, dev),))
    mod = res.module
    assert isinstance(mod, HipOmdModule) and mod.is_batched
    out = mod(_t(ts, dev))
    assert mod.fallbacks == 0
    f = oracle.omd_elem(_f64(ts), _f64(vals["a"]), _f64(vals["b"]))
    _gate(oracle.omd_apply(oracle.omd_compose(f, f), _f64(vals["h"])), out)


def test_a_bare_om_compose_root_returns_the_carrier(dev):
    s1, s2 = Var("s1", TensorType((4, 3))), Var("s2", TensorType((4, 5)))
    v1, v2 = Var("v1", TensorType((3, 6))), Var("v2", TensorType((5, 6)))
    bare = mk("om_compose", mk("om_elem", s1, v1), mk("om_elem", s2, v2))
    mod = HipStreamingOMModule(IR(bare, [s1, s2, v1, v2]), {})
    assert not mod.is_streaming
    rng = np.random.default_rng(40)
    ins = [rng.standard_normal(sh) for sh in ((4, 3), (4, 5), (3, 6), (5, 6))]
    out = mod(*[_t(x, dev) for x in ins])
    assert isinstance(out, tuple) and len(out) == 3
    a, b_, c, e = (_f64(x) for x in ins)
    ref = oracle.om_compose(oracle.om_elem(a, c), oracle.om_elem(b_, e))
    for r, o in zip(ref, out):
        _gate(np.asarray(r), o)
