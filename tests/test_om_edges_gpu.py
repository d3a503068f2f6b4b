"""Edge cases of the om executor that catopt's lowering tests pin
(tests/test_om_lower_edges.py of luisfuturist/catopt), on the HIP kernels.

* a leaf shared in the DAG, ``om_compose(leaf, leaf)``: the reduction sees it
  once per occurrence (softmax over the duplicated keys) and the leaf runs
  once (``_repeat_idx``, om_lower.py:642-655);
* one query (a Param) over an odd count of key blocks (the ``bmm_qk`` mode
  and the carried-up odd tail of the pair reduction, om_lower.py:800-832);
* a packaged ``om(m, l, a)`` carrier next to a ``q kᵀ`` leaf;
* rows with no key in every block: NaN rows exactly where the oracle has
  them (``om_apply`` is unclamped);
* a sequence shorter than any block, one leaf.

Every output is gated against the numpy oracle's ``om_elem`` /
``om_compose`` / ``om_apply`` on the same (rounded) inputs in float64:
fp32 <= 1e-4, bf16 <= 2e-2 (global relative error), NaN positions exact.
The shapes are the reference test's own (B = 2, T = 8, d = 4 and blocks of
3 or 4 keys) plus one at the kernels' working sizes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import _lib as L
from catopt_amd.executors import HipOMModule
from catopt_amd.ir import IR, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _gate_nan(ref, out, tol):
    on = _np(out)
    assert on.shape == ref.shape, (on.shape, ref.shape)
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    rep = oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, on, 0), rtol=tol)
    assert rep["passed"], rep


def _rand(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _qkt(q, k):
    return mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))


def _run(sink, ir, params, ins, dev):
    res = deliver(ir, params, sink, tuple(t.to(dev) for t in ins))
    mod = res.module
    assert isinstance(mod, HipOMModule) and res.stats["executor"] == "om_batched"
    out = mod(*[t.to(dev) for t in ins])
    assert mod.fallbacks == 0
    return mod, out


def _leaf(q, k, v):
    return oracle.om_elem(q @ np.swapaxes(k, -1, -2), v)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kind", ["attn", "scores"])
def test_a_leaf_shared_in_the_dag_runs_once(sink, dev, dtype, kind):
    B, T, d, n = 2, 8, 4, 4
    v = Var("v", TensorType((B, n, d)))
    if kind == "attn":
        q, k = Var("q", TensorType((B, T, d))), Var("k", TensorType((B, n, d)))
        leaf = mk("om_elem", _qkt(q, k), v)
        ins_vars = [q, k, v]
        ins = [_rand((B, T, d), 1, dtype), _rand((B, n, d), 2, dtype), _rand((B, n, d), 3, dtype)]
        one = _leaf(*(_np(t) for t in ins))
    else:
        s = Var("s", TensorType((B, T, n)))
        leaf = mk("om_elem", s, v)
        ins_vars = [s, v]
        ins = [_rand((B, T, n), 4, dtype, 2.0), _rand((B, n, d), 5, dtype)]
        one = oracle.om_elem(_np(ins[0]), _np(ins[1]))
    ir = IR(mk("om_apply", mk("om_compose", leaf, leaf)), ins_vars)
    mod, out = _run(sink, ir, {}, ins, dev)
    assert mod.leaf_kinds == [kind, kind]
    if kind == "attn":
        assert mod.kernel_leaves == 1  # evaluated once, composed twice
    # the reduction over the duplicated keys: the same softmax
    twice = oracle.om_compose(one, one)
    assert np.allclose(twice[1], 2 * one[1])
    _gate_nan(oracle.om_apply(twice), out, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,d,cuts", [(2, 8, 4, (4, 4, 4)), (1, 96, 64, (48, 80, 32))])
def test_one_query_over_an_odd_count_of_key_blocks(sink, dev, dtype, B, T, d, cuts):
    qp = Param("q", TensorType((B, T, d)))
    ks = [Var(f"k{i}", TensorType((B, c, d))) for i, c in enumerate(cuts)]
    vs = [Var(f"v{i}", TensorType((B, c, d))) for i, c in enumerate(cuts)]
    leaves = [mk("om_elem", _qkt(qp, k), v) for k, v in zip(ks, vs)]
    ir = IR(mk("om_apply", mk("om_compose", mk("om_compose", leaves[0], leaves[1]), leaves[2])), [*ks, *vs])
    tq = _rand((B, T, d), 10, dtype, d ** -0.5)
    tks = [_rand((B, c, d), 11 + i, dtype) for i, c in enumerate(cuts)]
    tvs = [_rand((B, c, d), 21 + i, dtype) for i, c in enumerate(cuts)]
    mod, out = _run(sink, ir, {"q": tq.to(dev)}, [*tks, *tvs], dev)
    assert mod.leaf_kinds == ["attn"] * 3 and mod.kernel_leaves == 3
    s = _np(tq) @ np.swapaxes(np.concatenate([_np(t) for t in tks], -2), -1, -2)
    dense = oracle.om_apply(oracle.om_elem(s, np.concatenate([_np(t) for t in tvs], -2)))
    _gate_nan(dense, out, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_a_packaged_carrier_next_to_a_product_leaf(sink, dev, dtype):
    B, T, d = 2, 8, 4
    q, k1, v1 = Var("q", TensorType((B, T, d))), Var("k1", TensorType((B, 4, d))), Var("v1", TensorType((B, 4, d)))
    m, lv, a = Var("m", TensorType((B, T, 1))), Var("l", TensorType((B, T, 1))), Var("a", TensorType((B, T, d)))
    ir = IR(mk("om_apply", mk("om_compose", mk("om_elem", _qkt(q, k1), v1), mk("om", m, lv, a))),
            [q, k1, v1, m, lv, a])
    tq, tk, tv = _rand((B, T, d), 30, dtype), _rand((B, 4, d), 31, dtype), _rand((B, 4, d), 32, dtype)
    # the carrier of three other keys, from the oracle
    rng = np.random.default_rng(33)
    f = oracle.om_elem(_np(tq) @ rng.standard_normal((B, d, 3)), rng.standard_normal((B, 3, d)))
    fm, fl, fa = (torch.from_numpy(np.ascontiguousarray(x)).float() for x in f)
    mod, out = _run(sink, ir, {}, [tq, tk, tv, fm, fl, fa], dev)
    assert mod.leaf_kinds == ["attn", "om"] and mod.kernel_leaves == 1
    ref = oracle.om_apply(oracle.om_compose(_leaf(_np(tq), _np(tk), _np(tv)), tuple(_np(t) for t in (fm, fl, fa))))
    _gate_nan(ref, out, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rows_with_no_key_in_any_block_are_nan(sink, dev, dtype):
    B, T, dv = 1, 6, 4
    s0, s1 = Var("s0", TensorType((B, T, 3))), Var("s1", TensorType((B, T, 3)))
    v0, v1 = Var("v0", TensorType((B, 3, dv))), Var("v1", TensorType((B, 3, dv)))
    ir = IR(mk("om_apply", mk("om_compose", mk("om_elem", s0, v0), mk("om_elem", s1, v1))), [s0, s1, v0, v1])
    ts0, ts1 = _rand((B, T, 3), 40, dtype, 2.0), _rand((B, T, 3), 41, dtype, 2.0)
    ts0[:, 2] = float("-inf")  # row 2: no key in either block
    ts1[:, 2] = float("-inf")
    ts1[:, 4] = float("-inf")  # row 4: keys in the first block only
    tv0, tv1 = _rand((B, 3, dv), 42, dtype), _rand((B, 3, dv), 43, dtype)
    mod, out = _run(sink, ir, {}, [ts0, ts1, tv0, tv1], dev)
    assert mod.leaf_kinds == ["scores", "scores"]
    ref = oracle.om_apply(oracle.om_compose(oracle.om_elem(_np(ts0), _np(tv0)), oracle.om_elem(_np(ts1), _np(tv1))))
    assert np.isnan(ref[:, 2]).all() and not np.isnan(ref[:, 4]).any()
    _gate_nan(ref, out, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_a_short_sequence_and_one_leaf(sink, dev, dtype):
    B, T, d, n = 1, 2, 4, 4
    q, k, v = Var("q", TensorType((B, T, d))), Var("k", TensorType((B, n, d))), Var("v", TensorType((B, n, d)))
    ir = IR(mk("om_apply", mk("om_elem", _qkt(q, k), v)), [q, k, v])
    ins = [_rand((B, T, d), 50, dtype), _rand((B, n, d), 51, dtype), _rand((B, n, d), 52, dtype)]
    n0 = L.call_count()
    mod, out = _run(sink, ir, {}, ins, dev)
    assert mod.leaf_kinds == ["attn"] and mod.kernel_leaves == 1 and L.call_count() > n0
    _gate_nan(oracle.om_apply(_leaf(*(_np(t) for t in ins))), out, TOL[dtype])
