"""The chunked decayed plan on the extracted spellings (CPU).

Mirrors catopt's lowering tests for ``ChunkedDecayModule``
(tests/test_decayed_lower.py of luisfuturist/catopt): the pair-product form
that extraction delivers (``decayed_lower.py:1-10``) in each of its spellings
must plan, with the integers ``(K, C)`` and the scale pinned; a term that
denotes another function must decline and run as written.  Both halves are
pinned by evaluating the term as written (the generic module on the CPU op
table, float64) against the quadratic retention oracle: every accepted
spelling equals it, every declined variant differs from it.
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest

import oracle
from catopt_amd.evaluator import HipIRModule
from catopt_amd.executors import HipChunkedDecayModule, build_decayed_plan
from catopt_amd.ir import Op, TensorType, Var
from catopt_amd.sink import HipSink, route_spec
from tests.cpu_table import cpu_table
from tests.decayed_terms import SAME_FUNCTION, DecayedTerms

mk = Op.make

SPELLINGS = [dict(zip(SAME_FUNCTION, combo)) for combo in itertools.product(*SAME_FUNCTION.values())]


def _np(t):
    return t.detach().double().numpy()


def _as_written(b: DecayedTerms, root, vals, x):
    return _np(HipIRModule(b.ir(root), vals, ops=cpu_table())(x))


def _retention(b: DecayedTerms, vals, x):
    q, k, v = b.projections(vals, x)
    return oracle.retention_quadratic(_np(q), _np(k), _np(v), _np(vals["g"]), 1.0 / b.scale)


def _pins(p, b: DecayedTerms):
    assert (p["K"], p["C"]) == (b.K, b.C)
    assert math.isclose(p["scale"], 1.0 / b.scale, rel_tol=1e-15)
    assert (p["q"], p["k"], p["v"], p["g"]) == (b.q, b.k, b.v, b.g)


@pytest.mark.parametrize("kw", SPELLINGS, ids=lambda kw: "-".join(kw.values()))
def test_every_spelling_of_the_extracted_form_plans(kw):
    b = DecayedTerms()
    _pins(build_decayed_plan(b.root(**kw)), b)


def test_spellings_mixed_across_summands_plan():
    # extraction picks each e-class's spelling on its own: one plan must take
    # a different spelling in every summand
    b = DecayedTerms(K=4, C=8)
    cyc = itertools.cycle(SPELLINGS[::5])
    arms = []
    for i in range(b.K):
        kw = next(cyc)
        t = b.intra(i, keys=kw["keys"], law=kw["assoc"] == "law")
        for j in range(i):
            t = mk("add", t, b.cross(i, j, **next(cyc)))
        arms.append(t)
    root = mk("concat", *arms, dim=-2)
    _pins(build_decayed_plan(root), b)
    vals, x = b.values()
    assert oracle.verify_equiv(_retention(b, vals, x), _as_written(b, root, vals, x), rtol=1e-12)["passed"]


@pytest.mark.parametrize("heads", [None, 3])
def test_every_accepted_spelling_denotes_retention(heads):
    # what makes the plan legitimate: each spelling, evaluated as written,
    # is scale · Σ_{s<=t} γ^(t-s) (q_t·k_s) v_s
    b = DecayedTerms(heads=heads)
    vals, x = b.values()
    ref = _retention(b, vals, x)
    for kw in SPELLINGS:
        assert oracle.verify_equiv(ref, _as_written(b, b.root(**kw), vals, x), rtol=1e-12)["passed"], kw


def _other_functions(b: DecayedTerms) -> dict:
    """Terms of the family that denote something other than retention."""
    out = {
        "no_row_gate": b.root(gate="none"),
        "ungated_state": b.root(state="no_mul"),
        "non_key_state": b.root(state="add"),
        "gated_intra": b.root(row=True),
    }
    # a second decay base in every arm after the first (the reference's
    # distinct-decays case)
    arms = [b.arm(i, decay=b.decay(b.g2) if i else None) for i in range(b.K)]
    out["distinct_decays"] = mk("concat", *arms, dim=-2)
    # a score that is not one q kᵀ
    twice = mk("add", mk("matmul", b.qi(0), b.kti(0)), mk("matmul", b.qi(0), b.kti(0)))
    out["non_product_score"] = mk("concat", b.arm(0, score=twice), *[b.arm(i) for i in range(1, b.K)], dim=-2)
    return out


def test_terms_of_another_function_decline_and_run_as_written():
    b = DecayedTerms()
    vals, x = b.values()
    ref = _retention(b, vals, x)
    for name, root in _other_functions(b).items():
        assert build_decayed_plan(root) is None, name
        written = _as_written(b, root, vals, x)
        # the decline is necessary: the term really is another function
        assert not oracle.verify_equiv(ref, written, rtol=1e-3)["passed"], name
        mod = HipChunkedDecayModule(b.ir(root), vals, ops=cpu_table())
        assert not mod.is_batched and mod.n_chunks == 0
        assert np.array_equal(_np(mod(x)), written), name


def test_structural_declines():
    b = DecayedTerms(K=3, C=8)
    good = [b.arm(i) for i in range(3)]
    # not a concat, or a concat on another axis
    assert build_decayed_plan(b.q) is None
    assert build_decayed_plan(mk("concat", *good, dim=-1)) is None
    # an arm without its intra element
    assert build_decayed_plan(mk("concat", good[0], b.cross(1, 0), good[2], dim=-2)) is None
    # two intra elements in one arm
    assert build_decayed_plan(mk("concat", good[0], mk("add", good[1], b.intra(1)), good[2], dim=-2)) is None
    # a cross block missing, repeated, or from the wrong source chunk
    assert build_decayed_plan(mk("concat", good[0], good[1], mk("add", b.intra(2), b.cross(2, 0)), dim=-2)) is None
    assert build_decayed_plan(mk("concat", good[0], mk("add", good[1], b.cross(1, 0)), good[2], dim=-2)) is None
    bad = mk("add", mk("add", b.intra(2), b.cross(2, 0)), b.cross(2, 0))
    assert build_decayed_plan(mk("concat", good[0], good[1], bad, dim=-2)) is None
    # the arms out of order
    assert build_decayed_plan(mk("concat", good[1], good[0], good[2], dim=-2)) is None
    # a v of another width in one intra element
    wide = Var("v_wide", TensorType((b.B, b.C, b.D + 1)))
    arm1 = mk("add", mk("div", mk("om_decayed", mk("matmul", b.qi(1), b.kti(1)), b.decay(), wide), b.S),
              b.cross(1, 0))
    assert build_decayed_plan(mk("concat", good[0], arm1, good[2], dim=-2)) is None
    # a cross term whose scale differs from the intra elements'
    odd = mk("add", b.intra(1), mk("mul", b.row(b.C), mk("div", b.pair(1, 0), mk("add", b.S, b.S))))
    assert build_decayed_plan(mk("concat", good[0], odd, good[2], dim=-2)) is None


@pytest.mark.parametrize("mistake", ["offset", "col_sign", "col_offset", "row_sign", "period"])
def test_planted_gate_integers_decline(mistake):
    b = DecayedTerms(K=3, C=8)

    def cross(i, j):
        off = (i - j) * b.C + (1 if mistake == "offset" else 0)
        t = b.C + 1 if mistake == "period" else b.C
        row = mk("unsqueeze", mk("decay_vec", b.g, t=t, sign=-1 if mistake == "row_sign" else 1, offset=off), dim=-1)
        col = mk("unsqueeze", mk("decay_vec", b.g, t=b.C, sign=1 if mistake == "col_sign" else -1,
                                 offset=1 if mistake == "col_offset" else 0), dim=-1)
        a = mk("transpose", mk("mul", b.ki(j), col), dim0=-1, dim1=-2)
        return mk("mul", row, mk("div", mk("matmul", b.qi(i), mk("matmul", a, b.vi(j))), b.S))

    arms = []
    for i in range(b.K):
        t = b.intra(i)
        for j in range(i):
            t = mk("add", t, cross(i, j))
        arms.append(t)
    assert build_decayed_plan(mk("concat", *arms, dim=-2)) is None


def test_the_sink_routes_the_extracted_form_to_the_chunked_executor():
    sink = HipSink(device="cpu", ops=cpu_table())
    b = DecayedTerms()
    assert route_spec(b.root(), sink).name == "om_decayed_chunked"
    assert route_spec(b.root(assoc="law", gate="row_in"), sink).name == "om_decayed_chunked"
    spec = route_spec(b.root(gate="none"), sink)
    assert spec is None or spec.name != "om_decayed_chunked"


def test_the_chunked_module_on_host_inputs_runs_the_term_as_written():
    # host tensors: the kernel cannot run, the module counts one fallback and
    # its output is the generic module's, bit for bit
    b = DecayedTerms()
    vals, x = b.values()
    mod = HipChunkedDecayModule(b.ir(b.root()), vals, ops=cpu_table())
    assert mod.is_batched and mod.n_chunks == b.K
    out = _np(mod(x))
    assert mod.fallbacks == 1
    assert np.array_equal(out, _as_written(b, b.root(), vals, x))
