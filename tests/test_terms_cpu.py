"""catopt's JSON term encoding, read and written on the host.

The committed ``tests/golden/terms.json`` holds delivered terms in the
encoding catopt's own tools persist (``catopt_core/ir.py:366-445``), laid
out as intake census records (``intake/ledger.py:127-138``).  Pinned here:
the file follows from the forms; every program record decodes to a term that
re-encodes to the same data; hand-written text in the reference's spelling
(``-Infinity`` constants, ``__tuple__`` / ``__list__`` attrs, ``mvar``
leaves) decodes to the terms it names; a rewrite pattern, which holds
metavariables, is refused by the loader with their names.  The GPU side
(``test_terms_gpu.py``) delivers the decoded programs through ``HipSink``.
"""

from __future__ import annotations

import json
import math

import pytest
import torch

from catopt_amd.executors import HipOMModule
from catopt_amd.ir import (IR, Const, Op, Param, TensorType, Var, ir_from_record, metavariables, postorder,
                           term_from_data, term_to_data)
from tests.cpu_table import cpu_table
from tests.golden import make_terms

mk = Op.make


def _file():
    return json.loads(make_terms.PATH.read_text())


def test_terms_file_follows_from_the_forms():
    assert _file() == json.loads(make_terms.dumps(make_terms.records()))


def test_program_records_decode_and_round_trip():
    recs = [r for r in _file()["workloads"] if r["name"] != "sdpa_cat_rule_rhs"]
    assert len(recs) == 7
    for rec in recs:
        ir = ir_from_record(rec)
        assert json.loads(json.dumps(term_to_data(ir.root))) == rec["term"], rec["name"]
        assert [(v.name, list(v.typ.shape)) for v in ir.inputs] == [(i["name"], i["shape"]) for i in rec["inputs"]]
        assert sorted({n.op for n in postorder(ir.root)}) == rec["ops"]
    # the -inf fill constant travels as JSON -Infinity and decodes to -inf
    text = make_terms.PATH.read_text()
    assert "-Infinity" in text
    c3 = ir_from_record(next(r for r in recs if r["name"] == "c3_causal_attention"))
    fills = [n.args[2] for n in postorder(c3.root) if n.op == "masked_fill"]
    assert len(fills) == 1 and isinstance(fills[0], Const) and fills[0].value == float("-inf")
    # tuple attrs come back as tuples (split sizes of the K-way form)
    c4 = ir_from_record(next(r for r in recs if r["name"] == "c4_retention"))
    sizes = {n.attrs["sizes"] for n in postorder(c4.root) if n.op == "split"}
    assert sizes == {(64, 64, 64, 64)}


REF_STYLE = """
{"op": "om_apply", "args": [{"op": "om_elem", "args": [
  {"op": "masked_fill", "args": [
    {"op": "mul", "args": [
      {"op": "matmul", "args": [{"var": "q", "shape": [1, 2, 64, 64]},
                                {"op": "transpose", "args": [{"var": "k", "shape": [1, 2, 64, 64]}],
                                 "attrs": {"dim0": -2, "dim1": -1}}], "attrs": {}},
      {"const": 0.125}], "attrs": {}},
    {"op": "split", "args": [{"op": "cmask", "args": [{"var": "q", "shape": [1, 2, 64, 64]}], "attrs": {"off": 0}}],
     "attrs": {"sizes": {"__tuple__": [64]}, "dim": -1, "index": 0}},
    {"const": -Infinity}], "attrs": {}},
  {"var": "v", "shape": [1, 2, 64, 64]}], "attrs": {}}], "attrs": {}}
"""


def test_reference_style_text_decodes_to_the_term_it_spells():
    q, k, v = (Var(n, TensorType((1, 2, 64, 64))) for n in "qkv")
    s = mk("mul", mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1)), Const(0.125))
    m = mk("split", mk("cmask", q, off=0), sizes=(64,), dim=-1, index=0)
    want = mk("om_apply", mk("om_elem", mk("masked_fill", s, m, Const(float("-inf"))), v))
    got = term_from_data(json.loads(REF_STYLE))
    assert got is want  # interned: the same node
    # and it plans as one causal attention leaf on the kernel
    mod = HipOMModule(IR(got, [q, k, v]), {}, ops=cpu_table())
    (lf,) = mod._plan["leaves"]
    assert lf["kind"] == "attn" and lf["mask_kind"] == "causal" and lf["causal_off"] == 0
    assert math.isclose(lf["scale"], 0.125)


def test_attr_markers_and_rejections():
    t = term_from_data({"op": "reshape", "args": [{"param": "w", "shape": [4, 4]}],
                        "attrs": {"shape": {"__list__": [2, 8]}, "dims": {"__tuple__": [{"__tuple__": [1, 2]}, 3]}}})
    assert t.attrs["shape"] == [2, 8] and t.attrs["dims"] == ((1, 2), 3)
    assert t.args[0] == Param("w", TensorType((4, 4)))
    with pytest.raises(ValueError, match="bad attr encoding"):
        term_from_data({"op": "x", "args": [], "attrs": {"a": {"__nope__": 1}}})
    with pytest.raises(ValueError, match="bad term encoding"):
        term_from_data({"leaf": 1})
    with pytest.raises(TypeError):
        term_to_data(mk("x", Var("a", TensorType((1,))), w=torch.zeros(2)))


def test_pattern_records_are_refused_with_their_metavariables():
    rec = next(r for r in _file()["workloads"] if r["name"] == "sdpa_cat_rule_rhs")
    term = term_from_data(rec["term"])  # decodes as a pattern: bare-name leaves
    assert metavariables(term) == ["q", "k1", "k2", "v1", "v2"]
    with pytest.raises(ValueError, match=r"pattern metavariables \['q', 'k1', 'k2', 'v1', 'v2'\]"):
        ir_from_record(rec)
    assert term_from_data({"mvar": "A"}) == "A" and term_to_data("A") == {"mvar": "A"}
