"""Writes ``terms.json``: delivered terms in catopt's JSON term encoding.

The encoding is the one catopt's own tools persist terms in
(``catopt_core/ir.py:366-445``: ``{"op", "args", "attrs"}`` nodes,
``{"var" | "param", "shape"}`` and ``{"const": v}`` leaves, ``{"mvar"}``
metavariables, ``{"__tuple__"}`` / ``{"__list__"}`` attrs, raw floats so
``-inf`` is written as JSON ``-Infinity``), laid out as the intake census
records it (``intake/ledger.py:127-138``: ``name``, ``ops``, ``term``,
``inputs``).  The terms are this package's spellings of the delivered forms
(``catopt_amd.forms``) at the shapes of the golden fixtures beside this
file, plus the OM_SPLIT spellings of the sdpa right-hand sides
(``om.py:1195-1340``) and one rewrite-rule pattern, which holds
metavariables and must be refused by a loader.

Run from the repository root: ``python tests/golden/make_terms.py``.
``records()`` returns the records without writing, so the tests can check
that the committed file still follows from the forms.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from catopt_amd import forms  # noqa: E402
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var, record_from_ir, term_to_data  # noqa: E402

PATH = HERE / "terms.json"
mk = Op.make
NEG_INF = Const(float("-inf"))


def _qkt(q, k):
    return mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))


def sdpa_cat_split(B=1, H=2, Tq=192, cuts=(80, 112), d=64, sc=0.125) -> IR:
    """``om_apply(om_compose(...))`` of the causal sdpa-cat right-hand side
    (``om.py:1205-1222``) after OM_SPLIT: one leaf per key block, each
    ``masked_fill(split(S), split(cmask(S)), -inf)`` over ``split(V)``."""
    q = Var("q", TensorType((B, H, Tq, d)))
    ks = [Var(f"k{i + 1}", TensorType((B, H, c, d))) for i, c in enumerate(cuts)]
    vs = [Var(f"v{i + 1}", TensorType((B, H, c, d))) for i, c in enumerate(cuts)]
    qs = mk("mul", q, mk("fill", q, value=sc))
    S = mk("concat", *[_qkt(qs, k) for k in ks], dim=-1)
    V = mk("concat", *vs, dim=-2)
    M = mk("cmask", S)
    leaves = []
    for i in range(len(cuts)):
        s_i = mk("masked_fill", mk("split", S, sizes=tuple(cuts), dim=-1, index=i),
                 mk("split", M, sizes=tuple(cuts), dim=-1, index=i), NEG_INF)
        leaves.append(mk("om_elem", s_i, mk("split", V, sizes=tuple(cuts), dim=-2, index=i)))
    tree = leaves[0]
    for lf in leaves[1:]:
        tree = mk("om_compose", tree, lf)
    return IR(mk("om_apply", tree), [q, *ks, *vs])


def attnbias_split(B=1, H=2, T=128, d=128, cuts=(48, 80)) -> IR:
    """The attn_mask right-hand side (``om.py:1315-1340``) after OM_SPLIT:
    ``add(split(S), split(attnbias(m)))`` leaves, ``m`` a weight."""
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    m = Param("m", TensorType((T, T)))
    S = mk("mul", _qkt(q, k), Const(d ** -0.5))
    bias = mk("attnbias", m)
    leaves = [mk("om_elem", mk("add", mk("split", S, sizes=cuts, dim=-1, index=i),
                               mk("split", bias, sizes=cuts, dim=-1, index=i)),
                 mk("split", v, sizes=cuts, dim=-2, index=i)) for i in range(len(cuts))]
    return IR(mk("om_apply", mk("om_compose", *leaves)), [q, k, v])


def sdpa_cat_pattern():
    """The sdpa-cat right-hand side as a rewrite rule holds it: metavariable
    leaves ``q``, ``k1``... and an attr metavariable ``SC``
    (``om.py:1205-1222``)."""
    qs = mk("mul", "q", mk("fill", "q", value="SC"))
    S = mk("concat", _qkt(qs, "k1"), _qkt(qs, "k2"), dim=-1)
    return mk("om_apply", mk("om_elem", S, mk("concat", "v1", "v2", dim=-2)))


def records() -> list[dict]:
    out = [
        record_from_ir("c1_weight_chain", forms.weight_chain_form(8, 128, 64)[0]),
        record_from_ir("c2_swiglu", forms.swiglu_block_form((1, 64), 256, 512)[0]),
        record_from_ir("c3_causal_attention", forms.causal_attention_form(1, 1, 256, 128, mask="cmask")[0]),
        record_from_ir("c4_retention", forms.retention_kway_form(1, 2, 256, 128, 64)[0]),
        record_from_ir("c5_ssm", forms.diag_ssm_form(2, 8, 16, 16)[0]),
        record_from_ir("sdpa_cat_split", sdpa_cat_split()),
        record_from_ir("attnbias_split", attnbias_split()),
    ]
    pat = sdpa_cat_pattern()
    out.append({"name": "sdpa_cat_rule_rhs", "ops": sorted({"om_apply", "om_elem", "concat", "matmul",
                                                            "transpose", "mul", "fill"}),
                "term": term_to_data(pat), "inputs": []})
    return out


def dumps(recs: list[dict]) -> str:
    """One record per line, compact (the unrolled scan terms repeat their
    prefix chains: the encoding keeps no DAG sharing)."""
    body = ",\n".join(json.dumps(r, separators=(",", ":")) for r in recs)
    return '{"format": 1, "workloads": [\n' + body + "\n]}\n"


def main() -> None:
    PATH.write_text(dumps(records()))
    print(f"{PATH.relative_to(ROOT)}: {PATH.stat().st_size} bytes")


if __name__ == "__main__":
    main()
