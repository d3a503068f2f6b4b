"""Terms in catopt's JSON encoding, decoded and delivered on the GPU.

Each program record of ``tests/golden/terms.json`` (catopt's term encoding,
``catopt_core/ir.py:366-445``, in the intake census layout) is decoded with
``ir_from_record`` and lowered through ``HipSink`` as catopt routes a term.
The five configs run on the inputs of their golden fixtures
(``tests/golden/*.npz``) and are compared with the stored float64 outputs;
the OM_SPLIT spellings and the small SSM are compared with the numpy oracle
on seeded inputs.  Gates: fp32 ≤ 1e-5, bf16 ≤ 2e-2 (the verify metric), NaN
positions exact.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.ir import ir_from_record
from catopt_amd.sink import HipSink, deliver
from tests.golden import make_golden as G
from tests.golden import make_terms

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sink():
    return HipSink()


@pytest.fixture(scope="module")
def records():
    return {r["name"]: r for r in json.loads(make_terms.PATH.read_text())["workloads"]}


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _gate(ref, out, tol):
    on = _np(out)
    assert on.shape == ref.shape
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    rep = oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, on, 0), rtol=tol)
    assert rep["passed"], rep


def _golden(name, dev):
    fx = G.load(name)
    t = {k: torch.from_numpy(v).to(torch.bfloat16 if k in fx["bf16"] else torch.float32).to(dev)
         for k, v in fx["inputs"].items()}
    return fx, t


def _deliver(sink, rec, params, ins):
    ir = ir_from_record(rec)
    res = deliver(ir, params, sink, tuple(ins))
    assert res.stats["hip_kernel"] and res.stats["torch_fallback_ops"] == 0, res.stats
    out = res.module(*ins)
    assert int(getattr(res.module, "fallbacks", 0)) == 0
    return res, out


@pytest.mark.parametrize("name,executor,tol", [
    ("c1_weight_chain", "generic", 1e-5),
    ("c2_swiglu", "generic", 2e-2),
    ("c3_causal_attention", "om_batched", 2e-2),
    ("c4_retention", "om_decayed_chunked", 2e-2),
])
def test_config_terms_on_their_golden_inputs(sink, dev, records, name, executor, tol):
    fx, t = _golden(name, dev)
    rec = records[name]
    in_names = [i["name"] for i in rec["inputs"]]
    params = {k: (v.cpu() if name == "c4_retention" else v) for k, v in t.items() if k not in in_names}
    res, out = _deliver(sink, rec, params, [t[n] for n in in_names])
    assert res.stats["executor"] == executor
    _gate(fx["expected"]["y"].astype(np.float64), out, tol)


def test_ssm_term(sink, dev, records):
    rec = records["c5_ssm"]
    rng = np.random.default_rng(15)
    B, T, D, N = 2, 8, 16, 16
    a = (1.0 / (1.0 + np.exp(rng.standard_normal((B, T, D, N))))).astype(np.float32)
    bx, c = (rng.standard_normal((B, T, N)).astype(np.float32) for _ in range(2))
    x = rng.standard_normal((B, T, D)).astype(np.float32)
    h = rng.standard_normal((B, D, N)).astype(np.float32)
    ins = [torch.from_numpy(z).to(dev) for z in (a, bx, c, x, h)]
    res, out = _deliver(sink, rec, {}, ins)
    assert res.stats["executor"] == "scan"
    y, _ = oracle.ssm_serial(*(z.astype(np.float64) for z in (a, bx, c, x, h)))
    _gate(y, out, 1e-5)


def _om_blocks(s, v, cuts):
    edges = [0, *np.cumsum(cuts)]
    leaves = [oracle.om_elem(s[..., a:b], v[..., a:b, :]) for a, b in zip(edges[:-1], edges[1:])]
    return oracle.fused_om_levels(*(np.stack([f[i] for f in leaves]) for i in range(3)))


def _bf16(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def test_sdpa_cat_split_term(sink, dev, records):
    rec = records["sdpa_cat_split"]
    shapes = {i["name"]: tuple(i["shape"]) for i in rec["inputs"]}
    ins = [_bf16(shapes[n], 200 + j) for j, n in enumerate(shapes)]
    res, out = _deliver(sink, rec, {}, [t.to(dev) for t in ins])
    assert res.stats["executor"] == "om_batched" and res.module.kernel_leaves == 2
    q = _np(ins[0])
    K = np.concatenate([_np(ins[1]), _np(ins[2])], -2)
    V = np.concatenate([_np(ins[3]), _np(ins[4])], -2)
    scq = float(torch.tensor(0.125, dtype=torch.bfloat16))  # q · fill(q, SC) in q's dtype
    s = np.where(oracle.cmask_keep(q.shape[-2], K.shape[-2]), scq * (q @ np.swapaxes(K, -1, -2)), -np.inf)
    _gate(_om_blocks(s, V, (80, 112)), out, 2e-2)


def test_attnbias_split_term(sink, dev, records):
    rec = records["attnbias_split"]
    shapes = {i["name"]: tuple(i["shape"]) for i in rec["inputs"]}
    ins = [_bf16(shapes[n], 300 + j) for j, n in enumerate(shapes)]
    T, d = shapes["q"][-2], shapes["q"][-1]
    rng = np.random.default_rng(4)
    keep = rng.random((T, T)) < 0.5
    keep[3] = False  # a row with no key: NaN, as dense softmax
    res, out = _deliver(sink, rec, {"m": torch.from_numpy(keep)}, [t.to(dev) for t in ins])
    assert res.stats["executor"] == "om_batched" and res.module.kernel_leaves == 2
    s = np.where(keep, d ** -0.5 * (_np(ins[0]) @ np.swapaxes(_np(ins[1]), -1, -2)), -np.inf)
    _gate(_om_blocks(s, _np(ins[2]), (48, 80)), out, 2e-2)


def test_pattern_record_is_not_lowered(sink, records):
    with pytest.raises(ValueError, match="pattern metavariables"):
        ir_from_record(records["sdpa_cat_rule_rhs"])
