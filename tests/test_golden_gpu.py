"""The delivered forms on the committed golden fixtures, on the GPU.

Each fixture's inputs (``tests/golden/*.npz``, written from their seeds by
``tests/golden/make_golden.py``) go through ``HipSink`` exactly as catopt
routes a term, and the module's output is compared with the stored float64
result of the numpy restatement.  Gates: fp32 ≤ 1e-5, bf16 ≤ 2e-2 (the
verify metric).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import forms
from catopt_amd.runner import HipGraphRunner
from catopt_amd.sink import HipSink, deliver
from tests.golden import make_golden as G

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _inputs(fx, dev):
    return {k: torch.from_numpy(v).to(torch.bfloat16 if k in fx["bf16"] else torch.float32).to(dev)
            for k, v in fx["inputs"].items()}


def _check(fx, out, tol):
    rep = oracle.verify_equiv(fx["expected"]["y"].astype(np.float64), out.detach().float().cpu().double().numpy(),
                              rtol=tol)
    assert rep["passed"], rep


def _run(sink, ir, params, ins, graph=True):
    res = deliver(ir, params, sink, ins, runner=HipGraphRunner() if graph else None)
    out = res.module(*ins).clone()
    assert int(getattr(res.module, "fallbacks", 0)) == 0, res.stats
    return res, out


def test_golden_c1_weight_chain(sink, dev):
    fx = G.load("c1_weight_chain")
    t = _inputs(fx, dev)
    ir, _ = forms.weight_chain_form(8, 128, 64)
    res, out = _run(sink, ir, {k: v for k, v in t.items() if k != "x"}, (t["x"],))
    assert [s[0] for s in res.module._tape.steps] == ["hip_linear"]
    _check(fx, out, 1e-5)


def test_golden_c2_swiglu(sink, dev):
    fx = G.load("c2_swiglu")
    t = _inputs(fx, dev)
    ir, _ = forms.swiglu_block_form((1, 64), 256, 512)
    res, out = _run(sink, ir, {k: v for k, v in t.items() if k != "x"}, (t["x"],))
    assert [s[0] for s in res.module._tape.steps] == ["rms_norm", "hip_swiglu", "hip_linear"]
    _check(fx, out, 2e-2)


def test_golden_c3_causal_attention(sink, dev):
    fx = G.load("c3_causal_attention")
    t = _inputs(fx, dev)
    ir, _ = forms.causal_attention_form(1, 1, 256, 128, mask="param")
    mask = torch.ones(256, 256, dtype=torch.bool).tril()
    res, out = _run(sink, ir, {"mask": mask}, (t["q"], t["k"], t["v"]))
    assert res.stats["executor"] == "om_batched" and res.stats["hip_kernel"]
    _check(fx, out, 2e-2)


def test_golden_c4_retention(sink, dev):
    fx = G.load("c4_retention")
    t = _inputs(fx, dev)
    ir, _ = forms.retention_kway_form(1, 2, 256, 128, 64)
    res, out = _run(sink, ir, {"gamma": t["gamma"].cpu()}, (t["q"], t["k"], t["v"]))
    assert res.stats["executor"] == "om_decayed_chunked" and res.stats["hip_kernel"]
    _check(fx, out, 2e-2)


def test_golden_c5_ssm(sink, dev):
    fx = G.load("c5_ssm")
    t = _inputs(fx, dev)
    ir, _ = forms.diag_ssm_form(2, 256, 16, 16)
    res, out = _run(sink, ir, {}, tuple(t[n] for n in ("a", "bx", "c", "x", "h")))
    assert res.stats["executor"] == "scan" and res.module.fused_readouts > 0
    _check(fx, out, 1e-5)


def test_golden_aff_linear_recurrence(sink, dev):
    fx = G.load("aff_linear_recurrence")
    t = _inputs(fx, dev)
    ir, _ = forms.dense_scan_form(32, 16, (4,), 1)
    res, out = _run(sink, ir, {}, (t["A"], t["b"], t["h"]))
    assert res.stats["executor"] == "scan" and res.stats["hip_kernel"]
    _check(fx, out, 1e-5)


def test_golden_omd_scan_attention(sink, dev):
    fx = G.load("omd_scan_attention")
    t = _inputs(fx, dev)
    ir, _ = forms.omd_scan_attention_form(128, 16, 16, 4, 16)
    res, out = _run(sink, ir, {}, tuple(t[n] for n in ("q", "k", "a", "x", "h")))
    assert res.stats["executor"] == "omd_batched" and res.stats["hip_kernel"]
    _check(fx, out, 1e-5)
