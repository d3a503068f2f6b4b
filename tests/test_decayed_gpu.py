"""The chunked decayed executor on the extracted spellings (GPU).

The pair-product form that extraction delivers (decayed_lower.py:1-10 of
luisfuturist/catopt) is built as catopt's lowering tests build it
(tests/test_decayed_lower.py): q/k/v projections of one input inside the
term, a scalar or per-head decay base.  Each accepted spelling must run the
HIP retention kernel (no fallback) and match the quadratic retention oracle
on the float64 projections of the same values; each term of another
function must run the generic module and match the term evaluated as
written on the CPU in float64.  Gates: bf16 <= 2e-2, fp32 <= 1e-5 (global
relative error).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import kernels as K
from catopt_amd.evaluator import HipIRModule
from catopt_amd.runner import HipGraphRunner
from catopt_amd.sink import HipSink, deliver
from tests.cpu_table import cpu_table
from tests.decayed_terms import DecayedTerms

pytestmark = pytest.mark.gpu

TOL_BF16, TOL_F32 = 2e-2, 1e-5


def _np(t):
    return t.detach().float().cpu().double().numpy() if t.dtype == torch.bfloat16 else t.detach().cpu().double().numpy()


def _gate(ref, out, tol):
    rep = oracle.verify_equiv(ref, _np(out), rtol=tol)
    assert rep["passed"], rep
    return rep


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _dev(vals, x, dev):
    return {n: t.to(dev) for n, t in vals.items()}, x.to(dev)


def _retention_ref(b, vals, x):
    q, k, v = b.projections({n: t.cpu() for n, t in vals.items()}, x.cpu())
    g = vals["g"].detach().cpu().double().numpy()
    return oracle.retention_quadratic(q.numpy(), k.numpy(), v.numpy(), g, 1.0 / b.scale)


CASES = [
    # (B, K, C, D, heads, spelling)
    (2, 4, 64, 64, None, {}),
    (1, 3, 64, 128, 4, {"gate": "row_in", "state": "colscale", "keys": "t_split"}),
    (2, 5, 32, 64, None, {"gate": "row_rev", "assoc": "left", "state": "parsed_rev"}),
    (1, 4, 64, 32, 2, {"assoc": "law"}),
    (2, 3, 16, 32, None, {}),          # the reference test's chunking: T = 48 runs zero-padded
    (1, 7, 24, 48, 3, {"gate": "row_in"}),  # ragged T = 168 and head width 48
]


@pytest.mark.parametrize("B,Kc,C,D,heads,kw", CASES)
def test_extracted_spellings_run_the_retention_kernel(sink, dev, B, Kc, C, D, heads, kw):
    b = DecayedTerms(B=B, K=Kc, C=C, D=D, heads=heads)
    # a per-head decay base stays fp32 (the bench's parameters); a scalar
    # one is rounded to bf16 with the weights (the kernel widens it)
    vals, x = b.values(dtype=torch.bfloat16, seed=B + Kc + C,
                       gamma_dtype=torch.float32 if heads else torch.bfloat16)
    vd, xd = _dev(vals, x, dev)
    res = deliver(b.ir(b.root(**kw)), vd, sink, (xd,))
    mod = res.module
    assert res.stats["executor"] == "om_decayed_chunked" and mod.is_batched and mod.n_chunks == Kc
    out = mod(xd)
    assert mod.fallbacks == 0 and out.shape == x.shape
    _gate(_retention_ref(b, vals, x), out, TOL_BF16)


def test_the_extracted_form_verifies_against_the_term_as_written(sink, dev):
    # verify gate of the drop-in path: the planned module against the same
    # term lowered generically (every op through the HIP bindings), fp32
    b = DecayedTerms(B=2, K=4, C=64, D=64)
    vals, x = b.values(dtype=torch.float32, seed=5)
    vd, xd = _dev(vals, x, dev)
    # fp32 operands run the fp32 retention kernel (no fallback) and equal
    # the written term evaluated op by op on the device
    res32 = deliver(b.ir(b.root()), vd, sink, (xd,), verify_ir=b.ir(b.root()), rtol=TOL_F32)
    assert res32.verified.passed, res32.verified
    mod = res32.module
    out = mod(xd)
    assert mod.is_batched and mod.fallbacks == 0
    _gate(_retention_ref(b, vals, x), out, TOL_F32)
    # bf16 operands: the kernel runs and agrees with the bf16 generic module
    vals16, x16 = b.values(dtype=torch.bfloat16, seed=5)
    vd16, xd16 = _dev(vals16, x16, dev)
    res = deliver(b.ir(b.root()), vd16, sink, (xd16,), verify_ir=b.ir(b.root()), rtol=TOL_BF16)
    assert res.module.is_batched and res.verified.passed, res.verified


@pytest.mark.parametrize("name", ["no_row_gate", "ungated_state", "gated_intra", "distinct_decays"])
def test_terms_of_another_function_run_as_written(sink, dev, name):
    from tests.test_decayed_plan_cpu import _other_functions

    b = DecayedTerms(B=2, K=3, C=32, D=32)
    root = _other_functions(b)[name]
    vals, x = b.values(dtype=torch.float32, seed=9)
    vd, xd = _dev(vals, x, dev)
    res = deliver(b.ir(root), vd, sink, (xd,))
    assert not getattr(res.module, "is_batched", False)
    ref = HipIRModule(b.ir(root), {n: t.double() for n, t in vals.items()}, ops=cpu_table())(x.double())
    _gate(ref.numpy(), res.module(xd), TOL_F32)


def test_graph_replays_of_the_extracted_form(sink, dev):
    b = DecayedTerms(B=1, K=4, C=64, D=128, heads=2)
    vals, x = b.values(dtype=torch.bfloat16, seed=21)
    vd, xd = _dev(vals, x, dev)
    res = deliver(b.ir(b.root(gate="row_rev")), vd, sink, (xd,), runner=HipGraphRunner())
    assert res.stats["cuda_graph"] is True and res.module.is_batched
    ref = _retention_ref(b, vals, x)
    for r in range(3):
        x_r = x if r % 2 == 0 else (x * 0.5).to(x.dtype)
        out = res.module(x_r.to(dev)).clone()
        torch.cuda.synchronize()
        _gate(ref if r % 2 == 0 else _retention_ref(b, vals, x_r), out, TOL_BF16)
        # eager work between replays
        torch.ones(1 << 20, device=dev).sum().item()
    assert res.module.fallbacks == 0


@pytest.mark.parametrize("T", [1, 12, 63, 65, 100, 1000])
def test_retention_kernel_on_ragged_steps(dev, T):
    # T not a multiple of the 64-step chunk runs zero-padded at the end
    B, H, d = 1, 3, 64
    g = torch.Generator().manual_seed(T)
    q, k, v = (torch.randn(B, H, T, d, generator=g).mul(d ** -0.5).to(torch.bfloat16) for _ in range(3))
    gam = np.array([0.9, 0.97, 0.995], dtype=np.float32)
    o = K.retention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(gam).to(dev), 0.5)
    assert o.shape == (B, H, T, d)
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.astype(np.float64), 0.5)
    _gate(ref, o, TOL_BF16)
