"""Mask planes that broadcast against the score, and bias values at the edge
of fp32, on the HIP attention kernel.

* A key-padding plane ``(1, 1, 1, Tk)`` (bool, or a 0 / -inf bias) keeps the
  same keys for every query row: torch broadcasts it over ``Tq``.  The plane
  has one row, so it must not be read as a one-row triangle (``j <= i + off``
  for every row ``i``).  Weight-only and input masks, through the om
  executor and through the ``sdpa`` binding.
* ``torch.finfo(float32).min`` in an additive bias (the usual HF-style
  padding value): a row masked entirely that way is the mean of ``v`` in
  torch (every scaled score rounds to the same finite value); a row masked in
  part gives the masked keys weight 0.  The kernel adds the bias to the
  scaled score, as torch does.
* An ``sdpa`` call whose batch is beyond one attention launch's grid runs as
  several launches.
* The omd fold leaves out a leaf with no finite score by select, so NaN or
  inf in that leaf's ``l`` and numerators do not reach the output
  (``torch.where`` in ``_fused_omd_reduce``, om_fused.py:99-125).

References: float64 numpy over the same bf16-rounded inputs
(``oracle.om_elem`` / ``fused_om_levels``), gate 2e-2 (bf16, global relative
error), NaN positions exact; the fold test is exact up to fp32 rounding
(1e-6) against the same fold without the empty leaf.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import _lib as L
from catopt_amd import kernels as K
from catopt_amd.bindings import torch_fallback_count
from catopt_amd.evaluator import HipIRModule
from catopt_amd.executors import HipOMModule
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make
TOL_BF16 = 2e-2
F32_MIN = float(np.finfo(np.float32).min)


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _rand(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def _gate_nan(ref, out, tol):
    on = _np(out)
    assert on.shape == ref.shape, (on.shape, ref.shape)
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    rep = oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, on, 0), rtol=tol)
    assert rep["passed"], rep


def _softmax_ref(s, v):
    """``om_apply(om_elem(s, v))`` in float64 (NaN rows where a row has no
    finite score)."""
    m, l_, a = oracle.om_elem(s, v)
    return oracle.om_apply((m, l_, a))


def _bias_ir(B, H, T, d, m_term):
    q, k, v = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    S = mk("mul", mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1)), Const(d ** -0.5))
    inputs = [q, k, v] + ([m_term] if isinstance(m_term, Var) else [])
    return IR(mk("om_apply", mk("om_elem", mk("add", S, mk("attnbias", m_term)), v)), inputs)


def _padding(T, kept):
    keep = np.zeros((1, 1, 1, T), dtype=bool)
    keep[..., :kept] = True
    return keep


@pytest.mark.parametrize("kind", ["param_bool", "param_zero_neg_inf", "input_bool", "input_zero_neg_inf"])
def test_key_padding_plane_keeps_the_same_keys_for_every_row(sink, dev, kind):
    B, H, T, d = 2, 2, 192, 128
    keep = _padding(T, 70)
    val = torch.from_numpy(keep) if kind.endswith("bool") else \
        torch.from_numpy(np.where(keep, 0.0, -np.inf).astype(np.float32))
    shape = TensorType((1, 1, 1, T))
    if kind.startswith("param"):
        m_term, params, extra = Param("m", shape), {"m": val}, []
    else:
        m_term, params, extra = Var("m", shape), {}, [val.to(dev)]
    ir = _bias_ir(B, H, T, d, m_term)
    q, k, v = (_rand((B, H, T, d), s) for s in (1, 2, 3))
    ins = [q.to(dev), k.to(dev), v.to(dev), *extra]
    res = deliver(ir, params, sink, tuple(ins))
    mod = res.module
    assert isinstance(mod, HipOMModule)
    out = mod(*ins)
    assert mod.fallbacks == 0 and mod.kernel_leaves == 1
    s = d ** -0.5 * (_np(q) @ np.swapaxes(_np(k), -1, -2))
    s = np.where(np.broadcast_to(keep, s.shape), s, -np.inf)
    _gate_nan(_softmax_ref(s, _np(v)), out, TOL_BF16)


@pytest.mark.parametrize("where", ["om", "sdpa"])
def test_finfo_min_bias_rows(sink, dev, where):
    B, H, T, d = 1, 2, 160, 128
    rng = np.random.default_rng(5)
    bias = (rng.standard_normal((T, T)) * 0.5).astype(np.float32)
    bias[3, :] = F32_MIN                      # masked entirely: the mean of v in torch
    bias[40, rng.random(T) < 0.6] = F32_MIN   # masked in part: those keys weigh 0
    bias[41, 7:] = F32_MIN
    q, k, v = (_rand((B, H, T, d), s) for s in (11, 12, 13))
    bt = torch.from_numpy(bias)
    if where == "om":
        ir = _bias_ir(B, H, T, d, Param("m", TensorType((T, T))))
        res = deliver(ir, {"m": bt}, sink, (q.to(dev), k.to(dev), v.to(dev)))
        out = res.module(q.to(dev), k.to(dev), v.to(dev))
        assert res.module.fallbacks == 0 and res.module.kernel_leaves == 1
    else:
        qv, kv, vv, m = (Var(n, TensorType(t)) for n, t in
                         (("q", (B, H, T, d)), ("k", (B, H, T, d)), ("v", (B, H, T, d)), ("m", (T, T))))
        mod = HipIRModule(IR(mk("sdpa", qv, kv, vv, m), [qv, kv, vv, m]), {}, device=dev)
        n_hip, n_torch = L.call_count(), torch_fallback_count()
        out = mod(q.to(dev), k.to(dev), v.to(dev), bt.to(dev))
        assert L.call_count() > n_hip and torch_fallback_count() == n_torch
    s = d ** -0.5 * (_np(q) @ np.swapaxes(_np(k), -1, -2)) + bias.astype(np.float64)
    ref = _softmax_ref(s, _np(v))
    assert np.isfinite(ref).all()
    vmean = _np(v).mean(axis=-2)
    np.testing.assert_allclose(ref[..., 3, :], vmean, rtol=1e-9, atol=1e-12)  # torch's value
    on = _np(out)
    assert np.isfinite(on).all()
    rep = oracle.verify_equiv(ref, on, rtol=TOL_BF16)
    assert rep["passed"], rep
    np.testing.assert_allclose(on[..., 3, :], vmean, atol=2e-2)


def test_sdpa_key_padding_plane_broadcasts(dev):
    B, H, T, d = 2, 3, 128, 64
    keep = _padding(T, 50)
    qv, kv, vv = (Var(n, TensorType((B, H, T, d))) for n in "qkv")
    m = Var("m", TensorType((1, 1, 1, T)))
    mod = HipIRModule(IR(mk("sdpa", qv, kv, vv, m), [qv, kv, vv, m]), {}, device=dev)
    q, k, v = (_rand((B, H, T, d), s) for s in (21, 22, 23))
    n_hip, n_torch = L.call_count(), torch_fallback_count()
    out = mod(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(keep).to(dev))
    assert L.call_count() > n_hip and torch_fallback_count() == n_torch
    s = d ** -0.5 * (_np(q) @ np.swapaxes(_np(k), -1, -2))
    s = np.where(np.broadcast_to(keep, s.shape), s, -np.inf)
    _gate_nan(_softmax_ref(s, _np(v)), out, TOL_BF16)


@pytest.mark.parametrize("rank", [3, 4])
def test_sdpa_batch_beyond_one_launch(dev, rank):
    # a batch past one launch's grid runs as several launches of the kernel
    # (torch's own kernels on this stack reject a 4-D operand that large)
    N, T, d = K.ATTENTION_MAX_GRID_AXIS + 7, 4, 8
    shape = (N, T, d) if rank == 3 else (N, 1, T, d)
    qv, kv, vv = (Var(n, TensorType(shape)) for n in "qkv")
    mod = HipIRModule(IR(mk("sdpa", qv, kv, vv), [qv, kv, vv]), {}, device=dev)
    q, k, v = (_rand(shape, s) for s in (31, 32, 33))
    n_hip, n_torch = L.call_count(), torch_fallback_count()
    out = mod(q.to(dev), k.to(dev), v.to(dev))
    assert L.call_count() >= n_hip + 2 and torch_fallback_count() == n_torch
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    assert (out.float().cpu() - ref).abs().max().item() < 2e-2


def test_omd_fold_leaves_out_an_empty_leaf_by_select(dev):
    Lc, Tq, d = 5, 70, 48
    g = torch.Generator().manual_seed(3)
    m = torch.randn(Lc, Tq, 1, generator=g)
    lv = torch.rand(Lc, Tq, 1, generator=g) + 0.5
    num = torch.randn(Lc, Tq, 2 * d, generator=g)
    h = torch.randn(d, generator=g)
    base = K.omd_fold_apply(*(t.to(dev) for t in (m[:4], lv[:4], num[:4], h)))
    m[4] = float("-inf")               # leaf 4 has no finite score ...
    lv[4, ::2] = float("nan")          # ... and junk in its statistics
    lv[4, 1::2] = float("inf")
    num[4, :, ::3] = float("inf")
    num[4, :, 1::3] = float("nan")
    out = K.omd_fold_apply(*(t.to(dev) for t in (m, lv, num, h)))
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out, base, rtol=1e-6, atol=1e-6)
