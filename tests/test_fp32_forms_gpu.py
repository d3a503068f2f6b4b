"""fp32 delivered forms on the fp32 kernels, with no T×T score in HBM.

* Masked attention leaves with fp32 operands run the fp32 carrier kernel's
  mask modes (``catopt_hip_attn_carrier_f32_masked``): the causal ``cmask``
  and a weight-only lower triangle (causal mode; key blocks of a split score
  fold their offset into it), a weight-only bool keep-plane, a float bias
  plane (including ``-inf`` entries and ``finfo(float32).min`` rows) and an
  input-dependent mask.  Through the om executor every leaf is a kernel leaf
  (``kernel_leaves``, ``fallbacks == 0``, no torch op); through the streaming
  executor every block is.
* The carrier kernel itself: ``(m, l, a)`` per row against
  ``oracle.om_elem`` for ragged ``Tq`` / ``Tk``, head dims 16..128 and value
  widths up to 256, causal offsets that mask whole key tiles (or every key),
  and the empty carrier ``(-inf, 0, 0)`` on rows with no kept key.
* Retention with fp32 operands runs the fp32 retention kernel: the K-way
  delivered form through the decayed executor (C = 64 and 128, ``d`` = 128
  and 64, ``fallbacks == 0``) and the kernel directly on a ragged ``T`` with
  ``dk != dv``.

* fp16 operands run the same fp32 kernels widened on the device, the output
  rounded to fp16: a masked om leaf, a streaming fold and the K-way
  retention form, with no fallback.

References: float64 numpy over the same fp32 (or fp16-rounded) inputs
(``oracle.om_elem`` / ``om_apply`` / ``fused_om_levels``,
``oracle.retention_quadratic`` / ``retention_kway``).  Gates: 1e-5 for fp32,
2e-3 for fp16 (its output rounding is 2^-11), global relative error (the
verify metric), NaN positions exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import forms
from catopt_amd import kernels as K
from catopt_amd.executors import HipOMModule, HipStreamingOMModule, to_streaming_om_module
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make
TOL = 1e-5
TOL_F16 = 2e-3
NEG_INF = Const(float("-inf"))
F32_MIN = float(np.finfo(np.float32).min)


@pytest.fixture(scope="module")
def sink():
    return HipSink()


def _np(t):
    return t.detach().cpu().double().numpy()


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g) * scale


def _gate_nan(ref, out, tol=TOL):
    on = _np(out) if isinstance(out, torch.Tensor) else out
    assert on.shape == ref.shape, (on.shape, ref.shape)
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    rep = oracle.verify_equiv(np.where(fin, ref, 0), np.where(fin, on, 0), rtol=tol)
    assert rep["passed"], rep


def _softmax_ref(s, v):
    return oracle.om_apply(oracle.om_elem(s, v))


def _qkt(q, k):
    return mk("matmul", q, mk("transpose", k, dim0=-2, dim1=-1))


# ------------------------------------------------------------- om executor


def _masked_ir(B, H, Tq, Tk, d, kind):
    """``om_apply(om_elem(<masked scale·q kᵀ>, v))`` with the mask spelled
    as ``kind``; returns the IR and the mask term's variable (if any)."""
    q = Var("q", TensorType((B, H, Tq, d)))
    k, v = (Var(n, TensorType((B, H, Tk, d))) for n in "kv")
    S = mk("mul", _qkt(q, k), Const(d ** -0.5))
    extra = []
    if kind == "cmask":
        s = mk("masked_fill", S, mk("cmask", S), NEG_INF)
    elif kind in ("tri_param", "bool_param"):
        s = mk("masked_fill", S, mk("logical_not", Param("m", TensorType((Tq, Tk)))), NEG_INF)
    elif kind == "bias_param":
        s = mk("add", S, mk("attnbias", Param("m", TensorType((Tq, Tk)))))
    elif kind == "input_bool":
        m = Var("m", TensorType((1, 1, Tq, Tk)))
        s = mk("masked_fill", S, mk("logical_not", m), NEG_INF)
        extra = [m]
    else:
        raise ValueError(kind)
    return IR(mk("om_apply", mk("om_elem", s, v)), [q, k, v, *extra])


def _plane(kind, Tq, Tk, rng):
    if kind in ("cmask", "tri_param"):
        return oracle.cmask_keep(Tq, Tk)
    if kind in ("bool_param", "input_bool"):
        keep = rng.random((Tq, Tk)) < 0.6
        keep[5, :] = False            # a row with no key: NaN, as dense softmax
        return keep
    bias = (rng.standard_normal((Tq, Tk)) * 0.5).astype(np.float32)
    bias[rng.random((Tq, Tk)) < 0.2] = -np.inf
    bias[3, :] = F32_MIN              # every key at -FLT_MAX: finite scores, the mean of v
    bias[7, :] = -np.inf              # no key: NaN
    return bias


@pytest.mark.parametrize("kind", ["cmask", "tri_param", "bool_param", "bias_param", "input_bool"])
def test_f32_masked_leaf_on_the_carrier_kernel(sink, dev, kind):
    B, H, Tq, Tk, d = 2, 3, 150, 200, 64
    rng = np.random.default_rng(len(kind))
    ir = _masked_ir(B, H, Tq, Tk, d, kind)
    plane = _plane(kind, Tq, Tk, rng)
    params = {}
    q, k, v = _rand((B, H, Tq, d), 1), _rand((B, H, Tk, d), 2), _rand((B, H, Tk, d), 3)
    ins = [q.to(dev), k.to(dev), v.to(dev)]
    if kind == "input_bool":
        ins.append(torch.from_numpy(plane).reshape(1, 1, Tq, Tk).to(dev))
    elif kind != "cmask":
        params["m"] = torch.from_numpy(plane)
    res = deliver(ir, params, sink, tuple(ins))
    mod = res.module
    assert isinstance(mod, HipOMModule) and res.stats["executor"] == "om_batched"
    out = mod(*ins)
    assert mod.fallbacks == 0 and mod.kernel_leaves == 1
    assert res.stats["hip_kernel"] and res.stats["torch_fallback_ops"] == 0
    s = d ** -0.5 * (_np(q) @ np.swapaxes(_np(k), -1, -2))
    if kind == "bias_param":
        s = s + plane.astype(np.float64)
    else:
        s = np.where(plane, s, -np.inf)
    ref = _softmax_ref(s, _np(v))
    if kind == "bias_param":
        np.testing.assert_allclose(ref[..., 3, :], _np(v).mean(axis=-2), rtol=1e-9, atol=1e-12)
    _gate_nan(ref, out)


def _split_causal_ir(B, H, Tq, cuts, d):
    q = Var("q", TensorType((B, H, Tq, d)))
    ks = [Var(f"k{i}", TensorType((B, H, c, d))) for i, c in enumerate(cuts)]
    vs = [Var(f"v{i}", TensorType((B, H, c, d))) for i, c in enumerate(cuts)]
    S = mk("concat", *[_qkt(q, k) for k in ks], dim=-1)
    M = mk("cmask", S)
    leaves = []
    for i in range(len(cuts)):
        s_i = mk("masked_fill", mk("split", S, sizes=tuple(cuts), dim=-1, index=i),
                 mk("split", M, sizes=tuple(cuts), dim=-1, index=i), NEG_INF)
        leaves.append(mk("om_elem", s_i, mk("split", mk("concat", *vs, dim=-2), sizes=tuple(cuts), dim=-2,
                                            index=i)))
    t = leaves[0]
    for lf in leaves[1:]:
        t = mk("om_compose", t, lf)
    return IR(mk("om_apply", t), [q, *ks, *vs])


def _split_inputs(B, H, Tq, cuts, d, dev):
    q = _rand((B, H, Tq, d), 4, 0.5)
    ks = [_rand((B, H, c, d), 10 + i, 0.5) for i, c in enumerate(cuts)]
    vs = [_rand((B, H, c, d), 20 + i) for i, c in enumerate(cuts)]
    s = _np(q) @ np.swapaxes(np.concatenate([_np(x) for x in ks], -2), -1, -2)
    s = np.where(oracle.cmask_keep(Tq, sum(cuts)), s, -np.inf)
    ref = _softmax_ref(s, np.concatenate([_np(x) for x in vs], -2))
    return [t.to(dev) for t in (q, *ks, *vs)], ref


def test_f32_split_causal_key_blocks_fold_their_offsets(sink, dev):
    # the second block's causal bound is shifted by the first block's width;
    # rows before it keep no key of that block (empty carriers in the fold)
    B, H, Tq, cuts, d = 1, 4, 160, (96, 64), 128
    ir = _split_causal_ir(B, H, Tq, cuts, d)
    ins, ref = _split_inputs(B, H, Tq, cuts, d, dev)
    res = deliver(ir, {}, sink, tuple(ins))
    mod = res.module
    assert isinstance(mod, HipOMModule)
    out = mod(*ins)
    assert mod.fallbacks == 0 and mod.kernel_leaves == 2
    _gate_nan(ref, out)


def test_f32_streaming_masked_blocks_fold_on_the_kernel(dev):
    B, H, Tq, cuts, d = 2, 2, 128, (64, 64, 32), 48
    mod = to_streaming_om_module(_split_causal_ir(B, H, Tq, cuts, d))
    assert isinstance(mod, HipStreamingOMModule) and mod.n_blocks == len(cuts)
    ins, ref = _split_inputs(B, H, Tq, cuts, d, dev)
    out = mod(*ins)
    assert mod.kernel_leaves == len(cuts)
    _gate_nan(ref, out)


# ------------------------------------------------------- the carrier kernel


def _carrier_ref(s, v):
    """om_elem in float64 with the kernel's empty carrier on rows with no
    finite score."""
    m, lv, a = oracle.om_elem(s, v)
    empty = ~np.isfinite(m)
    return m, np.where(empty, 0.0, lv), np.where(empty, 0.0, a), empty


def _check_carrier(got, s, v):
    m, lv, a = (_np(t) for t in got)
    rm, rl, ra, empty = _carrier_ref(s, v)
    assert np.array_equal(np.isneginf(m), empty) and not np.isnan(m).any()
    assert (lv[empty] == 0).all() and (np.broadcast_to(empty, a.shape) <= (a == 0)).all()
    fin = ~empty
    np.testing.assert_allclose(m[fin], rm[fin], rtol=1e-6, atol=1e-6)
    assert oracle.verify_equiv(rl, lv, rtol=TOL)["passed"]
    assert oracle.verify_equiv(ra, a, rtol=TOL)["passed"]


@pytest.mark.parametrize("dk,dv,Tq,Tk", [(16, 8, 40, 70), (48, 96, 130, 33), (128, 256, 257, 300)])
@pytest.mark.parametrize("off", [0, -45, 37])
def test_f32_carrier_causal_offsets(dev, dk, dv, Tq, Tk, off):
    q, k, v = _rand((3, Tq, dk), 5, 0.4), _rand((3, Tk, dk), 6, 0.4), _rand((3, Tk, dv), 7)
    sc = dk ** -0.5
    got = K.attn_carrier_f32(q.to(dev), k.to(dev), v.to(dev), sc, causal=True, causal_off=off)
    s = sc * (_np(q) @ np.swapaxes(_np(k), -1, -2))
    s = np.where(oracle.cmask_keep(Tq, Tk, -off), s, -np.inf)
    _check_carrier(got, s, _np(v))


def test_f32_carrier_causal_offset_that_masks_every_key(dev):
    Tq, Tk, d = 64, 96, 32
    q, k, v = _rand((2, Tq, d), 8), _rand((2, Tk, d), 9), _rand((2, Tk, d), 10)
    m, lv, a = K.attn_carrier_f32(q.to(dev), k.to(dev), v.to(dev), 1.0, causal=True, causal_off=-Tq)
    assert torch.isneginf(m).all() and (lv == 0).all() and (a == 0).all()


@pytest.mark.parametrize("mode", ["mask", "bias"])
def test_f32_carrier_planes_shared_over_the_batch(dev, mode):
    Tq, Tk, dk, dv = 97, 150, 64, 80
    rng = np.random.default_rng(11)
    q, k, v = _rand((4, Tq, dk), 12, 0.3), _rand((4, Tk, dk), 13, 0.3), _rand((4, Tk, dv), 14)
    s = _np(q) @ np.swapaxes(_np(k), -1, -2)
    if mode == "mask":
        keep = rng.random((Tq, Tk)) < 0.3
        keep[0, :] = False
        got = K.attn_carrier_f32(q.to(dev), k.to(dev), v.to(dev), 1.0, mask=torch.from_numpy(keep).to(dev))
        s = np.where(keep, s, -np.inf)
    else:
        bias = (rng.standard_normal((Tq, Tk)) * 2).astype(np.float32)
        bias[rng.random((Tq, Tk)) < 0.3] = -np.inf
        bias[2, :] = -np.inf
        bias[4, :] = F32_MIN
        got = K.attn_carrier_f32(q.to(dev), k.to(dev), v.to(dev), 1.0, bias=torch.from_numpy(bias).to(dev))
        s = s + bias.astype(np.float64)
    _check_carrier(got, s, _np(v))


# ---------------------------------------------------------------- retention


def _gammas(H):
    return torch.tensor([1 - 2.0 ** (-5 - h / 2) for h in range(H)], dtype=torch.float32)


@pytest.mark.parametrize("C,d", [(64, 128), (128, 128), (64, 64)])
def test_f32_retention_kway_executor(sink, dev, C, d):
    B, H, T = 2, 3, 512
    ir, _ = forms.retention_kway_form(B, H, T, d, C, scale=0.5)
    gam = _gammas(H)
    q, k, v = (_rand((B, H, T, d), 60 + i, 1 / math.sqrt(d)) for i in range(3))
    ins = tuple(t.to(dev) for t in (q, k, v))
    res = deliver(ir, {"gamma": gam}, sink, ins)
    assert res.stats["executor"] == "om_decayed_chunked" and res.stats["hip_kernel"]
    out = res.module(*ins)
    assert res.module.fallbacks == 0 and out.dtype == torch.float32
    g = gam.double().numpy()
    rep = oracle.verify_equiv(oracle.retention_quadratic(_np(q), _np(k), _np(v), g, 0.5), _np(out), rtol=TOL)
    assert rep["passed"], rep
    rep = oracle.verify_equiv(oracle.retention_kway(_np(q), _np(k), _np(v), g, T // C, 0.5), _np(out), rtol=TOL)
    assert rep["passed"], rep


@pytest.mark.parametrize("T,dk,dv", [(200, 40, 24), (64, 128, 128), (1000, 20, 20), (37, 8, 100)])
def test_f32_retention_kernel_ragged_steps_and_widths(dev, T, dk, dv):
    B, H = 1, 2
    gam = torch.tensor([0.9, 0.995], dtype=torch.float32)
    q, k = _rand((B, H, T, dk), 70, dk ** -0.5), _rand((B, H, T, dk), 71, dk ** -0.5)
    v = _rand((B, H, T, dv), 72)
    out = K.retention(q.to(dev), k.to(dev), v.to(dev), gam.to(dev), 0.75)
    assert out.shape == (B, H, T, dv) and out.dtype == torch.float32
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.double().numpy(), 0.75)
    rep = oracle.verify_equiv(ref, _np(out), rtol=TOL)
    assert rep["passed"], rep


# --------------------------------------------------------------------- fp16


@pytest.mark.parametrize("kind", ["cmask", "bias_param"])
def test_f16_masked_leaf_runs_the_fp32_kernel(sink, dev, kind):
    B, H, Tq, Tk, d = 1, 2, 130, 170, 64
    rng = np.random.default_rng(40 + len(kind))
    ir = _masked_ir(B, H, Tq, Tk, d, kind)
    plane = _plane(kind, Tq, Tk, rng)
    params = {} if kind == "cmask" else {"m": torch.from_numpy(plane)}
    q, k, v = (t.half() for t in (_rand((B, H, Tq, d), 41), _rand((B, H, Tk, d), 42), _rand((B, H, Tk, d), 43)))
    ins = [q.to(dev), k.to(dev), v.to(dev)]
    res = deliver(ir, params, sink, tuple(ins))
    mod = res.module
    out = mod(*ins)
    assert isinstance(mod, HipOMModule) and mod.fallbacks == 0 and mod.kernel_leaves == 1
    assert out.dtype == torch.float16
    s = d ** -0.5 * (_np(q) @ np.swapaxes(_np(k), -1, -2))
    s = s + plane.astype(np.float64) if kind == "bias_param" else np.where(plane, s, -np.inf)
    _gate_nan(_softmax_ref(s, _np(v)), out, TOL_F16)


def test_f16_streaming_blocks_fold_on_the_kernel(dev):
    B, H, Tq, cuts, d = 1, 2, 96, (64, 32), 32
    mod = to_streaming_om_module(_split_causal_ir(B, H, Tq, cuts, d))
    ins, ref = _split_inputs(B, H, Tq, cuts, d, dev)
    ins = [t.half() for t in ins]
    # the reference over the fp16-rounded inputs
    q, ks, vs = ins[0], ins[1:1 + len(cuts)], ins[1 + len(cuts):]
    s = _np(q) @ np.swapaxes(np.concatenate([_np(x) for x in ks], -2), -1, -2)
    s = np.where(oracle.cmask_keep(Tq, sum(cuts)), s, -np.inf)
    ref = _softmax_ref(s, np.concatenate([_np(x) for x in vs], -2))
    out = mod(*ins)
    assert mod.kernel_leaves == len(cuts) and out.dtype == torch.float16
    _gate_nan(ref, out, TOL_F16)


def test_f16_retention_kway_executor(sink, dev):
    B, H, T, d, C = 1, 2, 256, 64, 64
    ir, _ = forms.retention_kway_form(B, H, T, d, C, scale=0.5)
    gam = _gammas(H)
    q, k, v = (_rand((B, H, T, d), 80 + i, 1 / math.sqrt(d)).half() for i in range(3))
    ins = tuple(t.to(dev) for t in (q, k, v))
    res = deliver(ir, {"gamma": gam}, sink, ins)
    out = res.module(*ins)
    assert res.module.fallbacks == 0 and out.dtype == torch.float16
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.double().numpy(), 0.5)
    rep = oracle.verify_equiv(ref, _np(out), rtol=TOL_F16)
    assert rep["passed"], rep
