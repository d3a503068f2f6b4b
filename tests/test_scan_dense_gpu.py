"""Dense affine scans on the GPU (``catopt_hip_aff_scan`` and ``HipScanModule``).

The counterpart of the reference's ``tests/test_scan_batched.py``: the
``apply(<aff_compose tree>, h)`` term of ``LinearRecurrence`` equals the
sequential fold ``h_t = A h_{t-1} + x_t`` (T = 16, 32; d = 16), the batched
executor agrees with the serial lowering, hipGraph replays pick up new
inputs, and terms outside the kernels' envelope run the generic module.
Beyond those: batched column states (shared, per-slot and time-varying maps,
k > 1 columns), ragged d (tiles padded with zeros), both schedules
(streaming and chunk-parallel) and long sequences.  References: the numpy
oracle's serial recurrence in float64 (pinned by closed forms in
test_oracle.py).  Gates: fp32 ≤ 1e-5, bf16 ≤ 2e-2 (verify metric).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import _lib as L
from catopt_amd import forms
from catopt_amd import kernels as K
from catopt_amd.executors import HipScanModule, prefix_chunk_table
from catopt_amd.runner import HipGraphRunner
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _gate(ref, out, tol):
    rep = oracle.verify_equiv(ref, _np(out), rtol=tol)
    assert rep["passed"], rep
    return rep


def _maps(rng, shape, d):
    """Contractive maps (spectral radius about 0.9): long scans stay bounded."""
    return (rng.standard_normal((*shape, d, d)) * (0.9 / np.sqrt(d))).astype(np.float32)


@pytest.fixture(scope="module")
def sink():
    return HipSink()


# ------------------------------------------------------------------ kernel


@pytest.mark.parametrize("d", [16, 5, 33, 64])
@pytest.mark.parametrize("schedule", [L.SCAN_STREAM, L.SCAN_CHUNKED])
def test_kernel_lti_vector(dev, d, schedule):
    T = 300
    rng = np.random.default_rng(d)
    A = _maps(rng, (), d)
    b = rng.standard_normal((T, d)).astype(np.float32)
    h0 = rng.standard_normal((d, 1)).astype(np.float32)
    ref = oracle.serial_aff_scan(A.astype(np.float64), b.astype(np.float64), h0.astype(np.float64))
    At = torch.from_numpy(A).to(dev).reshape(1, 1, d, d)
    bt = torch.from_numpy(b).to(dev).reshape(T, 1, d)
    ht = torch.from_numpy(h0).to(dev).reshape(1, d, 1)
    states, hf = K.aff_scan(At, bt, ht, prefix_chunk_table(T), schedule=schedule)
    _gate(ref, states.reshape(T, d, 1), TOL_F32)
    _gate(ref[-1], hf.reshape(d, 1), TOL_F32)


@pytest.mark.parametrize("kind", ["shared_tv", "per_slot_tv", "per_slot_lti", "shared_b"])
@pytest.mark.parametrize("d,k", [(16, 1), (24, 3), (64, 1), (48, 17)])
@pytest.mark.parametrize("schedule", [L.SCAN_STREAM, L.SCAN_CHUNKED])
def test_kernel_batched_columns(dev, kind, d, k, schedule):
    T, P = 70, 37
    rng = np.random.default_rng(7 * d + k)
    if kind == "shared_tv":
        A = _maps(rng, (T, 1), d)
    elif kind == "per_slot_lti":
        A = _maps(rng, (1, P), d)
    else:
        A = _maps(rng, (T, P), d)
    b = rng.standard_normal((T, 1 if kind == "shared_b" else P, d)).astype(np.float32)
    h0 = rng.standard_normal((P, d, k)).astype(np.float32)
    Ao = np.broadcast_to(A, (T, P, d, d))
    ref = oracle.serial_aff_scan(Ao.astype(np.float64), np.broadcast_to(b, (T, P, d)).astype(np.float64),
                                 h0.astype(np.float64))
    f = lambda z: torch.from_numpy(np.ascontiguousarray(z)).to(dev)  # noqa: E731
    states, hf = K.aff_scan(f(A), f(b), f(h0), [0, 9, 10, 40, T], schedule=schedule)
    _gate(ref, states, TOL_F32)
    _gate(ref[-1], hf, TOL_F32)
    _, hf2 = K.aff_scan(f(A), f(b), f(h0), [0, 9, 10, 40, T], schedule=schedule, states=False)
    assert torch.equal(hf, hf2)


def test_kernel_long_sequence_auto_schedule(dev):
    """T = 6000, one column: AUTO picks the chunk-parallel schedule; it agrees
    with streaming and with the float64 recurrence."""
    T, d = 6000, 16
    rng = np.random.default_rng(3)
    A = _maps(rng, (T, 1), d)
    b = rng.standard_normal((T, 1, d)).astype(np.float32)
    h0 = rng.standard_normal((1, d, 1)).astype(np.float32)
    f = lambda z: torch.from_numpy(z).to(dev)  # noqa: E731
    table = prefix_chunk_table(T)
    s_auto, h_auto = K.aff_scan(f(A), f(b), f(h0), table)
    s_str, h_str = K.aff_scan(f(A), f(b), f(h0), table, schedule=L.SCAN_STREAM)
    ref = oracle.serial_aff_scan(A[:, 0].astype(np.float64), b[:, 0].astype(np.float64),
                                 h0[0].astype(np.float64))
    _gate(ref, s_auto[:, 0], TOL_F32)
    _gate(ref, s_str[:, 0], TOL_F32)
    _gate(ref[-1], h_auto[0], TOL_F32)
    # zero steps: the state passes through
    _, h_empty = K.aff_scan(f(A[:1]), f(b[:0]), f(h0), [0, 0], schedule=L.SCAN_STREAM)
    assert torch.equal(h_empty, f(h0))


# ---------------------------------------------------------------- executor


@pytest.mark.parametrize("steps", [16, 32])
def test_linear_recurrence_matches_sequential(sink, dev, steps):
    """test_batched_scan_matches_sequential (fp32, d = 16) through the sink."""
    d = 16
    torch.manual_seed(0)
    A = torch.randn(d, d) * 0.1
    h0 = torch.randn(d)
    x = torch.randn(steps, d)
    ir, _ = forms.linear_recurrence_form(steps, d)
    res = deliver(ir, {"p_a": A.to(dev), "p_h0": h0.to(dev)}, sink, (x.to(dev),))
    assert res.stats["executor"] == "scan" and res.stats["hip_kernel"]
    mod = res.module
    assert mod.is_batched and mod.n_levels <= int(np.ceil(np.log2(steps))) + 1
    out = mod(x.to(dev))
    assert mod.fallbacks == 0
    h = h0.double()
    for t in range(steps):  # the model's own loop (models/__init__.py:593-598)
        h = A.double() @ h + x[t].double()
    assert (out.double().cpu() - h).abs().max().item() < 1e-5
    # and the executor agrees with the serial lowering of the same term
    serial = sink.lower(ir, {"p_a": A.to(dev), "p_h0": h0.to(dev)})(x.to(dev))
    assert (out - serial).abs().max().item() < 1e-5


def test_batched_columns_through_the_sink_with_graph_replay(sink, dev):
    T, d, B, k = 48, 32, 6, 3
    rng = np.random.default_rng(11)
    ir, _ = forms.dense_scan_form(T, d, (B,), k, time_varying=True, per_slot=True)
    A = _maps(rng, (T, B), d)
    b = rng.standard_normal((T, B, d, 1)).astype(np.float32)
    h = rng.standard_normal((B, d, k)).astype(np.float32)
    ins = tuple(torch.from_numpy(z).to(dev) for z in (A, b, h))
    res = deliver(ir, {}, sink, ins, runner=HipGraphRunner())
    assert res.stats["executor"] == "scan" and res.stats["hip_kernel"]
    assert res.module.is_graph_captured
    out = res.module(*ins).clone()
    assert res.module.fallbacks == 0 and out.shape == (B, d, k)
    ref = oracle.serial_aff_scan(A.astype(np.float64), b[..., 0].astype(np.float64), h.astype(np.float64))
    _gate(ref[-1], out, TOL_F32)
    A2 = _maps(rng, (T, B), d)
    out2 = res.module(torch.from_numpy(A2).to(dev), ins[1], ins[2]).clone()
    ref2 = oracle.serial_aff_scan(A2.astype(np.float64), b[..., 0].astype(np.float64), h.astype(np.float64))
    _gate(ref2[-1], out2, TOL_F32)


@pytest.mark.parametrize("shared", [False, True])
def test_shared_map_broadcast_over_batched_states(dev, shared):
    """A shared (d, d) map rides along batched (B, d, 1) offsets and (B, d, k)
    states: one MFMA product over all B·k columns per step."""
    T, d, B, k = 40, 16, 50, 2
    rng = np.random.default_rng(5)
    ir, _ = forms.dense_scan_form(T, d, (B,), k, time_varying=not shared)
    A = _maps(rng, () if shared else (T,), d)
    b = rng.standard_normal((T, B, d, 1)).astype(np.float32)
    h = rng.standard_normal((B, d, k)).astype(np.float32)
    mod = HipScanModule(ir, {})
    out = mod(*(torch.from_numpy(z).to(dev) for z in (A, b, h)))
    assert mod.fallbacks == 0
    Ab = np.broadcast_to(A, (T, B, d, d)) if shared else np.broadcast_to(A[:, None], (T, B, d, d))
    ref = oracle.serial_aff_scan(Ab.astype(np.float64), b[..., 0].astype(np.float64), h.astype(np.float64))
    _gate(ref[-1], out, TOL_F32)


@pytest.mark.parametrize("dim", [0, 1])
def test_prefix_form_every_state(dev, dim):
    T, d = 200, 24
    rng = np.random.default_rng(9)
    ir, _ = forms.dense_scan_prefix_form(T, d, dim=dim)
    A = _maps(rng, (T,), d)
    b = rng.standard_normal((T, d)).astype(np.float32)
    h = rng.standard_normal(d).astype(np.float32)
    mod = HipScanModule(ir, {})
    assert mod._plan["mode"] == "prefix"
    out = mod(*(torch.from_numpy(z).to(dev) for z in (A, b, h)))
    assert mod.fallbacks == 0
    ref = oracle.serial_aff_scan(A.astype(np.float64), b.astype(np.float64), h[:, None].astype(np.float64))[..., 0]
    _gate(np.moveaxis(ref, 0, dim), out, TOL_F32)


def test_bf16_operands(dev):
    T, d, B = 64, 32, 8
    rng = np.random.default_rng(13)
    ir, _ = forms.dense_scan_form(T, d, (B,), 1, time_varying=True)
    A = torch.from_numpy(_maps(rng, (T,), d)).bfloat16()
    b = torch.from_numpy(rng.standard_normal((T, B, d, 1)).astype(np.float32)).bfloat16()
    h = torch.from_numpy(rng.standard_normal((B, d, 1)).astype(np.float32)).bfloat16()
    mod = HipScanModule(ir, {})
    out = mod(A.to(dev), b.to(dev), h.to(dev))
    assert mod.fallbacks == 0 and out.dtype == torch.bfloat16
    Ab = np.broadcast_to(_np(A)[:, None], (T, B, d, d))
    ref = oracle.serial_aff_scan(Ab, _np(b)[..., 0], _np(h))
    _gate(ref[-1], out, TOL_BF16)


def test_outside_the_envelope_runs_the_generic_module(dev):
    """fp64 operands and d > 64 run the embedded generic module (counted)."""
    T = 12
    for d, dtype in ((16, torch.float64), (80, torch.float32)):
        ir, _ = forms.linear_recurrence_form(T, d)
        A = torch.randn(d, d, dtype=dtype) * (0.5 / d ** 0.5)
        h0 = torch.randn(d, dtype=dtype)
        mod = HipScanModule(ir, {"p_a": A.to(dev), "p_h0": h0.to(dev)})
        x = torch.randn(T, d, dtype=dtype)
        out = mod(x.to(dev))
        assert mod.fallbacks == 1
        ref = oracle.serial_aff_scan(_np(A), _np(x), _np(h0)[:, None])[-1, :, 0]
        _gate(ref, out, 1e-5)
