"""Deferred-affine attention (omd) on the GPU (``HipOmdModule``).

The counterpart of the reference's ``tests/test_omd_lower.py`` /
``test_omd_lower_edges.py``: ``omd_apply(<omd_compose tree>, h)`` over key
blocks whose coefficients are stacked projections of one scan's prefix maps
equals softmax attention over that scan's states (diagonal and dense
carriers); a fully masked row of one block contributes nothing; packaged
``omd`` leaves fold in; hipGraph replays follow new inputs; fp64 runs the
generic module.  References: the float64 serial recurrence of the numpy
oracle (pinned by closed forms) under a dense softmax computed here — a
different formulation from the carrier algebra the executor uses.  Gates:
fp32 ≤ 1e-5, bf16 ≤ 2e-2 (verify metric).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import forms
from catopt_amd.executors import HipOmdModule
from catopt_amd.ir import IR, Const, Op, TensorType, Var
from catopt_amd.runner import HipGraphRunner
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu
mk = Op.make
TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def _np(t):
    return t.detach().float().cpu().double().numpy()


def _gate(ref, out, tol):
    rep = oracle.verify_equiv(ref, _np(out), rtol=tol)
    assert rep["passed"], rep
    return rep


def _softmax_rows(sc):
    w = np.exp(sc - sc.max(-1, keepdims=True))
    return w / w.sum(-1, keepdims=True)


def _inputs(T, d, Tq, dk, dense, seed, dtype=torch.float32):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((Tq, dk)) * 0.5
    k = rng.standard_normal((T, dk)) * 0.5
    a = (rng.standard_normal((T, d, d)) * (0.9 / np.sqrt(d))) if dense else rng.uniform(0.6, 1.0, (T, d))
    x = rng.standard_normal((T, d))
    h = rng.standard_normal(d)
    return [torch.from_numpy(z.astype(np.float32)).to(dtype) for z in (q, k, a, x, h)]


def _reference(q, k, a, x, h, dense):
    qn, kn, an, xn, hn = (_np(t) for t in (q, k, a, x, h))
    if dense:
        states = oracle.serial_aff_scan(an, xn, hn[:, None])[..., 0]
    else:
        states = oracle.serial_affd_scan(an, xn, hn)
    return _softmax_rows(qn @ kn.T) @ states


@pytest.fixture(scope="module")
def sink():
    return HipSink()


@pytest.mark.parametrize("dense", [False, True])
def test_omd_attention_over_scan_states(sink, dev, dense):
    T, d, Tq, nb, dk = (128, 16, 48, 4, 16) if dense else (512, 32, 64, 8, 16)
    ir, _ = forms.omd_scan_attention_form(T, d, Tq, nb, dk, dense=dense)
    ins = _inputs(T, d, Tq, dk, dense, 1)
    res = deliver(ir, {}, sink, tuple(t.to(dev) for t in ins))
    assert res.stats["executor"] == "omd_batched" and res.stats["hip_kernel"]
    mod = res.module
    assert mod.map_mode == "chain"
    out = mod(*(t.to(dev) for t in ins))
    assert mod.fallbacks == 0 and out.shape == (Tq, d) and out.dtype == torch.float32
    _gate(_reference(*ins, dense), out, TOL_F32)


def test_omd_bf16_operands(dev):
    T, d, Tq, nb, dk = 256, 32, 32, 4, 16
    ir, _ = forms.omd_scan_attention_form(T, d, Tq, nb, dk)
    ins = _inputs(T, d, Tq, dk, False, 2, torch.bfloat16)
    mod = HipOmdModule(ir, {})
    out = mod(*(t.to(dev) for t in ins))
    assert mod.fallbacks == 0 and out.dtype == torch.bfloat16
    _gate(_reference(*ins, False), out, TOL_BF16)


def test_omd_masked_block_rows_and_packaged_leaf(dev):
    """Block 0 hides every key from query row 1 (a -inf row: that block's
    carrier row is the empty one), and a packaged omd(m, l, fa, fb) leaf
    built from the oracle folds in with the kernel-made ones."""
    T, d, Tq, dk = 64, 8, 6, 8
    C = T // 2
    ins = _inputs(T, d, Tq, dk, False, 3)
    q_, k_, a_, x_, h_ = (Var(n, TensorType(tuple(t.shape))) for n, t in zip("qkaxh", ins))
    mask = Var("mask", TensorType((Tq, C)))
    fs = []
    for j in range(T):
        lf = mk("aff_diag", mk("select", a_, dim=0, index=j), mk("select", x_, dim=0, index=j))
        fs.append(lf if j == 0 else mk("affd_compose", lf, fs[-1]))

    def stacks(lo, hi):
        return (mk("stack", *[mk("affd_a", f) for f in fs[lo:hi]], dim=0),
                mk("stack", *[mk("affd_b", f) for f in fs[lo:hi]], dim=0))

    s0 = mk("masked_fill", mk("matmul", q_, mk("transpose", mk("chunk", k_, chunks=2, dim=0, index=0), dim0=0, dim1=1)),
            mask, Const(float("-inf")))
    e0 = mk("omd_elem", s0, *stacks(0, C))
    pm, pl, pa, pb = (Var(n, TensorType(sh)) for n, sh in
                      (("pm", (Tq, 1)), ("pl", (Tq, 1)), ("pa", (Tq, d)), ("pb", (Tq, d))))
    root = mk("omd_apply", mk("omd_compose", e0, mk("omd", pm, pl, pa, pb)), h_)
    mod = HipOmdModule(IR(root, [q_, k_, a_, x_, h_, mask, pm, pl, pa, pb]), {})
    assert mod.is_batched and mod.map_mode == "chain"
    mk_np = np.zeros((Tq, C), dtype=bool)
    mk_np[1] = True
    mk_np[3, ::2] = True
    # the second key block as a packaged carrier, from the oracle on the true prefix maps
    qn, kn, an, xn = (_np(t) for t in ins[:4])
    Pa, Pb = np.cumprod(an, axis=0), oracle.serial_affd_scan(an, xn, np.zeros(d))
    s1 = qn @ kn[C:].T
    pkg = oracle.omd_elem(s1, Pa[C:], Pb[C:])
    dev_ins = [t.to(dev) for t in ins] + [torch.from_numpy(mk_np).to(dev)] + \
        [torch.from_numpy(np.asarray(z, dtype=np.float32)).to(dev) for z in pkg]
    out = mod(*dev_ins)
    assert mod.fallbacks == 0
    states = oracle.serial_affd_scan(an, xn, _np(ins[4]))
    sc = qn @ kn.T
    sc[:, :C][mk_np] = -np.inf
    _gate(_softmax_rows(sc) @ states, out, TOL_F32)


def test_omd_graph_replay_and_fp64_fallback(sink, dev):
    T, d, Tq, nb, dk = 128, 16, 16, 4, 8
    ir, _ = forms.omd_scan_attention_form(T, d, Tq, nb, dk)
    ins = [t.to(dev) for t in _inputs(T, d, Tq, dk, False, 4)]
    res = deliver(ir, {}, sink, tuple(ins), runner=HipGraphRunner())
    assert res.module.is_graph_captured
    out = res.module(*ins).clone()
    _gate(_reference(*ins, False), out, TOL_F32)
    ins2 = [t.to(dev) for t in _inputs(T, d, Tq, dk, False, 5)]
    out2 = res.module(*ins2).clone()
    _gate(_reference(*ins2, False), out2, TOL_F32)
    mod = HipOmdModule(ir, {})
    out64 = mod(*(t.double() for t in ins))
    assert mod.fallbacks == 1 and out64.dtype == torch.float64
    rep = oracle.verify_equiv(_reference(*ins, False), out64.cpu().numpy(), rtol=1e-10)
    assert rep["passed"], rep


@pytest.mark.parametrize("dk,dv,Tq,Tk", [(64, 128, 300, 256), (5, 33, 17, 45), (128, 256, 130, 97),
                                         (16, 1, 64, 32), (32, 64, 1, 1)])
def test_attn_carrier_f32_matches_om_elem(dev, dk, dv, Tq, Tk):
    """The fused carrier kernel against the oracle's om_elem on the same
    fp32 scores: ragged query / key counts, widths that pad the templates,
    a batch with per-batch values, and a negative scale (whose max is the
    raw minimum)."""
    from catopt_amd import kernels as K

    rng = np.random.default_rng(dk * 7 + dv)
    for lead, shared_v, scale in (((), True, 0.3), ((2,), False, -0.7), ((3,), True, 1.0)):
        # attention-scaled queries: scores of order one, as in softmax attention (unscaled
        # unit-normal q·k at dk = 128 reach |s| ~ 40, where the fp32 rounding of the dot
        # product alone is 1e-5 of exp(s))
        q = (rng.standard_normal((*lead, Tq, dk)) / np.sqrt(dk)).astype(np.float32)
        k = rng.standard_normal((*lead, Tk, dk)).astype(np.float32)
        v = rng.standard_normal((Tk, dv) if shared_v else (*lead, Tk, dv)).astype(np.float32)
        m, lv, a = K.attn_carrier_f32(*(torch.from_numpy(z).to(dev) for z in (q, k, v)), scale)
        s = scale * (q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2))
        rm, rl, ra = oracle.om_elem(s, v.astype(np.float64))
        _gate(rm, m, TOL_F32)
        _gate(rl, lv, TOL_F32)
        _gate(ra, a, TOL_F32)
    # no keys: the empty carrier
    m, lv, a = K.attn_carrier_f32(torch.zeros(4, dk, device=dev), torch.zeros(0, dk, device=dev),
                                  torch.zeros(0, dv, device=dev))
    assert torch.isneginf(m).all() and not lv.any() and not a.any()


def test_omd_leaves_run_the_fused_kernel(dev):
    T, d, Tq, nb, dk = 256, 32, 40, 4, 16
    ir, _ = forms.omd_scan_attention_form(T, d, Tq, nb, dk)
    ins = _inputs(T, d, Tq, dk, False, 6)
    mod = HipOmdModule(ir, {})
    out = mod(*(t.to(dev) for t in ins))
    assert mod.fallbacks == 0 and mod.fused_leaves == nb and mod.fused_readout
    _gate(_reference(*ins, False), out, TOL_F32)


@pytest.mark.parametrize("L,Tq,d", [(16, 300, 64), (1, 7, 5), (5, 33, 128)])
def test_omd_fold_apply_matches_the_serial_fold(dev, L, Tq, d):
    """``catopt_hip_omd_fold_apply`` against the oracle's serial
    ``omd_compose`` fold and ``omd_apply`` in float64: carriers with an
    empty row in some leaves (m = -inf, l = 0, a = 0), a row empty in every
    leaf (NaN: 0 / 0), and carrier maxima far apart (weights that underflow
    to 0 beside 1)."""
    from catopt_amd import kernels as K

    rng = np.random.default_rng(L * 100 + d)
    m = rng.standard_normal((L, Tq)) * 30
    lv = rng.uniform(1.0, 5.0, (L, Tq))
    fa, fb = rng.standard_normal((L, Tq, d)), rng.standard_normal((L, Tq, d))
    h = rng.standard_normal(d)
    dead = [0] + ([Tq - 1] if Tq > 1 else [])
    m[0, Tq // 2] = -np.inf  # empty in leaf 0 only (all leaves when L = 1)
    lv[0, Tq // 2], fa[0, Tq // 2], fb[0, Tq // 2] = 0, 0, 0
    m[:, dead], lv[:, dead], fa[:, dead], fb[:, dead] = -np.inf, 0, 0, 0
    f32 = lambda z: np.asarray(z, np.float32).astype(np.float64)  # noqa: E731
    m, lv, fa, fb, h = (f32(z) for z in (m, lv, fa, fb, h))
    carriers = [(m[i][:, None], lv[i][:, None], fa[i], fb[i]) for i in range(L)]
    acc = carriers[0]
    for c in carriers[1:]:
        acc = oracle.omd_compose(acc, c)
    with np.errstate(invalid="ignore", divide="ignore"):
        ref = oracle.omd_apply(acc, h)
    assert np.isnan(ref[0]).all()
    num = torch.from_numpy(np.concatenate([fa, fb], -1).astype(np.float32)).to(dev)
    t = lambda z: torch.from_numpy(z.astype(np.float32)).to(dev)  # noqa: E731
    out = K.omd_fold_apply(t(m), t(lv), num, t(h))
    assert out.shape == (Tq, d)
    on = _np(out)
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    _gate(np.where(fin, ref, 0), torch.from_numpy(np.where(fin, on, 0)), TOL_F32)


# ------------------------------------------------------------ forest plans


def _restart_reference(q, k, a, x, h, blocks, dense):
    qn, kn, an, xn, hn = (_np(t) for t in (q, k, a, x, h))
    C = kn.shape[0] // blocks
    parts = []
    for i in range(blocks):
        sl = slice(i * C, (i + 1) * C)
        if dense:
            parts.append(oracle.serial_aff_scan(an[sl], xn[sl], hn[:, None])[..., 0])
        else:
            parts.append(oracle.serial_affd_scan(an[sl], xn[sl], hn))
    return _softmax_rows(qn @ kn.T) @ np.concatenate(parts)


@pytest.mark.parametrize("dense,bracket", [(False, "chain"), (False, "tree"), (True, "chain"), (True, "tree")])
def test_omd_forest_plan_block_restart(sink, dev, dense, bracket):
    """Maps of several leaf sequences (states restarted at every key block):
    the forest plan composes them level by level on the HIP slot kernels and
    the leaves run the fused carrier kernel, no generic-module fallback."""
    T, d, Tq, nb, dk = (64, 8, 24, 4, 16) if dense else (256, 32, 48, 8, 16)
    ir, _ = forms.omd_block_restart_form(T, d, Tq, nb, dk, dense=dense, bracket=bracket)
    ins = _inputs(T, d, Tq, dk, dense, 5)
    print(f"forest dense={dense} bracket={bracket} T={T}", flush=True)
    res = deliver(ir, {}, sink, tuple(t.to(dev) for t in ins))
    assert res.stats["executor"] == "omd_batched" and res.stats["hip_kernel"]
    mod = res.module
    assert mod.map_mode == "forest"
    out = mod(*[t.to(dev) for t in ins])
    assert mod.fallbacks == 0 and mod.fused_leaves == nb
    _gate(_restart_reference(*ins, nb, dense), out, TOL_F32)


def test_compose_slots_kernels(dev):
    """One launch per level over slot arrays.  Diagonal: bit-equal to the
    serial torch evaluation of ``(fa * ga, fa * gb + fb)`` on the device (no
    fused multiply-add).  Dense: ``(fa @ ga, fa @ gb + fb)`` against float64.
    An operand slot at or past the level's first output gives NaN."""
    from catopt_amd import kernels as K

    rng = np.random.default_rng(11)
    levels = [([1, 3, 5], [0, 2, 4]), ([7, 6], [6, 8]), ([10], [9])]
    n = 12  # 6 leaves, then 3 + 2 + 1 nodes
    # diagonal, a (2, 500) map per slot
    A = torch.zeros(n, 2, 500, device=dev)
    B = torch.zeros(n, 2, 500, device=dev)
    A[:6] = torch.from_numpy(rng.uniform(0.5, 1.5, (6, 2, 500)).astype(np.float32)).to(dev)
    B[:6] = torch.from_numpy(rng.standard_normal((6, 2, 500)).astype(np.float32)).to(dev)
    RA, RB = A.clone(), B.clone()
    out0 = 6
    for f, g in levels:
        fi = torch.tensor(f, device=dev)
        gi = torch.tensor(g, device=dev)
        K.compose_slots(A, B, fi, gi, out0, "diag")
        for j, (a_, b_) in enumerate(zip(f, g)):
            RA[out0 + j] = RA[a_] * RA[b_]
            RB[out0 + j] = RA[a_] * RB[b_] + RB[a_]
        out0 += len(f)
    torch.cuda.synchronize()
    assert torch.equal(A, RA) and torch.equal(B, RB)
    # dense, P = 3 maps of 24 x 24 per slot
    P, d = 3, 24
    Ad = torch.zeros(n, P, d, d, device=dev)
    Bd = torch.zeros(n, P, d, device=dev)
    Ad[:6] = torch.from_numpy((rng.standard_normal((6, P, d, d)) / np.sqrt(d)).astype(np.float32)).to(dev)
    Bd[:6] = torch.from_numpy(rng.standard_normal((6, P, d)).astype(np.float32)).to(dev)
    ref_a, ref_b = list(_np(Ad[:6])), list(_np(Bd[:6]))
    out0 = 6
    for f, g in levels:
        K.compose_slots(Ad, Bd, torch.tensor(f, device=dev), torch.tensor(g, device=dev), out0, "dense")
        for a_, b_ in zip(f, g):
            ref_a.append(ref_a[a_] @ ref_a[b_])
            ref_b.append((ref_a[a_] @ ref_b[b_][..., None])[..., 0] + ref_b[a_])
        out0 += len(f)
    _gate(np.stack(ref_a), Ad, TOL_F32)
    _gate(np.stack(ref_b), Bd, TOL_F32)
    # an operand slot that is not yet written: NaN in that output only
    K.compose_slots(A, B, torch.tensor([0, 9], device=dev), torch.tensor([1, 1], device=dev), 9, "diag")
    torch.cuda.synchronize()
    assert torch.equal(A[9], RA[0] * RA[1]) and bool(torch.isnan(A[10]).all()) and bool(torch.isnan(B[10]).all())
