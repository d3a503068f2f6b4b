"""Parity on the production code paths: the grids and shapes the configs run.

The edge-shape tests in ``test_kernels_gpu.py`` use small grids, which skip
branches that only the full workloads take: the GEMM's XCD-aware tile order
and its 8-M-tile grouping (active when the grid is a multiple of 8), and the
attention kernel's XCD remap in causal mode.  Here
those branches run, as do the persistent GEMM's multi-round tile streams
(C2's GEMMs), and C2–C5 are delivered through ``HipSink`` at their full
shapes, with every output element of sampled tiles compared against the
numpy oracle in float64 (the pinned parity), and every output element of
C2–C5 compared against an independent fp32 torch computation on the device
(the whole-output tests at the end):

* C2 (x[8,2048,4096] bf16): the first and the last 256-row M-tile, all
  4096 output columns (every N-tile of both GEMMs);
* C3 (q,k,v[4,32,4096,128] bf16): (b,h) = (0,0) and (3,31), all queries;
* C4 (q,k,v[4,16,8192,128] bf16): (b,h) = (0,0) and (3,15), all steps;
* C5 (B=16, T=16384, D=2048, N=16 fp32): batch 15, channels 2016–2047,
  every step (the last 4096 gated separately), plus batch 0, channels 0–31.

Gates: fp32 ≤ 1e-5, bf16 ≤ 2e-2 on ``max|Δ|/(max|ref|+1e-8)``.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import _lib as L
from catopt_amd import forms
from catopt_amd import kernels as K
from catopt_amd.sink import HipSink, deliver

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().double().numpy()


def _gate(ref, out, tol):
    rep = oracle.verify_equiv(ref, out if isinstance(out, np.ndarray) else _np(out), rtol=tol)
    assert rep["passed"], rep
    return rep


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dtype)


@pytest.fixture(scope="module")
def sink():
    return HipSink()


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.empty_cache()


# ------------------------------------------------------------- GEMM grids


# M = 2304: 9 M-tiles of 256, so the tile order has one full group of 8
# M-tiles and a partial last group of 1; N = 2048 (or 1024 paired outputs):
# 8 N-tiles, 72 workgroups, a multiple of 8, so the XCD remap runs.
@pytest.mark.parametrize("epi", [L.EPI_NONE, L.EPI_BIAS, L.EPI_BIAS_ADD2])
def test_linear_grouped_grid(dev, epi):
    M, N, Kd = 2304, 2048, 512
    x = _rand((M, Kd), torch.bfloat16, 40)
    w = _rand((N, Kd), torch.bfloat16, 41, 0.05)
    b = _rand((N,), torch.bfloat16, 42) if epi != L.EPI_NONE else None
    b2 = _rand((N,), torch.bfloat16, 43) if epi == L.EPI_BIAS_ADD2 else None
    y = K.linear(x.to(dev), w.to(dev), None if b is None else b.to(dev), None if b2 is None else b2.to(dev))
    ref = oracle.linear(_np(x), _np(w), None if b is None else _np(b))
    if b2 is not None:
        ref = ref + _np(b2)
    _gate(ref, y, TOL_BF16)


@pytest.mark.parametrize("epi", [L.EPI_SILU_MUL, L.EPI_GLU])
def test_linear_paired_grouped_grid(dev, epi):
    M, N, Kd = 2304, 1024, 512
    x = _rand((M, Kd), torch.bfloat16, 44)
    wg = _rand((N, Kd), torch.bfloat16, 45, 0.05)
    wu = _rand((N, Kd), torch.bfloat16, 46, 0.05)
    y = K.linear(x.to(dev), torch.cat([wg, wu], 0).to(dev), epilogue=epi)
    g, u = oracle.linear(_np(x), _np(wg)), oracle.linear(_np(x), _np(wu))
    ref = oracle.silu(g) * u if epi == L.EPI_SILU_MUL else g * (1 / (1 + np.exp(-u)))
    _gate(ref, y, TOL_BF16)


def test_linear_large_plain(dev):
    # M·N·K = 2^30, 16 tiles: the plain (no-epilogue) GEMM of the down
    # projection's kind on a grid whose workgroups take one tile each
    M = N = Kd = 1024
    x = _rand((M, Kd), torch.bfloat16, 47)
    w = _rand((N, Kd), torch.bfloat16, 48, 0.05)
    y = K.linear(x.to(dev), w.to(dev))
    _gate(oracle.linear(_np(x), _np(w)), y, TOL_BF16)


def test_linear_k_tail_grouped_grid(dev):
    # K % 64 != 0 on a grouped grid: the tail tile's zeroed chunks
    M, N, Kd = 2304, 2048, 520
    x = _rand((M, Kd), torch.bfloat16, 49)
    w = _rand((N, Kd), torch.bfloat16, 50, 0.05)
    y = K.linear(x.to(dev), w.to(dev))
    _gate(oracle.linear(_np(x), _np(w)), y, TOL_BF16)


@pytest.mark.parametrize("epi", [L.EPI_NONE, L.EPI_BIAS, L.EPI_SILU_MUL])
def test_linear_persistent_rounds_ragged(dev, epi):
    # 17 x 33 = 561 tiles: more than two rounds of the one-workgroup-per-CU
    # grid (the loads run ahead across tile boundaries and each tile's
    # stores overlap the next tile), with ragged M and N edges and a K tail
    # (K = 200: three full stages and one of 8)
    paired = epi == L.EPI_SILU_MUL
    M, Kd = 4160, 200
    N = 33 * 128 - 124 if paired else 33 * 256 - 248
    x = _rand((M, Kd), torch.bfloat16, 51)
    w = _rand(((2 if paired else 1) * N, Kd), torch.bfloat16, 52, 0.05)
    b = _rand((N,), torch.bfloat16, 53) if epi == L.EPI_BIAS else None
    y = K.linear(x.to(dev), w.to(dev), None if b is None else b.to(dev), epilogue=epi)
    if paired:
        ref = oracle.silu(oracle.linear(_np(x), _np(w[:N]))) * oracle.linear(_np(x), _np(w[N:]))
    else:
        ref = oracle.linear(_np(x), _np(w), None if b is None else _np(b))
    _gate(ref, y, TOL_BF16)


# ------------------------------------------------------- attention grid


# Grids that are multiples of 8 workgroups, so the XCD remaps and (causal)
# the tile orders run: d = 128, T = 256 is the 64-query kernel with one
# query tile per workgroup (8 workgroups), T = 512 the same kernel with the
# two tiles of a head's pair per workgroup (8 workgroups, 8 heads: one per
# XCD), and d = 64 the 32-query kernel (B·H·⌈T/128⌉ = 16 workgroups).
@pytest.mark.parametrize("T,d", [(256, 128), (512, 128), (256, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_remapped_grid(dev, causal, T, d):
    B, H = 1, 8
    q = _rand((B, H, T, d), torch.bfloat16, 60)
    k = _rand((B, H, T, d), torch.bfloat16, 61)
    v = _rand((B, H, T, d), torch.bfloat16, 62)
    scale = 1 / math.sqrt(d)
    o = K.attention(q.to(dev), k.to(dev), v.to(dev), scale, causal=causal)
    ref = oracle.attention_om(_np(q), _np(k), _np(v), scale, causal=causal)
    _gate(ref, o, TOL_BF16)


# ----------------------------------------------------- C2..C5 full shapes


def test_c2_full_shape_first_and_last_m_tiles(sink, dev):
    D, F = 4096, 11008
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    x = torch.randn(8, 2048, D, device=dev, generator=g).to(bf)
    vals = {
        "gamma": (1 + 0.02 * torch.randn(D, device=dev, generator=g)).to(bf),
        "W_gate": (0.02 * torch.randn(F, D, device=dev, generator=g)).to(bf),
        "W_up": (0.02 * torch.randn(F, D, device=dev, generator=g)).to(bf),
        "W_down": (0.02 * torch.randn(D, F, device=dev, generator=g)).to(bf),
    }
    ir, _ = forms.swiglu_block_form((8, 2048), D, F)
    res = deliver(ir, vals, sink, (x,))
    assert [s[0] for s in res.module._tape.steps] == ["rms_norm", "hip_swiglu", "hip_linear"]
    y = res.module(x).reshape(-1, D)
    torch.cuda.synchronize()
    M = y.shape[0]
    gam, wg, wu, wd = (_np(vals[n]) for n in ("gamma", "W_gate", "W_up", "W_down"))
    x2 = x.reshape(-1, D)
    for r0 in (0, M - 256):
        xs = _np(x2[r0:r0 + 256])
        ref = oracle.swiglu_fused(oracle.rms_norm(xs, gam, 1e-6), wg, wu, wd)
        _gate(ref, y[r0:r0 + 256], TOL_BF16)


def test_c3_full_shape_first_and_last_heads(sink, dev):
    B, H, T, d = 4, 32, 4096, 128
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn((B, H, T, d), device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    ir, _ = forms.causal_attention_form(B, H, T, d, mask="param")
    mask = torch.ones(T, T, dtype=torch.bool, device=dev).tril()
    res = deliver(ir, {"mask": mask}, sink, (q, k, v))
    assert res.module._plan["leaves"][0]["mask_kind"] == "causal"
    o = res.module(q, k, v)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (B - 1, H - 1)):
        ref = oracle.attention_om(_np(q[b, h]), _np(k[b, h]), _np(v[b, h]), 1 / math.sqrt(d), causal=True)
        _gate(ref, o[b, h], TOL_BF16)


def test_c4_full_shape_first_and_last_heads(sink, dev):
    B, H, T, d, C = 4, 16, 8192, 128, 64
    g = torch.Generator(device=dev).manual_seed(0)
    s = 1 / math.sqrt(d)
    q, k, v = ((torch.randn((B, H, T, d), device=dev, generator=g) * s).to(torch.bfloat16) for _ in range(3))
    gamma = torch.tensor([1 - 2.0 ** (-5 - h / 2) for h in range(H)], dtype=torch.float32, device=dev)
    ir, _ = forms.retention_kway_form(B, H, T, d, C)
    res = deliver(ir, {"gamma": gamma}, sink, (q, k, v))
    assert res.module.n_chunks == T // C and res.module.fallbacks == 0
    o = res.module(q, k, v)
    torch.cuda.synchronize()
    gam = gamma.cpu().double().numpy()
    for b, h in ((0, 0), (B - 1, H - 1)):
        ref = oracle.retention_kway(_np(q[b, h:h + 1]), _np(k[b, h:h + 1]), _np(v[b, h:h + 1]),
                                    gam[h:h + 1], T // C, 1.0)
        _gate(ref, o[b, h:h + 1], TOL_BF16)


def test_c5_full_shape_last_batch_and_channels(sink, dev):
    B, D, N, T = 16, 2048, 16, 16384
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn((B, T, D, N), device=dev, generator=g).neg_().sigmoid_()  # exp(-softplus(z))
    bx = torch.randn((B, T, N), device=dev, generator=g)
    c = torch.randn((B, T, N), device=dev, generator=g)
    x = torch.randn((B, T, D), device=dev, generator=g)
    h = torch.zeros((B, D, N), device=dev)
    ir, _ = forms.diag_ssm_form(B, T, D, N)
    res = deliver(ir, {}, sink, (a, bx, c, x, h))
    assert res.module.is_batched and res.module._plan["factors"] is not None
    y = res.module(a, bx, c, x, h)
    torch.cuda.synchronize()
    # a spans 2^33 elements: batch 15 lies past the 2^31-element mark
    for b, d0 in ((B - 1, D - 32), (0, 0)):
        sl = slice(d0, d0 + 32)
        ys, _ = oracle.ssm_serial(_np(a[b:b + 1, :, sl]), _np(bx[b:b + 1]), _np(c[b:b + 1]),
                                  _np(x[b:b + 1, :, sl]))
        got = _np(y[b:b + 1, :, sl])
        _gate(ys, got, TOL_F32)
        _gate(ys[:, 12288:], got[:, 12288:], TOL_F32)
    del a


# ------------------------------------------- whole outputs at full shapes
#
# Every output element of C2–C5 against an independent fp32 torch
# computation on the device, written from each model's definition (not from
# the kernels' algebra), chunked to bound memory: C2 fp32 rms_norm and
# matmuls per block of rows; C3 fp32 masked softmax attention per block of
# heads; C4 the quadratic decayed form per head (both chunk lengths the
# delivered K-way form takes); C5 the serial recurrence over every lane.
# The gate is the verify metric over the whole output, max|Δ| / max|ref|,
# taken across all blocks (the sampled oracle slices above stay the pinned
# parity).


class _WholeGate:
    """max|Δ| and max|ref| accumulated over blocks of one output."""

    def __init__(self):
        self.dmax = 0.0
        self.rmax = 0.0

    def add(self, ref: torch.Tensor, out: torch.Tensor) -> None:
        out = out.float()
        assert bool(torch.isfinite(out).all()), "non-finite output"
        self.dmax = max(self.dmax, (out - ref).abs().max().item())
        self.rmax = max(self.rmax, ref.abs().max().item())

    def check(self, tol: float) -> float:
        rel = self.dmax / (self.rmax + 1e-8)
        print(f"[whole-output] max_rel={rel:.3e} (gate {tol:g})", flush=True)
        assert rel <= tol, (rel, self.dmax, self.rmax)
        return rel


def test_c2_whole_output(sink, dev):
    D, F = 4096, 11008
    g = torch.Generator(device=dev).manual_seed(1)
    bf = torch.bfloat16
    x = torch.randn(8, 2048, D, device=dev, generator=g).to(bf)
    vals = {
        "gamma": (1 + 0.02 * torch.randn(D, device=dev, generator=g)).to(bf),
        "W_gate": (0.02 * torch.randn(F, D, device=dev, generator=g)).to(bf),
        "W_up": (0.02 * torch.randn(F, D, device=dev, generator=g)).to(bf),
        "W_down": (0.02 * torch.randn(D, F, device=dev, generator=g)).to(bf),
    }
    ir, _ = forms.swiglu_block_form((8, 2048), D, F)
    res = deliver(ir, vals, sink, (x,))
    y = res.module(x).reshape(-1, D)
    gam, wg, wu, wd = (vals[n].float() for n in ("gamma", "W_gate", "W_up", "W_down"))
    x2 = x.reshape(-1, D)
    gate = _WholeGate()
    for r0 in range(0, x2.shape[0], 2048):
        xs = x2[r0:r0 + 2048].float()
        h = xs * torch.rsqrt(xs.pow(2).mean(-1, keepdim=True) + 1e-6) * gam
        ref = (torch.nn.functional.silu(h @ wg.T) * (h @ wu.T)) @ wd.T
        gate.add(ref, y[r0:r0 + 2048])
    gate.check(TOL_BF16)


def test_c3_whole_output(sink, dev):
    B, H, T, d = 4, 32, 4096, 128
    g = torch.Generator(device=dev).manual_seed(1)
    q, k, v = (torch.randn((B, H, T, d), device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
    ir, _ = forms.causal_attention_form(B, H, T, d, mask="param")
    mask = torch.ones(T, T, dtype=torch.bool, device=dev).tril()
    res = deliver(ir, {"mask": mask}, sink, (q, k, v))
    o = res.module(q, k, v)
    gate = _WholeGate()
    keep = torch.ones(T, T, dtype=torch.bool, device=dev).tril()
    for b in range(B):
        for h0 in range(0, H, 8):
            qs, ks, vs = (t[b, h0:h0 + 8].float() for t in (q, k, v))
            s = (qs @ ks.transpose(-1, -2).contiguous()) / math.sqrt(d)
            ref = torch.softmax(s.masked_fill(~keep, float("-inf")), dim=-1) @ vs
            gate.add(ref, o[b, h0:h0 + 8])
            del s, ref
    gate.check(TOL_BF16)


@pytest.mark.parametrize("C", [64, 128])
def test_c4_whole_output(sink, dev, C):
    B, H, T, d = 4, 16, 8192, 128
    g = torch.Generator(device=dev).manual_seed(1)
    sd = 1 / math.sqrt(d)
    q, k, v = ((torch.randn((B, H, T, d), device=dev, generator=g) * sd).to(torch.bfloat16) for _ in range(3))
    gamma = torch.tensor([1 - 2.0 ** (-5 - h / 2) for h in range(H)], dtype=torch.float32, device=dev)
    ir, _ = forms.retention_kway_form(B, H, T, d, C)
    res = deliver(ir, {"gamma": gamma}, sink, (q, k, v))
    assert res.module.n_chunks == T // C and res.module.fallbacks == 0
    o = res.module(q, k, v)
    gate = _WholeGate()
    pos = torch.arange(T, device=dev, dtype=torch.float32)
    R = 2048  # query rows per block: o[t] = Σ_{s<=t} γ^(t-s) (q_t·k_s) v_s
    for h in range(H):
        lg = math.log2(float(gamma[h]))
        for r0 in range(0, T, R):
            t = pos[r0:r0 + R, None]
            s = pos[None, :r0 + R]
            dec = torch.where(s <= t, torch.exp2((t - s) * lg), torch.zeros((), device=dev))
            for b in range(B):
                qs = q[b, h, r0:r0 + R].float()
                ks, vs = k[b, h, :r0 + R].float(), v[b, h, :r0 + R].float()
                ref = ((qs @ ks.T) * dec) @ vs
                gate.add(ref, o[b, h, r0:r0 + R])
            del dec
    gate.check(TOL_BF16)


def test_c5_whole_output(sink, dev):
    B, D, N, T = 16, 2048, 16, 16384
    g = torch.Generator(device=dev).manual_seed(1)
    a = torch.randn((B, T, D, N), device=dev, generator=g).neg_().sigmoid_()  # exp(-softplus(z))
    bx = torch.randn((B, T, N), device=dev, generator=g)
    c = torch.randn((B, T, N), device=dev, generator=g)
    x = torch.randn((B, T, D), device=dev, generator=g)
    h0 = torch.zeros((B, D, N), device=dev)
    ir, _ = forms.diag_ssm_form(B, T, D, N)
    res = deliver(ir, {}, sink, (a, bx, c, x, h0))
    y = res.module(a, bx, c, x, h0)
    # h_t = a_t ⊙ h_{t-1} + x_t ⊗ bx_t, y_t = h_t · c_t, every lane, serially
    gate = _WholeGate()
    h = h0.clone()
    blk = 512
    ref = torch.empty((B, blk, D), device=dev)
    for t0 in range(0, T, blk):
        for i in range(blk):
            t = t0 + i
            h = a[:, t] * h + x[:, t, :, None] * bx[:, t, None, :]
            ref[:, i] = (h * c[:, t, None, :]).sum(-1)
        gate.add(ref, y[:, t0:t0 + blk])
    gate.check(TOL_F32)
    del a
