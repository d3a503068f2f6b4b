"""GPU parity of every C-ABI kernel against the numpy oracle.

Inputs are seeded on the host, rounded to the kernel dtype, and the oracle
runs on exactly those values in float64.  Gates (the north star's, as the
reference's verify metric ``max|Δ| / (max|ref| + 1e-8)``):
  fp32  ≤ 1e-5,   bf16  ≤ 2e-2,   integer tables bit-exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import _lib as L
from catopt_amd import kernels as K

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().double().numpy()


def _gate(ref, out, tol):
    rep = oracle.verify_equiv(ref, _np(out) if isinstance(out, torch.Tensor) else out, rtol=tol)
    assert rep["passed"], rep
    return rep


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * scale).to(dtype)


# ------------------------------------------------------------------ rmsnorm


@pytest.mark.parametrize("rows,cols", [(64, 4096), (33, 1000), (7, 4097), (5, 8192)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rmsnorm(dev, rows, cols, dtype):
    x = _rand((rows, cols), dtype, 1)
    w = (1 + 0.02 * _rand((cols,), torch.float32, 2)).to(dtype)
    y = K.rmsnorm(x.to(dev), w.to(dev), 1e-6)
    ref = oracle.rms_norm(_np(x), _np(w), 1e-6)
    _gate(ref, y, TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)


def test_rmsnorm_strided_rows_no_weight(dev):
    x = _rand((16, 2 * 512), torch.bfloat16, 3)[:, :512]
    y = K.rmsnorm(x.to(dev), None, 1e-5)
    _gate(oracle.rms_norm(_np(x), None, 1e-5), y, TOL_BF16)


# ------------------------------------------------------------------ linear


@pytest.mark.parametrize("M,N,Kd", [(512, 512, 512), (300, 520, 264), (17, 1000, 64), (1, 256, 4096)])
@pytest.mark.parametrize("with_bias", [0, 1, 2])
def test_linear_bf16(dev, M, N, Kd, with_bias):
    x = _rand((M, Kd), torch.bfloat16, 10)
    w = _rand((N, Kd), torch.bfloat16, 11, 0.05)
    b = _rand((N,), torch.bfloat16, 12) if with_bias else None
    b2 = _rand((N,), torch.bfloat16, 13) if with_bias == 2 else None
    y = K.linear(x.to(dev), w.to(dev), None if b is None else b.to(dev), None if b2 is None else b2.to(dev))
    ref = oracle.linear(_np(x), _np(w), None if b is None else _np(b))
    if b2 is not None:
        ref = ref + _np(b2)
    _gate(ref, y, TOL_BF16)


@pytest.mark.parametrize("M,N,Kd", [(256, 384, 512), (100, 200, 128), (513, 128, 4096)])
@pytest.mark.parametrize("epi", [L.EPI_SILU_MUL, L.EPI_GLU])
def test_linear_paired_epilogue(dev, M, N, Kd, epi):
    x = _rand((M, Kd), torch.bfloat16, 20)
    wg = _rand((N, Kd), torch.bfloat16, 21, 0.05)
    wu = _rand((N, Kd), torch.bfloat16, 22, 0.05)
    wcat = torch.cat([wg, wu], 0)
    y = K.linear(x.to(dev), wcat.to(dev), epilogue=epi)
    g = oracle.linear(_np(x), _np(wg))
    u = oracle.linear(_np(x), _np(wu))
    ref = oracle.silu(g) * u if epi == L.EPI_SILU_MUL else g * (1 / (1 + np.exp(-u)))
    _gate(ref, y, TOL_BF16)


def test_linear_paired_unaligned_falls_to_generic(dev):
    # K % 8 != 0 takes the generic kernel; the result must not change.
    x = _rand((40, 60), torch.bfloat16, 23)
    w = _rand((2 * 72, 60), torch.bfloat16, 24, 0.1)
    y = K.linear(x.to(dev), w.to(dev), epilogue=L.EPI_SILU_MUL)
    g, u = oracle.linear(_np(x), _np(w[:72])), oracle.linear(_np(x), _np(w[72:]))
    _gate(oracle.silu(g) * u, y, TOL_BF16)


@pytest.mark.parametrize("M,N,Kd", [(64, 512, 512), (7, 33, 129), (30, 100, 260), (1, 17, 4),
                                    (129, 40, 1000), (600, 700, 2048)])
def test_linear_fp32(dev, M, N, Kd):
    # (64,512,512), (30,100,260), (1,17,4), (129,40,1000): the skinny split-K
    # kernel (ragged tiles, K not a multiple of 64); (7,33,129): K % 4 != 0,
    # the tiled kernel; (600,700,2048): enough tiles for the tiled kernel.
    x = _rand((M, Kd), torch.float32, 30)
    w = _rand((N, Kd), torch.float32, 31, 1 / math.sqrt(Kd))
    b = _rand((N,), torch.float32, 32)
    y = K.linear(x.to(dev), w.to(dev), b.to(dev))
    _gate(oracle.linear(_np(x), _np(w), _np(b)), y, TOL_F32)
    b2 = _rand((N,), torch.float32, 33)
    y2 = K.linear(x.to(dev), w.to(dev), b.to(dev), b2.to(dev))
    _gate(oracle.linear(_np(x), _np(w), _np(b)) + _np(b2), y2, TOL_F32)
    y0 = K.linear(x.to(dev), w.to(dev))
    _gate(oracle.linear(_np(x), _np(w)), y0, TOL_F32)


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_matmul_layouts(dev, ta, tb, dtype):
    A = _rand((3, 70, 90), dtype, 40)
    B = _rand((3, 90, 50), dtype, 41)
    a = A.transpose(1, 2).contiguous().transpose(1, 2) if ta else A
    b = B.transpose(1, 2).contiguous().transpose(1, 2) if tb else B
    y = K.matmul(a.to(dev), b.to(dev))
    _gate(_np(A) @ _np(B), y, TOL_BF16 if dtype == torch.bfloat16 else TOL_F32)


def test_matmul_fold_chain_fp32(dev):
    Ws = [_rand((512, 512), torch.float32, 50 + i, 1 / math.sqrt(512)) for i in range(3)]
    y = K.matmul(K.matmul(Ws[2].to(dev), Ws[1].to(dev)), Ws[0].to(dev))
    _gate(_np(Ws[2]) @ _np(Ws[1]) @ _np(Ws[0]), y, TOL_F32)


def test_matmul_broadcast_batch(dev):
    A = _rand((4, 2, 64, 96), torch.bfloat16, 60)
    B = _rand((96, 128), torch.bfloat16, 61)
    y = K.matmul(A.to(dev), B.to(dev))
    _gate(_np(A) @ _np(B), y, TOL_BF16)


@pytest.mark.parametrize("c_off,sc_pad", [(0, 4), (4, 0), (4, 4)])
def test_matmul_bf16_c_rows_not_16_byte_aligned(dev, c_off, sc_pad):
    # a batch stride of C that is 4 elements off a multiple of 8, or C itself
    # 8 bytes off a 16-byte boundary: the epilogue stores column by column
    # (its 16-byte stores need every row of every batch 16-byte aligned);
    # the elements around each C[b] stay untouched
    nb, M, N, Kd = 3, 64, 128, 96
    A = _rand((nb, M, Kd), torch.bfloat16, 70).to(dev)
    Bt = _rand((nb, N, Kd), torch.bfloat16, 71).to(dev)  # B given as Nx K rows: transB = 1
    sC = M * N + sc_pad
    buf = torch.full((c_off + nb * sC + 8,), 7.0, dtype=torch.bfloat16, device=dev)
    lib = L.load()
    st = lib.catopt_hip_matmul(L.BF16, nb, M, N, Kd, A.data_ptr(), Kd, M * Kd, 0, Bt.data_ptr(), Kd, N * Kd,
                               1, buf.data_ptr() + 2 * c_off, N, sC, K._stream(A))
    L.check("catopt_hip_matmul", st)
    ref = _np(A) @ np.swapaxes(_np(Bt), 1, 2)
    host = buf.float().cpu()
    for b in range(nb):
        _gate(ref[b], host[c_off + b * sC: c_off + b * sC + M * N].reshape(M, N).double().numpy(), TOL_BF16)
        gap = host[c_off + b * sC + M * N: c_off + (b + 1) * sC]
        assert bool((gap == 7.0).all())
    assert bool((host[:c_off] == 7.0).all()) and bool((host[c_off + nb * sC:] == 7.0).all())


# ------------------------------------------------------------------ attention


def _qkv(B, H, T, d, seed, Tk=None):
    Tk = Tk or T
    return (_rand((B, H, T, d), torch.bfloat16, seed), _rand((B, H, Tk, d), torch.bfloat16, seed + 1),
            _rand((B, H, Tk, d), torch.bfloat16, seed + 2))


@pytest.mark.parametrize("T,d", [(256, 128), (200, 128), (384, 64), (64, 128)])
def test_attention_causal(dev, T, d):
    q, k, v = _qkv(1, 3, T, d, 70)
    scale = 1 / math.sqrt(d)
    o = K.attention(q.to(dev), k.to(dev), v.to(dev), scale, causal=True)
    ref = oracle.attention_om(_np(q), _np(k), _np(v), scale, causal=True, block=64)
    _gate(ref, o, TOL_BF16)
    assert not torch.isnan(o).any()


def test_attention_ml_carriers_and_unnormalised(dev):
    q, k, v = _qkv(2, 2, 128, 128, 80)
    scale = 0.1
    a, m, l = K.attention(q.to(dev), k.to(dev), v.to(dev), scale, causal=True, normalize=False, return_ml=True)
    out, mr, lr = oracle.attention_om(_np(q), _np(k), _np(v), scale, causal=True, block=32, return_ml=True)
    _gate(mr, m, 1e-5)
    _gate(lr, l, TOL_BF16)
    _gate(out * lr, a, TOL_BF16)


def test_attention_bool_mask_nan_rows(dev):
    T = 96
    q, k, v = _qkv(1, 2, T, 128, 90)
    rng = np.random.default_rng(0)
    keep = rng.random((T, T)) < 0.3
    keep[5, :] = False  # a fully masked row: om_apply gives NaN there
    o = K.attention(q.to(dev), k.to(dev), v.to(dev), 0.125, mask=torch.from_numpy(keep).to(dev))
    ref = oracle.attention_om(_np(q), _np(k), _np(v), 0.125, causal=False, mask=keep, block=32)
    on = _np(o)
    assert np.array_equal(np.isnan(on), np.isnan(ref))
    fin = ~np.isnan(ref)
    _gate(np.where(fin, ref, 0), np.where(fin, on, 0), TOL_BF16)


@pytest.mark.parametrize("d,dv,causal", [(32, 32, True), (96, 96, False), (80, 48, True), (128, 72, False)])
def test_attention_other_head_dims(dev, d, dv, causal):
    # widths other than 64 / 128 run zero-padded to the next of them
    B, H, T = 1, 2, 192
    q, k = _rand((B, H, T, d), torch.bfloat16, 130), _rand((B, H, T, d), torch.bfloat16, 131)
    v = _rand((B, H, T, dv), torch.bfloat16, 132)
    sc = 1 / math.sqrt(d)
    o, m, lsum = K.attention(q.to(dev), k.to(dev), v.to(dev), sc, causal=causal, return_ml=True)
    assert o.shape == (B, H, T, dv) and m.shape == (B, H, T, 1)
    ref = oracle.attention_om(_np(q), _np(k), _np(v), sc, causal=causal)
    _gate(ref, o, TOL_BF16)


def test_attention_causal_offset_and_cross_lengths(dev):
    q, k, v = _qkv(1, 2, 100, 128, 95, Tk=300)
    o = K.attention(q.to(dev), k.to(dev), v.to(dev), 0.08, causal=True, causal_off=200)
    ref = oracle.attention_om(_np(q), _np(k), _np(v), 0.08, causal=True, causal_off=200)
    _gate(ref, o, TOL_BF16)


# The 64-query kernel (attn_q64_kernel) takes d = 128, no mask or causal, and
# whole 64-key tiles; these cases reach its edges: query counts off a
# multiple of the 256-query workgroup and of a wave's 64, keys of one and of
# many tiles, causal offsets that start, end or empty rows, several heads per
# XCD and a head count off a multiple of 8 (the grid mappings), and odd and
# even query-tile counts (even counts run two tiles per workgroup).
@pytest.mark.parametrize("B,H,Tq,Tk,causal,off", [
    (1, 2, 256, 256, True, 0), (2, 3, 100, 320, True, 220), (1, 16, 300, 512, True, 0),
    (1, 2, 200, 64, False, 0), (1, 4, 512, 512, True, -130), (1, 2, 64, 1024, True, 960),
    (2, 8, 320, 384, False, 0), (1, 1, 1000, 1024, True, 24), (1, 4, 1024, 1024, True, 0),
])
def test_attention_q64_tiles(dev, B, H, Tq, Tk, causal, off):
    q, k, v = _qkv(B, H, Tq, 128, 300 + Tq + Tk, Tk=Tk)
    scale = 1 / math.sqrt(128)
    o, m, lsum = K.attention(q.to(dev), k.to(dev), v.to(dev), scale, causal=causal, causal_off=off,
                             return_ml=True)
    ref, mr, lr = oracle.attention_om(_np(q), _np(k), _np(v), scale, causal=causal, causal_off=off,
                                      return_ml=True)
    on = _np(o)
    assert np.array_equal(np.isnan(on), np.isnan(ref))  # rows with no key (negative offsets) are NaN
    fin = ~np.isnan(ref)
    _gate(np.where(fin, ref, 0), np.where(fin, on, 0), TOL_BF16)
    mf = np.isfinite(mr)
    assert np.array_equal(np.isfinite(_np(m)), mf)
    _gate(np.where(mf, mr, 0), np.where(mf, _np(m), 0), 1e-5)
    # a row with no key: the single-leaf oracle's l is exp(-inf - -inf) = NaN;
    # the kernel's carrier is the empty one, (m, l) = (-inf, 0)
    ln = _np(lsum)
    _gate(np.where(mf, lr, 0), np.where(mf, ln, 0), TOL_BF16)
    assert bool((ln[~mf] == 0).all())


def test_attention_q64_strided_and_zero_rows(dev):
    # (B, T, H, d) operands viewed as (B, H, T, d): row stride H·d, the head
    # ranges of the buffer resources far from the tensor start; a causal
    # offset that leaves the first rows without keys returns 0 there in the
    # sdpa convention
    B, T, H = 2, 448, 3
    base = [_rand((B, T, H, 128), torch.bfloat16, 400 + i).to(dev) for i in range(3)]
    q, k, v = (t.transpose(1, 2) for t in base)
    o = K.attention(q, k, v, 0.09, causal=True, causal_off=-40, empty_rows="zero")
    ref = oracle.attention_om(_np(q), _np(k), _np(v), 0.09, causal=True, causal_off=-40)
    ref = np.where(np.isnan(ref), 0.0, ref)
    _gate(ref, o, TOL_BF16)
    assert bool((o[:, :, :40] == 0).all())


# one query tile per workgroup (192 queries) and two (448: the paired path)
@pytest.mark.parametrize("Tq,Tk,causal", [(192, 256, False), (448, 512, True)])
def test_attention_q64_unnormalised_numerator(dev, Tq, Tk, causal):
    q, k, v = _qkv(1, 2, Tq, 128, 450, Tk=Tk)
    a, m, lsum = K.attention(q.to(dev), k.to(dev), v.to(dev), 0.1, causal=causal, normalize=False, return_ml=True)
    out, mr, lr = oracle.attention_om(_np(q), _np(k), _np(v), 0.1, causal=causal, return_ml=True)
    _gate(mr, m, 1e-5)
    _gate(lr, lsum, TOL_BF16)
    _gate(out * lr, a, TOL_BF16)


def test_om_compose_kernel(dev):
    rng = np.random.default_rng(1)
    m1 = rng.standard_normal((40, 1))
    m2 = rng.standard_normal((40, 1))
    m1[3] = -np.inf
    m2[7] = -np.inf
    m1[9] = m2[9] = -np.inf
    l1, l2 = rng.random((40, 1)), rng.random((40, 1))
    a1, a2 = rng.standard_normal((40, 16)), rng.standard_normal((40, 16))
    l1[m1 == -np.inf] = 0
    l2[m2 == -np.inf] = 0
    f = [torch.tensor(t, dtype=torch.float32, device=dev) for t in (m1, l1, a1)]
    g = [torch.tensor(t, dtype=torch.float32, device=dev) for t in (m2, l2, a2)]
    m, l, a = K.om_compose(f, g)
    rm, rl, ra = oracle.om_compose((m1, l1, a1), (m2, l2, a2))
    assert np.array_equal(np.isinf(_np(m)), np.isinf(rm))
    _gate(rl, l, TOL_F32)
    _gate(ra, a, TOL_F32)


# ------------------------------------------------------------------ retention


def _gammas(H):
    return np.array([1 - 2.0 ** (-5 - h / 2) for h in range(H)], dtype=np.float32)


# (1, 2, 128): two one-chunk segments; (5, 16, 256): more (head, slice) work
# items than CUs, so one segment per head
@pytest.mark.parametrize("B,H,T", [(1, 2, 512), (2, 3, 1024), (1, 1, 64), (1, 2, 128), (5, 16, 256)])
def test_retention_vs_kway_form(dev, B, H, T):
    scale = 1.0
    q = _rand((B, H, T, 128), torch.bfloat16, 100, 1 / math.sqrt(128))
    k = _rand((B, H, T, 128), torch.bfloat16, 101, 1 / math.sqrt(128))
    v = _rand((B, H, T, 128), torch.bfloat16, 102, 1 / math.sqrt(128))
    gam = _gammas(H)
    o = K.retention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(gam).to(dev), scale)
    g64 = gam.astype(np.float64)
    if T >= 128:  # the K-way delivered form with 64-row chunks
        ref = oracle.retention_kway(_np(q), _np(k), _np(v), g64, T // 64, scale)
    else:  # a single chunk is the quadratic form itself
        ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), g64, scale)
    _gate(ref, o, TOL_BF16)


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, TOL_BF16), (torch.float32, TOL_F32)])
def test_retention_decay_rates_zero_one_and_negative(dev, dtype, tol):
    # γ^k as pow gives it for integer k: 0^0 = 1 (a γ = 0 head is the
    # diagonal term alone), γ = 1 (no decay), a negative γ alternating in
    # sign; T = 1024 over 4 heads splits each head into segments, so the
    # start-state pieces are scaled by these powers too
    B, H, T, d = 1, 4, 1024, 128
    q = _rand((B, H, T, d), dtype, 140, 1 / math.sqrt(d))
    k = _rand((B, H, T, d), dtype, 141, 1 / math.sqrt(d))
    v = _rand((B, H, T, d), dtype, 142, 1 / math.sqrt(d))
    gam = np.array([0.0, 1.0, -0.9, 0.5], dtype=np.float32)
    o = K.retention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(gam).to(dev), 0.25)
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.astype(np.float64), 0.25)
    assert np.isfinite(ref).all() and np.isfinite(_np(o)).all()
    for h in range(H):  # per head: the heads' scales differ by orders of magnitude
        _gate(ref[:, h], o[:, h], tol)


@pytest.mark.parametrize("dk,dv", [(64, 64), (96, 64), (128, 80)])
def test_retention_narrow_heads(dev, dk, dv):
    # head dims below 128 run zero-padded to the kernel's width
    B, H, T = 1, 2, 256
    q = _rand((B, H, T, dk), torch.bfloat16, 120, 1 / math.sqrt(dk))
    k = _rand((B, H, T, dk), torch.bfloat16, 121, 1 / math.sqrt(dk))
    v = _rand((B, H, T, dv), torch.bfloat16, 122, 1 / math.sqrt(dv))
    gam = _gammas(H)
    o = K.retention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(gam).to(dev), 0.7)
    assert o.shape == (B, H, T, dv)
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.astype(np.float64), 0.7)
    _gate(ref, o, TOL_BF16)


@pytest.mark.parametrize("B,H,T,d", [(1, 3, 1000, 64), (2, 2, 200, 120), (1, 5, 4100, 128), (3, 1, 70, 8)])
def test_retention_ragged_steps_and_narrow_heads_in_the_kernel(dev, B, H, T, d):
    # a T off the 64-step chunk and head dims below 128 (multiples of 8) run
    # in place: the kernel's buffer ranges load zeros past T and past d and
    # drop the stores there (no padded copies); (1, 5, 4100, 128) spans
    # several segments, the last one ragged
    q = _rand((B, H, T, d), torch.bfloat16, 130, 1 / math.sqrt(d))
    k = _rand((B, H, T, d), torch.bfloat16, 131, 1 / math.sqrt(d))
    v = _rand((B, H, T, d), torch.bfloat16, 132, 1 / math.sqrt(d))
    gam = _gammas(H)
    o = K.retention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(gam).to(dev), 0.9)
    assert o.shape == (B, H, T, d)
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.astype(np.float64), 0.9)
    _gate(ref, o, TOL_BF16)


def test_retention_long_many_segments(dev):
    # 64 chunks over one (b,h): exercises the segment carry pass.
    B, H, T = 1, 2, 4096
    q = _rand((B, H, T, 128), torch.bfloat16, 110, 1 / math.sqrt(128))
    k = _rand((B, H, T, 128), torch.bfloat16, 111, 1 / math.sqrt(128))
    v = _rand((B, H, T, 128), torch.bfloat16, 112, 1 / math.sqrt(128))
    gam = _gammas(H)
    o = K.retention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(gam).to(dev), 0.5)
    ref = oracle.retention_quadratic(_np(q), _np(k), _np(v), gam.astype(np.float64), 0.5)
    _gate(ref, o, TOL_BF16)


def test_decay_generators(dev):
    gam = _gammas(4)
    g = torch.from_numpy(gam).to(dev)
    _gate(oracle.decay(gam.astype(np.float64), 64), K.decay(g, 64), TOL_F32)
    for off, sign in [(0, -1), (128, 1), (64, 0)]:
        _gate(oracle.decay_vec(gam.astype(np.float64), 64, off, sign), K.decay_vec(g, 64, off, sign), TOL_F32)


# ------------------------------------------------------------------ scans


@pytest.mark.parametrize("schedule", [L.SCAN_STREAM, L.SCAN_CHUNKED])
@pytest.mark.parametrize("lti", [False, True])
def test_affd_scan(dev, schedule, lti):
    rng = np.random.default_rng(5)
    T, S = 300, 1000
    a = rng.uniform(0.5, 1.0, (S,) if lti else (T, S)).astype(np.float32)
    u = rng.standard_normal((T, S)).astype(np.float32)
    h0 = rng.standard_normal(S).astype(np.float32)
    table = oracle.prefix_chunk_table(T)
    st, hf = K.affd_scan(torch.from_numpy(a).to(dev), torch.from_numpy(u).to(dev),
                         torch.from_numpy(h0).to(dev), table, schedule=schedule)
    ref = oracle.serial_affd_scan(a.astype(np.float64), u.astype(np.float64), h0.astype(np.float64))
    _gate(ref, st, TOL_F32)
    _gate(ref[-1], hf, TOL_F32)


@pytest.mark.parametrize("schedule", [L.SCAN_STREAM, L.SCAN_CHUNKED])
@pytest.mark.parametrize("N,D,aps", [(16, 64, True), (16, 70, True), (4, 40, False), (64, 16, True)])
def test_ssm_scan(dev, schedule, N, D, aps):
    rng = np.random.default_rng(6)
    B, T = 2, 257
    z = rng.standard_normal((B, T, D, N) if aps else (B, T, D))
    a = np.exp(-np.log1p(np.exp(z))).astype(np.float32)  # exp(-softplus(z)) in (0, 1)
    bx = rng.standard_normal((B, T, N)).astype(np.float32)
    c = rng.standard_normal((B, T, N)).astype(np.float32)
    x = rng.standard_normal((B, T, D)).astype(np.float32)
    h0 = rng.standard_normal((B, D, N)).astype(np.float32)
    table = oracle.prefix_chunk_table(T)
    t = lambda z_: torch.from_numpy(z_).to(dev)  # noqa: E731
    y, hf = K.ssm_scan(t(a), t(bx), t(c), t(x), t(h0), table, schedule=schedule, return_state=True)
    ry, rh = oracle.ssm_serial(*(z_.astype(np.float64) for z_ in (a, bx, c, x, h0)))
    _gate(ry, y, TOL_F32)
    _gate(rh, hf, TOL_F32)


def test_silu_kernels(dev):
    x = _rand((1000,), torch.bfloat16, 7)
    u = _rand((1000,), torch.bfloat16, 8)
    _gate(oracle.silu(_np(x)), K.silu(x.to(dev)), TOL_BF16)
    _gate(oracle.silu(_np(x)) * _np(u), K.silu_mul(x.to(dev), u.to(dev)), TOL_BF16)


def test_empty_inputs(dev):
    """Zero rows, steps, queries or keys at every entry point: empty outputs,
    the initial state passed through, and the empty carrier (m = -inf, l = 0,
    a / l = NaN) when there are no keys."""
    t = lambda *s, dt=torch.bfloat16: torch.randn(*s, device=dev).to(dt)  # noqa: E731
    for dt in (torch.bfloat16, torch.float32):
        assert K.linear(t(0, 64, dt=dt), t(32, 64, dt=dt)).shape == (0, 32)
    assert K.linear(t(0, 64), t(64, 64), epilogue=L.EPI_SILU_MUL).shape == (0, 32)
    assert K.matmul(t(0, 8, dt=torch.float32), t(8, 16, dt=torch.float32)).shape == (0, 16)
    assert K.rmsnorm(t(0, 256), t(256), 1e-6).shape == (0, 256)
    assert K.silu(t(0)).shape == (0,)
    # no queries / no steps
    assert K.attention(t(1, 2, 0, 64), t(1, 2, 0, 64), t(1, 2, 0, 64), 0.125, causal=True).shape == (1, 2, 0, 64)
    assert K.retention(t(1, 2, 0, 128), t(1, 2, 0, 128), t(1, 2, 0, 128),
                       torch.tensor([0.9, 0.95], device=dev)).shape == (1, 2, 0, 128)
    # no keys: om_apply of the empty carrier is 0 / 0
    q = t(1, 1, 5, 64)
    out = K.attention(q, t(1, 1, 0, 64), t(1, 1, 0, 64), 0.125)
    assert out.shape == (1, 1, 5, 64) and torch.isnan(out.float()).all()
    o2, m, lv = K.attention(q, t(1, 1, 0, 64), t(1, 1, 0, 64), 0.125, normalize=False, return_ml=True)
    assert torch.isneginf(m).all() and not lv.any() and not o2.float().any()
    # zero steps: the state passes through
    h0 = torch.randn(10, device=dev)
    st, hf = K.affd_scan(torch.zeros(0, 10, device=dev), torch.zeros(0, 10, device=dev), h0, [0, 0])
    assert st.shape == (0, 10) and torch.equal(hf, h0)
    hs = torch.randn(1, 8, 16, device=dev)
    y, hsf = K.ssm_scan(torch.zeros(1, 0, 8, 16, device=dev), torch.zeros(1, 0, 16, device=dev),
                        torch.zeros(1, 0, 16, device=dev), torch.zeros(1, 0, 8, device=dev), hs, [0, 0],
                        return_state=True)
    assert y.shape == (1, 0, 8) and torch.equal(hsf, hs)
    assert K.decay(torch.tensor([0.9, 0.8], device=dev), 0).shape == (2, 0, 0)
    e = torch.zeros(0, 1, device=dev)
    mc, lc, ac = K.om_compose((e, e, torch.zeros(0, 4, device=dev)), (e, e, torch.zeros(0, 4, device=dev)))
    assert mc.shape == (0, 1) and ac.shape == (0, 4)


@pytest.mark.parametrize("nbytes", [16, 4096, (1 << 20) + 48, 64 << 20])
def test_hbm_read_reads_every_word(dev, nbytes):
    """The read stream's sink is written only when some lane's XOR of the
    words it read equals the sentinel: with one sentinel word in zeros, at the
    start, the middle or the end of the buffer, the sink is written (that word
    was read); with none, it is not."""
    SENT = 0x9E3779B9
    n32 = nbytes // 4
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    buf = torch.zeros(n32, dtype=torch.int32, device=dev)
    K.hbm_read(buf, sink)
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    for pos in sorted({0, n32 // 2, n32 - 1}):
        buf.zero_()
        buf[pos] = torch.tensor(SENT, dtype=torch.int64).to(torch.int32)
        sink.zero_()
        K.hbm_read(buf, sink)
        torch.cuda.synchronize()
        assert int(sink.item()) & 0xFFFFFFFF == SENT, (nbytes, pos)
