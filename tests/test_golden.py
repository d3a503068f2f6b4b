"""The committed golden fixtures (``tests/golden/*.npz``) on the CPU.

Each fixture holds seeded inputs of one config at a small shape and the
expected output, written by ``tests/golden/make_golden.py`` from the numpy
restatement in float64.  Here:

* the inputs still follow bit for bit from the fixture's seed, and the
  restatement still reproduces the stored output (a change to either shows);
* every stored output agrees with an independent float64 computation in
  torch, written from the model's definition rather than from the
  restatement: the literal ``nn.Linear`` chain, ``F.rms_norm`` and
  ``F.silu``, ``F.scaled_dot_product_attention``, the quadratic decayed
  retention, and serial loops for the scans.

The GPU side (``test_golden_gpu.py``) runs the delivered forms on these
inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests.golden import make_golden as G

NAMES = list(G.FIXTURES)


def _t(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float64))


def _close(ref, out, rtol=1e-6):
    rep = oracle.verify_equiv(np.asarray(ref, dtype=np.float64), np.asarray(out, dtype=np.float64), rtol=rtol)
    assert rep["passed"], rep


@pytest.mark.parametrize("name", NAMES)
def test_fixture_follows_from_its_seed(name):
    fx, gen = G.load(name), G.generate(name)
    assert fx["seed"] == gen["seed"] and set(fx["bf16"]) == set(gen["bf16"])
    assert set(fx["inputs"]) == set(gen["inputs"])
    for k, v in gen["inputs"].items():
        assert fx["inputs"][k].dtype == np.float32 and np.array_equal(fx["inputs"][k], np.asarray(v, np.float32)), k
    for k, v in gen["expected"].items():
        _close(v, fx["expected"][k])


def test_bf16_bits_round_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e-39, 65504.0], dtype=np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(G.to_bf16_bits(x), want)
    assert np.array_equal(G.from_bf16_bits(want), torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_c1_literal_chain():
    fx = G.load("c1_weight_chain")
    i = fx["inputs"]
    h = _t(i["x"])
    for n in range(8):
        h = F.linear(h, _t(i[f"W{n + 1}"]), _t(i[f"b{n + 1}"]))
    _close(h.numpy(), fx["expected"]["y"])


def test_c2_rms_norm_swiglu():
    fx = G.load("c2_swiglu")
    i = {k: _t(v) for k, v in fx["inputs"].items()}
    h = F.rms_norm(i["x"], (i["x"].shape[-1],), i["gamma"], 1e-6)
    y = F.linear(F.silu(F.linear(h, i["W_gate"])) * F.linear(h, i["W_up"]), i["W_down"])
    _close(y.numpy(), fx["expected"]["y"])


def test_c3_sdpa_causal():
    fx = G.load("c3_causal_attention")
    q, k, v = (_t(fx["inputs"][n]) for n in "qkv")
    y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    _close(y.numpy(), fx["expected"]["y"])


def test_c4_quadratic_retention():
    fx = G.load("c4_retention")
    q, k, v = (_t(fx["inputs"][n]) for n in "qkv")
    g = _t(fx["inputs"]["gamma"])
    T = q.shape[-2]
    i = torch.arange(T, dtype=torch.float64)
    diff = i[:, None] - i[None, :]
    dec = torch.where(diff >= 0, g[:, None, None] ** diff.clamp_min(0), torch.zeros(()))
    y = ((q @ k.transpose(-1, -2)) * dec) @ v
    _close(y.numpy(), fx["expected"]["y"])


def test_c5_serial_ssm():
    fx = G.load("c5_ssm")
    a, bx, c, x, h = (_t(fx["inputs"][n]) for n in ("a", "bx", "c", "x", "h"))
    ys = []
    for t in range(x.shape[1]):
        h = a[:, t] * h + x[:, t, :, None] * bx[:, t, None, :]
        ys.append((h * c[:, t, None, :]).sum(-1))
    _close(torch.stack(ys, 1).numpy(), fx["expected"]["y"])


def test_aff_serial_recurrence():
    fx = G.load("aff_linear_recurrence")
    A, b, h = (_t(fx["inputs"][n]) for n in ("A", "b", "h"))
    for t in range(b.shape[0]):
        h = A @ h + b[t]
    _close(h.numpy(), fx["expected"]["y"])


def test_omd_softmax_over_scan_states():
    fx = G.load("omd_scan_attention")
    q, k, a, x, h = (_t(fx["inputs"][n]) for n in ("q", "k", "a", "x", "h"))
    states = []
    for t in range(a.shape[0]):
        h = a[t] * h + x[t]
        states.append(h)
    w = torch.softmax(q @ k.T, dim=-1)
    _close((w @ torch.stack(states)).numpy(), fx["expected"]["y"])


def test_fixture_sizes_stay_small():
    total = sum(G.path_of(n).stat().st_size for n in NAMES)
    assert total < 4 * 2 ** 20, total
