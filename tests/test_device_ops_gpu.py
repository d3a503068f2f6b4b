"""The device ops around the delivered forms run on the ROCm device (GPU).

A generic module whose term mixes the HIP-backed ops (``linear``) with the
table's device ops (``layer_norm``, ``clamp``, ``cumsum``, a creator)
evaluates on the device, with no host round trip: the output and every
created tensor live on the device, and the value matches the float64 numpy
composition of the same term.  Gate fp32 <= 1e-5 (global relative error).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd.bindings import HIP_BINDINGS
from catopt_amd.ir import IR, Const, Op, Param, TensorType, Var
from catopt_amd.sink import HipSink

pytestmark = pytest.mark.gpu
mk = Op.make


def test_a_term_of_device_ops_runs_on_the_device(dev):
    n, d, e = 16, 32, 24
    x, w = Var("x", TensorType((n, d))), Param("w", TensorType((e, d)))
    h = mk("layer_norm", mk("linear", x, w), dim=[e], eps=0.25)
    t = mk("cumsum", mk("clamp", h, min=-0.5, max=0.75), dim=1)
    t = mk("add", t, mk("ones", shape=[n, e]))
    rng = np.random.default_rng(3)
    wv, xv = rng.standard_normal((e, d)) * 0.2, rng.standard_normal((n, d))
    mod = HipSink().lower(IR(t, [x]), {"w": torch.from_numpy(wv).float().to(dev)})
    out = mod(torch.from_numpy(xv).float().to(dev))
    assert out.device.type == "cuda"
    xf, wf = (np.asarray(a, np.float32).astype(np.float64) for a in (xv, wv))
    y = xf @ wf.T
    ln = (y - y.mean(-1, keepdims=True)) / np.sqrt(y.var(-1, keepdims=True) + 0.25)
    ref = np.cumsum(np.clip(ln, -0.5, 0.75), 1) + 1.0
    rep = oracle.verify_equiv(ref, out.double().cpu().numpy(), rtol=1e-5)
    assert rep["passed"], rep


def test_creators_allocate_on_the_device(dev):
    for name, args, kw in (("zeros", (), {"shape": [3]}), ("randn", (), {"shape": [2, 2]}),
                           ("full", (torch.tensor(2.0),), {"shape": [4]}),
                           ("arange", (torch.tensor(0), torch.tensor(5)), {})):
        assert HIP_BINDINGS[name](*args, **kw).device.type == "cuda", name
    assert HIP_BINDINGS["arange"](torch.tensor(0), torch.tensor(5)).tolist() == [0, 1, 2, 3, 4]
    g = torch.arange(6.0, device=dev)
    assert HIP_BINDINGS["gt"](g, torch.tensor(2.5)).sum().item() == 3  # a host 0-dim Const beside a device tensor
    assert torch.equal(HIP_BINDINGS["where"](HIP_BINDINGS["ge"](g, Const(3).value * torch.ones((), device=dev)),
                                             g, torch.zeros((), device=dev)),
                       torch.tensor([0, 0, 0, 3, 4, 5.0], device=dev))
