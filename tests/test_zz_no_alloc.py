"""The entry point that allocates nothing: ``catopt_hip_affd_scan_noalloc``.

It runs the kernels of ``catopt_hip_affd_scan`` with the chunk-parallel
schedule's workspace in a static device array instead of a caller buffer.
Both entry points are called through the C ABI on the same seeded inputs,
twice in a row (the second call smaller, so it runs over what the first left
in the array), and their outputs must agree bit for bit; each is also gated
against the oracle's serial recurrence (fp32 ≤ 1e-5).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from catopt_amd import _lib as L

pytestmark = pytest.mark.gpu


def _inputs(T, S, seed, dev):
    g = torch.Generator().manual_seed(seed)
    a = torch.rand((T, S), generator=g) * 0.9 + 0.05
    u = torch.randn((T, S), generator=g)
    h0 = torch.randn((S,), generator=g)
    return a.to(dev), u.to(dev), h0.to(dev)


def _table(T, n):
    starts = sorted({0, *[(i * T) // n for i in range(1, n)], T})
    return torch.tensor(starts, dtype=torch.int64)


def _run(lib, noalloc, a, u, h0, cs, nc, schedule, dev, stream=None):
    T, S = u.shape
    states = torch.full((T, S), float("nan"), device=dev)
    hf = torch.full((S,), float("nan"), device=dev)
    torch.cuda.synchronize(dev)  # inputs in place before a side stream reads them
    stream = (stream or torch.cuda.current_stream(dev)).cuda_stream
    if noalloc:
        st = lib.catopt_hip_affd_scan_noalloc(T, S, a.data_ptr(), S, u.data_ptr(), S, h0.data_ptr(),
                                              cs.data_ptr(), nc, schedule, states.data_ptr(), hf.data_ptr(),
                                              stream)
    else:
        wsb = lib.catopt_hip_affd_scan_workspace_bytes(T, S, nc, schedule)
        ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=dev)
        st = lib.catopt_hip_affd_scan(T, S, a.data_ptr(), S, u.data_ptr(), S, h0.data_ptr(), cs.data_ptr(), nc,
                                      schedule, states.data_ptr(), hf.data_ptr(), ws.data_ptr(), wsb, stream)
    L.check("catopt_hip_affd_scan_noalloc" if noalloc else "catopt_hip_affd_scan", st)
    torch.cuda.synchronize(dev)
    return states, hf


@pytest.mark.parametrize("schedule", [L.SCAN_CHUNKED, L.SCAN_AUTO, L.SCAN_STREAM])
def test_noalloc_matches_the_workspace_entry_twice(dev, schedule):
    lib = L.load()
    for T, S, n, seed in ((3000, 1200, 55, 1), (700, 300, 26, 2)):  # second call smaller
        a, u, h0 = _inputs(T, S, seed, dev)
        cs = _table(T, n).to(dev)
        nc = cs.numel() - 1
        ref_states, ref_hf = _run(lib, False, a, u, h0, cs, nc, schedule, dev)
        got_states, got_hf = _run(lib, True, a, u, h0, cs, nc, schedule, dev)
        assert torch.equal(got_states, ref_states) and torch.equal(got_hf, ref_hf), (T, S, schedule)
        serial = oracle.serial_affd_scan(a.cpu().double().numpy(), u.cpu().double().numpy(),
                                         h0.cpu().double().numpy())
        rep = oracle.verify_equiv(serial, got_states.cpu().double().numpy(), rtol=1e-5)
        assert rep["passed"], rep
        assert oracle.verify_equiv(serial[-1], got_hf.cpu().double().numpy(), rtol=1e-5)["passed"]


def test_noalloc_rejects_a_workspace_beyond_its_array(dev):
    lib = L.load()
    cap = lib.catopt_hip_affd_scan_noalloc_max_bytes()
    assert cap == 16 * 1024 * 1024
    # chunked workspace 2·S·n_chunks·4 B: S = 4096, 513 chunks -> 16.03 MiB > cap;
    # rejected on the host, before any device work (the pointers are never read)
    T, S, nc = 513, 4096, 513
    assert lib.catopt_hip_scan_workspace_bytes(S, nc) > cap
    cs = torch.arange(T + 1, dtype=torch.int64, device=dev)
    x = torch.zeros((T, S), device=dev)
    st = lib.catopt_hip_affd_scan_noalloc(T, S, x.data_ptr(), S, x.data_ptr(), S, None, cs.data_ptr(), nc,
                                          L.SCAN_CHUNKED, None, None, torch.cuda.current_stream(dev).cuda_stream)
    assert st == L.E_WORKSPACE
    # one chunk fewer fits (2·4096·512·4 B = 16 MiB exactly) and runs
    T2 = 512
    cs2 = torch.arange(T2 + 1, dtype=torch.int64, device=dev)
    a, u, h0 = _inputs(T2, S, 3, dev)
    got_states, got_hf = _run(lib, True, a, u, h0, cs2, T2, L.SCAN_CHUNKED, dev)
    ref_states, ref_hf = _run(lib, False, a, u, h0, cs2, T2, L.SCAN_CHUNKED, dev)
    assert torch.equal(got_states, ref_states) and torch.equal(got_hf, ref_hf)
    assert np.isfinite(got_hf.cpu().numpy()).all()


def test_noalloc_on_a_side_stream(dev):
    # the scratch address is resolved on the stream's device (here a stream
    # of default priority other than the current one)
    lib = L.load()
    side = torch.cuda.Stream(device=dev)
    T, S, n = 2000, 800, 40
    a, u, h0 = _inputs(T, S, 4, dev)
    cs = _table(T, n).to(dev)
    nc = cs.numel() - 1
    ref_states, ref_hf = _run(lib, False, a, u, h0, cs, nc, L.SCAN_CHUNKED, dev)
    got_states, got_hf = _run(lib, True, a, u, h0, cs, nc, L.SCAN_CHUNKED, dev, stream=side)
    assert torch.equal(got_states, ref_states) and torch.equal(got_hf, ref_hf)
