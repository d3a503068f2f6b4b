"""The graph runner's contract and the failure classifier (CPU).

Mirrors catopt's runner tests (tests/test_runners.py:162-255 of
luisfuturist/catopt) with the same stand-in executor, which records capture
and drop attempts: host inputs, a module without ``capture_cuda_graph``,
tuple and non-tensor inputs all degrade quietly to ``cuda_graph = False``;
an earlier compiling runner leaves capture unattempted; and the classifier
buckets failures with the reference's precedence (failures.py:74-122).
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from catopt_amd import _lib as L
from catopt_amd.ports import FailureClass, classify, is_nonfinite
from catopt_amd.runner import HipGraphRunner


class Capturable(nn.Module):
    """Stand-in planned executor: records capture / drop attempts."""

    def __init__(self) -> None:
        super().__init__()
        self.captured = False
        self.dropped = False

    def capture_cuda_graph(self, *xs: torch.Tensor) -> None:
        self.captured = True

    def drop_cuda_graph(self) -> None:
        self.dropped = True

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x


def test_host_input_degrades_quietly():
    mod, stats = Capturable(), {}
    assert HipGraphRunner().apply(mod, torch.randn(2, 4), stats) is mod
    assert stats["cuda_graph"] is False and not mod.captured


def test_a_module_without_capture_degrades_quietly():
    mod, stats = nn.Linear(4, 4), {}
    assert HipGraphRunner().apply(mod, torch.randn(2, 4), stats) is mod
    assert stats["cuda_graph"] is False


def test_tuple_and_non_tensor_inputs_degrade():
    mod = Capturable()
    for ex in ((torch.randn(2, 4),), ("not-a-tensor",), [], ()):
        stats: dict = {}
        assert HipGraphRunner().apply(mod, ex, stats) is mod
        assert stats["cuda_graph"] is False
    assert not mod.captured


def test_a_compiled_module_is_left_alone():
    mod, stats = Capturable(), {"compiled": True}
    assert HipGraphRunner().apply(mod, torch.randn(2, 4), stats) is mod
    assert "cuda_graph" not in stats and not mod.captured


def test_failure_classes_follow_the_reference_precedence():
    C = FailureClass
    assert classify(RuntimeError("CUDA out of memory")) is C.OOM
    assert classify(RuntimeError("OOM while allocating")) is C.OOM
    assert classify(MemoryError()) is C.OOM
    assert classify(TimeoutError()) is C.TIMEOUT
    assert classify(RuntimeError("operation timed out")) is C.TIMEOUT
    # unavailable outranks kernel: a missing device is a feasibility gap
    assert classify(RuntimeError("no CUDA device present")) is C.UNAVAILABLE
    assert classify(RuntimeError("device not available")) is C.UNAVAILABLE
    assert classify(RuntimeError("CUDA error: an illegal memory access")) is C.KERNEL
    assert classify(RuntimeError("device-side assert triggered")) is C.KERNEL
    assert classify(RuntimeError("HIP error: invalid device function")) is C.KERNEL
    assert classify(RuntimeError("capture broke")) is C.UNKNOWN
    assert classify(ValueError("shape mismatch")) is C.UNKNOWN
    # this library's own errors classify by type
    assert classify(L.HipExtensionMissing("x")) is C.UNAVAILABLE
    assert classify(L.HipKernelError("catopt_hip_linear", L.E_INVAL)) is C.KERNEL
    # process-control signals are re-raised, never classified
    with pytest.raises(KeyboardInterrupt):
        classify(KeyboardInterrupt())
    with pytest.raises(SystemExit):
        classify(SystemExit(1))
    assert is_nonfinite(float("nan")) and is_nonfinite(float("-inf")) and not is_nonfinite(1.0)


def test_delivery_records_its_runner_and_unpacks():
    # optimize.py:2340-2372 and pipeline.py:238-241: the runner's name is
    # always recorded (identity by default, member names for a chain), and
    # the result unpacks as (module, stats)
    from catopt_amd import forms
    from catopt_amd.runner import IdentityRunner
    from catopt_amd.sink import HipSink, deliver
    from tests.cpu_table import cpu_table

    sink = HipSink(device="cpu", ops=cpu_table())
    ir, _ = forms.scan_final_form(4, (2,))
    res = deliver(ir, {}, sink)
    mod, stats = res
    assert mod is res.module and stats is res.stats
    assert stats["runner"] == "identity" and stats["lowering"] == "batched"
    assert IdentityRunner().apply(mod, None, {}) is mod

    class Chain:
        names = ("identity", "hip_graph")

        def apply(self, module, x, stats):
            return module

    assert deliver(ir, {}, sink, runner=Chain()).stats["runner"] == ["identity", "hip_graph"]
    assert deliver(ir, {}, sink, runner=Capturable()).stats["runner"] == "Capturable"
