"""The graph runner on device inputs (GPU): catopt's capture cases
(tests/test_runners.py:209-234 of luisfuturist/catopt) with the stand-in
executor of ``tests/test_runner_cpu.py``, and a planned executor whose plan
declined (its own capture declines, so the runner reports no graph)."""

from __future__ import annotations

import pytest
import torch

from catopt_amd.executors import HipChunkedDecayModule
from catopt_amd.ir import IR, Op, TensorType, Var
from catopt_amd.ports import FailureClass
from catopt_amd.runner import HipGraphRunner
from tests.test_runner_cpu import Capturable

pytestmark = pytest.mark.gpu


def test_a_device_input_is_captured(dev):
    mod, stats = Capturable(), {}
    assert HipGraphRunner().apply(mod, torch.randn(2, 4, device=dev), stats) is mod
    assert stats["cuda_graph"] is True and mod.captured


def test_a_failed_capture_is_dropped_and_classified(dev):
    class Failing(Capturable):
        def capture_cuda_graph(self, *xs):
            raise RuntimeError("capture broke")

    mod, stats = Failing(), {}
    assert HipGraphRunner().apply(mod, torch.randn(2, 4, device=dev), stats) is mod
    assert stats["cuda_graph"] is False and mod.dropped
    assert stats["cuda_graph_failure"] is FailureClass.UNKNOWN


def test_a_declined_plan_reports_no_graph(dev):
    x = Var("x", TensorType((4,)))
    mod = HipChunkedDecayModule(IR(Op.make("relu", x), [x]), {})
    assert not mod.is_batched
    stats: dict = {}
    assert HipGraphRunner().apply(mod, torch.randn(4, device=dev), stats) is mod
    assert stats["cuda_graph"] is False and not mod.is_graph_captured
    assert torch.equal(mod(torch.full((4,), -1.0, device=dev)), torch.zeros(4, device=dev))
