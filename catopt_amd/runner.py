"""``HipGraphRunner``: record a delivered executor into a hipGraph.

The ROCm counterpart of ``CudaGraphRunner`` (luisfuturist/catopt
``packages/catopt-cuda/src/catopt_cuda/runners.py:37-89``), conforming to the
``Runner`` port: ``apply(module, example_input, stats) -> module``.

* Only planned executors expose ``capture_cuda_graph``; the generic module
  degrades quietly (``stats["cuda_graph"] = False``).
* A capture that raises is classified (``FailureClass``) into
  ``stats["cuda_graph_failure"]`` and the partial graph is dropped, so
  delivery continues eagerly.
* ``stats["compiled"]`` set means another runner already owns the module:
  capture is skipped.

Replay collapses a form's launches (for the weight chain: one GEMM plus the
Python dispatch around it) into one graph launch.
"""

from __future__ import annotations

from typing import Any

import torch

from .ports import classify

__all__ = ["HipGraphRunner", "IdentityRunner"]


class IdentityRunner:
    """The default delivery: the routed executor as it is."""

    name = "identity"

    def apply(self, module: torch.nn.Module, example_input: Any, stats: dict) -> torch.nn.Module:
        return module


class HipGraphRunner:
    name = "hip_graph"

    def apply(self, module: torch.nn.Module, example_input: Any, stats: dict) -> torch.nn.Module:
        if stats.get("compiled"):
            return module
        stats["cuda_graph"] = False
        xs = tuple(example_input) if isinstance(example_input, (tuple, list)) else (example_input,)
        capture = getattr(module, "capture_cuda_graph", None)
        # the capture copies every input into a static device buffer, so all
        # of them (not only the first, as runners.py:66-72 checks) must be
        # device tensors; a planned executor whose plan is None declines
        # inside its own capture_cuda_graph
        if capture is None or not xs or not all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in xs):
            return module
        try:
            capture(*xs)
            # a module reporting its capture state is taken at its report
            stats["cuda_graph"] = bool(getattr(module, "is_graph_captured", True))
        except Exception as exc:
            stats["cuda_graph_failure"] = classify(exc)
            module.drop_cuda_graph()
        return module
