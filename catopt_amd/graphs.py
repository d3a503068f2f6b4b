"""hipGraph recording shared by the executors (``torch.cuda.CUDAGraph``
records a hipGraph on ROCm)."""

from __future__ import annotations

from typing import Callable

import torch

__all__ = ["global_module_hooks", "record_graph", "signature"]


def signature(xs: tuple) -> tuple:
    """Shape/dtype/device/stride key of a call's inputs (graph replay guard)."""
    return tuple((tuple(t.shape), t.dtype, t.device, tuple(t.stride())) if isinstance(t, torch.Tensor)
                 else (type(t), t) for t in xs)


def record_graph(fn: Callable, example_inputs: tuple, warmup: int = 3) -> tuple:
    """Warm ``fn`` up on a side stream, then record one call into a graph.

    Returns ``(graph, static_inputs, static_output, signature)``."""
    if not all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in example_inputs):
        raise ValueError("graph capture requires device inputs (CUDA/HIP tensors)")
    static_ins = [t.detach().clone() for t in example_inputs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(1, warmup)):
            fn(*static_ins)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn(*static_ins)
    return g, static_ins, out, signature(tuple(static_ins))


def global_module_hooks() -> bool:
    """Whether any process-wide nn.Module hook is registered (the executors
    then take nn.Module's full call path, so the hooks run)."""
    m = torch.nn.modules.module
    return bool(m._global_forward_hooks or m._global_forward_pre_hooks or m._global_backward_hooks
                or m._global_backward_pre_hooks or getattr(m, "_global_forward_hooks_always_called", None))
