"""Shared machinery of the planned HIP executors.

The counterpart of ``BatchedExecutorBase`` (luisfuturist/catopt
``packages/catopt-torch/src/catopt_torch/executors/base.py:120-304``): the
``_plan`` / ``eval_mod`` fallback contract, the input environment, the
memoised leaf evaluator, a device/dtype-keyed constant cache, and HIP-graph
capture with the same ``capture_cuda_graph`` / ``drop_cuda_graph`` /
``is_graph_captured`` API (the name is the port's; on ROCm,
``torch.cuda.CUDAGraph`` records a hipGraph).

Capture rules: inputs must be device tensors; a call whose shapes, dtypes or
devices differ from the captured ones runs eagerly; parameters are baked in
by address; the returned tensor is the static output buffer, overwritten by
the next replay.  The HIP kernels launch on torch's current stream and make
no allocation of their own, so they record into the graph as plain kernel
nodes (no memset nodes: torch's fills are kernels).
"""

from __future__ import annotations

from typing import Any, Callable

import torch

from ..graphs import global_module_hooks, record_graph, signature
from ..ir import is_op

__all__ = ["HipExecutorBase"]


class HipExecutorBase:
    """Mixin: ``class X(HipExecutorBase, nn.Module)``.

    The concrete ``__init__`` sets ``_inputs``, ``eval_mod``, ``_plan`` and
    ``_const_cache``, then calls :meth:`_init_graph_state`; it supplies
    ``_forward_impl``.
    """

    _inputs: list
    _plan: dict | None
    eval_mod: Any
    _const_cache: dict
    _forward_impl: Callable

    def _init_graph_state(self) -> None:
        self._graph = None
        self._graph_inputs: list = []
        self._graph_out = None
        self._graph_sig = None

    @property
    def is_batched(self) -> bool:
        return self._plan is not None

    @property
    def is_graph_captured(self) -> bool:
        return self._graph is not None

    @property
    def _root(self) -> Any:
        return self.eval_mod._root

    @property
    def _param_map(self) -> dict:
        return self.eval_mod._param_map

    def capture_cuda_graph(self, *example_inputs: torch.Tensor, warmup: int = 3):
        """Record the planned forward into a hipGraph; returns ``self``.  A
        no-op without a device or without a plan; host inputs on a machine
        with a device raise ``ValueError`` (executors/base.py:180-220)."""
        if self._plan is None or not torch.cuda.is_available():
            return self
        self._graph, self._graph_inputs, self._graph_out, self._graph_sig = record_graph(
            self._forward_impl, example_inputs, warmup)
        return self

    def drop_cuda_graph(self) -> None:
        self._init_graph_state()

    def __call__(self, *xs: Any) -> Any:
        # skip nn.Module's hook dispatch when no hook is registered: it costs
        # microseconds per call, the order of a small step's kernels
        if self._forward_hooks or self._forward_pre_hooks or global_module_hooks():
            return super().__call__(*xs)
        return self.forward(*xs)

    def forward(self, *xs: Any) -> Any:
        if self._graph is not None and signature(xs) == self._graph_sig:
            for dst, src in zip(self._graph_inputs, xs):
                dst.copy_(src)
            self._graph.replay()
            return self._graph_out
        return self._forward_impl(*xs)

    # -- eval plumbing ---------------------------------------------------------

    def _input_env(self, xs: tuple) -> tuple[Any, dict]:
        x = xs[0] if xs else None
        env: dict = {"self": x}
        for i, inp in enumerate(self._inputs):
            env[inp.name] = xs[i] if i < len(xs) else x
        return x, env

    def ev_factory(self, env: dict, x: Any, memo: dict | None = None) -> Callable[[Any], Any]:
        """``ev(t)``: evaluate a leaf operand through ``eval_mod`` with a
        shared memo, so DAG-shared subterms run once per forward."""
        memo = {} if memo is None else memo
        eval_mod = self.eval_mod

        def ev(t: Any) -> Any:
            if is_op(t) and t in memo:
                return memo[t]
            return eval_mod._eval(t, env, x, memo)

        return ev

    def _cached(self, key: tuple, like: torch.Tensor, make: Callable, dtype: torch.dtype | None = None):
        want = dtype or like.dtype
        t = self._const_cache.get(key)
        if t is None or t.device != like.device or t.dtype != want:
            t = make(like)
            self._const_cache[key] = t
        return t
