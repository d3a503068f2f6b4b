"""``HipSink``: the drop-in sink that lowers catopt's delivered terms to HIP.

It presents the reference's ``Sink`` port (luisfuturist/catopt
``packages/catopt-core/src/catopt_core/ports.py:557-605``), the surface
``TorchSink`` implements (``packages/catopt-torch/src/catopt_torch/adapters.py:56-284``):

* ``supported_ops`` — the op names this sink lowers (the extraction
  feasibility bound: anything outside prices at +inf, ports.py:522-554);
* ``ops`` — the binding registry (:class:`~catopt_amd.bindings.HipOpTable`);
* ``executors`` — the ordered ``ExecutorSpec`` table; mapping order is
  routing order and carrier executors precede the generic one
  (adapters.py:197-283 orders ``om_decayed_chunked, scan, om_batched,
  omd_batched, om_streaming, …, generic``);
* ``lower(ir, params)`` — the generic executor;
* ``verify(ref, opt, inputs, rtol, atol)`` — the global relative-error gate
  ``max|ref − out| / (max|ref| + 1e-8) < rtol`` (``report.py:128-207``).

Below the sink sit the orchestration steps of ``Optimizer.lower``
(``catopt_orchestrator/optimize.py:460-500, 2257-2415``), restated as plain
functions so a caller without the orchestrator can run them:
:func:`route_spec`, :func:`lower_extracted` and :func:`deliver`
(route → lower → runner → verify → ``LowerResult``).

The sink needs the HIP library: constructing one loads it and raises
:class:`~catopt_amd._lib.HipExtensionMissing` when it is absent.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Any, Mapping

import torch

from . import _lib as L
from .bindings import HipOpTable, torch_fallback_count
from .evaluator import HipIRModule
from .folds import specialize_causal
from .executors import (
    HipChunkedDecayModule,
    HipOMModule,
    HipOmdModule,
    HipScanModule,
    HipStreamingOMModule,
    is_decayed_term,
    is_om_term,
    is_omd_term,
    is_scan_term,
)
from .ir import IR
from .ports import ExecutorSpec, LowerResult, VerifyReport, classify
from .runner import IdentityRunner

__all__ = ["HipSink", "verify_equiv", "verify_module", "route_spec", "lower_extracted", "deliver"]

_REL_FLOOR = 1e-8


def _pair(ref: Any, out: Any, rtol: float, atol: float | None) -> VerifyReport:
    ref_t = torch.as_tensor(ref).detach()
    out_t = torch.as_tensor(out).detach().to(ref_t.device)
    diff = (ref_t.double() - out_t.double()).abs()
    max_abs = float(diff.max()) if diff.numel() else 0.0
    denom = float(ref_t.double().abs().max()) if ref_t.numel() else 0.0
    max_rel = max_abs / (denom + _REL_FLOOR)
    passed = bool(max_rel < rtol) and (atol is None or bool(max_abs <= atol))
    return VerifyReport(max_abs=max_abs, max_rel=max_rel, passed=passed)


def verify_equiv(ref: Any, out: Any, rtol: float = 1e-4, atol: float | None = None) -> VerifyReport:
    """``report.verify_equiv`` (report.py:143-165): NaN anywhere fails;
    tuple outputs are compared output by output (worst case reported)."""
    if isinstance(ref, (tuple, list)):
        reps = [_pair(r, o, rtol, atol) for r, o in zip(ref, out)]
        return VerifyReport(max_abs=max(r.max_abs for r in reps), max_rel=max(r.max_rel for r in reps),
                            passed=all(r.passed for r in reps) and len(ref) == len(out),
                            per_output=tuple(r.max_abs for r in reps))
    return _pair(ref, out, rtol, atol)


def verify_module(ref_mod: Any, opt_mod: Any, inputs: Any, rtol: float = 1e-4,
                  atol: float | None = None) -> VerifyReport:
    """Run both modules on clones of ``inputs`` under ``no_grad`` and compare
    (report.py:168-207)."""
    args = inputs if isinstance(inputs, tuple) else (inputs,)
    with torch.no_grad():
        ref = ref_mod(*[a.clone() if isinstance(a, torch.Tensor) else a for a in args])
        out = opt_mod(*[a.clone() if isinstance(a, torch.Tensor) else a for a in args])
        if isinstance(out, torch.Tensor):
            out = out.clone()  # a graph-replayed module returns its static buffer
    return verify_equiv(ref, out, rtol=rtol, atol=atol)


class HipSink:
    """The MI355X sink (module docstring).

    ``device`` is where lowered modules keep their parameters (default
    ``cuda:0``); ``ops`` replaces the binding table (the reference's
    ``TorchBackend(ops=…)`` seam, ops.py:338-389).
    """

    def __init__(self, device: Any = None, ops: HipOpTable | None = None) -> None:
        L.load()  # loud when the HIP library is missing: there is no CPU path
        self.device = torch.device(device) if device is not None else torch.device("cuda", 0)
        self._ops = ops if ops is not None else HipOpTable()

    # -- Capabilities ---------------------------------------------------------

    @property
    def supported_ops(self) -> frozenset:
        return frozenset(self._ops.torch_bindings)

    @property
    def ops(self) -> HipOpTable:
        return self._ops

    # -- Sink -------------------------------------------------------------------

    def lower(self, ir: IR, params: dict | None = None) -> HipIRModule:
        return HipIRModule(ir, params, ops=self._ops, device=self.device)

    def specialize_causal(self, term: Any, params: dict, memo: dict) -> Any:
        """The causal-mask const fold (``adapters.py:102-113``):
        ``sdpa(q, k, v, mask) → sdpa(q, k, v, arg5=True)`` where the
        parameter-only mask is the causal keep-mask, evaluated on this
        sink's device; ``memo["_hit"]`` records a rewrite."""
        return specialize_causal(term, params, memo, ops=self._ops, device=self.device)

    def verify(self, ref: Any, opt: Any, inputs: Any, *, rtol: float = 1e-4,
               atol: float | None = None) -> VerifyReport:
        return verify_module(ref, opt, inputs, rtol=rtol, atol=atol)

    @property
    def executors(self) -> Mapping[str, ExecutorSpec]:
        dev, ops = self.device, self._ops

        def planned(cls):
            return lambda ir, params=None: cls(ir, params, device=dev, ops=ops)

        return OrderedDict([
            ("om_decayed_chunked", ExecutorSpec(
                "om_decayed_chunked", planned(HipChunkedDecayModule), is_decayed_term,
                lambda m: bool(getattr(m, "is_batched", False)),
                (frozenset({"concat", "om_decayed"}),
                 frozenset({"add", "mul", "div", "matmul", "split", "transpose", "unsqueeze"}),
                 frozenset({"decay", "decay_vec"})))),
            ("scan", ExecutorSpec(
                "scan", planned(HipScanModule), is_scan_term,
                lambda m: bool(getattr(m, "is_batched", False)),
                (frozenset({"apply", "applyd"}),
                 frozenset({"aff_compose", "affd_compose", "stack", "aff_A", "aff_b", "affd_a", "affd_b"}),
                 frozenset({"aff", "aff_diag"})))),
            ("om_batched", ExecutorSpec(
                "om_batched", planned(HipOMModule), is_om_term,
                lambda m: bool(getattr(m, "is_batched", False)),
                (frozenset({"om_apply"}), frozenset({"om_compose"}), frozenset({"om", "om_elem"})))),
            ("omd_batched", ExecutorSpec(
                "omd_batched", planned(HipOmdModule), is_omd_term,
                lambda m: bool(getattr(m, "is_batched", False)),
                (frozenset({"omd_apply", "omd_applym"}), frozenset({"omd_compose"}),
                 frozenset({"omd", "omd_elem"})))),
            # after om_batched with the same acceptance, as in the reference:
            # never the routed choice, selectable by name
            ("om_streaming", ExecutorSpec(
                "om_streaming", planned(HipStreamingOMModule), is_om_term,
                lambda m: bool(getattr(m, "is_streaming", False)),
                (frozenset({"om_apply"}), frozenset({"om_compose"}), frozenset({"om", "om_elem"})))),
            ("generic", ExecutorSpec(
                "generic", lambda ir, params=None: self.lower(ir, params), lambda t: True,
                lambda m: True, None)),
        ])


# ------------------------------------------------------------- orchestration


def route_spec(term: Any, sink: Any) -> ExecutorSpec | None:
    """First carrier spec whose ``accepts`` holds (optimize.py:485-500)."""
    table = getattr(sink, "executors", None) or {}
    return next((s for s in table.values() if s.carrier is not None and s.accepts(term)), None)


def lower_extracted(term: Any, ir: IR, params: dict | None, sink: Any) -> Any:
    """Route ``term`` through the executor table, else ``sink.lower``
    (optimize.py:460-482)."""
    spec = route_spec(term, sink)
    if spec is not None:
        return spec.lower(ir, params)
    return sink.lower(ir, params)


def deliver(ir: IR, params: dict | None, sink: Any, example_inputs: Any = None, *,
            runner: Any = None, verify_ir: IR | None = None, rtol: float = 1e-4,
            atol: float | None = None) -> LowerResult:
    """Lower a delivered IR the way ``Optimizer.lower`` does
    (optimize.py:2257-2415): route to an executor, let ``runner`` wrap it
    (e.g. :class:`~catopt_amd.runner.HipGraphRunner`), and verify against
    ``verify_ir`` (the un-optimised program) lowered generically.

    ``stats`` carries the reference's keys — ``lowering`` ("batched" or
    "generic"), ``executor``, ``runner``, ``cuda_graph``,
    ``cuda_graph_failure`` — plus ``fallbacks`` (the planned executor's
    generic-path calls or leaves) and, with ``example_inputs``, the record of
    one counted eager call: ``hip_calls`` (HIP entry points it ran),
    ``torch_fallback_ops`` (HIP-backed bindings that took their torch device
    op) and ``hip_kernel`` (``hip_calls > 0``; without inputs, whether a
    planned executor engaged).
    """
    stats: dict = {}
    spec = route_spec(ir.root, sink)
    try:
        module = spec.lower(ir, params) if spec is not None else sink.lower(ir, params)
    except Exception as exc:
        stats["lower_failure"] = classify(exc)
        raise
    engaged = bool(getattr(module, "is_batched", False))
    stats["executor"] = spec.name if spec is not None else "generic"
    stats["lowering"] = "batched" if engaged else "generic"
    stats["hip_kernel"] = engaged
    if example_inputs is not None:
        # one eager call, counted: HIP entry points that ran, and HIP-backed
        # bindings that took their torch device op instead
        xs = example_inputs if isinstance(example_inputs, (tuple, list)) else (example_inputs,)
        n_hip, n_torch = L.call_count(), torch_fallback_count()
        with torch.no_grad():
            module(*xs)
        stats["hip_calls"] = L.call_count() - n_hip
        stats["torch_fallback_ops"] = torch_fallback_count() - n_torch
        stats["hip_kernel"] = stats["hip_calls"] > 0
    # the runner's name is recorded even when no input lets it run
    # (optimize.py:2340-2372: identity by default, the member names of a chain)
    if runner is None:
        runner = IdentityRunner()
    names = getattr(runner, "names", None)
    stats["runner"] = list(names) if names is not None else getattr(runner, "name", type(runner).__name__)
    if example_inputs is not None:
        module = runner.apply(module, example_inputs, stats)
    verified = None
    if verify_ir is not None and example_inputs is not None:
        ref = sink.lower(verify_ir, params)
        verified = sink.verify(ref, module, example_inputs, rtol=rtol, atol=atol)
        stats["verify_max_rel"] = verified.max_rel
    stats["fallbacks"] = int(getattr(module, "fallbacks", 0))
    return LowerResult(module=module, stats=stats, verified=verified)
