"""The plug-in surface this package presents to catopt's orchestrator.

catopt routes an extracted term through its sink's executor table
(``Sink`` / ``ExecutorSpec`` / ``Binding`` / ``Executor`` ports,
luisfuturist/catopt ``packages/catopt-core/src/catopt_core/ports.py:189-605``).
Those ports are structural (``typing.Protocol``), so this module re-declares
the records with the same field names and meaning instead of importing them:

* :class:`ExecutorSpec` — ``(name, lower, accepts, engaged, carrier)``
  (ports.py:282-311); mapping order of ``Sink.executors`` is routing order.
* :class:`VerifyReport` — ``max_abs / max_rel / passed`` (ports.py:393-427,
  ``report.VerifyReport``).
* :class:`LowerResult` — ``(module, stats, verified)``
  (``catopt_core/pipeline.py:217``).
* :class:`FailureClass` / :func:`classify` — the failure buckets of
  ``catopt_core/failures.py:34-123`` that a delivery records instead of
  swallowing (graph-capture failures, kernel errors).
"""

from __future__ import annotations

import enum
import math
from dataclasses import dataclass, field
from typing import Any, Callable, Protocol, runtime_checkable

__all__ = [
    "Binding",
    "Executor",
    "ExecutorSpec",
    "VerifyReport",
    "LowerResult",
    "FailureClass",
    "classify",
]


@runtime_checkable
class Binding(Protocol):
    """One op's lowering: ``fn(*operand_values, **attrs)`` (ports.py:189-207)."""

    def __call__(self, *args: Any, **attrs: Any) -> Any: ...


@runtime_checkable
class Executor(Protocol):
    """A lowered module: ``forward(*xs)`` (ports.py:218-237)."""

    def forward(self, *xs: Any) -> Any: ...


@dataclass(frozen=True)
class ExecutorSpec:
    """One entry of ``Sink.executors`` (ports.py:282-311).

    ``lower(ir, params) -> Executor``; ``accepts(term) -> bool`` is the
    term-level probe the router asks; ``engaged(module) -> bool`` reports
    whether the built module took its planned (HIP) path; ``carrier`` names
    ``(root_ops, inner_ops, leaf_ops)`` or is ``None`` for the generic
    evaluator.
    """

    name: str
    lower: Callable
    accepts: Callable
    engaged: Callable
    carrier: Any = None


@dataclass(frozen=True)
class VerifyReport:
    """The verify gate's result (report.py:35-60)."""

    max_abs: float
    max_rel: float
    passed: bool
    per_output: tuple = ()


@dataclass
class LowerResult:
    """A delivered module, its stats and the verify outcome
    (pipeline.py:217-241); unpacks as ``(module, stats)``."""

    module: Any
    stats: dict = field(default_factory=dict)
    verified: Any = None

    def __iter__(self):
        yield self.module
        yield self.stats


class FailureClass(str, enum.Enum):
    """Failure buckets (failures.py:34-47); ``OK`` is the no-failure
    sentinel and :func:`classify` never returns it."""

    OK = "ok"
    OOM = "oom"
    TIMEOUT = "timeout"
    KERNEL = "kernel"
    NONFINITE = "nonfinite"
    UNAVAILABLE = "unavailable"
    UNKNOWN = "unknown"


def is_nonfinite(value: float) -> bool:
    """A NaN or infinite measurement (failures.py:125-135): the NONFINITE
    check a caller applies to a measured result."""
    return not math.isfinite(value)


def classify(exc: BaseException) -> FailureClass:
    """Bucket an exception with the precedence of failures.py:74-122, first
    match wins: a process-control signal is re-raised; ``MemoryError`` or an
    "out of memory" / "oom" message is OOM; ``TimeoutError`` or a "timed
    out" / "timeout" message is TIMEOUT; a message naming a device as
    unavailable is UNAVAILABLE (it outranks KERNEL, so "no CUDA device"
    reads as a feasibility gap); a "cuda" / "device-side" / "kernel"
    message is KERNEL; anything else UNKNOWN.  This library's own errors
    classify by type first: a missing or mismatched library is UNAVAILABLE,
    a failed entry point KERNEL; a HIP runtime error text ("hip error",
    "hiperror…") counts as a kernel message like a CUDA one."""
    from . import _lib

    if isinstance(exc, (KeyboardInterrupt, SystemExit)):
        raise exc
    if isinstance(exc, _lib.HipExtensionMissing):
        return FailureClass.UNAVAILABLE
    if isinstance(exc, _lib.HipKernelError):
        return FailureClass.KERNEL
    msg = str(exc).lower()
    if isinstance(exc, MemoryError) or "out of memory" in msg or "oom" in msg:
        return FailureClass.OOM
    if isinstance(exc, TimeoutError) or "timed out" in msg or "timeout" in msg:
        return FailureClass.TIMEOUT
    if "device" in msg and ("not available" in msg or "unavailable" in msg or "no cuda" in msg):
        return FailureClass.UNAVAILABLE
    if "cuda" in msg or "device-side" in msg or "kernel" in msg or "hip error" in msg or "hiperror" in msg:
        return FailureClass.KERNEL
    return FailureClass.UNKNOWN
