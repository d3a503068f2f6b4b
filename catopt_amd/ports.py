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
    """A delivered module, its stats and the verify outcome (pipeline.py:217)."""

    module: Any
    stats: dict = field(default_factory=dict)
    verified: Any = None


class FailureClass(str, enum.Enum):
    """Failure buckets (failures.py:34-60)."""

    OOM = "oom"
    TIMEOUT = "timeout"
    KERNEL = "kernel"
    NONFINITE = "nonfinite"
    UNAVAILABLE = "unavailable"
    UNKNOWN = "unknown"


def classify(exc: BaseException) -> FailureClass:
    """Bucket an exception the way failures.py:62-123 does."""
    from . import _lib

    if isinstance(exc, _lib.HipExtensionMissing):
        return FailureClass.UNAVAILABLE
    if isinstance(exc, _lib.HipKernelError):
        return FailureClass.KERNEL
    if isinstance(exc, MemoryError):
        return FailureClass.OOM
    if isinstance(exc, TimeoutError):
        return FailureClass.TIMEOUT
    text = f"{type(exc).__name__}: {exc}".lower()
    if "out of memory" in text or "outofmemory" in text:
        return FailureClass.OOM
    if "timed out" in text or "timeout" in text:
        return FailureClass.TIMEOUT
    if "nan" in text and "finite" in text:
        return FailureClass.NONFINITE
    if "hip" in text or "cuda" in text or "kernel" in text:
        return FailureClass.KERNEL
    if "not available" in text or "unavailable" in text:
        return FailureClass.UNAVAILABLE
    return FailureClass.UNKNOWN
