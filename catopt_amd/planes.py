"""Mask and bias planes for the attention kernel's mask modes.

The kernel takes one ``(Tq, Tk)`` plane shared over the batch and head axes.
A mask term's value can be smaller than the score it masks: torch
broadcasts a ``(…, 1, Tk)`` key-padding mask or a ``(Tq, 1)`` row mask over
the missing extent.  These helpers find the one plane a tensor holds over its
leading axes and fit it to the score's ``(Tq, Tk)`` at call time, so a plane
with one query row is never read as a ``Tq``-row pattern.

Sharing over the leading axes is decided from shape and strides where they
settle it (every leading axis of extent 1 or stride 0, as ``expand`` gives).
Otherwise the planes are compared by value, which reads the tensor on the
host, so the comparison is skipped while a stream is being captured into a
graph (the caller then takes its score path).
"""
from __future__ import annotations

import torch

__all__ = ["fit_plane", "shared_plane"]


def _capturing() -> bool:
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def shared_plane(t: torch.Tensor, *, compare: bool = True) -> torch.Tensor | None:
    """The one plane (its last two axes) ``t`` holds over its leading axes,
    as a view; ``None`` when they may carry different planes.  NaN entries
    count as equal."""
    if not isinstance(t, torch.Tensor) or t.dim() < 2:
        return None
    lead = t.dim() - 2
    if all(t.shape[i] == 1 or t.stride(i) == 0 for i in range(lead)):
        return t[(0,) * lead]
    if not compare or _capturing():
        return None
    t3 = t.reshape(-1, *t.shape[-2:])
    first = t3[:1]
    same = t3 == first
    if t3.is_floating_point():
        same = same | (t3.isnan() & first.isnan())
    return t3[0] if bool(same.all()) else None


def fit_plane(plane: torch.Tensor, tq: int, tk: int) -> torch.Tensor | None:
    """``plane`` as a contiguous ``(tq, tk)`` plane, broadcast as torch
    broadcasts a mask against its score; ``None`` when it does not broadcast
    to exactly that shape."""
    if plane.dim() != 2:
        return None
    if tuple(plane.shape) == (tq, tk):
        return plane.contiguous()
    try:
        shape = torch.broadcast_shapes(tuple(plane.shape), (tq, tk))
    except RuntimeError:
        return None
    if tuple(shape) != (tq, tk):
        return None
    return plane.expand(tq, tk).contiguous()
