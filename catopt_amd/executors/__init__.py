"""Planned HIP executors for the carrier forms catopt delivers."""

from .base import HipExecutorBase
from .decayed import HipChunkedDecayModule, build_decayed_plan, is_decayed_term
from .om import HipOMModule, build_om_plan, is_om_term
from .scan import HipScanModule, build_scan_plan, is_scan_term, prefix_chunk_table

__all__ = [
    "HipExecutorBase",
    "HipOMModule",
    "HipChunkedDecayModule",
    "HipScanModule",
    "build_om_plan",
    "build_decayed_plan",
    "build_scan_plan",
    "is_om_term",
    "is_decayed_term",
    "is_scan_term",
    "prefix_chunk_table",
]
