"""Planned HIP executors for the carrier forms catopt delivers."""

from .base import HipExecutorBase
from .decayed import HipChunkedDecayModule, build_decayed_plan, is_decayed_term
from .om import HipOMModule, build_om_plan, is_om_term
from .omd import HipOmdModule, build_omd_plan, is_omd_term, to_batched_omd_module
from .scan import HipScanModule, build_scan_plan, is_scan_term, prefix_chunk_table
from .stream import (HipStreamingOMModule, build_stream_plan, om_apply_state, om_empty_state, om_step,
                     om_step_qk, to_streaming_om_module)

__all__ = [
    "HipExecutorBase",
    "HipOMModule",
    "HipChunkedDecayModule",
    "HipScanModule",
    "HipOmdModule",
    "HipStreamingOMModule",
    "build_om_plan",
    "build_decayed_plan",
    "build_scan_plan",
    "build_stream_plan",
    "build_omd_plan",
    "is_omd_term",
    "to_batched_omd_module",
    "is_om_term",
    "is_decayed_term",
    "is_scan_term",
    "prefix_chunk_table",
    "om_apply_state",
    "om_empty_state",
    "om_step",
    "om_step_qk",
    "to_streaming_om_module",
]
