"""Planned HIP executors for the carrier forms catopt delivers."""

from .base import HipExecutorBase
from .decayed import (HipChunkedDecayModule, build_decayed_plan, is_decayed_chunked_term, is_decayed_term,
                      to_chunked_decayed_module)
from .om import HipOMModule, build_om_plan, is_om_apply_term, is_om_term, to_batched_om_module
from .omd import HipOmdModule, build_omd_plan, is_omd_apply_term, is_omd_term, to_batched_omd_module
from .scan import (HipScanModule, build_scan_plan, is_scan_apply_term, is_scan_term, prefix_chunk_table,
                   to_batched_scan_module)
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
    # the reference's constructor and probe names
    "to_batched_om_module",
    "to_batched_scan_module",
    "to_chunked_decayed_module",
    "is_om_apply_term",
    "is_scan_apply_term",
    "is_omd_apply_term",
    "is_decayed_chunked_term",
]
