"""MI355X (gfx950) ChunkGatedDeltaRuleFwdH: the chunked gated delta-rule state recurrence.

Drop-in for the reference's FwdH operator path; see ``fwd_h`` for the two Python
signatures and ``include/cgdr_fwd_h.h`` for the C ABI they call.
"""

from .fwd_h import CHUNK_SIZE, chunk_gated_delta_rule_fwd_h, plan, run
from . import _abi

prepare_chunk_offsets = _abi.prepare_chunk_offsets
prepare_chunk_indices = _abi.prepare_chunk_indices

__all__ = [
    "CHUNK_SIZE",
    "chunk_gated_delta_rule_fwd_h",
    "run",
    "plan",
    "prepare_chunk_offsets",
    "prepare_chunk_indices",
]
