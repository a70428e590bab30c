"""MI355X (gfx950) ChunkGatedDeltaRuleFwdH: the chunked gated delta-rule state recurrence.

Drop-in for the reference's FwdH operator path; see ``fwd_h`` for the two Python
signatures and ``include/cgdr_fwd_h.h`` for the C ABI they call.  ``chunk_o`` is the
chunk output built on FwdH's h and v_new (``include/cgdr_chunk_o.h``), ``wy`` the producer
of FwdH's w, u and g (``include/cgdr_wy.h``) and the full chunked forward built from the three.
"""

from .fwd_h import CHUNK_SIZE, chunk_gated_delta_rule_fwd_h, plan, run
from .chunk_o import chunk_fwd_o
from .wy import chunk_gated_delta_rule_fwd, wy_fwd
from . import _abi

prepare_chunk_offsets = _abi.prepare_chunk_offsets
prepare_chunk_indices = _abi.prepare_chunk_indices

__all__ = [
    "CHUNK_SIZE",
    "chunk_gated_delta_rule_fwd_h",
    "chunk_fwd_o",
    "wy_fwd",
    "chunk_gated_delta_rule_fwd",
    "run",
    "plan",
    "prepare_chunk_offsets",
    "prepare_chunk_indices",
]
