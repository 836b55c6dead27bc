"""MI355X-native execution backend of the gdn2 (GatedDeltaNet2) token mixer.

Kernel-level ops (``chunk_gdn2``, ``fused_recurrent_gdn2``) run hand-written
CDNA4 HIP kernels from ``libgdn2_hip.so`` through a C ABI.
"""

from .ops import ChunkGDN2Function, chunk_gdn2, fused_recurrent_gdn2, fused_recurrent_gdn2_fwd

__all__ = ["ChunkGDN2Function", "chunk_gdn2", "fused_recurrent_gdn2", "fused_recurrent_gdn2_fwd"]
