"""MI355X-native execution backend of the gdn2 (GatedDeltaNet2) token mixer.

* ``GatedDeltaNet2`` -- drop-in mixer module (reference constructor, forward
  and cache contract) whose recurrence runs on HIP kernels;
* ``chunk_gdn2`` / ``fused_recurrent_gdn2`` -- kernel-level ops mirroring the
  reference op signatures, backed by ``libgdn2_hip.so`` through a C ABI;
* ``BLOCKS`` / ``build_block`` -- the block-registry entries for gdn2.
"""

from .config import GDN2Config
from .gdn2 import GDN2_BACKENDS, GatedDeltaNet2, RMSNormGated, ShortConvolution, resolve_gdn2_backend
from .host import Block, GDN2Host
from .ops import ChunkGDN2Function, chunk_gdn2, fused_recurrent_gdn2, fused_recurrent_gdn2_fwd
from .registry import BLOCKS, build_block

__all__ = [
    "BLOCKS",
    "Block",
    "ChunkGDN2Function",
    "GDN2Config",
    "GDN2Host",
    "GDN2_BACKENDS",
    "GatedDeltaNet2",
    "RMSNormGated",
    "ShortConvolution",
    "build_block",
    "chunk_gdn2",
    "fused_recurrent_gdn2",
    "fused_recurrent_gdn2_fwd",
    "resolve_gdn2_backend",
]
