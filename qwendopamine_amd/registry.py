"""Block registry for the gdn2 mixer (reference ``models/blocks/registry.py:16-45``).

Only the gdn2 entries are provided: the other reference blocks (GDN-1, Qwen3.5
decoder layer, reward encoder) are outside this backend.
"""

from __future__ import annotations

from typing import Any

from torch import nn

from .gdn2 import GatedDeltaNet2

BLOCKS: dict[str, type] = {
    "gdn2": GatedDeltaNet2,
    "qwen35_gdn2": GatedDeltaNet2,
}


def build_block(block_type: str, config: Any, layer_idx: int) -> nn.Module:
    """Instantiate ``BLOCKS[block_type](config, layer_idx)``; ``KeyError`` for unknown names.

    The two arguments are passed positionally, as the reference does: for
    ``GatedDeltaNet2`` the layer index lands in the ``hidden_size`` slot, which
    the config branch overrides, so the module's ``layer_idx`` stays ``None``.
    """
    if block_type not in BLOCKS:
        raise KeyError(f"Unknown block type: {block_type}. Available: {list(BLOCKS)}")
    return BLOCKS[block_type](config, layer_idx)
