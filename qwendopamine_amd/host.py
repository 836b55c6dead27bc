"""Minimal all-gdn2 decoder host (reference ``models/gdn2/host.py:24-84``).

Embedding -> N x (RMSNorm -> GatedDeltaNet2 + residual) -> RMSNorm -> LM head.
Used to exercise the mixer's cache plumbing inside a model.
"""

from __future__ import annotations

from typing import Any

import torch
from torch import nn

from .config import GDN2Config
from .gdn2 import GatedDeltaNet2


class RMSNorm(nn.Module):
    """``weight * x * rsqrt(mean(x^2) + eps)`` (reference ``models/normalization.py:9-50``)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps

    def reset_parameters(self) -> None:
        nn.init.ones_(self.weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps))


class Block(nn.Module):
    """Pre-norm residual block around one ``GatedDeltaNet2``."""

    def __init__(self, config: GDN2Config, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.norm = RMSNorm(config.hidden_size, eps=config.norm_eps)
        self.attn = GatedDeltaNet2(config, layer_idx=layer_idx)

    def forward(self, x: torch.Tensor, past_key_values: Any | None = None, use_cache: bool = False):
        out, _, past_key_values = self.attn(self.norm(x), past_key_values=past_key_values,
                                            use_cache=use_cache)
        return x + out, past_key_values


class GDN2Host(nn.Module):
    """GPT-style decoder of gdn2 blocks only."""

    def __init__(self, config: GDN2Config) -> None:
        super().__init__()
        self.config = config
        self.embed = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([Block(config, i) for i in range(getattr(config, "num_layers", 24))])
        self.norm = RMSNorm(config.hidden_size, eps=config.norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.apply(self._init_weights)

    def _init_weights(self, module: nn.Module) -> None:
        if getattr(module, "_is_hf_initialized", False):
            return
        if isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=0.02)
        elif isinstance(module, nn.Linear):
            nn.init.xavier_uniform_(module.weight, gain=2**-2.5)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, RMSNorm):
            module.reset_parameters()
        module._is_hf_initialized = True

    def forward(self, input_ids: torch.Tensor, past_key_values: Any | None = None):
        x = self.embed(input_ids)
        for layer in self.layers:
            x, past_key_values = layer(x, past_key_values=past_key_values)
        return self.lm_head(self.norm(x)), past_key_values


__all__ = ["Block", "GDN2Host", "RMSNorm"]
