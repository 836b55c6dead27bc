"""Hybrid gdn2 / softmax-attention decoder with streaming caches (the config-3 host).

The layer stack, parameter names and initialisation follow the reference's
lit-gpt style ``GDN2GPT`` (``models/gdn2_gpt/model.py:176-430``, presets
``config.py:9-114``): token embedding ``wte``, blocks ``h.<i>`` of
``norm_1 -> mixer -> residual -> norm_2 -> SwiGLU -> residual``, then ``ln_f`` and an
untied ``lm_head``. A state dict of the reference model loads into this one.

What differs from the reference host, deliberately:

* **Streaming gdn2 state.** ``GDN2GPT`` calls its gdn2 mixers without a cache
  (``model.py:232``), so its incremental decode restarts every gdn2 layer from a
  zero state. Here each gdn2 layer owns the reference cache dict
  (``{"recurrent_state", "conv_state"}``, ``gdn2.py:698-701``) and decode continues the
  prefill's recurrence exactly.
* **Attention KV caches** are kept in the model dtype (the reference allocates them
  in the default dtype, ``model.py:421-424``), at a fixed ``max_seq_length``; decode
  masks the unused tail.
* **Decode as one HIP graph.** ``GreedyDecoder`` captures a whole decode step
  (embedding, 24 layers, LM head, argmax, position update) once and replays it;
  the gdn2 caches are refreshed in place at the end of every step, so replays
  advance the recurrence.
* **Fused elementwise passes** (inference on the GPU). Each residual add runs with the
  RMSNorm that reads its result (``ops.add_rms_norm``), and SwiGLU's ``silu(a) * b``
  is one pass (``ops.silu_mul``); both round as the torch ops they replace, and the
  logits are bit-identical to the unfused host's.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
from torch import nn
from torch.nn import functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import ops
from ._stacked import drop, stacked_rows
from .gdn2 import GatedDeltaNet2, _inference


@dataclass
class HybridConfig:
    """Field names and meanings of the reference ``GDN2GPTConfig`` (``config.py:9-48``)."""

    name: str = "c3"
    block_size: int = 4096
    vocab_size: int = 151936
    padded_vocab_size: int | None = None
    n_layer: int = 24
    n_head: int = 16
    n_embd: int = 1024
    head_size: int = 64
    n_query_groups: int = 16
    intermediate_size: int = 3072
    norm_eps: float = 1e-5
    bias: bool = False
    rotary_percentage: float = 1.0
    rope_base: float = 10000.0
    condense_ratio: float = 1.0
    gdn2_layers: list[int] | None = field(default=None)
    gdn2_per_layer: int = 0
    conv_size: int = 4
    expand_v: float = 1.0
    use_short_conv: bool = True
    chunk_size: int = 64
    allow_neg_eigval: bool = False
    backend: str = "auto"
    fp32_decay: bool = True

    def __post_init__(self) -> None:
        if self.padded_vocab_size is None:
            self.padded_vocab_size = self.vocab_size

    @classmethod
    def c3(cls, **kwargs) -> "HybridConfig":
        """The benchmark's config 3: 24 layers, three gdn2 layers then one attention
        layer, hidden 1024, 16 heads x 64, SwiGLU 3072, vocab 151936 (about 0.68 B
        parameters)."""
        base = dict(gdn2_layers=[i for i in range(24) if i % 4 != 3])
        base.update(kwargs)
        return cls(**base)

    def is_gdn2(self, layer_idx: int) -> bool:
        """Layer selection of the reference ``Block`` (``model.py:184-189``)."""
        if self.gdn2_layers is not None:
            return layer_idx in self.gdn2_layers
        if self.gdn2_per_layer > 0:
            return layer_idx % self.gdn2_per_layer == 0
        return layer_idx == self.n_layer // 2


def build_rope_cache(seq_len: int, n_elem: int, device, base: float = 10000.0,
                     condense_ratio: float = 1.0) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos / sin tables ``[seq_len, n_elem / 2]`` (reference ``model.py:20-37``)."""
    theta = 1.0 / (base ** (torch.arange(0, n_elem, 2, device=device, dtype=torch.float32) / n_elem))
    pos = torch.arange(seq_len, device=device, dtype=torch.float32) / condense_ratio
    ang = torch.outer(pos, theta)
    return torch.cos(ang), torch.sin(ang)


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Interleaved-pair rotation of the first ``2 * cos.shape[-1]`` channels of
    ``x [B, T, heads, D]``, in fp32, result in ``x``'s dtype (reference ``model.py:40-61``)."""
    rot = 2 * cos.shape[-1]
    xf = x.float()
    if rot == x.shape[-1] and x.shape[1] == 1:
        # Single-token (decode) calls are bound by launches: the pair rotation
        # (x1 c - x2 s, x1 s + x2 c) is the complex product of x1 + i x2 with
        # c + i s, three launches instead of about ten.  Long prefills keep the
        # real form (torch's broadcast complex product measured slower there).
        xc = torch.view_as_complex(xf.contiguous().view(*x.shape[:-1], rot // 2, 2))
        rc = torch.complex(cos.float(), sin.float())[None, :, None, :]
        return torch.view_as_real(xc * rc).flatten(-2).to(x.dtype)
    x1, x2 = xf[..., :rot:2], xf[..., 1:rot:2]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    y = torch.stack((x1 * c - x2 * s, x1 * s + x2 * c), dim=-1).flatten(-2)
    y = torch.cat((y, xf[..., rot:]), dim=-1)
    return y.to(x.dtype)


class RMSNorm(nn.Module):
    """``weight * x * rsqrt(mean(x^2) + eps)`` in the input dtype (reference
    ``models/normalization.py:40-51``)."""

    def __init__(self, size: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _inference(x, self.weight):
            # One HIP pass with the same per-op rounding (six torch launches otherwise).
            return ops.rms_norm(x, self.weight, self.eps)
        return self.weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps))


class SwiGLU(nn.Module):
    """``w3(silu(w1 x) * w2 x)`` (reference ``model.py:64-78``)."""

    def __init__(self, n_embd: int, hidden: int, bias: bool = False) -> None:
        super().__init__()
        self.w1 = nn.Linear(n_embd, hidden, bias=bias)
        self.w2 = nn.Linear(n_embd, hidden, bias=bias)
        self.w3 = nn.Linear(hidden, n_embd, bias=bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if torch.is_grad_enabled() and any(t.requires_grad for t in (x, self.w1.weight, self.w2.weight)):
            return self.w3(F.silu(self.w1(x)) * self.w2(x))
        # Inference: w1 and w2 as one GEMM (the same dot products, one launch).
        ab = ops.linear(x, *self._fused12())
        if ab.is_cuda:
            # silu(a) * b in one HIP pass with torch's roundings (three launches otherwise).
            return ops.linear(ops.silu_mul(ab), self.w3.weight, self.w3.bias)
        a, b = ab.chunk(2, dim=-1)
        return self.w3(F.silu(a) * b)

    def _fused12(self) -> tuple[torch.Tensor, torch.Tensor | None]:
        """[w1; w2] weights (and biases) as one tensor each; w1 and w2 are row views of it."""
        w = stacked_rows(self, "_cache12", [self.w1.weight, self.w2.weight])
        bias = None if self.w1.bias is None else stacked_rows(self, "_cache12b", [self.w1.bias, self.w2.bias])
        return w, bias

    def _apply(self, fn, *args, **kwargs):
        drop(self, "_cache12", "_cache12b")
        return super()._apply(fn, *args, **kwargs)


class LLaMAMLP(nn.Module):
    def __init__(self, config: HybridConfig) -> None:
        super().__init__()
        self.swiglu = SwiGLU(config.n_embd, config.intermediate_size, bias=config.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.swiglu(x)


class CausalSelfAttention(nn.Module):
    """Grouped-query attention with RoPE and a static KV cache (reference ``model.py:89-173``):
    fused ``attn`` projection laid out ``[groups, q_per_kv + 2, head_size]``, output ``proj``.

    The cache is ``[B, groups, max_seq_length, head_size]`` per tensor. A multi-token
    cached call is a prefill from position 0: it attends within its own tokens
    (causal SDPA, flash or memory-efficient kernels only) and stores k, v. A single-token
    call attends over the cache up to its position; its products are issued with
    contiguous right operands."""

    def __init__(self, config: HybridConfig, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_size, self.n_head, self.n_query_groups = config.head_size, config.n_head, config.n_query_groups
        if self.n_head % self.n_query_groups != 0:
            raise ValueError(f"n_head ({self.n_head}) must be divisible by n_query_groups ({self.n_query_groups}).")
        self.attn = nn.Linear(config.n_embd, (self.n_head + 2 * self.n_query_groups) * self.head_size,
                              bias=config.bias)
        self.proj = nn.Linear(self.n_head * self.head_size, config.n_embd, bias=config.bias)
        self.kv_cache: tuple[torch.Tensor, torch.Tensor] | None = None

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                input_pos: torch.Tensor | None = None, mask: torch.Tensor | None = None) -> torch.Tensor:
        return self.forward_qkv(ops.linear(x, self.attn.weight, self.attn.bias), cos, sin, input_pos, mask)

    def forward_qkv(self, qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    input_pos: torch.Tensor | None = None, mask: torch.Tensor | None = None) -> torch.Tensor:
        """``forward`` from the fused ``attn`` projection's output ``[B, T, (n_head + 2 G) D]``."""
        b, t, _ = qkv.shape
        G, qpk, D = self.n_query_groups, self.n_head // self.n_query_groups, self.head_size
        if (t == 1 and input_pos is not None and self.kv_cache is not None and _inference(qkv)
                and ops.attention_decode_supported(qkv, qpk, D)):
            # RoPE, the cache store and the attention of the token in one HIP launch.
            o = ops.attention_decode(qkv, cos, sin, input_pos, *self.kv_cache, self.n_head)
            return ops.linear(o.reshape(b, 1, self.n_head * D), self.proj.weight, self.proj.bias)
        if input_pos is not None and cos.shape[0] != t:
            # Whole rotation tables without a mask: the caller expected the fused decode
            # launch above, which this call cannot take (its predicate reads the weights,
            # this one the projection output).  Select the rows of input_pos and build the
            # causal mask over the cache here.
            cos, sin = cos.index_select(0, input_pos), sin.index_select(0, input_pos)
            if mask is None and self.kv_cache is not None:
                L = self.kv_cache[0].shape[2]
                mask = (torch.arange(L, device=qkv.device)[None, :] <= input_pos[:, None]).reshape(1, 1, t, L)
        qkv = qkv.view(b, t, G, qpk + 2, D)
        q, k, v = qkv.split((qpk, 1, 1), dim=-2)
        q = apply_rotary_emb(q.reshape(b, t, self.n_head, D), cos, sin)
        k = apply_rotary_emb(k.reshape(b, t, G, D), cos, sin)
        v = v.reshape(b, t, G, D)
        if input_pos is not None:
            if self.kv_cache is None:
                raise RuntimeError("KV cache not set up: call HybridDecoder.setup_caches first")
            ck, cv = self.kv_cache
            ck.index_copy_(2, input_pos, k.transpose(1, 2))
            cv.index_copy_(2, input_pos, v.transpose(1, 2))
            if t == 1:
                return ops.linear(self._decode(q, ck, cv, mask).reshape(b, 1, self.n_head * D), self.proj.weight,
                                  self.proj.bias)
        q, k, v = (z.transpose(1, 2) for z in (q, k, v))
        if qpk > 1:
            k, v = k.repeat_interleave(qpk, dim=1), v.repeat_interleave(qpk, dim=1)
        # No math fallback in 16-bit: it multiplies by a transposed key view.
        backends = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]
        if q.dtype == torch.float32:
            backends.append(SDPBackend.MATH)
        with sdpa_kernel(backends):
            o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.proj(o.transpose(1, 2).reshape(b, t, self.n_head * D))

    def _decode(self, q: torch.Tensor, ck: torch.Tensor, cv: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        """Softmax attention of one token ``q [B, 1, heads, D]`` over the cache; ``mask``
        ``[1, 1, 1, L]`` marks the valid positions. Returns ``[B, heads, D]``."""
        b, G, L, D = ck.shape
        qpk = self.n_head // G
        qt = q.reshape(b, G, qpk, D).transpose(-1, -2).contiguous()            # [B, G, D, qpk]
        s = torch.matmul(ck, qt).float() * (1.0 / math.sqrt(D))               # [B, G, L, qpk]
        s = s.masked_fill(~mask.reshape(1, 1, L, 1), float("-inf"))
        pt = torch.softmax(s, dim=2).to(cv.dtype).transpose(-1, -2).contiguous()  # [B, G, qpk, L]
        return torch.matmul(pt, cv).reshape(b, self.n_head, D)


class Block(nn.Module):
    """Pre-norm residual block: gdn2 or attention mixer, then SwiGLU (reference ``model.py:176-248``)."""

    def __init__(self, config: HybridConfig, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.use_gdn2 = config.is_gdn2(layer_idx)
        self.norm_1 = RMSNorm(config.n_embd, eps=config.norm_eps)
        if self.use_gdn2:
            self.attn = GatedDeltaNet2(
                hidden_size=config.n_embd, num_heads=config.n_head, head_dim=config.head_size,
                num_v_heads=config.n_head, layer_idx=layer_idx, norm_eps=config.norm_eps,
                conv_size=config.conv_size, expand_v=config.expand_v, use_short_conv=config.use_short_conv,
                chunk_size=config.chunk_size, allow_neg_eigval=config.allow_neg_eigval,
                backend=config.backend, fp32_decay=config.fp32_decay,
            )
        else:
            self.attn = CausalSelfAttention(config, layer_idx)
        self.norm_2 = RMSNorm(config.n_embd, eps=config.norm_eps)
        self.mlp = LLaMAMLP(config)
        # gdn2 layers: the reference cache dict of this layer (None until a
        # cached forward has run).
        self.gdn2_cache: dict | None = None

    def forward(self, x: torch.Tensor, cos, sin, input_pos=None, mask=None) -> torch.Tensor:
        n1 = self.norm_1(x)
        h = self._mix(n1, cos, sin, input_pos, mask)
        x = x + h
        return x + self.mlp(self.norm_2(x))

    def forward_pending(self, x: torch.Tensor, pending: torch.Tensor | None, cos, sin, input_pos=None,
                        mask=None) -> tuple[torch.Tensor, torch.Tensor]:
        """``forward`` with its last residual add left to the caller: returns ``(x', m)``
        such that ``forward`` would return ``x' + m``, and takes the previous block's
        pending ``m`` (or None).  Each residual add then runs in one HIP pass with the
        norm that reads its result (``ops.add_rms_norm``, bit-identical to the add and
        the norm apart).  Inference on GPU tensors only."""
        decode_rows = x.shape[0] * x.shape[1] <= 4
        fused = None
        if (pending is not None and decode_rows and self.use_gdn2 and input_pos is not None
                and self.gdn2_cache is not None and x.shape[1] == 1):
            # gdn2 layer's decode step: the add and norm_1 formed while the mixer's
            # input projections stage their input (one launch less, the same bits).
            step = dict(self.gdn2_cache)
            fused = self.attn.decode_step_from_residual(x, pending, self.norm_1.weight, self.norm_1.eps, step)
            if fused is not None:
                self._keep_cache(step)
        if fused is not None:
            x, h = fused
        elif pending is None:
            h = self._mix(self.norm_1(x), cos, sin, input_pos, mask)
        elif decode_rows and not self.use_gdn2 and input_pos is not None:
            # Attention layer on decode-sized rows: the add and norm_1 formed while
            # the qkv product stages its input (one launch less, the same bits).
            at = self.attn
            qkv, x = ops.linear_addnorm(x, pending, self.norm_1.weight, self.norm_1.eps, at.attn.weight, at.attn.bias)
            h = at.forward_qkv(qkv, cos, sin, input_pos, mask)
        else:
            x, n1 = ops.add_rms_norm(x, pending, self.norm_1.weight, self.norm_1.eps)
            h = self._mix(n1, cos, sin, input_pos, mask)
        if decode_rows:
            # Decode-sized rows: the add and norm_2 formed while SwiGLU's w1 / w2
            # product stages its input (one launch less, the same bits).
            sw = self.mlp.swiglu
            gated, x = ops.linear_addnorm(x, h, self.norm_2.weight, self.norm_2.eps, *sw._fused12(), swiglu=True)
            return x, ops.linear(gated, sw.w3.weight, sw.w3.bias)
        x, n2 = ops.add_rms_norm(x, h, self.norm_2.weight, self.norm_2.eps)
        return x, self.mlp(n2)

    def _mix(self, n1: torch.Tensor, cos, sin, input_pos, mask) -> torch.Tensor:
        if self.use_gdn2:
            if input_pos is None:
                h, _, _ = self.attn(n1)
                return h
            return self._gdn2_cached(n1)
        return self.attn(n1, cos, sin, input_pos, mask)

    def _gdn2_cached(self, x: torch.Tensor) -> torch.Tensor:
        """Run the mixer on this layer's cache. Once the cache exists, its tensors are
        updated in place (the mixer returns fresh ones), so that their addresses stay
        fixed across decode steps and a captured step can be replayed."""
        if self.gdn2_cache is None:
            cache: dict = {}
            h, _, cache = self.attn(x, past_key_values=cache, use_cache=True)
            self.gdn2_cache = cache
            return h
        step = dict(self.gdn2_cache)
        h, _, step = self.attn(x, past_key_values=step, use_cache=True, update_cache_in_place=True)
        self._keep_cache(step)
        return h

    def _keep_cache(self, step: dict) -> None:
        """Decode steps update the cache where it lies; other calls return fresh tensors,
        which are copied into the cache's own (so its addresses stay fixed)."""
        if step["recurrent_state"] is not self.gdn2_cache["recurrent_state"]:
            self.gdn2_cache["recurrent_state"].copy_(step["recurrent_state"])
        for dst, src in zip(self.gdn2_cache["conv_state"], step["conv_state"]):
            if src is not dst:
                dst.copy_(src)


class HybridDecoder(nn.Module):
    """The reference ``GDN2GPT`` layer stack with streaming caches (``model.py:251-430``)."""

    def __init__(self, config: HybridConfig) -> None:
        super().__init__()
        self.config = config
        self.wte = nn.Embedding(config.padded_vocab_size, config.n_embd)
        self.h = nn.ModuleList([Block(config, i) for i in range(config.n_layer)])
        self.ln_f = RMSNorm(config.n_embd, eps=config.norm_eps)
        self.lm_head = nn.Linear(config.n_embd, config.padded_vocab_size, bias=False)
        self.rope: tuple[torch.Tensor, torch.Tensor] | None = None
        self.mask_cache: torch.Tensor | None = None
        self.max_seq_length = 0
        self.apply(self._init_weights)

    def _init_weights(self, module: nn.Module) -> None:
        """Normal(0, sqrt(2 / 5 / n_embd)) for embeddings and every Linear, zero biases
        (reference ``model.py:273-295``, ``mamba_init=False``)."""
        std = math.sqrt(2.0 / 5 / self.config.n_embd)
        if isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=std)
        elif isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=std)
            if module.bias is not None:
                nn.init.zeros_(module.bias)

    def _rope_tables(self, n: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        if self.rope is None or self.rope[0].shape[0] < n or self.rope[0].device != device:
            c = self.config
            self.rope = build_rope_cache(max(n, c.block_size), int(c.rotary_percentage * c.head_size), device,
                                         c.rope_base, c.condense_ratio)
        return self.rope

    def _attention_decode_fused(self) -> bool:
        """Whether every attention layer's single-token step takes ``ops.attention_decode``
        (the condition ``CausalSelfAttention.forward_qkv`` tests, on the weights)."""
        for blk in self.h:
            if blk.use_gdn2:
                continue
            at = blk.attn
            w = at.attn.weight
            G, qpk, D = at.n_query_groups, at.n_head // at.n_query_groups, at.head_size
            if at.kv_cache is None or not _inference(w) or not ops.attention_decode_supported(w, qpk, D):
                return False
        return True

    def setup_caches(self, batch: int, max_seq_length: int) -> None:
        """Allocate the attention KV caches ``[batch, groups, max_seq_length, head_size]``
        and the causal mask, and drop every gdn2 cache (the next cached forward is a
        prefill)."""
        p = self.lm_head.weight
        c = self.config
        self.max_seq_length = max_seq_length
        self.mask_cache = torch.tril(torch.ones(max_seq_length, max_seq_length, dtype=torch.bool,
                                                device=p.device))[None, None]
        self._rope_tables(max_seq_length, p.device)
        for blk in self.h:
            blk.gdn2_cache = None
            if not blk.use_gdn2:
                shape = (batch, c.n_query_groups, max_seq_length, c.head_size)
                blk.attn.kv_cache = (torch.zeros(shape, dtype=p.dtype, device=p.device),
                                     torch.zeros(shape, dtype=p.dtype, device=p.device))

    def forward(self, idx: torch.Tensor, input_pos: torch.Tensor | None = None,
                last_only: bool = False) -> torch.Tensor:
        """Logits ``[B, T, vocab]``. With ``input_pos`` (positions of ``idx``'s tokens,
        a device tensor), the caches are read and extended: the first cached call after
        ``setup_caches`` is the prefill, later ones continue it.  ``last_only`` applies the
        final norm and the LM head to the last position only (logits ``[B, 1, vocab]``):
        what greedy decoding reads of a prefill, without the ``T x vocab`` product."""
        t = idx.shape[1]
        cos, sin = self._rope_tables(t, idx.device)
        mask = None
        if input_pos is None:
            cos, sin = cos[:t], sin[:t]
        else:
            if self.mask_cache is None:
                raise RuntimeError("call setup_caches before a cached forward")
            if not (t == 1 and self._attention_decode_fused()):
                cos, sin = cos.index_select(0, input_pos), sin.index_select(0, input_pos)
                mask = self.mask_cache.index_select(2, input_pos)
            # else: every attention layer takes the fused decode kernel, which reads
            # the rotation tables' row input_pos itself and needs no mask.
        x = self.wte(idx)
        if _inference(x, self.ln_f.weight) and ops.add_rms_norm_supported(x):
            # The residual adds fused with the norms that follow them.
            pending = None
            for blk in self.h:
                x, pending = blk.forward_pending(x, pending, cos, sin, input_pos, mask)
            if last_only:
                x = x[:, -1:]
                pending = None if pending is None else pending[:, -1:]
            if pending is None:
                return ops.linear(self.ln_f(x), self.lm_head.weight)
            _, xn = ops.add_rms_norm(x, pending, self.ln_f.weight, self.ln_f.eps)
            return ops.linear(xn, self.lm_head.weight)
        for blk in self.h:
            x = blk(x, cos, sin, input_pos, mask)
        if last_only:
            x = x[:, -1:]
        return self.lm_head(self.ln_f(x))


class GreedyDecoder:
    """Prefill, then greedy decode with the step captured once as a HIP graph.

    ``generate(prompt, n)`` returns the ``n`` generated token ids ``[B, n]``. The
    captured step reads the previous token and position from static device tensors,
    writes the next token and advances the position, so the host only replays it.
    """

    def __init__(self, model: HybridDecoder, use_graph: bool = True, keep_logits: bool = False) -> None:
        self.model = model
        self.use_graph = use_graph
        self.keep_logits = keep_logits
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None  # last step's fp32 logits [B, vocab] (keep_logits)

    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        B, T = prompt.shape
        dev = prompt.device
        self.model.setup_caches(B, T + max_new_tokens)
        self.graph = None
        logits = self.model(prompt, input_pos=torch.arange(T, device=dev), last_only=True)[:, -1]
        self.tok = logits.argmax(-1, keepdim=True)
        self.pos = torch.full((1,), T, dtype=torch.long, device=dev)
        if self.keep_logits:
            self.logits = logits.float()
        return self.tok

    def _step(self) -> None:
        logits = self.model(self.tok, input_pos=self.pos)[:, -1]
        ops.argmax_rows(logits, out=self.tok)  # one launch (torch's reduction is about 50 µs here)
        self.pos.add_(1)
        if self.keep_logits:
            self.logits.copy_(logits)

    @torch.no_grad()
    def step(self) -> torch.Tensor:
        """One decode step; returns the static next-token tensor ``[B, 1]``."""
        if not self.use_graph:
            self._step()
            return self.tok
        if self.graph is None:
            # The first step runs eagerly on a side stream (library handles and
            # workspaces get created outside the capture); it is a real step.
            # Capture only records the second one, which the replay below runs.
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._step()
            torch.cuda.current_stream().wait_stream(side)
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self._step()
            return self.tok
        self.graph.replay()
        return self.tok

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        out = [self.prefill(prompt, max_new_tokens).clone()]
        for _ in range(max_new_tokens - 1):
            out.append(self.step().clone())
        return torch.cat(out, dim=1)


def count_parameters(config: HybridConfig) -> int:
    """Parameters of ``HybridDecoder(config)`` from the config alone (the closed form of
    reference ``compute_model_params``, ``model.py:433-501``, with the gdn2 mixer's
    q/k/v conv weights, ``A_log``, ``dt_bias``, ``f_proj``/``g_proj`` low-rank pairs and
    ``o_norm``)."""
    c = config
    d, k_dim = c.n_embd, c.n_head * c.head_size
    hv = int(c.head_size * c.expand_v)
    v_dim = c.n_head * hv
    mlp = 3 * d * c.intermediate_size
    norms = 2 * d
    attn = d * (c.n_head + 2 * c.n_query_groups) * c.head_size + c.n_head * c.head_size * d
    gdn2 = (d * k_dim * 2 + d * v_dim                                      # q, k, v projections
            + ((2 * k_dim + v_dim) * c.conv_size if c.use_short_conv else 0)
            + d * hv + hv * k_dim                                          # f_proj
            + d * k_dim + d * v_dim                                        # b_proj, w_proj
            + d * hv + hv * v_dim + v_dim                                  # g_proj (second with bias)
            + v_dim * d + hv + c.n_head + k_dim)                           # o_proj, o_norm, A_log, dt_bias
    n_gdn2 = sum(c.is_gdn2(i) for i in range(c.n_layer))
    return (2 * c.padded_vocab_size * d + d + (mlp + norms) * c.n_layer
            + attn * (c.n_layer - n_gdn2) + gdn2 * n_gdn2)


__all__ = ["Block", "CausalSelfAttention", "GreedyDecoder", "HybridConfig", "HybridDecoder",
           "apply_rotary_emb", "build_rope_cache", "count_parameters"]
