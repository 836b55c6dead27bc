r"""Drop-in ``GatedDeltaNet2`` token mixer whose recurrence runs on the MI355X HIP kernels.

Interface contract (reference ``src/qwendopamine/models/gdn2/gdn2.py``):

* constructor ``GatedDeltaNet2(hidden_size_or_config, hidden_size, num_heads,
  head_dim, layer_idx, mode, expand_v, num_v_heads, use_short_conv,
  allow_neg_eigval, conv_size, conv_bias, norm_eps, chunk_size, backend,
  compile_backend, fp32_decay, **kwargs)`` (``gdn2.py:491-653``), including the
  config-object aliases (``gdn2.py:515-538``) and the same parameter names,
  shapes, registration order and initialisation, so ``load_state_dict`` and
  seeded construction line up with the reference module;
* ``forward(hidden_states, attention_mask, past_key_values, use_cache,
  output_attentions, **kwargs) -> (out, None, past_key_values)``
  (``gdn2.py:780-1004``) with the same dict / ``transformers`` Cache layout
  (``gdn2.py:655-778``): ``recurrent_state [B, HV, d_k, d_v]`` and a 3-tuple of
  short-conv caches ``[B, D, conv_size-1]``.

What changes is the execution backend: the gdn2 recurrence itself always runs
on the hand-written HIP kernels (``qwendopamine_amd.ops``), chunkwise for
prefill/training and token-serial for decode.  The reference backend names are
accepted for compatibility and select only the algorithm:

    "auto", "hip", "torch", "triton", "fla"  follow the mode (chunk, or
                                              token-serial when seq_len <= 64
                                              in eval, as ``gdn2.py:790``)
    "torch-chunk", "compiled"                always chunkwise
    "torch-recurrent"                        always token-serial

Tensors on a non-GPU device raise ``RuntimeError``: there is no CPU path.  The
recurrent state is kept in float32 (the reference's accelerated ops return
float32 states; its pure-torch ops return the input dtype).
"""

from __future__ import annotations

import math
import warnings
from typing import Any, Literal

import torch
import torch.nn.functional as F
from torch import nn

from ._stacked import drop, stacked_rows
from . import ops

try:  # transformers is optional: only needed for HF Cache objects
    from transformers.cache_utils import Cache as _HFCache
except ImportError:  # pragma: no cover
    _HFCache = None
try:
    from transformers.cache_utils import LinearAttentionCacheLayerMixin as _LinearLayer
except ImportError:  # pragma: no cover
    _LinearLayer = None

__all__ = [
    "GDN2_BACKENDS",
    "GatedDeltaNet2",
    "RMSNormGated",
    "ShortConvolution",
    "resolve_gdn2_backend",
]

GDN2_BACKENDS = ("auto", "torch", "torch-chunk", "torch-recurrent", "compiled", "triton", "fla", "hip")

_WARNED: set[str] = set()


def _warn_once(msg: str) -> None:
    if msg not in _WARNED:
        _WARNED.add(msg)
        warnings.warn(f"[gdn2] {msg}", stacklevel=3)


def resolve_gdn2_backend(requested: str, *, training: bool, seq_len: int) -> str:
    """Validate a backend name (reference ``gdn2.py:69-97``).

    Raises ``ValueError`` for unknown names.  Forced names pass through
    unchanged; ``"auto"`` resolves to ``"hip"`` -- the HIP kernels are the
    execution backend of this package on every supported device.
    """
    if requested not in GDN2_BACKENDS:
        raise ValueError(f"gdn2 backend {requested!r} is not one of {', '.join(GDN2_BACKENDS)}")
    del training, seq_len
    return "hip" if requested == "auto" else requested


def _inference(*tensors: torch.Tensor | None) -> bool:
    """True for GPU tensors through which no gradient flows.  The prologue and
    epilogue then run on their HIP kernels, which are forward only.  Otherwise
    they use torch's differentiable ops, as the reference does.  This covers
    training, and standalone CPU use of these two nn.Modules.  The mixer's
    recurrence itself has no CPU path."""
    live = [t for t in tensors if t is not None]
    if not all(t.is_cuda for t in live):
        return False
    return not (torch.is_grad_enabled() and any(t.requires_grad for t in live))


class ShortConvolution(nn.Module):
    """Causal depthwise conv1d + optional SiLU with a rolling cache (reference ``gdn2.py:372-430``).

    Prefill pads ``kernel_size - 1`` zeros on the left; a single-token call with
    a cache ``[B, D, kernel_size-1]`` convolves ``cat(cache, x)``.  With
    ``output_final_state`` the new cache holds the last ``kernel_size - 1``
    inputs.
    """

    def __init__(self, hidden_size: int, kernel_size: int = 4, bias: bool = False,
                 activation: str | None = "silu") -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.kernel_size = kernel_size
        self.activation = activation
        self.conv1d = nn.Conv1d(hidden_size, hidden_size, kernel_size, groups=hidden_size,
                                bias=bias, padding=kernel_size - 1)
        # Training prefill (no cache) runs the HIP forward and backward kernels;
        # False uses torch's conv1d and SiLU.
        self.hip_backward = True

    def forward(self, x: torch.Tensor, cache: torch.Tensor | None = None,
                output_final_state: bool = False, cu_seqlens: torch.Tensor | None = None):
        if _inference(x, self.conv1d.weight):
            ys, new = ops.short_convolution([x], [self.conv1d.weight], [self.conv1d.bias],
                                            None if cache is None else [cache], output_final_state,
                                            self.activation)
            return ys[0], None if new is None else new[0]
        bsz, seq, dim = x.shape
        keep = self.kernel_size - 1
        if (self.hip_backward and x.is_cuda and cache is None and self.kernel_size <= 8
                and self.activation in (None, "silu") and (seq > 1 or not output_final_state)):
            # Differentiable path (training) on the HIP kernels.
            y = ops.short_conv_autograd(x, self.conv1d.weight, self.conv1d.bias, self.activation)
            new_cache = x.transpose(1, 2)[:, :, -keep:] if output_final_state else None
            return y, new_cache
        # Differentiable path (training): torch's depthwise conv.
        xt = x.transpose(1, 2)
        wgt, bias = self.conv1d.weight, self.conv1d.bias
        if cache is None and output_final_state and seq == 1:
            cache = x.new_zeros(bsz, dim, keep)
        if cache is not None and seq == 1:
            window = torch.cat([cache.to(x.dtype), xt], dim=-1)
            y = F.conv1d(window, wgt, bias, groups=dim)
            new_cache = window[:, :, 1:] if output_final_state else None
        else:
            y = F.conv1d(xt, wgt, bias, padding=keep, groups=dim)[..., :seq]
            new_cache = xt[:, :, -keep:] if output_final_state else None
        if self.activation == "silu":
            y = F.silu(y)
        return y.transpose(1, 2), new_cache


class RMSNormGated(nn.Module):
    """``x * rsqrt(mean(x^2) + eps) * weight * silu(z)`` computed in the input dtype.

    Reference ``gdn2.py:433-452``: the gdn2-local variant deliberately does not
    promote to float32.
    """

    def __init__(self, hidden_size: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))
        # Training runs the HIP forward and backward kernels (rows of up to 256
        # values); False uses torch ops.
        self.hip_backward = True

    def forward(self, x: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
        if _inference(x, z, self.weight):
            return ops.gated_rmsnorm(x, z, self.weight, self.eps)
        if self.hip_backward and x.is_cuda and x.shape[-1] <= 256 and z.shape == x.shape:
            return ops.gated_rmsnorm_autograd(x, z, self.weight, self.eps)
        # Differentiable path (training): torch ops, same rounding.
        inv = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)
        return x * inv * self.weight * F.silu(z)


def _get_unpad_data(attention_mask: torch.Tensor):
    """Packed-token indices of a 0/1 padding mask: ``(indices, cu_seqlens, max_len)``."""
    lens = attention_mask.sum(dim=-1, dtype=torch.int32)
    indices = torch.nonzero(attention_mask.flatten(), as_tuple=False).flatten()
    cu = torch.zeros(lens.numel() + 1, dtype=torch.int32, device=attention_mask.device)
    cu[1:] = torch.cumsum(lens, dim=0, dtype=torch.int32)
    return indices, cu, int(lens.max().item())


def _index_first_axis(x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, *x.shape[2:])[indices]


def _pad_input(packed: torch.Tensor, indices: torch.Tensor, batch: int, seqlen: int) -> torch.Tensor:
    out = packed.new_zeros(batch * seqlen, *packed.shape[1:])
    out[indices] = packed
    return out.reshape(batch, seqlen, *packed.shape[1:])


def _split_heads(x: torch.Tensor, d: int) -> torch.Tensor:
    return x.reshape(*x.shape[:-1], x.shape[-1] // d, d)


class GatedDeltaNet2(nn.Module):
    """Gated DeltaNet 2 (GDN-2) token-mixing layer on the MI355X HIP backend."""

    def __init__(
        self,
        hidden_size_or_config: int | Any = 2048,
        hidden_size: int | None = None,
        num_heads: int | None = None,
        head_dim: int | None = None,
        layer_idx: int | None = None,
        mode: Literal["chunk", "fused_recurrent"] = "chunk",
        expand_v: float = 1.0,
        num_v_heads: int | None = None,
        use_short_conv: bool = True,
        allow_neg_eigval: bool = False,
        conv_size: int = 4,
        conv_bias: bool = False,
        norm_eps: float = 1e-5,
        chunk_size: int = 64,
        backend: str = "auto",
        compile_backend: bool = False,
        fp32_decay: bool = True,
        **kwargs: Any,
    ) -> None:
        super().__init__()
        cfg = hidden_size_or_config
        if hasattr(cfg, "hidden_size") or hasattr(cfg, "n_embd"):
            # Config object with the reference's alias lookups (gdn2.py:515-538).
            hidden_size = getattr(cfg, "hidden_size", getattr(cfg, "n_embd", 2048))
            num_heads = getattr(cfg, "num_heads", getattr(cfg, "n_head", 16))
            head_dim = getattr(cfg, "head_dim", getattr(cfg, "head_size", 128))
            num_v_heads = getattr(cfg, "num_v_heads", getattr(cfg, "n_query_groups", num_v_heads or num_heads))
            conv_size = getattr(cfg, "conv_size", getattr(cfg, "conv_kernel_size", conv_size))
            norm_eps = getattr(cfg, "norm_eps", getattr(cfg, "rms_norm_eps", norm_eps))
            allow_neg_eigval = getattr(cfg, "allow_neg_eigval", allow_neg_eigval)
            expand_v = getattr(cfg, "expand_v", expand_v)
            chunk_size = getattr(cfg, "chunk_size", getattr(cfg, "train_chunk_size", chunk_size))
            backend = getattr(cfg, "backend", backend)
            compile_backend = getattr(cfg, "compile_backend", compile_backend)
            fp32_decay = getattr(cfg, "fp32_decay", fp32_decay)
        elif hidden_size is None:
            hidden_size = int(cfg)

        if backend not in GDN2_BACKENDS:
            raise ValueError(f"GatedDeltaNet2: unknown backend {backend!r}; choose one of {sorted(GDN2_BACKENDS)}")

        self.hidden_size = hidden_size
        self.num_heads = 16 if num_heads is None else num_heads
        self.head_dim = 128 if head_dim is None else head_dim
        self.num_v_heads = self.num_heads if num_v_heads is None else num_v_heads
        if self.num_v_heads > self.num_heads and self.num_v_heads % self.num_heads != 0:
            raise ValueError(
                f"GatedDeltaNet2: {self.num_v_heads} value heads cannot be grouped over "
                f"{self.num_heads} key heads (need a whole multiple)"
            )
        self.layer_idx = layer_idx
        self.mode = mode
        self.use_short_conv = use_short_conv
        self.allow_neg_eigval = allow_neg_eigval
        self.conv_size = conv_size
        self.conv_bias = conv_bias
        self.norm_eps = norm_eps
        self.expand_v = expand_v
        self.chunk_size = chunk_size
        self.backend = backend
        self.compile_backend = compile_backend
        self.fp32_decay = fp32_decay
        # Single-token inference calls run the fused decode kernel (conv, gates,
        # recurrence and output norm in one launch) when its conditions hold;
        # False runs the same steps as separate passes.
        self.fused_decode = True
        # Chunked inference applies the gated output norm in the scan's output
        # stage when one scan workgroup owns a whole value row anyway (bf16,
        # head_v_dim in {16, 32, 64}, at least 256 sequence-heads or 16-wide
        # heads); False always runs the norm as its own pass.  With fewer
        # sequence-heads the scan splits value rows over more workgroups and the
        # norm pass is faster.
        self.fused_norm = True
        # Chunked inference prefill convolves q, k and v inside the chunk
        # kernels (bf16, width-4 convolutions without bias, whole key widths of
        # 32 / 64 / 128, no packed sequences); False runs the convolution pass.
        self.fused_conv = True

        self.head_k_dim = self.head_dim
        self.head_v_dim = int(self.head_dim * self.expand_v)
        self.key_dim = int(self.num_heads * self.head_k_dim)
        self.value_dim = int(self.num_v_heads * self.head_v_dim)

        D, kd, vd, hv = self.hidden_size, self.key_dim, self.value_dim, self.head_v_dim
        # Registration order fixes both state_dict keys and the RNG order of
        # seeded initialisation (reference gdn2.py:573-622).
        self.q_proj = nn.Linear(D, kd, bias=False)
        self.k_proj = nn.Linear(D, kd, bias=False)
        self.v_proj = nn.Linear(D, vd, bias=False)
        if self.use_short_conv:
            self.q_conv1d = ShortConvolution(kd, kernel_size=conv_size, bias=conv_bias)
            self.k_conv1d = ShortConvolution(kd, kernel_size=conv_size, bias=conv_bias)
            self.v_conv1d = ShortConvolution(vd, kernel_size=conv_size, bias=conv_bias)
        self.f_proj = nn.Sequential(nn.Linear(D, hv, bias=False), nn.Linear(hv, kd, bias=False))
        self.b_proj = nn.Linear(D, kd, bias=False)
        self.w_proj = nn.Linear(D, vd, bias=False)
        # A ~ U(1, 16) per head; dt log-uniform in [1e-3, 1e-1] per key channel,
        # stored as its softplus inverse.
        self.A_log = nn.Parameter(torch.empty(self.num_heads, dtype=torch.float32).uniform_(1, 16).log())
        self.A_log._no_weight_decay = True
        lo, hi = math.log(1e-3), math.log(1e-1)
        dt = torch.exp(torch.rand(kd, dtype=torch.float32) * (hi - lo) + lo).clamp(min=1e-4)
        self.dt_bias = nn.Parameter(dt + torch.log(-torch.expm1(-dt)))
        self.dt_bias._no_weight_decay = True
        self.g_proj = nn.Sequential(nn.Linear(D, hv, bias=False), nn.Linear(hv, vd, bias=True))
        self.o_norm = RMSNormGated(hv, eps=norm_eps)
        self.o_proj = nn.Linear(vd, D, bias=False)
        self.apply(self._initialize_weights)
        if self.compile_backend:
            _warn_once("compile_backend has no effect: the recurrence runs on HIP kernels")

    def _initialize_weights(self, module: nn.Module) -> None:
        """Xavier(gain 2^-2.5) linears, Kaiming(a=sqrt 5) convs, unit norms (gdn2.py:640-653)."""
        if getattr(module, "_is_hf_initialized", False):
            return
        if isinstance(module, nn.Linear):
            nn.init.xavier_uniform_(module.weight, gain=2**-2.5)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Conv1d):
            nn.init.kaiming_uniform_(module.weight, a=math.sqrt(5))
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, RMSNormGated):
            nn.init.ones_(module.weight)
        module._is_hf_initialized = True

    # ------------------------------------------------------------------ cache
    def _get_cache(self, past_key_values):
        """``(recurrent_state, (conv_q, conv_k, conv_v))`` from a dict or HF Cache (gdn2.py:655-703)."""
        if past_key_values is None:
            return None, None
        if isinstance(past_key_values, dict):
            return past_key_values.get("recurrent_state"), past_key_values.get("conv_state")
        if _HFCache is not None and isinstance(past_key_values, _HFCache):
            layers = getattr(past_key_values, "layers", [])
            if self.layer_idx is None or self.layer_idx >= len(layers):
                return None, None
            lc = layers[self.layer_idx]
            rs = getattr(lc, "recurrent_states", None)
            if rs is None:
                rec = getattr(lc, "recurrent_state", None)
            elif isinstance(rs, torch.Tensor):
                rec = rs
            elif isinstance(rs, dict):
                rec = rs.get(0)
            elif isinstance(rs, (list, tuple)) and rs:
                rec = rs[0]
            else:
                rec = None
            cs = getattr(lc, "conv_states", None)
            if cs is None:
                conv = getattr(lc, "conv_state", None)
            elif isinstance(cs, dict):
                conv = (cs.get(0), cs.get(1), cs.get(2))
            elif isinstance(cs, (list, tuple)) and len(cs) == 3:
                conv = tuple(cs)
            else:
                conv = None
            return rec, conv
        return None, None

    def _update_cache(self, past_key_values, recurrent_state, conv_state) -> None:
        """Store the new states into a dict or HF Cache (gdn2.py:705-778)."""
        if past_key_values is None:
            return
        if isinstance(past_key_values, dict):
            if recurrent_state is not None:
                past_key_values["recurrent_state"] = recurrent_state
            if conv_state is not None:
                past_key_values["conv_state"] = conv_state
            return
        if self.layer_idx is None or _HFCache is None or not isinstance(past_key_values, _HFCache):
            return
        layers = getattr(past_key_values, "layers", [])
        if self.layer_idx >= len(layers):
            return
        lc = layers[self.layer_idx]
        recurrent_layer = (
            (_LinearLayer is not None and isinstance(lc, _LinearLayer))
            or hasattr(lc, "update_recurrent_state")
            or hasattr(lc, "recurrent_states")
        )
        caught = (TypeError, ValueError, AttributeError, RuntimeError, IndexError)
        if recurrent_state is not None:
            if recurrent_layer and hasattr(past_key_values, "update_recurrent_state"):
                try:
                    past_key_values.update_recurrent_state(recurrent_state, self.layer_idx)
                except caught as e:
                    _warn_once(f"update_recurrent_state failed: {e}")
            else:
                rs = getattr(lc, "recurrent_states", None)
                if isinstance(rs, dict):
                    rs[0] = recurrent_state
                elif hasattr(lc, "recurrent_state"):
                    lc.recurrent_state = recurrent_state
        if conv_state is not None:
            if recurrent_layer and hasattr(past_key_values, "update_conv_state"):
                try:
                    past_key_values.update_conv_state(conv_state, self.layer_idx)
                except caught as e:
                    _warn_once(f"update_conv_state failed: {e}")
            else:
                cs = getattr(lc, "conv_states", None)
                if isinstance(cs, dict):
                    cs[0], cs[1], cs[2] = conv_state
                elif hasattr(lc, "conv_state"):
                    lc.conv_state = conv_state

    # ---------------------------------------------------------------- forward
    def _gate_params(self, rep: int) -> tuple[torch.Tensor, torch.Tensor]:
        """float32 ``A_log [HV]`` and ``dt_bias [HV * d_k]`` for the in-kernel gate, each
        key head's parameters repeated for its ``rep`` value heads.  Cached until either
        parameter changes, so a decode step launches no conversion kernels."""
        key = (self.A_log.data_ptr(), self.A_log._version, self.dt_bias.data_ptr(), self.dt_bias._version,
               self.A_log.dtype, self.dt_bias.dtype, rep)
        cached = getattr(self, "_gate_cache", None)
        if cached is None or cached[0] != key:
            a = self.A_log.detach().float()
            d = self.dt_bias.detach().float().view(self.num_heads, self.head_k_dim)
            if rep > 1:
                a, d = a.repeat_interleave(rep), d.repeat_interleave(rep, dim=0)
            cached = (key, a.contiguous(), d.reshape(-1).contiguous())
            self._gate_cache = cached
        return cached[1], cached[2]

    def _fused_input_weight(self) -> tuple[torch.Tensor, list[int]]:
        """The first-stage input projections stacked as one weight, ``[q; k; v; b; w;
        f_proj[0]; g_proj[0]]`` (none has a bias), and their output widths.  Used by the
        inference path for a single GEMM.  The seven parameters are row views of the
        stacked tensor, so the module holds one copy of these weights."""
        ws = [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.b_proj.weight,
              self.w_proj.weight, self.f_proj[0].weight, self.g_proj[0].weight]
        return stacked_rows(self, "_in_cache", ws), [int(t.shape[0]) for t in ws]

    def _apply(self, fn, *args, **kwargs):
        # Parameters are about to be converted or moved: the caches would hold the old copies.
        drop(self, "_in_cache", "_gate_cache")
        return super()._apply(fn, *args, **kwargs)

    def _fused_decode_ok(self, x: torch.Tensor) -> bool:
        """Whether a single-token inference call on ``x`` can take the fused decode kernel
        (the caller has checked the token count, padding and ``cu_seqlens``)."""
        convs = (self.q_conv1d, self.k_conv1d, self.v_conv1d) if self.use_short_conv else ()
        return bool(
            self.fused_decode and self.use_short_conv and self.fp32_decay and not self.allow_neg_eigval
            and self.num_v_heads == self.num_heads and self.head_k_dim == self.head_v_dim
            and self.head_k_dim in (64, 128) and self.conv_size == 4
            and all(c.activation == "silu" for c in convs)
            and self._algorithm("fused_recurrent" if not self.training else self.mode,
                                resolve_gdn2_backend(self.backend, training=self.training, seq_len=1),
                                False) == "recurrent"
            and _inference(x, self.A_log, self.dt_bias, self.b_proj.weight, self.w_proj.weight,
                           *(c.conv1d.weight for c in convs), self.o_norm.weight,
                           self.f_proj[1].weight, self.g_proj[1].weight))

    def _decode_fused(self, x, past_key_values, recurrent_state, conv_states, want_state, in_place,
                      use_cache):
        """Single-token inference step on the fused decode kernel (``ops.decode_step_fused``):
        the short convolutions, the gate and b / w activations, the recurrence and the gated
        output norm in one launch, between the input projections and ``o_proj``.  Same
        result and cache updates as the separate passes of ``forward``."""
        batch = x.shape[0]
        W_in, sizes = self._fused_input_weight()
        y = ops.linear(x.reshape(batch, x.shape[-1]), W_in)  # [B, sum(sizes)]
        return self._decode_fused_rows(y, x.dtype, past_key_values, recurrent_state, conv_states, want_state,
                                       in_place, use_cache)

    def decode_step_from_residual(self, residual: torch.Tensor, delta: torch.Tensor, norm_weight: torch.Tensor,
                                  eps: float, cache: dict) -> tuple[torch.Tensor, torch.Tensor] | None:
        """A host block's single-token step from its pre-norm inputs: ``s = residual +
        delta``, ``x = RMSNorm(s)`` (the block's norm_1) and this mixer on ``x``, with the
        add and the norm formed while the input projections stage their input
        (``ops.linear_addnorm``, bit for bit the separate ops).  ``cache`` is the layer's
        cache dict; its tensors are updated where they lie (as ``update_cache_in_place``)
        and the dict's entries set to the new states.  Returns
        ``(s, mixer output)``, or None when the fused decode path does not apply (the
        caller then runs the ops apart).  No counterpart in the reference."""
        batch, seq_len, _ = residual.shape
        state = cache.get("recurrent_state") if cache else None
        conv = cache.get("conv_state") if cache else None
        if (seq_len != 1 or state is None or conv is None or any(c is None for c in conv)
                or state.dtype != torch.float32 or not state.is_contiguous()
                or not _inference(residual, delta, norm_weight) or not self._fused_decode_ok(residual)):
            return None
        W_in, sizes = self._fused_input_weight()
        y, s = ops.linear_addnorm(residual.reshape(batch, -1), delta.reshape(batch, -1), norm_weight, eps, W_in)
        out, _, _ = self._decode_fused_rows(y, residual.dtype, cache, state, tuple(conv), True, True, True)
        return s.view_as(residual), out

    def _decode_fused_rows(self, y, dt, past_key_values, recurrent_state, conv_states, want_state, in_place,
                           use_cache):
        """The fused decode step from the input projections' output ``y`` [B, sum(sizes)]."""
        batch = y.shape[0]
        _, sizes = self._fused_input_weight()
        qr, kr, vr, b, w, f0, g0 = y.split(sizes, dim=-1)
        g, z = ops.linear_pair(f0, self.f_proj[1].weight, self.f_proj[1].bias, g0, self.g_proj[1].weight,
                               self.g_proj[1].bias)
        caches = list(conv_states) if all(c is not None for c in conv_states) else None
        if caches is not None and not all(c.dtype == dt and c.is_contiguous() for c in caches):
            caches, in_place = [c.to(dt).contiguous() for c in caches], False
        h0 = recurrent_state
        if h0 is not None and (h0.dtype != torch.float32 or not h0.is_contiguous()):
            h0, in_place = h0.float().contiguous(), False
        if in_place and caches is None:
            in_place = False
        A_log, dt_bias = self._gate_params(1)
        convs = (self.q_conv1d, self.k_conv1d, self.v_conv1d)
        o, state, new_caches = ops.decode_step_fused(
            [qr, kr, vr], [c.conv1d.weight for c in convs], [c.conv1d.bias for c in convs], caches,
            g, b, w, h0, z, self.o_norm.weight, self.o_norm.eps,
            num_heads=self.num_heads, head_dim=self.head_k_dim, A_log=A_log, dt_bias=dt_bias,
            update_cache_in_place=in_place, output_final_state=want_state)
        if use_cache or past_key_values is not None:
            self._update_cache(past_key_values, state, tuple(new_caches))
        out = ops.linear(o.reshape(batch, 1, -1), self.o_proj.weight, self.o_proj.bias)
        return out, None, past_key_values

    def _algorithm(self, mode: str, backend: str, needs_grad: bool) -> str:
        if backend in ("torch-chunk", "compiled"):
            algo = "chunk"
        elif backend == "torch-recurrent":
            algo = "recurrent"
        else:
            algo = "chunk" if mode == "chunk" else "recurrent"
        # The token-serial kernel is inference-only; gradients go through the
        # chunkwise kernels, which compute the same recurrence.
        if algo == "recurrent" and needs_grad:
            algo = "chunk"
        return algo

    def forward(
        self,
        hidden_states: torch.Tensor,
        attention_mask: torch.Tensor | None = None,
        past_key_values: Any = None,
        use_cache: bool | None = False,
        output_attentions: bool | None = False,
        **kwargs: Any,
    ):
        """Reference ``GatedDeltaNet2.forward`` (``gdn2.py:780-1004``).

        Extension keyword (no counterpart in the reference): ``update_cache_in_place=True``
        makes a single-token inference call with an existing cache write the new recurrent
        and conv states into the cache's own tensors instead of fresh ones, so their
        addresses stay fixed (hosts that replay a captured decode step use it).
        """
        batch, seq_len, _ = hidden_states.shape
        if not hidden_states.is_cuda:
            raise RuntimeError(
                "GatedDeltaNet2 runs its recurrence on the MI355X HIP kernels; move the module "
                "and inputs to a ROCm GPU (there is no CPU path)."
            )
        mode = "fused_recurrent" if (seq_len <= 64 and not self.training) else self.mode
        want_state = bool(use_cache)
        recurrent_state, conv_states = self._get_cache(past_key_values)
        cq, ck, cv = conv_states if conv_states is not None else (None, None, None)
        cu_seqlens = kwargs.get("cu_seqlens")
        in_place = bool(kwargs.get("update_cache_in_place")) and want_state and seq_len == 1 \
            and cu_seqlens is None and recurrent_state is not None \
            and recurrent_state.dtype == torch.float32 and recurrent_state.is_contiguous()

        # Padding: drop masked tokens, run packed, scatter back (gdn2.py:799-813).
        padded = (
            attention_mask is not None
            and seq_len > 1
            and past_key_values is None
            and bool((attention_mask == 0).any())
        )
        indices = None
        if padded:
            indices, cu_seqlens, _ = _get_unpad_data(attention_mask)
            hidden_states = _index_first_axis(hidden_states, indices).unsqueeze(0)

        x = hidden_states
        # Inference with the in-kernel activations: g, b and w go to the kernels
        # as raw projections (see below).
        fuse = (_inference(x, self.A_log, self.dt_bias, self.f_proj[1].weight, self.b_proj.weight,
                           self.w_proj.weight)
                and self.fp32_decay and not self.allow_neg_eigval)
        convs = (self.q_conv1d, self.k_conv1d, self.v_conv1d) if self.use_short_conv else ()
        if fuse and seq_len == 1 and not padded and cu_seqlens is None and self._fused_decode_ok(x):
            return self._decode_fused(x, past_key_values, recurrent_state, (cq, ck, cv), want_state,
                                      in_place, use_cache)
        g0 = None
        conv_raw = None  # raw q, k, v rows when the chunk kernels convolve them
        if fuse and self.use_short_conv and _inference(x, *(c.conv1d.weight for c in convs)):
            # The seven first-stage input projections as one GEMM; q, k and v
            # are convolved in place as column ranges of its output.
            W_in, sizes = self._fused_input_weight()
            y = F.linear(x.reshape(-1, x.shape[-1]), W_in)  # [tokens, sum(sizes)]
            qr, kr, vr, b, w, f0, g0 = (t.view(*x.shape[:-1], -1) if i < 5 else t
                                        for i, t in enumerate(y.split(sizes, dim=-1)))
            backend0 = resolve_gdn2_backend(self.backend, training=self.training, seq_len=seq_len)
            if (self.fused_conv and x.dtype == torch.bfloat16 and cu_seqlens is None and seq_len >= 4
                    and self._algorithm(mode, backend0, False) == "chunk"
                    and self.num_v_heads == self.num_heads and self.head_k_dim in (32, 64, 128)
                    and self.head_v_dim % 16 == 0 and self.conv_size == 4
                    and all(c.conv1d.bias is None and c.activation == self.q_conv1d.activation
                            and c.conv1d.weight.dtype == x.dtype for c in convs)
                    and self.q_conv1d.activation in (None, "silu")):
                # Prefill: the chunk kernels convolve the raw rows (below); the
                # new conv caches are the last three raw rows.
                conv_raw = (qr, kr, vr)
                q, k, v = qr, kr, vr
                if want_state:
                    cq, ck, cv = (t[:, -3:, :].transpose(1, 2).contiguous() for t in conv_raw)
                else:
                    cq = ck = cv = None
            else:
                conv_in = None if cq is None else [cq, ck, cv]
                conv_out = conv_in if in_place and conv_in is not None and all(
                    c.dtype == qr.dtype and c.is_contiguous() for c in conv_in) else None
                (q, k, v), new = ops.short_convolution(
                    [qr, kr, vr], [c.conv1d.weight for c in convs], [c.conv1d.bias for c in convs],
                    conv_in, want_state, self.q_conv1d.activation, out_caches=conv_out)
                cq, ck, cv = new if new is not None else (None, None, None)
            # The low-rank second stages read their 2-D column ranges in place.
            g = self.f_proj[1](f0).view(*x.shape[:-1], -1)
        elif self.use_short_conv and _inference(x, *(c.conv1d.weight for c in convs)):
            # q, k and v convolutions in one launch.
            raw = [self.q_proj(x), self.k_proj(x), self.v_proj(x)]
            (q, k, v), new = ops.short_convolution(
                raw, [c.conv1d.weight for c in convs], [c.conv1d.bias for c in convs],
                None if cq is None else [cq, ck, cv], want_state, self.q_conv1d.activation)
            cq, ck, cv = new if new is not None else (None, None, None)
        elif self.use_short_conv:
            q, cq = self.q_conv1d(self.q_proj(x), cache=cq, output_final_state=want_state, cu_seqlens=cu_seqlens)
            k, ck = self.k_conv1d(self.k_proj(x), cache=ck, output_final_state=want_state, cu_seqlens=cu_seqlens)
            v, cv = self.v_conv1d(self.v_proj(x), cache=cv, output_final_state=want_state, cu_seqlens=cu_seqlens)
        else:
            q, k, v = F.silu(self.q_proj(x)), F.silu(self.k_proj(x)), F.silu(self.v_proj(x))

        # Decay g = -exp(A_log) * softplus(f_proj(x) + dt_bias), always in fp32;
        # b = sigmoid(b_proj(x)), w = sigmoid(w_proj(x)) (gdn2.py:840-866).  In
        # inference these activations run inside the kernels on the raw
        # projections (same fp32 formula for g).
        if g0 is not None:
            pass  # g, b, w came from the fused projection above
        elif fuse:
            g, b, w = self.f_proj(x), self.b_proj(x), self.w_proj(x)
        else:
            A = self.A_log.float().exp().repeat_interleave(self.head_k_dim)
            g = -A * F.softplus(self.f_proj(x).float() + self.dt_bias)
            if not self.fp32_decay:
                g = g.to(x.dtype)
            b = self.b_proj(x).sigmoid()
            w = self.w_proj(x).sigmoid()

        q, k, g, b = (_split_heads(t, self.head_k_dim) for t in (q, k, g, b))
        v, w = _split_heads(v, self.head_v_dim), _split_heads(w, self.head_v_dim)
        rep = self.num_v_heads // self.num_heads
        if rep > 1:
            q, k, g, b = (t.repeat_interleave(rep, dim=-2) for t in (q, k, g, b))
        if self.allow_neg_eigval:
            b = b * 2.0

        backend = resolve_gdn2_backend(self.backend, training=self.training, seq_len=seq_len)
        needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v, g, b, w))
        algo = self._algorithm(mode, backend, needs_grad)
        h0 = None if recurrent_state is None else recurrent_state.float()
        dt = q.dtype
        gate_kw: dict = {}
        if fuse:
            A_log, dt_bias = self._gate_params(rep)
            gate_kw = dict(use_gate_in_kernel=True, A_log=A_log, dt_bias=dt_bias, bw_logits=True)
        b, w, v, k = b.to(dt), w.to(dt), v.to(dt), k.to(dt)
        normed = None
        n_seq = batch if cu_seqlens is None else cu_seqlens.numel() - 1
        norm_in_scan = (algo == "chunk" and fuse and self.fused_norm and dt == torch.bfloat16
                        and self.head_v_dim in (16, 32, 64) and self.o_norm.weight.dtype == dt
                        and (n_seq * self.num_v_heads >= 256 or self.head_v_dim == 16)
                        and _inference(self.o_norm.weight, *(p for p in self.g_proj.parameters())))
        if conv_raw is not None:
            # Convolutions in the chunk kernels (and the gated output norm in
            # the scan where it applies); bit-identical to the separate passes.
            gate = None
            if norm_in_scan:
                gate = self.g_proj(x) if g0 is None else self.g_proj[1](g0).view(*x.shape[:-1], -1)
            o, recurrent_state = ops.chunk_gdn2_conv(
                *conv_raw, [c.conv1d.weight for c in convs], g, b, w, num_heads=self.num_heads,
                activation=self.q_conv1d.activation, gate=gate,
                norm_weight=self.o_norm.weight if norm_in_scan else None, eps=self.o_norm.eps,
                initial_state=h0, output_final_state=want_state, use_qk_l2norm_in_kernel=True, **gate_kw,
            )
            if norm_in_scan:
                normed = o
        elif norm_in_scan:
            # The gated output norm in the scan's output stage (bit-identical to
            # the separate pass).
            gate = self.g_proj(x) if g0 is None else self.g_proj[1](g0).view(*x.shape[:-1], -1)
            normed, recurrent_state = ops.chunk_gdn2_gated_norm(
                q, k, v, g, b, w, gate, self.o_norm.weight, self.o_norm.eps, initial_state=h0,
                output_final_state=want_state, use_qk_l2norm_in_kernel=True, cu_seqlens=cu_seqlens,
                **gate_kw,
            )
        elif algo == "chunk":
            o, recurrent_state = ops.chunk_gdn2(
                q, k, v, g, b, w, initial_state=h0, output_final_state=want_state,
                use_qk_l2norm_in_kernel=True, cu_seqlens=cu_seqlens, **gate_kw,
            )
        elif in_place:
            # The decode kernel updates the cached state where it lies.
            o, recurrent_state = ops.fused_recurrent_gdn2_fwd(
                q=q, k=k, v=v, g=g, b=b, w=w, initial_state=recurrent_state, output_final_state=True,
                inplace_final_state=True, use_qk_l2norm_in_kernel=True, **gate_kw,
            )
        else:
            o, recurrent_state = ops.fused_recurrent_gdn2(
                q, k, v, g, b, w, initial_state=h0, output_final_state=want_state,
                use_qk_l2norm_in_kernel=True, cu_seqlens=cu_seqlens, **gate_kw,
            )

        if use_cache or past_key_values is not None:
            self._update_cache(past_key_values, recurrent_state,
                               (cq, ck, cv) if self.use_short_conv else None)

        if normed is not None:
            o = normed
        else:
            gate = _split_heads(self.g_proj(x) if g0 is None else self.g_proj[1](g0).view(*x.shape[:-1], -1),
                                self.head_v_dim)
            o = self.o_norm(o, gate)
        out = self.o_proj(o.reshape(*o.shape[:-2], -1))
        if padded:
            out = _pad_input(out.squeeze(0), indices, batch, seq_len)
        return out, None, past_key_values
