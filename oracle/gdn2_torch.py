r"""PyTorch CPU restatement of the gdn2 recurrence, float32 -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` import this module:
it is the CPU baseline that BASELINE's plan times (the reference's own CPU path
is PyTorch), never a fallback of the product package.

* ``recurrent_fwd`` restates ``torch_recurrent_gdn2`` (reference
  ``models/gdn2/gdn2.py:100-184``) in the precision it computes in: inputs
  upcast to float32 (``:132-137``), ``F.normalize(eps=1e-6)`` on q and k
  (``:139-141``), q scaled after the norm (``:143-144``), then per token
  ``S <- S * exp(g)``, ``r = S^T (b * k)``, ``u = w * v - r``, ``S <- S + k u^T``,
  ``o = S^T q`` (``:156-179``), batched over (sequence, head).  The output is
  returned in the input dtype, the final state in float32.
* ``chunk_fwd`` is the numerically safe chunkwise form (relative decays
  ``exp(G_r - G_i) <= 1`` only, chunk 64) of the same recurrence: the reference's
  own chunk form (``gdn2.py:243-369``) divides by absolute decays and underflows
  under BASELINE's decay distribution.  The WY system ``(I + L)`` is solved with
  ``torch.linalg.solve_triangular`` as the reference's helper does
  (``gdn2.py:187-213``).

Both are pinned against the float64 oracle (``oracle/gdn2_oracle.py``, itself
pinned by closed forms, the third-party scalar gated delta rule and finite
differences) in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["recurrent_fwd", "chunk_fwd"]


def _prep(q, k, v, g, b, w, scale, l2norm):
    q, k, v, g, b, w = (x.float() for x in (q, k, v, g, b, w))
    if l2norm:
        q = F.normalize(q, p=2, dim=-1, eps=1e-6)
        k = F.normalize(k, p=2, dim=-1, eps=1e-6)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    # [B, T, H, D] -> [B, H, T, D]
    return tuple(x.transpose(1, 2).contiguous() for x in (q * scale, k, v, g, b, w))


@torch.no_grad()
def recurrent_fwd(q, k, v, g, b, w, initial_state=None, scale=None, use_qk_l2norm_in_kernel=True):
    """Token-by-token recurrence; ``[B,T,H,*]`` in, ``(o [B,T,H,V], S [B,H,K,V] float32)`` out."""
    dt = q.dtype
    B, T, H, K = q.shape
    V = v.shape[-1]
    q, k, v, g, b, w = _prep(q, k, v, g, b, w, scale, use_qk_l2norm_in_kernel)
    S = torch.zeros(B, H, K, V) if initial_state is None else initial_state.float().clone()
    o = torch.empty(B, H, T, V)
    for t in range(T):
        S.mul_(g[:, :, t].exp().unsqueeze(-1))
        r = torch.einsum("bhkv,bhk->bhv", S, b[:, :, t] * k[:, :, t])
        u = w[:, :, t] * v[:, :, t] - r
        S.add_(k[:, :, t].unsqueeze(-1) * u.unsqueeze(-2))
        o[:, :, t] = torch.einsum("bhkv,bhk->bhv", S, q[:, :, t])
    return o.transpose(1, 2).to(dt), S


@torch.no_grad()
def chunk_fwd(q, k, v, g, b, w, initial_state=None, scale=None, use_qk_l2norm_in_kernel=True,
              chunk_size=64):
    """Chunkwise WY form with relative decays (same outputs as ``recurrent_fwd``)."""
    dt = q.dtype
    B, T, H, K = q.shape
    V = v.shape[-1]
    q, k, v, g, b, w = _prep(q, k, v, g, b, w, scale, use_qk_l2norm_in_kernel)
    S = torch.zeros(B, H, K, V) if initial_state is None else initial_state.float().clone()
    o = torch.empty(B, H, T, V)
    for t0 in range(0, T, chunk_size):
        t1 = min(T, t0 + chunk_size)
        C = t1 - t0
        qc, kc, vc, bc, wc = (x[:, :, t0:t1] for x in (q, k, v, b, w))
        G = g[:, :, t0:t1].cumsum(2)  # [B,H,C,K]
        causal = torch.ones(C, C, dtype=torch.bool).tril()
        diff = G.unsqueeze(3) - G.unsqueeze(2)  # (r, i): G_r - G_i, [B,H,C,C,K]
        rel = torch.where(causal[:, :, None], diff, torch.full_like(diff, float("-inf"))).exp()
        e = bc * kc
        Aqk = torch.einsum("bhrd,bhid,bhrid->bhri", qc, kc, rel)
        L = torch.einsum("bhrd,bhid,bhrid->bhri", e, kc, rel).tril(-1)
        IL = L + torch.eye(C)
        eG = G.exp()
        Wm = torch.linalg.solve_triangular(IL, e * eG, upper=False, unitriangular=True)
        U0 = torch.linalg.solve_triangular(IL, wc * vc, upper=False, unitriangular=True)
        U = U0 - Wm @ S
        o[:, :, t0:t1] = (qc * eG) @ S + Aqk @ U
        Gl = G[:, :, -1]  # [B,H,K]
        S = Gl.exp().unsqueeze(-1) * S + (kc * (Gl.unsqueeze(2) - G).exp()).transpose(-1, -2) @ U
    return o.transpose(1, 2).to(dt), S
