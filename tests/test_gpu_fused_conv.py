"""GPU parity of the chunk forward with the short convolutions inside the kernels
(``ops.chunk_gdn2_conv``, C entry ``gdn2_chunk_fwd_conv``).

* **Separate passes.** prep convolves q and k while landing their rows and the scan's copy
  waves convolve v while forming ``w * v``, with the order and roundings of
  ``short_conv_vec_kernel``; the result must equal ``ops.short_convolution`` followed by
  ``ops.chunk_gdn2`` (or ``ops.chunk_gdn2_gated_norm``) bit for bit: key widths 32 / 64 / 128,
  value widths 16 .. 128 (one or two value slices), ragged lengths, T = 1, an initial state,
  SiLU on and off, the in-kernel gate with b / w logits, and q / k / v read as column ranges of
  one wider projection output (the module's layout).
* **Packed sequences.** With ``cu_seqlens`` every sequence starts from zero history: equal to
  convolving each sequence on its own, then the packed chunk op.
* **Oracle.** Against ``oracle.short_conv`` -> ``oracle.recurrent_fwd`` (-> ``gated_rmsnorm``)
  in float64 on the same bf16 inputs, at the bf16 bar (rel. L2 <= 2e-2).
* **Module.** ``GatedDeltaNet2`` bf16 prefill takes the fused convolution, and its outputs and
  caches equal the ``fused_conv = False`` path bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as orc
from tests._helpers import rel_l2

pytestmark = pytest.mark.gpu


def _inputs(dev, B, T, H, K, V, seed, gate_logits=False, pad=24):
    """Raw projections as column ranges of one [B, T, 2HK + HV + pad] tensor, conv taps, g, b, w."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    HK, HV = H * K, H * V
    y = torch.randn(B, T, 2 * HK + HV + pad, generator=gen).to(torch.bfloat16).to(dev)
    raw = (y[..., :HK], y[..., HK:2 * HK], y[..., 2 * HK:2 * HK + HV])
    taps = [(torch.randn(d, 1, 4, generator=gen) * 0.5).to(torch.bfloat16).to(dev) for d in (HK, HK, HV)]
    if gate_logits:
        g = torch.randn(B, T, H, K, generator=gen).to(torch.bfloat16).to(dev)
        b = torch.randn(B, T, H, K, generator=gen).to(torch.bfloat16).to(dev)
        w = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    else:
        g = (-torch.nn.functional.softplus(torch.randn(B, T, H, K, generator=gen) + 2)).to(dev)
        b = torch.rand(B, T, H, K, generator=gen).to(torch.bfloat16).to(dev)
        w = torch.rand(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    return raw, taps, g, b, w


def _gate_kw(dev, H, K, seed):
    gen = torch.Generator(device="cpu").manual_seed(seed + 7)
    A_log = torch.log(torch.rand(H, generator=gen) * 15 + 1).to(dev)
    dt_bias = (torch.randn(H * K, generator=gen) * 0.5).to(dev)
    return dict(use_gate_in_kernel=True, A_log=A_log, dt_bias=dt_bias, bw_logits=True)


def _separate(raw, taps, g, b, w, H, K, V, act, h0, gate=None, nw=None, **kw):
    from qwendopamine_amd import ops

    B, T = raw[0].shape[:2]
    (q, k, v), _ = ops.short_convolution(list(raw), taps, [None] * 3, None, False, act)
    args = (q.view(B, T, H, K), k.view(B, T, H, K), v.view(B, T, H, V), g, b, w)
    if gate is not None:
        return ops.chunk_gdn2_gated_norm(*args, gate, nw, 1e-5, initial_state=h0, output_final_state=True,
                                         use_qk_l2norm_in_kernel=True, **kw)
    return ops.chunk_gdn2(*args, initial_state=h0, output_final_state=True, use_qk_l2norm_in_kernel=True, **kw)


@pytest.mark.parametrize("B,T,H,K,V,h0,act,logits", [
    (2, 200, 3, 64, 64, True, "silu", False),
    (1, 129, 2, 128, 128, False, "silu", False),
    (3, 65, 2, 32, 32, True, None, False),
    (2, 1, 2, 64, 64, True, "silu", False),
    (1, 300, 2, 128, 64, True, "silu", True),
    (2, 150, 4, 64, 16, False, "silu", True),
    (8, 512, 16, 128, 128, True, "silu", True),
])
def test_fused_conv_equals_separate_passes(gpu_device, B, T, H, K, V, h0, act, logits):
    from qwendopamine_amd import ops

    print(f"[case] fused conv vs separate passes B={B} T={T} H={H} K={K} V={V} h0={h0} act={act} "
          f"logits={logits}", flush=True)
    dev = gpu_device
    raw, taps, g, b, w = _inputs(dev, B, T, H, K, V, seed=T + K + V, gate_logits=logits)
    s0 = torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(3)).to(dev) * 0.1 if h0 else None
    kw = _gate_kw(dev, H, K, T) if logits else {}
    with torch.no_grad():
        o_sep, ht_sep = _separate(raw, taps, g, b, w, H, K, V, act, s0, **kw)
        o, ht = ops.chunk_gdn2_conv(*raw, taps, g, b, w, num_heads=H, activation=act, initial_state=s0,
                                    output_final_state=True, use_qk_l2norm_in_kernel=True, **kw)
    torch.cuda.synchronize()
    print(f"  bit-identical fraction {(o == o_sep).float().mean().item():.6f}", flush=True)
    assert o.shape == (B, T, H, V) and o.dtype == torch.bfloat16
    assert torch.equal(o, o_sep)
    assert torch.equal(ht, ht_sep)


@pytest.mark.parametrize("K,V,T", [(64, 64, 200), (128, 32, 97), (64, 16, 64)])
def test_fused_conv_with_gated_norm_equals_separate_passes(gpu_device, K, V, T):
    from qwendopamine_amd import ops

    B, H = 2, 3
    print(f"[case] fused conv + gated norm vs separate passes K={K} V={V} T={T}", flush=True)
    dev = gpu_device
    raw, taps, g, b, w = _inputs(dev, B, T, H, K, V, seed=K * V + T, gate_logits=True)
    gen = torch.Generator(device="cpu").manual_seed(T)
    gate = torch.randn(B, T, H * V + 40, generator=gen).to(torch.bfloat16).to(dev)[..., 8:8 + H * V]
    nw = (torch.randn(V, generator=gen) * 0.3 + 1).to(torch.bfloat16).to(dev)
    kw = _gate_kw(dev, H, K, T)
    with torch.no_grad():
        o_sep, ht_sep = _separate(raw, taps, g, b, w, H, K, V, "silu", None, gate=gate, nw=nw, **kw)
        o, ht = ops.chunk_gdn2_conv(*raw, taps, g, b, w, num_heads=H, gate=gate, norm_weight=nw,
                                    output_final_state=True, use_qk_l2norm_in_kernel=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(o, o_sep) and torch.equal(ht, ht_sep)


def test_fused_conv_packed_sequences_start_from_zero_history(gpu_device):
    from qwendopamine_amd import ops

    cu = [0, 70, 71, 200, 263, 330]
    H, K, V = 2, 64, 64
    print("[case] fused conv varlen", flush=True)
    dev = gpu_device
    raw, taps, g, b, w = _inputs(dev, 1, cu[-1], H, K, V, seed=31)
    convd = []
    for t in raw:
        parts = [ops.short_convolution([t[:, s:e].contiguous()], [taps[len(convd)]], [None], None, False,
                                       "silu")[0][0] for s, e in zip(cu[:-1], cu[1:])]
        convd.append(torch.cat(parts, dim=1))
    cu_t = torch.tensor(cu, dtype=torch.int64, device=dev)
    h0 = torch.randn(len(cu) - 1, H, K, V, device=dev) * 0.1
    T = cu[-1]
    with torch.no_grad():
        o_sep, ht_sep = ops.chunk_gdn2(convd[0].view(1, T, H, K), convd[1].view(1, T, H, K),
                                       convd[2].view(1, T, H, V), g, b, w, initial_state=h0,
                                       output_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t)
        o, ht = ops.chunk_gdn2_conv(*raw, taps, g, b, w, num_heads=H, initial_state=h0, output_final_state=True,
                                    use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert torch.equal(o, o_sep) and torch.equal(ht, ht_sep)


@pytest.mark.parametrize("V,norm", [(64, False), (32, True)])
def test_fused_conv_matches_oracle(gpu_device, V, norm):
    from qwendopamine_amd import ops

    B, T, H, K = 2, 170, 2, 64
    print(f"[case] fused conv vs oracle V={V} norm={norm}", flush=True)
    dev = gpu_device
    raw, taps, g, b, w = _inputs(dev, B, T, H, K, V, seed=V + 11)
    h0 = torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(5)).to(dev) * 0.1
    gate = nw = None
    if norm:
        gen = torch.Generator(device="cpu").manual_seed(9)
        gate = torch.randn(B, T, H * V, generator=gen).to(torch.bfloat16).to(dev)
        nw = (torch.randn(V, generator=gen) * 0.3 + 1).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        o, ht = ops.chunk_gdn2_conv(*raw, taps, g, b, w, num_heads=H, gate=gate, norm_weight=nw,
                                    initial_state=h0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    np64 = lambda t: t.detach().double().cpu().numpy()  # noqa: E731
    cq, ck, cv = (orc.short_conv(np64(x), np64(wt).reshape(-1, 4))[0] for x, wt in zip(raw, taps))
    o_ref, s_ref = orc.recurrent_fwd(cq.reshape(B, T, H, K), ck.reshape(B, T, H, K), cv.reshape(B, T, H, V),
                                     np64(g), np64(b), np64(w), np64(h0))
    if norm:
        o_ref = orc.gated_rmsnorm(o_ref, np64(gate).reshape(B, T, H, V), np64(nw), 1e-5)
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2


def test_fused_conv_gate_logits_matches_oracle(gpu_device):
    """The in-kernel gate on random logits with decay rates up to 16 (as the config-3 bench
    line): most 16-token diagonal blocks span more than 2^115 and a share of their 4-token
    quarters too, so the quarter-referred products and the exact within-quarter pair sums
    both run.  Against the float64 oracle on g = -exp(A_log) softplus(logit + dt_bias),
    b = sigmoid(logit), w = sigmoid(logit)."""
    from qwendopamine_amd import ops

    B, T, H, K, V = 2, 200, 4, 64, 64
    print(f"[case] fused conv, gate logits with wide decays, vs oracle B={B} T={T} H={H}", flush=True)
    dev = gpu_device
    raw, taps, g, b, w = _inputs(dev, B, T, H, K, V, seed=21, gate_logits=True)
    gen = torch.Generator(device="cpu").manual_seed(23)
    A_log = torch.log(torch.linspace(4.0, 16.0, H))
    dt_bias = torch.randn(H * K, generator=gen) * 0.5
    kw = dict(use_gate_in_kernel=True, A_log=A_log.to(dev), dt_bias=dt_bias.to(dev), bw_logits=True)
    with torch.no_grad():
        o, ht = ops.chunk_gdn2_conv(*raw, taps, g, b, w, num_heads=H, initial_state=None,
                                    output_final_state=True, use_qk_l2norm_in_kernel=True, **kw)
    torch.cuda.synchronize()
    np64 = lambda t: t.detach().double().cpu().numpy()  # noqa: E731
    x = np64(g) + dt_bias.double().numpy().reshape(H, K)
    g_ref = -np.exp(A_log.double().numpy()).reshape(H, 1) * np.logaddexp(0.0, x)
    sig = lambda t: 1.0 / (1.0 + np.exp(-np64(t)))  # noqa: E731
    G2 = g_ref[:, : T // 16 * 16].reshape(B, T // 16, 16, H, K) / np.log(2.0)
    wide16 = float((-G2.sum(2) > 115).mean())
    wide4 = float((-G2.reshape(B, T // 16, 4, 4, H, K).sum(3) > 115).any(2).mean())
    cq, ck, cv = (orc.short_conv(np64(xx), np64(wt).reshape(-1, 4))[0] for xx, wt in zip(raw, taps))
    o_ref, s_ref = orc.recurrent_fwd(cq.reshape(B, T, H, K), ck.reshape(B, T, H, K), cv.reshape(B, T, H, V),
                                     g_ref, sig(b), sig(w), None)
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  wide 16-token blocks {wide16:.3f}, with a wide quarter {wide4:.4f}; "
          f"rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert wide16 > 0.3 and wide4 > 0.0
    assert eo <= 2e-2 and es <= 2e-2


def test_fused_conv_rejects_unsupported(gpu_device):
    from qwendopamine_amd import ops

    dev = gpu_device
    raw, taps, g, b, w = _inputs(dev, 1, 70, 2, 64, 64, seed=1)
    with pytest.raises(NotImplementedError):  # width 3
        ops.chunk_gdn2_conv(*raw, [t[..., :3] for t in taps], g, b, w, num_heads=2)
    with pytest.raises(NotImplementedError):  # fp32 rows
        ops.chunk_gdn2_conv(*(t.float() for t in raw), taps, g, b.float(), w.float(), num_heads=2)
    raw96, taps96, g96, b96, w96 = _inputs(dev, 1, 70, 2, 96, 64, seed=1)
    with pytest.raises(NotImplementedError):  # key width 96 (not a whole kernel key width)
        ops.chunk_gdn2_conv(*raw96, taps96, g96, b96, w96, num_heads=2)


@pytest.mark.parametrize("B,heads,head_dim", [(2, 4, 64), (64, 4, 64), (2, 2, 128)])
def test_module_prefill_fused_conv_equals_separate(gpu_device, monkeypatch, B, heads, head_dim):
    """GatedDeltaNet2 bf16 prefill convolves q, k, v inside the chunk kernels; outputs and caches
    equal the separate convolution pass bit for bit."""
    from qwendopamine_amd import GatedDeltaNet2, ops

    print(f"[case] module prefill fused conv B={B} heads={heads} head_dim={head_dim}", flush=True)
    calls = []
    real = ops.chunk_gdn2_conv

    def counting(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    monkeypatch.setattr(ops, "chunk_gdn2_conv", counting)
    torch.manual_seed(0)
    hidden = heads * head_dim
    m = GatedDeltaNet2(hidden_size=hidden, num_heads=heads, head_dim=head_dim).to(gpu_device)
    m = m.to(torch.bfloat16).eval()
    x = torch.randn(B, 150, hidden, device=gpu_device).to(torch.bfloat16)
    res = {}
    for fused in (True, False):
        m.fused_conv = fused
        cache: dict = {}
        with torch.no_grad():
            out, _, cache = m(x, past_key_values=cache, use_cache=True)
        torch.cuda.synchronize()
        res[fused] = (out, cache["recurrent_state"], cache["conv_state"])
    assert len(calls) == 1
    assert torch.equal(res[True][0], res[False][0])
    assert torch.equal(res[True][1], res[False][1])
    for a, b_ in zip(res[True][2], res[False][2]):
        assert torch.equal(a, b_)
    assert np.isfinite(res[True][0].float().cpu().numpy()).all()
