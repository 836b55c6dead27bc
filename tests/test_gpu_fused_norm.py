"""GPU parity of the chunk forward with the gated output norm in the scan's output stage
(``ops.chunk_gdn2_gated_norm``, C entry ``gdn2_chunk_fwd_gated_norm``).

* **Separate passes.** The fused op reproduces ``gated_rmsnorm_vec_kernel``'s summation order
  and roundings, so it must equal ``ops.chunk_gdn2`` followed by ``ops.gated_rmsnorm`` bit for
  bit: value head dims 16 / 32 / 64, ragged lengths (a last chunk of 1 token included),
  varlen, an initial state, the in-kernel gate with b / w logits, and a gate read as a column
  range of a wider tensor.
* **Oracle.** Against the float64 composition ``oracle.recurrent_fwd`` -> ``oracle.gated_rmsnorm``
  on the same bf16-rounded inputs, at the bf16 bar (rel. L2 <= 2e-2).
* **Module.** ``GatedDeltaNet2`` bf16 prefill takes the fused norm exactly when a scan workgroup
  owns whole value rows anyway (16-wide heads, or >= 256 sequence-heads), through
  ``chunk_gdn2_gated_norm`` or, with the convolutions also in the kernels, ``chunk_gdn2_conv``;
  with ``fused_norm`` on and off, outputs and caches are then bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as orc
from tests._helpers import rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu
NAMES = ("q", "k", "v", "g", "b", "w")


def _gate(dev, B, T, H, V, seed, wide=0):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    z = torch.randn(B, T, H * V + wide, generator=gen).to(torch.bfloat16).to(dev)
    return z[..., wide // 2: wide // 2 + H * V] if wide else z


def _nw(dev, V, seed):
    gen = torch.Generator(device="cpu").manual_seed(seed + 1)
    return (torch.randn(V, generator=gen) * 0.3 + 1.0).to(torch.bfloat16).to(dev)


@pytest.mark.parametrize("K,V,T,h0", [(64, 64, 200, True), (128, 64, 129, False), (32, 32, 65, True),
                                      (64, 16, 64, False), (128, 64, 1, True), (64, 64, 4096, True)])
def test_fused_norm_equals_separate_passes(gpu_device, K, V, T, h0):
    from qwendopamine_amd import ops

    B, H = 2, 3
    print(f"[case] fused norm vs separate passes K={K} V={V} T={T} h0={h0}", flush=True)
    inp = rand_inputs(B, T, H, K, V, seed=K + V + T, h0_std=0.1 if h0 else 0.0)
    t, _ = to_device(inp, gpu_device, torch.bfloat16)
    z, nw = _gate(gpu_device, B, T, H, V, seed=T), _nw(gpu_device, V, seed=T)
    args = [t[n] for n in NAMES]
    with torch.no_grad():
        o_sep, ht_sep = ops.chunk_gdn2(*args, initial_state=t["h0"], output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)
        on_sep = ops.gated_rmsnorm(o_sep, z.view(B, T, H, V), nw, 1e-5)
        on, ht = ops.chunk_gdn2_gated_norm(*args, z, nw, 1e-5, initial_state=t["h0"], output_final_state=True,
                                           use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    same = (on == on_sep).float().mean().item()
    print(f"  bit-identical fraction {same:.6f}", flush=True)
    assert on.dtype == torch.bfloat16 and on.shape == (B, T, H, V)
    assert torch.equal(on, on_sep)
    assert torch.equal(ht, ht_sep)


def test_fused_norm_gate_logits_wide_gate_rows(gpu_device):
    """In-kernel gate with b / w logits (the module's inference call) and a gate read as a
    column range of a wider tensor."""
    from qwendopamine_amd import ops

    B, T, H, K, V = 2, 150, 4, 64, 64
    print("[case] fused norm, in-kernel gate, b / w logits, strided gate rows", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(5)
    dev = gpu_device
    q, k = (torch.randn(B, T, H, K, generator=gen).to(torch.bfloat16).to(dev) for _ in range(2))
    v = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    f = torch.randn(B, T, H, K, generator=gen).to(torch.bfloat16).to(dev)
    bl = torch.randn(B, T, H, K, generator=gen).to(torch.bfloat16).to(dev)
    wl = torch.randn(B, T, H, V, generator=gen).to(torch.bfloat16).to(dev)
    A_log = torch.log(torch.rand(H, generator=gen) * 15 + 1).to(dev)
    dt_bias = (torch.randn(H * K, generator=gen) * 0.5).to(dev)
    z = _gate(dev, B, T, H, V, seed=9, wide=40)
    nw = _nw(dev, V, seed=9)
    kw = dict(use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, A_log=A_log, dt_bias=dt_bias,
              bw_logits=True)
    with torch.no_grad():
        o_sep, ht_sep = ops.chunk_gdn2(q, k, v, f, bl, wl, output_final_state=True, **kw)
        on_sep = ops.gated_rmsnorm(o_sep, z.reshape(B, T, H, V), nw, 1e-5)
        on, ht = ops.chunk_gdn2_gated_norm(q, k, v, f, bl, wl, z, nw, 1e-5, output_final_state=True, **kw)
    torch.cuda.synchronize()
    assert z.stride(1) == H * V + 40
    assert torch.equal(on, on_sep) and torch.equal(ht, ht_sep)


def test_fused_norm_varlen(gpu_device):
    from qwendopamine_amd import ops

    cu = [0, 70, 70, 71, 200, 263]
    H, K, V = 2, 64, 64
    print("[case] fused norm varlen", flush=True)
    inp = rand_inputs(1, cu[-1], H, K, V, seed=21, h0_std=0.0)
    t, _ = to_device(inp, gpu_device, torch.bfloat16)
    z, nw = _gate(gpu_device, 1, cu[-1], H, V, seed=21), _nw(gpu_device, V, seed=21)
    cu_t = torch.tensor(cu, dtype=torch.int64, device=gpu_device)
    h0 = torch.randn(len(cu) - 1, H, K, V, device=gpu_device) * 0.1
    args = [t[n] for n in NAMES]
    with torch.no_grad():
        o_sep, ht_sep = ops.chunk_gdn2(*args, initial_state=h0, output_final_state=True,
                                       use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t)
        on_sep = ops.gated_rmsnorm(o_sep, z.view(1, cu[-1], H, V), nw, 1e-5)
        on, ht = ops.chunk_gdn2_gated_norm(*args, z, nw, 1e-5, initial_state=h0, output_final_state=True,
                                           use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert torch.equal(on, on_sep) and torch.equal(ht, ht_sep)


@pytest.mark.parametrize("V", [16, 64])
def test_fused_norm_matches_oracle(gpu_device, V):
    from qwendopamine_amd import ops

    B, T, H, K = 2, 170, 2, 64
    print(f"[case] fused norm vs oracle V={V}", flush=True)
    inp = rand_inputs(B, T, H, K, V, seed=V + 3)
    t, r = to_device(inp, gpu_device, torch.bfloat16)
    z, nw = _gate(gpu_device, B, T, H, V, seed=V), _nw(gpu_device, V, seed=V)
    with torch.no_grad():
        on, ht = ops.chunk_gdn2_gated_norm(*(t[n] for n in NAMES), z, nw, 1e-5, initial_state=t["h0"],
                                           output_final_state=True, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES), r["h0"])
    zr = z.double().cpu().numpy().reshape(B, T, H, V)
    on_ref = orc.gated_rmsnorm(o_ref, zr, nw.double().cpu().numpy(), 1e-5)
    eo, es = rel_l2(on, on_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2


def test_fused_norm_rejects_unsupported(gpu_device):
    from qwendopamine_amd import ops

    inp = rand_inputs(1, 70, 2, 64, 128, seed=1)
    t, _ = to_device(inp, gpu_device, torch.bfloat16)
    z, nw = _gate(gpu_device, 1, 70, 2, 128, seed=1), _nw(gpu_device, 128, seed=1)
    with pytest.raises(NotImplementedError):
        ops.chunk_gdn2_gated_norm(*(t[n] for n in NAMES), z, nw)
    t32, _ = to_device(rand_inputs(1, 70, 2, 64, 64, seed=1), gpu_device, torch.float32)
    with pytest.raises(NotImplementedError):
        ops.chunk_gdn2_gated_norm(*(t32[n] for n in NAMES), z[..., :128].float(), nw[:64].float())


@pytest.mark.parametrize("B,heads,head_dim,padded", [(2, 4, 16, False), (64, 4, 64, False), (64, 4, 64, True),
                                                     (2, 4, 64, False)])
def test_module_prefill_fused_norm_equals_separate(gpu_device, monkeypatch, B, heads, head_dim, padded):
    """GatedDeltaNet2 bf16 prefill: the module takes the fused norm exactly when a scan
    workgroup owns whole value rows anyway (16-wide heads, or >= 256 sequence-heads), and
    its outputs and caches then equal the separate norm pass bit for bit."""
    from qwendopamine_amd import GatedDeltaNet2, ops

    print(f"[case] module prefill fused norm B={B} heads={heads} head_dim={head_dim} padded={padded}",
          flush=True)
    calls = []
    real, real_conv = ops.chunk_gdn2_gated_norm, ops.chunk_gdn2_conv

    def counting(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    def counting_conv(*a, **kw):  # the norm in the scan of the conv-fused prefill
        if kw.get("gate") is not None:
            calls.append(1)
        return real_conv(*a, **kw)

    monkeypatch.setattr(ops, "chunk_gdn2_gated_norm", counting)
    monkeypatch.setattr(ops, "chunk_gdn2_conv", counting_conv)
    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=256, num_heads=heads, head_dim=head_dim).to(gpu_device).to(torch.bfloat16).eval()
    x = torch.randn(B, 150, 256, device=gpu_device).to(torch.bfloat16)
    mask = None
    if padded:
        mask = torch.ones(B, 150, dtype=torch.long, device=gpu_device)
        mask[1, :37] = 0
    res = {}
    for fused in (True, False):
        m.fused_norm = fused
        cache: dict = {}
        with torch.no_grad():
            out, _, cache = m(x, attention_mask=mask, past_key_values=cache, use_cache=True)
        torch.cuda.synchronize()
        res[fused] = (out, cache["recurrent_state"])
    expect = head_dim == 16 or B * heads >= 256
    assert len(calls) == (1 if expect else 0)
    assert torch.equal(res[True][0], res[False][0])
    assert torch.equal(res[True][1], res[False][1])
