"""GPU tests of the drop-in GatedDeltaNet2 module (reference tests/models/test_gdn2.py
behaviours), with the recurrence on the HIP kernels."""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import rel_l2

pytestmark = pytest.mark.gpu


def _layer(dev, **kw):
    from qwendopamine_amd import GatedDeltaNet2

    torch.manual_seed(kw.pop("seed", 0))
    kw.setdefault("hidden_size", 64)
    kw.setdefault("num_heads", 2)
    kw.setdefault("head_dim", 32)
    return GatedDeltaNet2(**kw).to(dev)


def _oracle_module_forward(m, x):
    """The module forward composed from its own torch prologue/epilogue and the
    float64 oracle recurrence (reference gdn2.py:815-999), no cache."""
    with torch.no_grad():
        xf = x.float()
        mf = m.float()
        if mf.use_short_conv:
            q, _ = mf.q_conv1d(mf.q_proj(xf))
            k, _ = mf.k_conv1d(mf.k_proj(xf))
            v, _ = mf.v_conv1d(mf.v_proj(xf))
        else:
            q, k, v = F.silu(mf.q_proj(xf)), F.silu(mf.k_proj(xf)), F.silu(mf.v_proj(xf))
        A = mf.A_log.exp().repeat_interleave(mf.head_k_dim)
        g = -A * F.softplus(mf.f_proj(xf) + mf.dt_bias)
        b, w = mf.b_proj(xf).sigmoid(), mf.w_proj(xf).sigmoid()
        rep = mf.num_v_heads // mf.num_heads  # grouped value heads (gdn2.py:859-863)
        sp = lambda t, d, r=1: t.reshape(*t.shape[:-1], -1, d).repeat_interleave(r, dim=-2).double().cpu().numpy()  # noqa: E731
        o, _ = orc.recurrent_fwd(sp(q, mf.head_k_dim, rep), sp(k, mf.head_k_dim, rep), sp(v, mf.head_v_dim),
                                 sp(g, mf.head_k_dim, rep), sp(b, mf.head_k_dim, rep), sp(w, mf.head_v_dim))
        o = torch.from_numpy(o).float().to(x.device)
        gate = mf.g_proj(xf).reshape(*o.shape)
        o = mf.o_norm(o, gate)
        return mf.o_proj(o.reshape(*o.shape[:-2], -1))


@pytest.mark.parametrize("T,training", [(16, False), (150, False), (150, True)])
def test_module_matches_oracle_composition(gpu_device, T, training):
    print(f"[case] module parity T={T} training={training}", flush=True)
    m = _layer(gpu_device, hidden_size=128, num_heads=4, head_dim=32)
    m.train(training)
    x = torch.randn(2, T, 128, device=gpu_device)
    with torch.no_grad():
        out, attn, _ = m(x)
    assert out.shape == (2, T, 128) and attn is None
    ref = _oracle_module_forward(m, x)
    assert rel_l2(out, ref) <= 1e-4


def test_backends_agree(gpu_device):
    """Reference test_gdn2.py:68-93: every backend name gives the same output."""
    print("[case] backends agree", flush=True)
    from qwendopamine_amd import GatedDeltaNet2

    made = {}
    for be in ("torch", "torch-chunk", "torch-recurrent", "auto", "hip", "triton"):
        torch.manual_seed(0)
        made[be] = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32, backend=be,
                                  chunk_size=8, use_short_conv=False).to(gpu_device).eval()
    for layer in made.values():
        layer.load_state_dict(made["torch"].state_dict())
    x = torch.randn(1, 16, 64, device=gpu_device)
    with torch.no_grad():
        ref = made["torch"](x)[0]
        for be, layer in made.items():
            assert torch.allclose(layer(x)[0], ref, atol=1e-5), be


def test_config_init_forward(gpu_device):
    from qwendopamine_amd import GatedDeltaNet2
    from tests.test_module_cpu import DummyConfig

    m = GatedDeltaNet2(DummyConfig(hidden_size=128, num_heads=4, head_dim=32), layer_idx=0).to(gpu_device)
    out, _, _ = m(torch.randn(2, 8, 128, device=gpu_device))
    assert out.shape == (2, 8, 128)


def test_dict_cache_decode_continues_prefill(gpu_device):
    """Prefill with a dict cache, then single-token decode steps, equals one long forward."""
    print("[case] cache continuation", flush=True)
    m = _layer(gpu_device, layer_idx=0).eval()
    x = torch.randn(1, 40, 64, device=gpu_device)
    with torch.no_grad():
        full, _, _ = m(x)
        cache: dict = {}
        pre, _, _ = m(x[:, :37], past_key_values=cache, use_cache=True)
        assert cache["recurrent_state"].dtype == torch.float32
        assert cache["recurrent_state"].shape == (1, 2, 32, 32)
        assert len(cache["conv_state"]) == 3 and cache["conv_state"][0].shape == (1, 64, 3)
        steps = [m(x[:, t:t + 1], past_key_values=cache, use_cache=True)[0] for t in range(37, 40)]
    assert rel_l2(pre, full[:, :37]) <= 1e-4
    assert rel_l2(torch.cat(steps, 1), full[:, 37:]) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_updates_cache_in_place(gpu_device, dtype):
    """update_cache_in_place (an extension keyword): decode steps write the new recurrent
    and conv states into the cache's own tensors, with results identical to the default
    (fresh tensors) path."""
    print(f"[case] in-place cache update {dtype}", flush=True)
    m = _layer(gpu_device, layer_idx=0).to(dtype).eval()
    x = torch.randn(2, 24, 64, device=gpu_device, dtype=dtype)
    with torch.no_grad():
        c_ref: dict = {}
        c_inp: dict = {}
        m(x[:, :20], past_key_values=c_ref, use_cache=True)
        m(x[:, :20], past_key_values=c_inp, use_cache=True)
        state, convs = c_inp["recurrent_state"], c_inp["conv_state"]
        for t in range(20, 24):
            o_ref, _, _ = m(x[:, t:t + 1], past_key_values=c_ref, use_cache=True)
            o_inp, _, _ = m(x[:, t:t + 1], past_key_values=c_inp, use_cache=True, update_cache_in_place=True)
            assert c_inp["recurrent_state"] is state
            assert all(a is b for a, b in zip(c_inp["conv_state"], convs))
            assert torch.equal(o_inp, o_ref)
            assert torch.equal(state, c_ref["recurrent_state"])
            assert all(torch.equal(a, b) for a, b in zip(convs, c_ref["conv_state"]))


def test_incremental_decoding_updates_state(gpu_device):
    m = _layer(gpu_device, layer_idx=0)
    cache: dict = {}
    m(torch.randn(1, 1, 64, device=gpu_device), past_key_values=cache, use_cache=True)
    s1 = cache["recurrent_state"]
    m(torch.randn(1, 1, 64, device=gpu_device), past_key_values=cache, use_cache=True)
    s2 = cache["recurrent_state"]
    assert not torch.allclose(s1, s2)
    assert "conv_state" in cache


def test_dynamic_cache_runs(gpu_device):
    cu = pytest.importorskip("transformers.cache_utils")
    m = _layer(gpu_device, layer_idx=0)
    out, _, past = m(torch.randn(1, 1, 64, device=gpu_device), past_key_values=cu.DynamicCache(),
                     use_cache=True)
    assert out.shape == (1, 1, 64) and past is not None


def test_padding_tokens_are_zeroed(gpu_device):
    """Reference test_gdn2.py:367-379.  The packed run resets the recurrent state
    per sequence (cu_seqlens), while the short convolution ignores cu_seqlens as
    in the reference (gdn2.py:400), so only the first packed sequence is
    independent of its neighbours and must equal its standalone run."""
    m = _layer(gpu_device, chunk_size=8)
    x = torch.randn(2, 6, 64, device=gpu_device)
    mask = torch.tensor([[1, 1, 1, 1, 1, 1], [1, 1, 1, 0, 0, 0]], device=gpu_device)
    out, _, _ = m(x, attention_mask=mask)
    assert torch.all(out[1, 3:] == 0)
    assert not torch.allclose(out, m(x)[0])
    alone, _, _ = m(x[0:1])
    assert rel_l2(out[0], alone[0]) <= 1e-4


def test_bf16_forward_finite(gpu_device):
    m = _layer(gpu_device).to(torch.bfloat16)
    out, _, _ = m(torch.randn(2, 8, 64, device=gpu_device, dtype=torch.bfloat16))
    assert out.dtype == torch.bfloat16 and torch.isfinite(out.float()).all()


@pytest.mark.parametrize("T", [20, 150])
def test_gva_module(gpu_device, T):
    """Grouped value heads (num_v_heads = 2 num_heads) in inference, where the decay
    activation runs in-kernel with each key head's A_log / dt_bias repeated for its value
    heads (and, at T <= 64, the b / w sigmoids too), against the oracle composition."""
    print(f"[case] GVA module T={T}", flush=True)
    m = _layer(gpu_device, hidden_size=64, num_heads=2, head_dim=16, num_v_heads=4).eval()
    x = torch.randn(1, T, 64, device=gpu_device)
    with torch.no_grad():
        out, _, _ = m(x)
    assert out.shape == (1, T, 64) and torch.isfinite(out).all()
    assert rel_l2(out, _oracle_module_forward(m, x)) <= 1e-4
