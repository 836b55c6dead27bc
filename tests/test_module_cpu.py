"""CPU tests of the drop-in boundary's host logic (no kernel launches).

Mirrors the reference's construction / registry / config / cache tests
(tests/models/test_gdn2.py, test_gdn2_model.py, test_gdn2_params.py).  The
recurrence itself needs a GPU; running the module on CPU tensors must raise.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from qwendopamine_amd import (
    BLOCKS,
    GDN2_BACKENDS,
    GatedDeltaNet2,
    GDN2Config,
    GDN2Host,
    RMSNormGated,
    ShortConvolution,
    build_block,
    resolve_gdn2_backend,
)
from qwendopamine_amd.gdn2 import _get_unpad_data, _index_first_axis, _pad_input


class DummyConfig:
    def __init__(self, hidden_size=128, num_heads=4, head_dim=32, conv_size=4, rms_norm_eps=1e-5):
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.n_head = num_heads
        self.head_size = head_dim
        self.conv_size = conv_size
        self.norm_eps = rms_norm_eps
        self.rms_norm_eps = rms_norm_eps
        self.allow_neg_eigval = False
        self.expand_v = 1.0


def test_parameter_names_and_shapes_match_reference_layout():
    m = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32)
    shapes = {n: tuple(p.shape) for n, p in m.named_parameters()}
    assert shapes == {
        "A_log": (2,), "dt_bias": (64,),
        "q_proj.weight": (64, 64), "k_proj.weight": (64, 64), "v_proj.weight": (64, 64),
        "q_conv1d.conv1d.weight": (64, 1, 4), "k_conv1d.conv1d.weight": (64, 1, 4),
        "v_conv1d.conv1d.weight": (64, 1, 4),
        "f_proj.0.weight": (32, 64), "f_proj.1.weight": (64, 32),
        "b_proj.weight": (64, 64), "w_proj.weight": (64, 64),
        "g_proj.0.weight": (32, 64), "g_proj.1.weight": (64, 32), "g_proj.1.bias": (64,),
        "o_norm.weight": (32,), "o_proj.weight": (64, 64),
    }


def test_1_3b_layer_parameter_count():
    """Reference test_gdn2_params.py:36-68 (18 heads x 128)."""
    m = GatedDeltaNet2(hidden_size=2304, num_heads=18, head_dim=128, num_v_heads=18, expand_v=1.0,
                       use_short_conv=True, conv_size=4, layer_idx=0)
    kd = vd = 18 * 128
    hv = 128
    expected = (2304 * kd * 2 + 2304 * vd + kd * 4 * 2 + vd * 4 + 2304 * hv + hv * kd + 2304 * kd
                + 2304 * vd + 2304 * hv + hv * vd + vd + vd * 2304 + hv + 18 + kd)
    assert sum(p.numel() for p in m.parameters()) == expected


def test_config_object_aliases_and_layer_idx():
    m = GatedDeltaNet2(DummyConfig(hidden_size=128, num_heads=4, head_dim=32), layer_idx=3)
    assert (m.hidden_size, m.num_heads, m.head_dim, m.num_v_heads, m.layer_idx) == (128, 4, 32, 4, 3)
    assert m.conv_size == 4 and m.norm_eps == 1e-5


def test_registry_and_positional_build_block_quirk():
    assert BLOCKS["gdn2"] is GatedDeltaNet2 and BLOCKS["qwen35_gdn2"] is GatedDeltaNet2
    m = build_block("gdn2", DummyConfig(hidden_size=64, num_heads=2, head_dim=32), layer_idx=5)
    assert isinstance(m, GatedDeltaNet2)
    assert m.layer_idx is None  # the positional layer index lands in hidden_size, then overridden
    with pytest.raises(KeyError):
        build_block("nope", DummyConfig(), 0)


def test_constructor_validation():
    with pytest.raises(ValueError):
        GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32, backend="nope")
    with pytest.raises(ValueError):
        GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32, num_v_heads=3)


def test_backend_resolution():
    for be in GDN2_BACKENDS:
        expect = "hip" if be == "auto" else be
        assert resolve_gdn2_backend(be, training=True, seq_len=64) == expect
    with pytest.raises(ValueError):
        resolve_gdn2_backend("cuda", training=False, seq_len=1)


def test_init_ranges_and_flags():
    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32)
    a = m.A_log.exp()
    assert bool((a >= 1.0).all() and (a <= 16.0).all())
    dt = torch.nn.functional.softplus(m.dt_bias)
    assert bool((dt >= 1e-4 * 0.999).all() and (dt <= 0.1 * 1.001).all())
    assert m.fp32_decay is True
    assert getattr(m.A_log, "_no_weight_decay", False) and getattr(m.dt_bias, "_no_weight_decay", False)
    assert getattr(m.q_proj, "_is_hf_initialized", False)
    bound = 2**-2.5 * math.sqrt(6.0 / (64 + 64))
    assert float(m.q_proj.weight.abs().max()) <= bound + 1e-7
    assert torch.all(m.o_norm.weight == 1) and torch.all(m.g_proj[1].bias == 0)


def test_config_presets_and_host_init():
    assert GDN2Config.from_name("gdn2_1.3B").hidden_size == 2304
    with pytest.raises(KeyError):
        GDN2Config.from_name("nope")
    cfg = GDN2Config(hidden_size=64, num_heads=2, head_dim=32, num_layers=2)
    host = GDN2Host(cfg)
    assert host.embed.weight.shape == (cfg.vocab_size, 64)
    assert not torch.all(host.embed.weight == 0)
    assert torch.allclose(host.norm.weight, torch.ones_like(host.norm.weight))
    assert getattr(host.layers[0].attn.q_proj, "_is_hf_initialized", False)


def test_module_on_cpu_raises_no_cpu_path():
    m = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32)
    with pytest.raises(RuntimeError, match="no CPU path"):
        m(torch.randn(1, 4, 64))


def test_ops_on_cpu_raise():
    from qwendopamine_amd import chunk_gdn2, fused_recurrent_gdn2

    x = torch.randn(1, 4, 2, 16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        chunk_gdn2(x, x, x, -x.abs(), x.sigmoid(), x.sigmoid())
    with pytest.raises(RuntimeError, match="no CPU path"):
        fused_recurrent_gdn2(x, x, x, -x.abs(), x.sigmoid(), x.sigmoid())


def test_short_convolution_matches_direct_causal_sum():
    torch.manual_seed(1)
    conv = ShortConvolution(6, kernel_size=4, bias=True)
    x = torch.randn(2, 9, 6)
    y, cache = conv(x, output_final_state=True)
    wgt, bias = conv.conv1d.weight[:, 0], conv.conv1d.bias
    ref = torch.zeros_like(x)
    for t in range(9):
        for j in range(4):
            s = t - 3 + j
            if s >= 0:
                ref[:, t] += wgt[:, j] * x[:, s]
    ref = torch.nn.functional.silu(ref + bias)
    assert torch.allclose(y, ref, atol=1e-6)
    assert torch.equal(cache, x.transpose(1, 2)[:, :, -3:])
    # one more token through the cache equals the prefill of 10 tokens
    x1 = torch.randn(2, 1, 6)
    y1, cache1 = conv(x1, cache=cache, output_final_state=True)
    yfull, _ = conv(torch.cat([x, x1], 1))
    assert torch.allclose(y1[:, 0], yfull[:, -1], atol=1e-6)
    assert torch.equal(cache1[:, :, -1], x1[:, 0])


def test_rms_norm_gated_formula():
    n = RMSNormGated(8, eps=1e-5)
    with torch.no_grad():
        n.weight.copy_(torch.linspace(0.5, 1.5, 8))
    x, z = torch.randn(3, 8), torch.randn(3, 8)
    ref = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-5) * n.weight * z * torch.sigmoid(z)
    assert torch.allclose(n(x, z), ref, atol=1e-6)


def test_unpad_pad_roundtrip():
    mask = torch.tensor([[1, 1, 1, 0], [1, 0, 0, 0]])
    idx, cu, mx = _get_unpad_data(mask)
    assert idx.tolist() == [0, 1, 2, 4] and cu.tolist() == [0, 3, 1 + 3] and mx == 3
    x = torch.randn(2, 4, 5)
    packed = _index_first_axis(x, idx)
    back = _pad_input(packed, idx, 2, 4)
    assert torch.equal(back[mask.bool()], x[mask.bool()]) and torch.all(back[~mask.bool()] == 0)


def test_dict_and_hf_cache_roundtrip_on_cpu():
    m = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32, layer_idx=0)
    rec = torch.randn(1, 2, 32, 32)
    conv = (torch.randn(1, 64, 3), torch.randn(1, 64, 3), torch.randn(1, 64, 3))
    d: dict = {}
    m._update_cache(d, rec, conv)
    r2, c2 = m._get_cache(d)
    assert r2 is rec and c2 is conv
    cache_utils = pytest.importorskip("transformers.cache_utils")
    if not hasattr(cache_utils, "LinearAttentionCacheLayerMixin"):
        pytest.skip("LinearAttentionCacheLayerMixin not available")

    class Layer(cache_utils.LinearAttentionCacheLayerMixin):
        def __init__(self):
            super().__init__(number_of_states=1)

        def lazy_initialization(self, conv_states=None, recurrent_states=None, state_idx=0):
            pass

        def update_recurrent_state(self, recurrent_states, state_idx=0, **kw):
            self.recurrent_states[state_idx] = recurrent_states
            return recurrent_states

        def update_conv_state(self, conv_states, state_idx=0, **kw):
            for i, s in enumerate(conv_states):
                self.conv_states[i] = s
            return conv_states

    layer = Layer()
    cache = cache_utils.Cache(layers=[layer])
    m._update_cache(cache, rec, conv)
    r3, c3 = m._get_cache(cache)
    assert r3 is rec and all(a is b for a, b in zip(c3, conv))


def test_product_package_never_touches_the_oracle():
    """No file of the product package imports, loads or runs anything under oracle/."""
    from pathlib import Path

    pkg = Path(__file__).resolve().parents[1] / "qwendopamine_amd"
    files = [p for p in pkg.rglob("*") if p.suffix in (".py", ".hip", ".h")]
    assert files
    for p in files:
        text = p.read_text()
        for needle in ("from oracle", "import oracle", "libgdn2_cpu", "gdn2_oracle", "cpu_lib"):
            assert needle not in text, f"{p.name} references {needle}"
    assert np is not None


def test_stacked_input_weight_is_the_only_copy():
    """The inference path's stacked projection weight holds the parameters' storage (one
    copy), survives an inference-mode build for later training, follows optimiser steps
    and load_state_dict in place, and is rebuilt after a dtype conversion."""
    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32)
    sd = {k: v.clone() for k, v in m.state_dict().items()}
    with torch.inference_mode():
        W, sizes = m._fused_input_weight()
    assert not W.is_inference() and sum(sizes) == W.shape[0]
    assert m.q_proj.weight.data_ptr() == W.data_ptr()
    assert m.g_proj[0].weight.data_ptr() == W[-sizes[-1]:].data_ptr()
    assert all(torch.equal(sd[k], v) for k, v in m.state_dict().items())
    x = torch.randn(3, 64)
    (m.q_proj(x).sum() + m.w_proj(x).sum()).backward()
    torch.optim.SGD(m.parameters(), lr=0.1).step()
    W2, _ = m._fused_input_weight()
    assert W2 is W and torch.equal(W2[:64], m.q_proj.weight.detach())
    assert not torch.equal(W2[:64], sd["q_proj.weight"])
    m.load_state_dict(sd)
    assert torch.equal(m._fused_input_weight()[0][:64], sd["q_proj.weight"])
    m.double()
    W3, _ = m._fused_input_weight()
    assert W3.dtype == torch.float64 and m.q_proj.weight.data_ptr() == W3.data_ptr()


def test_state_dict_round_trip_after_stacking():
    """After the stacking that the first inference call does, a ``torch.save`` /
    ``torch.load`` round trip of the state dict keeps every value and shape and loads into
    a fresh module; a single stacked parameter saved on its own carries the whole stack's
    storage (torch saves a view's storage), so it is cloned first when it is saved alone."""
    import io

    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32)
    ref = {k: v.clone() for k, v in m.state_dict().items()}
    with torch.inference_mode():
        W, _ = m._fused_input_weight()
    sd = m.state_dict()
    assert sd["q_proj.weight"].untyped_storage().data_ptr() == W.untyped_storage().data_ptr()
    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    back = torch.load(buf, weights_only=True)
    assert back.keys() == ref.keys()
    for k, v in ref.items():
        assert back[k].shape == v.shape and torch.equal(back[k], v), k
    fresh = GatedDeltaNet2(hidden_size=64, num_heads=2, head_dim=32)
    fresh.load_state_dict(back)
    assert all(torch.equal(fresh.state_dict()[k], v) for k, v in ref.items())
    one, alone = io.BytesIO(), io.BytesIO()
    torch.save(m.q_proj.weight, one)
    torch.save(m.q_proj.weight.detach().clone(), alone)
    assert len(one.getvalue()) > len(alone.getvalue()) + W.numel() * W.element_size() // 2
    one.seek(0)
    assert torch.equal(torch.load(one, weights_only=True), ref["q_proj.weight"])


def test_ops_are_not_traced_by_torch_compile():
    """As the reference's ops (chunk_gdn2.py:1267, fused_recurrent_gdn2.py:344), the public
    ops carry torch.compiler.disable: a compiled caller runs them eagerly, so the op's own
    error for CPU tensors comes through instead of a tracing failure in the ctypes shim."""
    from qwendopamine_amd import ops

    x = torch.randn(1, 8, 2, 16)

    def f(q):
        o, _ = ops.chunk_gdn2(q, q, q, -q.abs(), q.sigmoid(), q.sigmoid())
        return o * 2

    with pytest.raises(RuntimeError, match="no CPU path"):
        torch.compile(f, backend="eager")(x)
    for name in ("chunk_gdn2", "fused_recurrent_gdn2", "fused_recurrent_gdn2_fwd", "decode_step_fused"):
        assert getattr(getattr(ops, name), "_torchdynamo_disable", False), name
