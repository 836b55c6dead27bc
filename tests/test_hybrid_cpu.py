"""CPU checks of the config-3 hybrid decoder host (``qwendopamine_amd.hybrid``).

* The parameter count of the built model equals the closed form of the reference's
  ``compute_model_params`` (``models/gdn2_gpt/model.py:433-501``), and the config-3
  model has the stated ~0.68 B parameters, built on the meta device.
* Parameter names are those of the reference ``GDN2GPT`` (``model.py:176-270``), so
  state dicts are interchangeable.
* RoPE is pinned by what fixes it mathematically: position 0 is the identity, each
  channel pair is rotated (norm preserved), and the score of a rotated query and key
  depends only on the difference of their positions.
* Streaming attention: an all-attention stack (which runs on the CPU) gives the same
  logits from prefill + single-token cached steps as from one uncached forward. The
  gdn2 layers of the same host need the GPU and are checked in ``test_gpu_hybrid.py``.
"""

from __future__ import annotations

import torch

from qwendopamine_amd.hybrid import (
    HybridConfig,
    HybridDecoder,
    apply_rotary_emb,
    build_rope_cache,
    count_parameters,
)


def test_c3_parameter_count_and_layer_pattern():
    cfg = HybridConfig.c3()
    with torch.device("meta"):
        m = HybridDecoder(cfg)
    n = sum(p.numel() for p in m.parameters())
    assert n == count_parameters(cfg)
    assert 0.6e9 <= n <= 0.7e9
    kinds = [blk.use_gdn2 for blk in m.h]
    assert kinds == [i % 4 != 3 for i in range(24)]
    assert sum(kinds) == 18


def test_parameter_names_follow_gdn2gpt():
    cfg = HybridConfig(n_layer=2, n_embd=64, n_head=2, head_size=32, n_query_groups=2, intermediate_size=96,
                       vocab_size=50, gdn2_layers=[0])
    with torch.device("meta"):
        names = set(HybridDecoder(cfg).state_dict())
    expected = {"wte.weight", "ln_f.weight", "lm_head.weight"}
    for i in range(2):
        expected |= {f"h.{i}.norm_1.weight", f"h.{i}.norm_2.weight",
                     *(f"h.{i}.mlp.swiglu.w{j}.weight" for j in (1, 2, 3))}
    expected |= {"h.1.attn.attn.weight", "h.1.attn.proj.weight"}
    assert expected <= names
    gdn2 = {n for n in names if n.startswith("h.0.attn.")}
    for p in ("q_proj.weight", "k_proj.weight", "v_proj.weight", "A_log", "dt_bias", "o_proj.weight",
              "o_norm.weight", "b_proj.weight", "w_proj.weight"):
        assert f"h.0.attn.{p}" in gdn2, p
    assert names - expected - gdn2 == set()


def test_rope_rotation_properties():
    D, L = 16, 12
    cos, sin = build_rope_cache(L, D, "cpu")
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, L, 1, D, generator=g, dtype=torch.float64)
    k = torch.randn(1, L, 1, D, generator=g, dtype=torch.float64)
    q[:] = q[:, :1]  # the same query and key at every position
    k[:] = k[:, :1]
    rq = apply_rotary_emb(q, cos.double(), sin.double())
    rk = apply_rotary_emb(k, cos.double(), sin.double())
    assert torch.allclose(rq[:, 0], q[:, 0])
    pair = lambda x: x.reshape(*x.shape[:-1], D // 2, 2).norm(dim=-1)  # noqa: E731
    assert torch.allclose(pair(rq), pair(q))
    scores = torch.einsum("d,ed->e", rq[0, 5, 0], rk[0, :, 0])
    shifted = torch.einsum("d,ed->e", rq[0, 8, 0], rk[0, :, 0])
    # <R(5) q, R(j) k> = <R(8) q, R(j + 3) k>
    assert torch.allclose(scores[:9], shifted[3:12])


def test_rope_complex_product_equals_pair_formula():
    """The single-token full-width rotation (a complex product) against the interleaved-pair formula of
    reference model.py:40-61, written out here with separate real products, in fp32."""
    D, L = 64, 1
    cos, sin = build_rope_cache(9, D, "cpu")
    cos, sin = cos[5:6], sin[5:6]  # one decode position
    x = torch.randn(7, L, 3, D, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    xf = x.float()
    x1, x2 = xf[..., 0::2], xf[..., 1::2]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    ref = torch.stack((x1 * c - x2 * s, x1 * s + x2 * c), dim=-1).flatten(-2)
    out = apply_rotary_emb(x, cos, sin)
    assert out.dtype == torch.bfloat16
    torch.testing.assert_close(out.float(), ref.to(torch.bfloat16).float(), rtol=2 ** -7, atol=1e-6)


def test_streaming_attention_matches_uncached_forward():
    torch.manual_seed(0)
    cfg = HybridConfig(n_layer=3, n_embd=128, n_head=4, head_size=32, n_query_groups=2, intermediate_size=256,
                       vocab_size=97, gdn2_layers=[], block_size=64)
    m = HybridDecoder(cfg).eval()
    idx = torch.randint(0, 97, (2, 12))
    with torch.no_grad():
        full = m(idx)
        m.setup_caches(2, 16)
        outs = [m(idx[:, :9], input_pos=torch.arange(9))]
        for t in range(9, 12):
            outs.append(m(idx[:, t:t + 1], input_pos=torch.tensor([t])))
    inc = torch.cat(outs, 1)
    assert (inc - full).abs().max() <= 1e-5 * full.abs().max()
