"""GPU checks of the config-3 hybrid decoder host (``qwendopamine_amd.hybrid``).

* **Streaming = uncached.** Prefill (the chunk kernels, T > 64) followed by single-token
  cached steps (the decode kernel, the conv cache, the attention KV cache) gives the
  logits of one uncached forward over the whole sequence: relative L2 <= 1e-4 in
  float32 and <= 2e-2 in bf16, at every position. This is the reference's split /
  resume invariance (``tests/models/test_gdn2.py:111-152``) at model level, and it is
  what the reference host ``GDN2GPT`` does not have (it decodes gdn2 layers without a
  cache, ``models/gdn2_gpt/model.py:232``).
* **Graph decode = eager decode.** The decode step captured once as a HIP graph and
  replayed gives the eager step's tokens and logits.
* **Config 3 at full size** (0.68 B parameters, float32): streaming = uncached on a
  short prompt.
"""

from __future__ import annotations

import pytest
import torch

from tests._helpers import rel_l2

pytestmark = pytest.mark.gpu


def _small(dtype, dev, gdn2_layers=(0, 1, 2), n_layer=4):
    from qwendopamine_amd.hybrid import HybridConfig, HybridDecoder

    torch.manual_seed(0)
    cfg = HybridConfig(n_layer=n_layer, n_embd=256, n_head=4, head_size=64, n_query_groups=2,
                       intermediate_size=512, vocab_size=1000, gdn2_layers=list(gdn2_layers), block_size=512)
    return HybridDecoder(cfg).to(dev, dtype).eval()


def _streaming_vs_uncached(m, idx, n_prefill):
    with torch.no_grad():
        full = m(idx).float()
        m.setup_caches(idx.shape[0], idx.shape[1])
        outs = [m(idx[:, :n_prefill], input_pos=torch.arange(n_prefill, device=idx.device))]
        for t in range(n_prefill, idx.shape[1]):
            outs.append(m(idx[:, t:t + 1], input_pos=torch.tensor([t], device=idx.device)))
    torch.cuda.synchronize()
    return torch.cat(outs, 1).float(), full


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_streaming_matches_uncached(gpu_device, dtype):
    print(f"[case] hybrid streaming vs uncached {dtype}", flush=True)
    m = _small(dtype, gpu_device)
    idx = torch.randint(0, 1000, (3, 106), device=gpu_device)
    inc, full = _streaming_vs_uncached(m, idx, 100)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for t in (0, 50, 99, 100, 103, 105):
        err = rel_l2(inc[:, t], full[:, t].double().cpu().numpy())
        assert err <= tol, (t, err)


def test_graph_decode_matches_eager(gpu_device):
    from qwendopamine_amd.hybrid import GreedyDecoder

    print("[case] hybrid graph decode vs eager", flush=True)
    m = _small(torch.bfloat16, gpu_device)
    prompt = torch.randint(0, 1000, (2, 70), device=gpu_device)
    runs = []
    for use_graph in (False, True):
        dec = GreedyDecoder(m, use_graph=use_graph, keep_logits=True)
        toks, logits = [dec.prefill(prompt, 12).clone()], [dec.logits.clone()]
        for _ in range(11):
            toks.append(dec.step().clone())
            logits.append(dec.logits.clone())
        torch.cuda.synchronize()
        runs.append((torch.cat(toks, 1), torch.stack(logits)))
    (t0, l0), (t1, l1) = runs
    assert torch.equal(t0, t1)
    for s in range(12):
        assert rel_l2(l1[s], l0[s].double().cpu().numpy()) <= 1e-3, s


def test_c3_full_size_streaming(gpu_device):
    """In float32: two bf16 runs of a 24-layer random model that tile their products
    differently (128 vs 132 tokens) already differ by ~2% in the logits, which would
    hide a cache error of the same size."""
    from qwendopamine_amd.hybrid import HybridConfig, HybridDecoder

    print("[case] hybrid config 3 full size streaming", flush=True)
    torch.manual_seed(3)
    m = HybridDecoder(HybridConfig.c3()).to(gpu_device, torch.float32).eval()
    idx = torch.randint(0, 151936, (2, 132), device=gpu_device)
    inc, full = _streaming_vs_uncached(m, idx, 128)
    for t in (0, 127, 128, 131):
        err = rel_l2(inc[:, t], full[:, t].double().cpu().numpy())
        assert err <= 1e-4, (t, err)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_last_only_logits(gpu_device, dtype):
    """``last_only`` (the prefill of greedy decoding) gives the full forward's last
    position: the same rows through the final norm, the LM head on one row instead of T
    (torch's GEMM may tile them differently, hence the tolerance)."""
    print(f"[case] hybrid last_only logits {dtype}", flush=True)
    m = _small(dtype, gpu_device)
    idx = torch.randint(0, 1000, (2, 70), device=gpu_device)
    with torch.no_grad():
        full = m(idx)
        last = m(idx, last_only=True)
        m.setup_caches(2, 70)
        cached = m(idx, input_pos=torch.arange(70, device=gpu_device), last_only=True)
    torch.cuda.synchronize()
    assert last.shape == (2, 1, 1000) and cached.shape == (2, 1, 1000)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel_l2(last[:, 0], full[:, -1].double().cpu().numpy()) <= tol
    assert rel_l2(cached[:, 0], full[:, -1].double().cpu().numpy()) <= (1e-4 if dtype == torch.float32 else 2e-2)


def test_decode_with_frozen_attention_and_grad_enabled(gpu_device):
    """A cached single-token step with autograd on, the attention weights frozen and the
    rest trainable: the decoder's fused-attention decision (made on the weights) says
    fused, but each attention layer sees a projection output that carries a gradient and
    takes its torch path, which must then select the rotation rows and build the mask
    itself.  The logits equal the no-grad run's to the bf16 bar (the two runs take
    different kernels: chunk vs token-serial gdn2, torch vs fused attention)."""
    print("[case] hybrid decode, frozen attention, grad enabled", flush=True)
    m = _small(torch.bfloat16, gpu_device)
    for blk in m.h:
        if not blk.use_gdn2:
            blk.attn.requires_grad_(False)
    idx = torch.randint(0, 1000, (2, 72), device=gpu_device)
    outs = {}
    for grad in (False, True):
        m.setup_caches(2, 72)
        assert m._attention_decode_fused()
        with torch.set_grad_enabled(grad):
            pre = m(idx[:, :70], input_pos=torch.arange(70, device=gpu_device))
            steps = [m(idx[:, t:t + 1], input_pos=torch.tensor([t], device=gpu_device)) for t in (70, 71)]
        torch.cuda.synchronize()
        outs[grad] = torch.cat([pre[:, -1:], *steps], 1).detach()
    assert outs[True].shape == (2, 3, 1000)
    assert rel_l2(outs[True], outs[False].double().cpu().numpy()) <= 2e-2
