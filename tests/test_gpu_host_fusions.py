"""GPU checks of the decoder hosts' fused elementwise passes.

Kernels:
* ``ops.add_rms_norm``: a block's residual add with the RMSNorm that reads its result
  (``gdn2_add_rms_norm_fwd``);
* ``ops.silu_mul``: SwiGLU's ``silu(a) * b`` on the fused w1 / w2 projection
  (``gdn2_silu_mul_fwd``).

Checks:
* **Two ops = one pass.** ``add_rms_norm`` against torch's add followed by the unfused
  norm entry point (``ops.rms_norm``), bit for bit, for both outputs, in bf16, fp16 and
  fp32, with an fp32 weight, and on row counts that leave a workgroup part-filled.
* **Reference rounding.** Both kernels against the reference's torch formulas evaluated
  in the io dtype (``models/normalization.py:48-50``, ``gdn2_gpt/model.py:74-77``).
* **Oracle.** ``add_rms_norm`` against the float64 oracle of the RMSNorm on the rounded sum.
* **Model.** The config-3 host's forward with the fused passes against the same model
  with them switched off, bit for bit, uncached and on a cached decode step.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rel_l2

pytestmark = pytest.mark.gpu


def _bits_equal(a: torch.Tensor, b: torch.Tensor) -> None:
    assert a.dtype == b.dtype and a.shape == b.shape
    diff = (a != b) & ~(torch.isnan(a) & torch.isnan(b))
    assert not bool(diff.any()), f"{int(diff.sum())} of {a.numel()} elements differ"


@pytest.mark.parametrize("dtype,N,rows", [(torch.bfloat16, 1024, 37 * 5), (torch.bfloat16, 2048, 3),
                                          (torch.bfloat16, 64, 1001), (torch.float16, 512, 65),
                                          (torch.float32, 1024, 130), (torch.float32, 16, 7)])
def test_add_rms_norm_equals_add_then_norm(gpu_device, dtype, N, rows):
    from qwendopamine_amd.ops import add_rms_norm, rms_norm

    print(f"[case] add_rms_norm dtype={dtype} N={N} rows={rows}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(N + rows)
    x = (torch.randn(rows, N, generator=g) * 2).to(gpu_device, dtype)
    h = (torch.randn(rows, N, generator=g) * 0.5).to(gpu_device, dtype)
    w = torch.randn(N, generator=g).to(gpu_device, dtype)
    s, out = add_rms_norm(x, h, w, 1e-5)
    s_ref = x + h
    out_ref = rms_norm(s_ref, w, 1e-5)
    torch.cuda.synchronize()
    _bits_equal(s, s_ref)
    _bits_equal(out, out_ref)
    ref = orc.rmsnorm(s_ref.double().cpu().numpy(), w.double().cpu().numpy(), 1e-5)
    assert rel_l2(out, ref) <= REL_TOL[dtype]
    if dtype != torch.float32:
        s32, out32 = add_rms_norm(x, h, w.float(), 1e-5)
        ref32 = rms_norm(s_ref, w.float(), 1e-5)
        torch.cuda.synchronize()
        assert out32.dtype == torch.float32
        _bits_equal(s32, s_ref)
        _bits_equal(out32, ref32)


def test_add_rms_norm_rounds_like_the_reference(gpu_device):
    """``x = x + h; norm_2(x)`` of reference Block.forward in bf16 by torch against the pass."""
    from qwendopamine_amd.ops import add_rms_norm

    print("[case] add_rms_norm reference rounding", flush=True)
    torch.manual_seed(5)
    x = torch.randn(4, 300, 1024, device=gpu_device, dtype=torch.bfloat16) * 3
    h = torch.randn(4, 300, 1024, device=gpu_device, dtype=torch.bfloat16)
    w = torch.randn(1024, device=gpu_device, dtype=torch.bfloat16)
    s, out = add_rms_norm(x, h, w, 1e-5)
    xs = x + h
    ref = w * (xs * torch.rsqrt(xs.pow(2).mean(-1, keepdim=True) + 1e-5))
    torch.cuda.synchronize()
    _bits_equal(s, xs)
    a, b = out.float(), ref.float()
    same = (a == b).float().mean().item()
    worst = ((a - b).abs() / (b.abs() + 1e-2)).max().item()
    print(f"  bit-identical {same:.5f}, worst relative diff {worst:.2e}", flush=True)
    assert same >= 0.99 and worst <= 2.0 ** -7


def test_add_rms_norm_rejects(gpu_device):
    from qwendopamine_amd.ops import add_rms_norm, add_rms_norm_supported

    print("[case] add_rms_norm rejects", flush=True)
    x = torch.zeros(4, 1000, device=gpu_device, dtype=torch.bfloat16)
    assert not add_rms_norm_supported(x)
    with pytest.raises(NotImplementedError):
        add_rms_norm(x, x, torch.ones(1000, device=gpu_device, dtype=torch.bfloat16))
    y = torch.zeros(4, 1024, device=gpu_device, dtype=torch.bfloat16)
    assert add_rms_norm_supported(y)
    with pytest.raises(ValueError):
        add_rms_norm(y, y[:, :512], torch.ones(1024, device=gpu_device, dtype=torch.bfloat16))


@pytest.mark.parametrize("dtype,H,rows", [(torch.bfloat16, 3072, 17), (torch.bfloat16, 512, 1000),
                                          (torch.float16, 64, 3), (torch.float32, 3072, 5)])
def test_silu_mul_matches_torch(gpu_device, dtype, H, rows):
    """Against ``F.silu(a) * b`` in the io dtype: the same two roundings.  torch's silu
    and the kernel's both evaluate x / (1 + exp(-x)) in float, so the rounded results
    agree except where the two float exps differ in the last bit across a rounding
    boundary: at most one unit in the last place of the io dtype, on a tiny share."""
    from qwendopamine_amd.ops import silu_mul

    print(f"[case] silu_mul dtype={dtype} H={H} rows={rows}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(H + rows)
    ab = (torch.randn(rows, 2 * H, generator=g) * 3).to(gpu_device, dtype)
    out = silu_mul(ab)
    a, b = ab.chunk(2, dim=-1)
    ref = F.silu(a) * b
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (rows, H)
    o, r = out.float(), ref.float()
    same = (o == r).float().mean().item()
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -22}[dtype]
    worst = ((o - r).abs() / (r.abs() + 1e-6)).max().item()
    print(f"  bit-identical {same:.6f}, worst relative diff {worst:.2e}", flush=True)
    assert same >= 0.999
    assert worst <= ulp
    # Strided rows: a column range of a wider row, as a fused projection with a bias-free
    # third block would hand over.
    wide = torch.randn(rows, 2 * H + 64, generator=g).to(gpu_device, dtype)
    view = wide[:, : 2 * H]
    torch.cuda.synchronize()
    _bits_equal(silu_mul(view), silu_mul(view.contiguous()))


def _small(dtype, dev):
    from qwendopamine_amd.hybrid import HybridConfig, HybridDecoder

    torch.manual_seed(0)
    cfg = HybridConfig(n_layer=4, n_embd=256, n_head=4, head_size=64, n_query_groups=2,
                       intermediate_size=512, vocab_size=1000, gdn2_layers=[0, 1, 2], block_size=512)
    return HybridDecoder(cfg).to(dev, dtype).eval()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_hybrid_forward_fused_equals_unfused(gpu_device, dtype, monkeypatch):
    """The host's residual adds fused with the following norms change no bit of the
    logits: uncached, a cached prefill and a cached decode step."""
    from qwendopamine_amd import ops

    print(f"[case] hybrid fused vs unfused host {dtype}", flush=True)
    m = _small(dtype, gpu_device)
    idx = torch.randint(0, 1000, (2, 80), device=gpu_device)

    def run():
        with torch.no_grad():
            full = m(idx)
            m.setup_caches(2, 81)
            pre = m(idx, input_pos=torch.arange(80, device=gpu_device))
            step = m(idx[:, -1:], input_pos=torch.tensor([80], device=gpu_device))
        torch.cuda.synchronize()
        return full, pre, step

    calls = {"n": 0}
    real = ops.add_rms_norm

    def counted(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(ops, "add_rms_norm", counted)
    fused = run()
    assert calls["n"] == 3 * 2 * 4  # two per block, three forwards
    monkeypatch.setattr(ops, "add_rms_norm_supported", lambda x: False)
    plain = run()
    for f, p in zip(fused, plain):
        _bits_equal(f, p)
