"""GPU parity of the mixer's prologue / epilogue kernels.

Kernels:
* the fused q/k/v short convolution (``ops.short_convolution``);
* the gated RMS norm (``ops.gated_rmsnorm``), and the same entry point without the gate
  (``ops.rms_norm``, the decoder hosts' RMSNorm).

Checks:
* **Oracle.** Against the float64 oracle (``oracle.short_conv``, ``oracle.gated_rmsnorm``,
  ``oracle.rmsnorm``)
  at relative L2 <= 1e-4 (float32) / 2e-2 (bf16, fp16).
* **Reference rounding (norm).** Against the reference's own torch formula evaluated in
  the input dtype on the GPU (gdn2.py:448-452; models/normalization.py:48-50). The norm kernel rounds after every op as
  that code does, so the two agree to within one bf16 unit in the last place.
* **Conv accuracy.** The conv kernel accumulates in fp32 and rounds once, as the
  reference's cuDNN target does; torch's bf16 depthwise conv on this image rounds
  intermediates. So the conv is held to the float64 oracle, and to at least torch's
  accuracy.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rel_l2

pytestmark = pytest.mark.gpu


def _same_rounding(a: torch.Tensor, b: torch.Tensor) -> None:
    """Two bf16 results of the same rounding sequence: nearly every element is bit-identical.
    The rest (a different fp32 summation order flipping a rounding) differ by at most one
    bf16 unit in the last place, i.e. 2^-7 relative to the magnitude, plus a small absolute
    floor near zero."""
    a, b = a.float(), b.float()
    same = (a == b).float().mean().item()
    worst = ((a - b).abs() / (b.abs() + 1e-2)).max().item()
    print(f"  bit-identical {same:.5f}, worst relative diff {worst:.2e}", flush=True)
    assert same >= 0.99
    assert worst <= 2.0 ** -7


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,with_cache,bias", [(130, False, True), (1, True, False), (1, False, True),
                                               (2, False, False), (64, False, False)])
def test_short_conv_matches_oracle(gpu_device, dtype, T, with_cache, bias):
    from qwendopamine_amd.ops import short_convolution

    print(f"[case] short conv dtype={dtype} T={T} cache={with_cache} bias={bias}", flush=True)
    rng = np.random.default_rng(T + 7)
    B, W, dims = 3, 4, (64, 64, 96)
    xs = [rng.standard_normal((B, T, d)) for d in dims]
    ws = [rng.standard_normal((d, 1, W)) * 0.5 for d in dims]
    bs = [rng.standard_normal(d) * 0.1 for d in dims] if bias else [None] * 3
    cs = [rng.standard_normal((B, d, W - 1)) for d in dims] if with_cache else None
    dev = lambda a: None if a is None else torch.from_numpy(a).to(gpu_device, dtype)  # noqa: E731
    ys, new = short_convolution([dev(x) for x in xs], [dev(w) for w in ws], [dev(b) for b in bs],
                                None if cs is None else [dev(c) for c in cs], output_final_state=True)
    torch.cuda.synchronize()
    rd = lambda a: None if a is None else dev(a).double().cpu().numpy()  # noqa: E731
    for i in range(3):
        y_ref, c_ref = orc.short_conv(rd(xs[i]), rd(ws[i]), rd(bs[i]),
                                      None if cs is None else rd(cs[i]), output_final_state=True)
        assert ys[i].dtype == dtype and tuple(ys[i].shape) == (B, T, dims[i])
        assert rel_l2(ys[i], y_ref) <= REL_TOL[dtype], i
        # The new cache is a copy of inputs: exact.
        assert np.array_equal(new[i].double().cpu().numpy(), c_ref), i


def test_short_conv_bf16_at_least_as_accurate_as_torch(gpu_device):
    """bf16: the kernel accumulates in fp32 and rounds the conv output once before the SiLU.
    Its error against the float64 oracle is no larger than that of torch's bf16 conv on
    this image, whose depthwise kernel rounds intermediates. The new cache is a copy of
    inputs, identical in both."""
    from qwendopamine_amd.gdn2 import ShortConvolution

    print("[case] short conv bf16 accuracy vs torch", flush=True)
    torch.manual_seed(0)
    conv = ShortConvolution(256, kernel_size=4, bias=True).to(gpu_device, torch.bfloat16)
    x = torch.randn(2, 96, 256, device=gpu_device, dtype=torch.bfloat16)
    with torch.no_grad():
        y_hip, c_hip = conv(x, output_final_state=True)
    # The same module with gradients enabled takes torch's differentiable path.
    y_torch, c_torch = conv(x.requires_grad_(True), output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(c_hip, c_torch.detach())
    w = conv.conv1d.weight.detach().double().cpu().numpy()
    bias = conv.conv1d.bias.detach().double().cpu().numpy()
    y_ref, _ = orc.short_conv(x.detach().double().cpu().numpy(), w, bias)
    e_hip, e_torch = rel_l2(y_hip, y_ref), rel_l2(y_torch.detach(), y_ref)
    print(f"  rel_l2 vs oracle: hip {e_hip:.3e}  torch {e_torch:.3e}", flush=True)
    assert e_hip <= 2e-2 and e_hip <= e_torch * 1.05


@pytest.mark.parametrize("dtype,N", [(torch.float32, 128), (torch.bfloat16, 64), (torch.bfloat16, 128),
                                     (torch.float16, 100), (torch.bfloat16, 256), (torch.bfloat16, 1024),
                                     (torch.float32, 1024), (torch.float16, 1000)])
def test_gated_rmsnorm_matches_oracle(gpu_device, dtype, N):
    from qwendopamine_amd.ops import gated_rmsnorm

    print(f"[case] gated rmsnorm dtype={dtype} N={N}", flush=True)
    rng = np.random.default_rng(N)
    x, z, w = rng.standard_normal((37, 5, N)) * 2, rng.standard_normal((37, 5, N)), rng.standard_normal(N)
    xt, zt, wt = (torch.from_numpy(a).to(gpu_device, dtype) for a in (x, z, w))
    out = gated_rmsnorm(xt, zt, wt, 1e-5)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    ref = orc.gated_rmsnorm(*(t.double().cpu().numpy() for t in (xt, zt, wt)), 1e-5)
    assert rel_l2(out, ref) <= REL_TOL[dtype]


def test_gated_rmsnorm_rounds_like_the_reference(gpu_device):
    """The reference formula evaluated in bf16 by torch (gdn2.py:448-452) against the kernel;
    an fp32 weight promotes the result to fp32 in both."""
    from qwendopamine_amd.ops import gated_rmsnorm

    print("[case] gated rmsnorm reference rounding", flush=True)
    torch.manual_seed(1)
    x = torch.randn(4096, 128, device=gpu_device, dtype=torch.bfloat16) * 3
    z = torch.randn(4096, 128, device=gpu_device, dtype=torch.bfloat16)
    w = torch.randn(128, device=gpu_device, dtype=torch.bfloat16)

    def ref_formula(x, z, w):
        variance = x.pow(2).mean(-1, keepdim=True)
        normed = x * torch.rsqrt(variance + 1e-5) * w
        return normed * F.silu(z)

    out = gated_rmsnorm(x, z, w, 1e-5)
    ref = ref_formula(x, z, w)
    torch.cuda.synchronize()
    _same_rounding(out, ref)
    out32 = gated_rmsnorm(x, z, w.float(), 1e-5)
    ref32 = ref_formula(x, z, w.float())
    assert out32.dtype == torch.float32 == ref32.dtype
    assert rel_l2(out32, ref32) <= 1e-5


@pytest.mark.parametrize("dtype,N", [(torch.bfloat16, 1024), (torch.bfloat16, 2048), (torch.float32, 1024),
                                     (torch.float16, 1000), (torch.bfloat16, 64), (torch.float32, 2000)])
def test_rms_norm_matches_oracle(gpu_device, dtype, N):
    """The gated norm's entry point without z: the decoder hosts' RMSNorm."""
    from qwendopamine_amd.ops import rms_norm

    print(f"[case] rms_norm dtype={dtype} N={N}", flush=True)
    rng = np.random.default_rng(N + 1)
    x, w = rng.standard_normal((37, 5, N)) * 2, rng.standard_normal(N)
    xt, wt = (torch.from_numpy(a).to(gpu_device, dtype) for a in (x, w))
    out = rms_norm(xt, wt, 1e-5)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    ref = orc.rmsnorm(xt.double().cpu().numpy(), wt.double().cpu().numpy(), 1e-5)
    assert rel_l2(out, ref) <= REL_TOL[dtype]


@pytest.mark.parametrize("N", [1024, 1000])
def test_rms_norm_rounds_like_the_reference(gpu_device, N):
    """Reference RMSNorm.forward (models/normalization.py:40-51) evaluated in bf16 by torch
    against the kernel, vectorised (N = 1024) and element-wise (N = 1000); an fp32 weight
    promotes the result to fp32 in both."""
    from qwendopamine_amd.ops import rms_norm

    print(f"[case] rms_norm reference rounding N={N}", flush=True)
    torch.manual_seed(2)
    x = torch.randn(2048, N, device=gpu_device, dtype=torch.bfloat16) * 3
    w = torch.randn(N, device=gpu_device, dtype=torch.bfloat16)

    def ref_formula(x, w):
        variance = x.pow(2).mean(-1, keepdim=True)
        return w * (x * torch.rsqrt(variance + 1e-5))

    out = rms_norm(x, w, 1e-5)
    ref = ref_formula(x, w)
    torch.cuda.synchronize()
    _same_rounding(out, ref)
    out32 = rms_norm(x, w.float(), 1e-5)
    ref32 = ref_formula(x, w.float())
    assert out32.dtype == torch.float32 == ref32.dtype
    assert rel_l2(out32, ref32) <= 1e-5


def test_module_inference_prologue_matches_training_path(gpu_device):
    """GatedDeltaNet2 under no_grad (HIP conv and norm) against the same module with
    gradients enabled (torch's differentiable conv and norm), prefill and one decode step."""
    from qwendopamine_amd import GatedDeltaNet2

    print("[case] module HIP prologue vs torch prologue", flush=True)
    torch.manual_seed(2)
    m = GatedDeltaNet2(hidden_size=512, num_heads=4, head_dim=64, mode="chunk").to(gpu_device, torch.bfloat16)
    x = torch.randn(2, 100, 512, device=gpu_device, dtype=torch.bfloat16)
    with torch.no_grad():
        cache_a = {}
        out_a, _, cache_a = m(x, past_key_values=cache_a, use_cache=True)
        step_a, _, _ = m(x[:, -1:], past_key_values=cache_a, use_cache=True)
    cache_b = {}
    out_b, _, cache_b = m(x, past_key_values=cache_b, use_cache=True)
    step_b, _, _ = m(x[:, -1:], past_key_values=cache_b, use_cache=True)
    torch.cuda.synchronize()
    assert rel_l2(out_a, out_b.detach()) <= 2e-2
    assert rel_l2(step_a, step_b.detach()) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,with_cache", [(3, 130, False), (4, 1, True), (1, 37, False)])
def test_short_conv_reads_column_ranges_in_place(gpu_device, dtype, B, T, with_cache):
    """q, k and v as column ranges of one wider [B, T, N] tensor (the module's fused input
    projection) give bit-identical outputs and caches to contiguous copies of them."""
    from qwendopamine_amd.ops import short_convolution

    print(f"[case] strided conv {dtype} B={B} T={T} cache={with_cache}", flush=True)
    W, dims = 4, (64, 64, 96)
    gen = torch.Generator(device=gpu_device).manual_seed(7)
    wide = torch.randn(B, T, sum(dims) + 40, generator=gen, device=gpu_device).to(dtype)
    offs = np.cumsum((0,) + dims[:-1])
    views = [wide[..., o:o + d] for o, d in zip(offs, dims)]
    assert not views[1].is_contiguous()
    ws = [torch.randn(d, 1, W, generator=gen, device=gpu_device).to(dtype) * 0.3 for d in dims]
    bs = [torch.randn(d, generator=gen, device=gpu_device).to(dtype) * 0.1 for d in dims]
    caches = [torch.randn(B, d, W - 1, generator=gen, device=gpu_device).to(dtype) for d in dims] \
        if with_cache else None
    ys, new = short_convolution(views, ws, bs, caches, True)
    ys_ref, new_ref = short_convolution([v.contiguous() for v in views], ws, bs, caches, True)
    torch.cuda.synchronize()
    for a, b in zip(ys + new, ys_ref + new_ref):
        assert torch.equal(a, b)
