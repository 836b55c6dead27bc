"""GPU parity of the HIP backward of the mixer's prologue and epilogue (training):
``ops.short_conv_autograd`` (C entry ``gdn2_short_conv_bwd``) and ``ops.gated_rmsnorm_autograd``
(``gdn2_gated_rmsnorm_bwd``).

The reference runs both through torch's autograd (``gdn2.py:395-452``).  The check here is
float64 autograd of the same functions on the CPU, on the same rounded inputs: rel. L2 <= 1e-4
for float32, <= 2e-2 for bfloat16 (where torch itself rounds every intermediate).  The module
test compares a float32 GatedDeltaNet2 training step with the HIP backward against the torch
ops path (``hip_backward = False``).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests._helpers import REL_TOL, rel_l2

pytestmark = pytest.mark.gpu


def _conv_ref(x, w, b, silu):
    """float64 CPU autograd of the prefill short convolution."""
    xd = x.detach().double().cpu().requires_grad_(True)
    wd = w.detach().double().cpu().requires_grad_(True)
    bd = None if b is None else b.detach().double().cpu().requires_grad_(True)
    T = x.shape[1]
    y = F.conv1d(xd.transpose(1, 2), wd, bd, padding=w.shape[-1] - 1, groups=x.shape[-1])[..., :T]
    if silu:
        y = F.silu(y)
    return y.transpose(1, 2), (xd, wd, bd)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,D,W,bias,silu,strided", [(2, 100, 96, 4, True, True, False),
                                                        (1, 33, 40, 3, False, False, False),
                                                        (3, 70, 64, 4, True, True, True),
                                                        (2, 1, 32, 4, False, True, False),
                                                        (1, 257, 200, 2, True, True, False)])
def test_short_conv_backward_vs_float64_autograd(gpu_device, dtype, B, T, D, W, bias, silu, strided):
    from qwendopamine_amd import ops

    print(f"[case] conv backward {dtype} B={B} T={T} D={D} W={W} bias={bias} silu={silu} strided={strided}",
          flush=True)
    gen = torch.Generator(device="cpu").manual_seed(T + D + W)
    xw = torch.randn(B, T, D + (24 if strided else 0), generator=gen).to(dtype).to(gpu_device)
    x = xw[..., 8:8 + D] if strided else xw
    w = (torch.randn(D, 1, W, generator=gen) * 0.5).to(dtype).to(gpu_device).requires_grad_(True)
    b = (torch.randn(D, generator=gen) * 0.1).to(dtype).to(gpu_device).requires_grad_(True) if bias else None
    dy = torch.randn(B, T, D, generator=gen).to(dtype).to(gpu_device)
    xl = x.detach().clone().requires_grad_(True) if not strided else x.detach().requires_grad_(True)
    y = ops.short_conv_autograd(xl, w, b, "silu" if silu else None)
    y.backward(dy)
    torch.cuda.synchronize()
    y_ref, (xd, wd, bd) = _conv_ref(x, w, b, silu)
    y_ref.backward(dy.double().cpu())
    tol = REL_TOL[dtype]
    errs = {"y": rel_l2(y, y_ref), "dx": rel_l2(xl.grad, xd.grad), "dw": rel_l2(w.grad, wd.grad)}
    if bias:
        errs["db"] = rel_l2(b.grad, bd.grad)
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e <= tol, (k, e)


def _norm_ref(x, z, w, eps):
    xd, zd, wd = (t.detach().double().cpu().requires_grad_(True) for t in (x, z, w))
    out = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + eps) * wd * F.silu(zd)
    return out, (xd, zd, wd)


@pytest.mark.parametrize("dtype,w_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                           (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("shape", [(2, 70, 3, 64), (3, 41, 128), (1, 5, 2, 100), (2, 9, 256)])
def test_gated_rmsnorm_backward_vs_float64_autograd(gpu_device, dtype, w_dtype, shape):
    from qwendopamine_amd import ops

    print(f"[case] gated norm backward {dtype} weight {w_dtype} shape={shape}", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(sum(shape))
    N = shape[-1]
    x = torch.randn(*shape, generator=gen).to(dtype).to(gpu_device).requires_grad_(True)
    z = torch.randn(*shape, generator=gen).to(dtype).to(gpu_device).requires_grad_(True)
    w = (torch.randn(N, generator=gen) * 0.3 + 1).to(w_dtype).to(gpu_device).requires_grad_(True)
    out = ops.gated_rmsnorm_autograd(x, z, w, 1e-5)
    dy = torch.randn(out.shape, generator=gen).to(out.dtype).to(gpu_device)
    out.backward(dy)
    torch.cuda.synchronize()
    ref, (xd, zd, wd) = _norm_ref(x, z, w, 1e-5)
    ref.backward(dy.double().cpu())
    tol = REL_TOL[dtype]
    errs = {"out": rel_l2(out, ref), "dx": rel_l2(x.grad, xd.grad), "dz": rel_l2(z.grad, zd.grad),
            "dw": rel_l2(w.grad, wd.grad)}
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    assert x.grad.dtype == dtype and w.grad.dtype == w_dtype
    for k, e in errs.items():
        assert e <= tol, (k, e)


def test_module_training_step_hip_prologue_matches_torch_ops(gpu_device):
    """float32 GatedDeltaNet2 training step: every parameter gradient with the HIP conv / norm
    backward equals the torch-ops path to float32 rounding."""
    from qwendopamine_amd import GatedDeltaNet2

    print("[case] module training step, HIP conv / norm backward vs torch ops", flush=True)
    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=256, num_heads=4, head_dim=64).to(gpu_device).float().train()
    x = torch.randn(2, 150, 256, device=gpu_device)
    grads = {}
    for hip in (True, False):
        for mod in m.modules():
            if hasattr(mod, "hip_backward"):
                mod.hip_backward = hip
        m.zero_grad(set_to_none=True)
        out, _, _ = m(x)
        (out * torch.linspace(-1, 1, out.shape[-1], device=gpu_device)).sum().backward()
        torch.cuda.synchronize()
        grads[hip] = {n: p.grad.detach().clone() for n, p in m.named_parameters()}
    for n in grads[True]:
        e = rel_l2(grads[True][n], grads[False][n])
        assert e <= 1e-4, (n, e)
