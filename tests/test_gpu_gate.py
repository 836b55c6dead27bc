"""The decay gate of the training path on its HIP kernels (``ops.gate_activation``:
``gdn2_gate_fwd`` / ``gdn2_gate_bwd``, reference ``kda_gate_fwd`` / ``kda_gate_bwd``,
``chunk_kda.py:3223-3292``) against float64 torch autograd of the same formula:

* forward ``y = -exp(A_log) softplus(g + dt_bias)`` and the bounded form
  ``lower_bound sigmoid(exp(A_log) (g + dt_bias))``, with and without ``dt_bias``;
* gradients of ``g``, ``A_log`` and ``dt_bias`` (sums over many 64-token blocks), for
  float32 / bf16 / fp16 ``g`` and key widths that are and are not multiples of 4;
* the backward is deterministic (two runs bit-identical).
"""

from __future__ import annotations

import pytest
import torch

from tests._helpers import rel_l2

pytestmark = pytest.mark.gpu


def _ref(g, A_log, dt_bias, lb, dy):
    gr = g.detach().double().cpu().requires_grad_(True)
    ar = A_log.detach().double().cpu().requires_grad_(True)
    dr = None if dt_bias is None else dt_bias.detach().double().cpu().requires_grad_(True)
    H, K = g.shape[-2:]
    x = gr if dr is None else gr + dr.reshape(H, K)
    a = ar.exp().reshape(H, 1)
    y = lb * torch.sigmoid(a * x) if lb is not None else -a * torch.nn.functional.softplus(x)
    y.backward(dy.detach().double().cpu())
    return y.detach(), gr.grad, ar.grad, None if dr is None else dr.grad


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lb", [None, -3.0])
@pytest.mark.parametrize("K,tokens,bias", [(128, 1000, True), (100, 300, True), (256, 65, False), (32, 1, True)])
def test_gate_forward_backward(gpu_device, dtype, lb, K, tokens, bias):
    from qwendopamine_amd.ops import gate_activation

    print(f"[case] gate {dtype} lb={lb} K={K} tokens={tokens} bias={bias}", flush=True)
    H = 3
    gen = torch.Generator(device="cpu").manual_seed(K + tokens)
    g = (torch.randn(tokens, H, K, generator=gen) * 2).to(dtype).to(gpu_device).requires_grad_(True)
    A_log = torch.log(torch.rand(H, generator=gen) * 15 + 1).to(gpu_device).requires_grad_(True)
    dt_bias = (torch.randn(H * K, generator=gen) * 0.5).to(gpu_device).requires_grad_(True) if bias else None
    dy = torch.randn(tokens, H, K, generator=gen).to(gpu_device)
    y = gate_activation(g, A_log, dt_bias, lb)
    y.backward(dy)
    torch.cuda.synchronize()
    y_ref, dg_ref, da_ref, db_ref = _ref(g, A_log, dt_bias, lb, dy)
    assert y.dtype == torch.float32 and g.grad.dtype == dtype
    errs = {"y": rel_l2(y, y_ref), "dg": rel_l2(g.grad, dg_ref), "dA_log": rel_l2(A_log.grad, da_ref)}
    if bias:
        errs["ddt_bias"] = rel_l2(dt_bias.grad, db_ref)
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    tol_dg = 1e-5 if dtype == torch.float32 else 4e-3  # dg is returned in g's dtype
    assert errs["y"] <= 1e-5 and errs["dg"] <= tol_dg and errs["dA_log"] <= 1e-5
    if bias:
        assert errs["ddt_bias"] <= 1e-5


def test_gate_backward_deterministic(gpu_device):
    from qwendopamine_amd.ops import gate_activation

    print("[case] gate backward deterministic", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(1)
    g = torch.randn(4096, 16, 128, generator=gen).to(gpu_device)
    A_log = torch.log(torch.rand(16, generator=gen) * 15 + 1).to(gpu_device)
    dt_bias = torch.randn(16 * 128, generator=gen).to(gpu_device)
    dy = torch.randn(4096, 16, 128, generator=gen).to(gpu_device)
    grads = []
    for _ in range(2):
        leaves = [t.detach().clone().requires_grad_(True) for t in (g, A_log, dt_bias)]
        gate_activation(*leaves, None).backward(dy)
        grads.append([t.grad.clone() for t in leaves])
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)
