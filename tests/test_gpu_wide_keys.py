"""Key head dims 129..256 in the chunk kernels (reference ``chunk_gdn2.py:1380-1382``
accepts d_k <= 256): the KP = 256 instantiations of prep, scan and the backward, for
bf16 / fp16 inputs, against the float64 oracle at the 16-bit bar (rel. L2 <= 2e-2).

float32 inputs beyond d_k = 128 take the token-serial wide path instead (a 231 KB fp32
blob does not fit the scans' LDS); its tests are in ``test_gpu_wide_keys_fp32.py``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu
NAMES = ("q", "k", "v", "g", "b", "w")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K,V,T,decay", [(256, 128, 200, "paper"), (192, 64, 130, "paper"),
                                          (256, 64, 128, "extreme"), (144, 48, 77, "paper")])
def test_chunk_forward_wide_keys(gpu_device, dtype, K, V, T, decay):
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] chunk forward d_k={K} d_v={V} T={T} {decay} {dtype}", flush=True)
    inp = rand_inputs(2, T, 2, K, V, seed=K + T, decay=decay)
    t, r = to_device(inp, gpu_device, dtype)
    with torch.no_grad():
        o, ht = chunk_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                           use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES), r["h0"])
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert torch.isfinite(o.float()).all()
    assert eo <= REL_TOL[dtype] and es <= REL_TOL[dtype]


def test_chunk_forward_wide_keys_varlen(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] chunk forward d_k=256 varlen bf16", flush=True)
    cu = [0, 70, 70, 71, 200]
    inp = rand_inputs(1, cu[-1], 2, 256, 64, seed=3, h0_std=0.0)
    t, r = to_device(inp, gpu_device, torch.bfloat16)
    cu_t = torch.tensor(cu, dtype=torch.int64, device=gpu_device)
    with torch.no_grad():
        o, ht = chunk_gdn2(*(t[n] for n in NAMES), output_final_state=True, use_qk_l2norm_in_kernel=True,
                           cu_seqlens=cu_t)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES), None, cu_seqlens=cu)
    assert rel_l2(o, o_ref) <= 2e-2 and rel_l2(ht, s_ref) <= 2e-2


@pytest.mark.parametrize("K,V,T,decay", [(256, 128, 150, "paper"), (192, 64, 100, "paper"),
                                          (256, 64, 128, "extreme")])
def test_chunk_backward_wide_keys(gpu_device, K, V, T, decay):
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] chunk backward d_k={K} d_v={V} T={T} {decay} bf16", flush=True)
    inp = rand_inputs(2, T, 2, K, V, seed=K + 5, decay=decay)
    rng = np.random.default_rng(K)
    inp["do"] = rng.standard_normal((2, T, 2, V))
    inp["dht"] = rng.standard_normal((2, 2, K, V))
    t, r = to_device(inp, gpu_device, torch.bfloat16)
    leaves = [t[n].detach().clone().requires_grad_(True) for n in NAMES]
    h0 = t["h0"].detach().clone().requires_grad_(True)
    o, ht = chunk_gdn2(*leaves, initial_state=h0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    ((o.float() * t["do"].float()).sum() + (ht * t["dht"]).sum()).backward()
    torch.cuda.synchronize()
    ref = orc.recurrent_vjp(*(r[n] for n in NAMES), r["do"], r["dht"], r["h0"])
    errs = {f"d{n}": rel_l2(x.grad, g) for n, x, g in zip((*NAMES, "h0"), (*leaves, h0), ref)}
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e <= 2e-2, (k, e)


def test_module_head_dim_256_prefill_and_training(gpu_device):
    """GatedDeltaNet2(head_dim=256) in bf16: a 150-token prefill (chunk kernels) against the
    oracle composition, and a training step whose gradients reach every parameter."""
    from qwendopamine_amd import GatedDeltaNet2

    print("[case] module head_dim=256 bf16 prefill + training", flush=True)
    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=256, num_heads=2, head_dim=256).to(gpu_device).to(torch.bfloat16)
    x = torch.randn(2, 150, 256, device=gpu_device).to(torch.bfloat16)
    m.eval()
    with torch.no_grad():
        out, _, _ = m(x)
        xf = x.float()
        mf = {n: p.float() for n, p in m.named_parameters()}
        conv = lambda name, y: F.silu(F.conv1d(y.transpose(1, 2), mf[name + ".conv1d.weight"], padding=3,  # noqa: E731
                                               groups=y.shape[-1])[..., :150]).transpose(1, 2)
        q = conv("q_conv1d", xf @ mf["q_proj.weight"].t())
        k = conv("k_conv1d", xf @ mf["k_proj.weight"].t())
        v = conv("v_conv1d", xf @ mf["v_proj.weight"].t())
        f = (xf @ mf["f_proj.0.weight"].t()) @ mf["f_proj.1.weight"].t()
        g = -mf["A_log"].exp().repeat_interleave(256) * F.softplus(f + mf["dt_bias"])
        b = (xf @ mf["b_proj.weight"].t()).sigmoid()
        w = (xf @ mf["w_proj.weight"].t()).sigmoid()
        sp = lambda a: a.reshape(2, 150, 2, 256).double().cpu().numpy()  # noqa: E731
        o, _ = orc.recurrent_fwd(sp(q), sp(k), sp(v), sp(g), sp(b), sp(w))
        o = torch.from_numpy(o).float().to(gpu_device)
        gate = ((xf @ mf["g_proj.0.weight"].t()) @ mf["g_proj.1.weight"].t() + mf["g_proj.1.bias"]).reshape(o.shape)
        on = o * torch.rsqrt(o.square().mean(-1, keepdim=True) + m.o_norm.eps) * mf["o_norm.weight"] * F.silu(gate)
        ref = on.reshape(2, 150, -1) @ mf["o_proj.weight"].t()
    e = rel_l2(out, ref)
    print(f"  inference rel_l2={e:.2e}", flush=True)
    assert e <= 3e-2
    m.train()
    out, _, _ = m(x)
    out.float().square().mean().backward()
    torch.cuda.synchronize()
    for n, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad.float()).all(), n
