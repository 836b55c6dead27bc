"""Full-size GPU checks at the BASELINE shapes, through size-independent properties.

* C1 (B8 T4096 H16 K=V=128, bf16): the chunkwise kernels equal the token-serial
  kernel (a different algorithm) on the same inputs, and split/resume at a
  chunk boundary equals the single pass.
* C2 (N64 H16 K=V=128 decode): one step equals a float32 torch evaluation of
  the reference update (gdn2.py:164-178); 256 decode steps equal the chunkwise
  prefill of the same 256 tokens.
* C4 forward shape (B4 T8192 H16): chunk vs token-serial kernel.
* C4 backward (B4 T8192 H16, bf16, dO ~ N(0,1)): the bf16 gradients equal the
  float32 kernels' gradients on the same (upcast) inputs -- the float32
  backward is itself pinned to the float64 oracle VJP at 1e-6 on small shapes
  -- for dq, dk, dv, dbeta = sum_K db + sum_V dw (b = w = beta broadcast) and
  the scalar dg = sum_K dg.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests._helpers import rel_l2

pytestmark = pytest.mark.gpu


def _inputs(dev, B, T, H, K, V, seed, dtype=torch.bfloat16):
    gen = torch.Generator(device=dev).manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, K, generator=gen, device=dev), dim=-1).to(dtype)
    k = F.normalize(torch.randn(B, T, H, K, generator=gen, device=dev), dim=-1).to(dtype)
    v = torch.randn(B, T, H, V, generator=gen, device=dev).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, 1, generator=gen, device=dev))
    g = (-F.softplus(torch.randn(B, T, H, 1, generator=gen, device=dev) + 2.0)).expand(B, T, H, K).contiguous()
    b = beta.expand(B, T, H, K).to(dtype).contiguous()
    w = beta.expand(B, T, H, V).to(dtype).contiguous()
    return q, k, v, g, b, w


@pytest.mark.parametrize("shape", [(8, 4096, 16, 128, 128), (4, 8192, 16, 128, 128)], ids=["C1", "C4fwd"])
def test_chunk_equals_token_serial_kernel_full_size(gpu_device, shape):
    from qwendopamine_amd.ops import chunk_gdn2, fused_recurrent_gdn2

    B, T, H, K, V = shape
    print(f"[case] full-size chunk vs recurrent {shape}", flush=True)
    q, k, v, g, b, w = _inputs(gpu_device, B, T, H, K, V, seed=1)
    with torch.no_grad():
        oc, sc = chunk_gdn2(q, k, v, g, b, w, output_final_state=True, use_qk_l2norm_in_kernel=True)
        orr, sr = fused_recurrent_gdn2(q, k, v, g, b, w, output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    eo, es = rel_l2(oc.float(), orr.float()), rel_l2(sc, sr)
    print(f"  rel_l2 o={eo:.3e} state={es:.3e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2
    assert torch.isfinite(oc.float()).all()


def test_split_resume_full_size(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] split/resume C1", flush=True)
    q, k, v, g, b, w = _inputs(gpu_device, 8, 4096, 16, 128, 128, seed=3)
    with torch.no_grad():
        o, s = chunk_gdn2(q, k, v, g, b, w, output_final_state=True, use_qk_l2norm_in_kernel=True)
        cut = 2048
        o1, s1 = chunk_gdn2(*(x[:, :cut] for x in (q, k, v, g, b, w)), output_final_state=True,
                            use_qk_l2norm_in_kernel=True)
        o2, s2 = chunk_gdn2(*(x[:, cut:] for x in (q, k, v, g, b, w)), initial_state=s1,
                            output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert rel_l2(torch.cat([o1, o2], 1).float(), o.float()) <= 1e-5
    assert rel_l2(s2, s) <= 1e-5


def test_decode_step_matches_torch_fp32(gpu_device):
    from qwendopamine_amd.ops import fused_recurrent_gdn2_fwd

    print("[case] C2 one decode step vs torch fp32", flush=True)
    N, H, K, V = 64, 16, 128, 128
    gen = torch.Generator(device=gpu_device).manual_seed(2)
    state = torch.randn(N, H, K, V, generator=gen, device=gpu_device) * 0.02
    q, k, v, g, b, w = _inputs(gpu_device, N, 1, H, K, V, seed=4)
    ref_state = state.clone()
    out, _ = fused_recurrent_gdn2_fwd(q, k, v, g, b, w, initial_state=state, inplace_final_state=True,
                                      use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    # torch float32 evaluation of the reference update on the same (bf16-rounded) inputs
    qf = F.normalize(q.float()[:, 0], dim=-1, eps=1e-6) * K**-0.5
    kf = F.normalize(k.float()[:, 0], dim=-1, eps=1e-6)
    S = ref_state * g[:, 0].exp().unsqueeze(-1)
    r = torch.einsum("nhkv,nhk->nhv", S, b.float()[:, 0] * kf)
    u = w.float()[:, 0] * v.float()[:, 0] - r
    S = S + kf.unsqueeze(-1) * u.unsqueeze(-2)
    o_ref = torch.einsum("nhkv,nhk->nhv", S, qf)
    assert rel_l2(state, S) <= 1e-5
    assert rel_l2(out[:, 0].float(), o_ref) <= 2e-2  # output rounded to bf16


def test_decode_loop_equals_prefill(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2, fused_recurrent_gdn2_fwd

    print("[case] C2 256 decode steps vs prefill", flush=True)
    N, H, K, V, T = 64, 16, 128, 128, 256
    q, k, v, g, b, w = _inputs(gpu_device, N, T, H, K, V, seed=5)
    gen = torch.Generator(device=gpu_device).manual_seed(6)
    h0 = torch.randn(N, H, K, V, generator=gen, device=gpu_device) * 0.02
    state = h0.clone()
    outs = []
    for t in range(T):
        o_t, _ = fused_recurrent_gdn2_fwd(*(x[:, t:t + 1] for x in (q, k, v, g, b, w)),
                                          initial_state=state, inplace_final_state=True,
                                          use_qk_l2norm_in_kernel=True)
        outs.append(o_t)
    with torch.no_grad():
        oc, sc = chunk_gdn2(q, k, v, g, b, w, initial_state=h0, output_final_state=True,
                            use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    od = torch.cat(outs, 1)
    eo, es = rel_l2(oc.float(), od.float()), rel_l2(sc, state)
    print(f"  rel_l2 o={eo:.3e} state={es:.3e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2


def _rel(a, b):
    a, b = a.double(), b.double()
    return float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b))


def test_backward_full_size_bf16_vs_fp32(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    B, T, H, K, V = 4, 8192, 16, 128, 128
    print("[case] full-size C4 backward bf16 vs fp32 kernels", flush=True)
    q, k, v, g, b, w = _inputs(gpu_device, B, T, H, K, V, seed=4)
    gen = torch.Generator(device=gpu_device).manual_seed(41)
    do = torch.randn(B, T, H, V, generator=gen, device=gpu_device).to(torch.bfloat16)
    grads = {}
    for dt in (torch.bfloat16, torch.float32):
        leaves = [x.to(dt).detach().requires_grad_(True) for x in (q, k, v, g, b, w)]
        o, _ = chunk_gdn2(*leaves, use_qk_l2norm_in_kernel=True)
        (o.float() * do.float()).sum().backward()
        torch.cuda.synchronize()
        dq, dk, dv, dg, db, dw = (x.grad.float() for x in leaves)
        grads[dt] = dict(dq=dq, dk=dk, dv=dv, dbeta=db.sum(-1) + dw.sum(-1), dg=dg.sum(-1))
        del leaves, o
    errs = {n: _rel(grads[torch.bfloat16][n], grads[torch.float32][n]) for n in grads[torch.float32]}
    print("  rel_l2 " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()), flush=True)
    for n, e in errs.items():
        assert e <= 2e-2, (n, e)
        assert torch.isfinite(grads[torch.bfloat16][n]).all(), n
