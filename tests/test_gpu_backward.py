"""GPU parity of the chunkwise backward (autograd through ``chunk_gdn2``) against
the float64 oracle VJP (``oracle.recurrent_vjp``, itself pinned by finite
differences), on seeded small cases.

Tolerances (north star): relative L2 <= 1e-4 for float32 inputs, <= 2e-2 for
bf16 / fp16 inputs, against the oracle run on the same rounded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dv", "dg", "db", "dw", "dh0")


def _grads(dev, dtype, B, T, H, K, V, seed=0, decay="paper", h0_std=0.1, l2=True, with_dht=True,
           g_dtype=torch.float32):
    from qwendopamine_amd.ops import chunk_gdn2

    inp = rand_inputs(B, T, H, K, V, seed=seed, decay=decay, h0_std=h0_std)
    rng = np.random.default_rng(seed + 100)
    inp["do"] = rng.standard_normal((B, T, H, V))
    inp["dht"] = rng.standard_normal((B, H, K, V)) if with_dht else None
    t, r = to_device(inp, dev, dtype, g_dtype=g_dtype)
    leaves = {n: t[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "g", "b", "w")}
    h0 = None if t["h0"] is None else t["h0"].detach().clone().requires_grad_(True)
    o, ht = chunk_gdn2(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["b"], leaves["w"],
                       initial_state=h0, output_final_state=True, use_qk_l2norm_in_kernel=l2)
    loss = (o.float() * t["do"].float()).sum()
    if with_dht:
        loss = loss + (ht * t["dht"].float()).sum()
    loss.backward()
    torch.cuda.synchronize()
    got = [leaves[n].grad for n in ("q", "k", "v", "g", "b", "w")] + [None if h0 is None else h0.grad]
    ref = orc.recurrent_vjp(r["q"], r["k"], r["v"], r["g"], r["b"], r["w"], r["do"], r["dht"], r["h0"],
                            use_qk_l2norm_in_kernel=l2)
    return got, ref


def _check(got, ref, tol, skip_h0=False):
    errs = {}
    for name, a, b in zip(NAMES, got, ref):
        if name == "dh0" and skip_h0:
            assert a is None
            continue
        assert a is not None, name
        assert torch.isfinite(a.float()).all(), name
        errs[name] = rel_l2(a, b)
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for name, e in errs.items():
        assert e <= tol, (name, e)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K,V,T", [(32, 32, 64), (64, 48, 130), (128, 128, 200), (40, 24, 77),
                                   (16, 16, 33)])
def test_chunk_bwd_matches_oracle(gpu_device, dtype, K, V, T):
    print(f"[case] chunk bwd dtype={dtype} K={K} V={V} T={T}", flush=True)
    got, ref = _grads(gpu_device, dtype, 2, T, 2, K, V)
    assert got[0].dtype == dtype and got[3].dtype == torch.float32
    _check(got, ref, REL_TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chunk_bwd_extreme_decay(gpu_device, dtype):
    """Decay spans > 80 per 16 tokens: the exact diagonal-block path of the backward."""
    print(f"[case] chunk bwd extreme decay {dtype}", flush=True)
    got, ref = _grads(gpu_device, dtype, 1, 128, 2, 64, 64, seed=3, decay="extreme")
    _check(got, ref, REL_TOL[dtype])


def test_chunk_bwd_no_l2norm_no_state(gpu_device):
    print("[case] chunk bwd without l2norm / h0 / dht", flush=True)
    got, ref = _grads(gpu_device, torch.float32, 1, 90, 3, 32, 32, seed=5, h0_std=0.0, l2=False,
                      with_dht=False)
    _check(got, ref, 1e-4, skip_h0=True)


def test_chunk_bwd_fp16_and_bf16_gate(gpu_device):
    print("[case] chunk bwd fp16 inputs", flush=True)
    got, ref = _grads(gpu_device, torch.float16, 1, 100, 2, 64, 64, seed=6)
    _check(got, ref, 2e-2)
    print("[case] chunk bwd bf16 inputs with bf16 g", flush=True)
    got, ref = _grads(gpu_device, torch.bfloat16, 2, 96, 2, 64, 64, seed=7, g_dtype=torch.bfloat16)
    assert got[3].dtype == torch.bfloat16
    _check(got, ref, 2e-2)


def test_chunk_bwd_varlen(gpu_device):
    """Packed sequences (cu_seqlens), one of them empty: per-sequence oracle VJPs."""
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] chunk bwd varlen", flush=True)
    cu = [0, 70, 70, 71, 200, 264]
    T, H, K, V = cu[-1], 2, 64, 32
    N = len(cu) - 1
    inp = rand_inputs(1, T, H, K, V, seed=11, h0_std=0.0)
    rng = np.random.default_rng(12)
    inp["h0"] = rng.standard_normal((N, H, K, V)) * 0.1
    inp["do"] = rng.standard_normal((1, T, H, V))
    inp["dht"] = rng.standard_normal((N, H, K, V))
    t, r = to_device(inp, gpu_device, torch.float32)
    leaves = {n: t[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "g", "b", "w", "h0")}
    cu_t = torch.tensor(cu, dtype=torch.int64, device=gpu_device)
    o, ht = chunk_gdn2(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["b"], leaves["w"],
                       initial_state=leaves["h0"], output_final_state=True,
                       use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t)
    ((o * t["do"]).sum() + (ht * t["dht"]).sum()).backward()
    torch.cuda.synchronize()
    ref = [np.zeros_like(r[n]) for n in ("q", "k", "v", "g", "b", "w")] + [np.zeros_like(r["h0"])]
    for s in range(N):
        a, e = cu[s], cu[s + 1]
        if e == a:
            # An empty sequence passes its final-state gradient straight to its initial state.
            ref[6][s] = r["dht"][s]
            continue
        sl = slice(a, e)
        gr = orc.recurrent_vjp(*(r[n][:, sl] for n in ("q", "k", "v", "g", "b", "w")), r["do"][:, sl],
                               r["dht"][s:s + 1], r["h0"][s:s + 1])
        for i in range(6):
            ref[i][:, sl] = gr[i]
        ref[6][s] = gr[6][0]
    got = [leaves[n].grad for n in ("q", "k", "v", "g", "b", "w", "h0")]
    _check(got, ref, 1e-4)


def test_chunk_bwd_gate_in_kernel(gpu_device):
    """use_gate_in_kernel with gradients: the gate runs as torch ops before the kernels, so
    dA_log / ddt_bias come from autograd; checked against the oracle VJP pushed through
    the same gate in float64."""
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] chunk bwd gate in kernel", flush=True)
    B, T, H, K, V = 1, 100, 2, 64, 32
    inp = rand_inputs(B, T, H, K, V, seed=13)
    rng = np.random.default_rng(17)
    graw = rng.standard_normal((B, T, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    do = rng.standard_normal((B, T, H, V))
    inp["g"] = graw
    t, r = to_device(inp, gpu_device, torch.float32)
    leaves = {n: t[n].detach().clone().requires_grad_(True) for n in ("q", "k", "v", "g", "b", "w")}
    a_t = torch.tensor(A_log, dtype=torch.float32, device=gpu_device, requires_grad=True)
    d_t = torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device, requires_grad=True)
    o, _ = chunk_gdn2(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["b"], leaves["w"],
                      initial_state=t["h0"], use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                      A_log=a_t, dt_bias=d_t)
    (o * torch.tensor(do, dtype=torch.float32, device=gpu_device)).sum().backward()
    torch.cuda.synchronize()
    g64 = torch.tensor(r["g"], dtype=torch.float64, requires_grad=True)
    a64 = torch.tensor(A_log, dtype=torch.float64, requires_grad=True)
    d64 = torch.tensor(dt_bias, dtype=torch.float64, requires_grad=True)
    gact = -torch.exp(a64).reshape(H, 1) * torch.nn.functional.softplus(g64 + d64.reshape(H, K))
    gr = orc.recurrent_vjp(r["q"], r["k"], r["v"], gact.detach().numpy(), r["b"], r["w"], do, None,
                           r["h0"])
    gact.backward(torch.from_numpy(gr[3]))
    errs = [rel_l2(leaves["g"].grad, g64.grad.numpy()), rel_l2(a_t.grad, a64.grad.numpy()),
            rel_l2(d_t.grad, d64.grad.numpy()), rel_l2(leaves["q"].grad, gr[0])]
    print("  rel_l2 dg_raw={:.2e} dA_log={:.2e} ddt_bias={:.2e} dq={:.2e}".format(*errs), flush=True)
    # Kernel outputs at the fp32 bar; dA_log and ddt_bias are torch sums of dg over
    # every token (a handful of numbers), checked at 1e-3.
    assert errs[0] <= 1e-4 and errs[3] <= 1e-4
    assert errs[1] <= 1e-3 and errs[2] <= 1e-3
