"""GPU checks of the chunk op's API variants (reference chunk_gdn2.py:1268-1434).

* ``transpose_state_layout``: states are ``[N, H, V, K]``. The kernels run the same
  arithmetic, so outputs and gradients are bit-identical to the ``[K, V]`` run, with
  the states transposed.
* ``return_intermediate_states`` (inference mode): ``h [B, NT, H, K, V]`` holds each
  chunk's start state. It is checked against the float64 oracle recurrence's state
  after the chunk's preceding token (relative L2 <= 1e-4 in float32, 2e-2 in bf16),
  for fixed-length and packed (varlen) batches.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu

NAMES = ("q", "k", "v", "g", "b", "w")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_transposed_state_layout_forward_and_backward(gpu_device, dtype):
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] chunk transposed states {dtype}", flush=True)
    B, T, H, K, V = 2, 150, 2, 64, 32
    inp = rand_inputs(B, T, H, K, V, seed=91)
    t, _ = to_device(inp, gpu_device, dtype)
    rng = np.random.default_rng(92)
    do = torch.from_numpy(rng.standard_normal((B, T, H, V))).to(gpu_device, dtype)
    dht = torch.from_numpy(rng.standard_normal((B, H, K, V))).to(gpu_device, torch.float32)

    def run(transpose):
        leaves = {n: t[n].detach().clone().requires_grad_(True) for n in NAMES}
        h0 = t["h0"].transpose(-1, -2).contiguous() if transpose else t["h0"].clone()
        h0.requires_grad_(True)
        o, ht = chunk_gdn2(*(leaves[n] for n in NAMES), initial_state=h0, output_final_state=True,
                           use_qk_l2norm_in_kernel=True, transpose_state_layout=transpose)
        d = dht.transpose(-1, -2).contiguous() if transpose else dht
        ((o.float() * do.float()).sum() + (ht * d).sum()).backward()
        torch.cuda.synchronize()
        grads = [leaves[n].grad for n in NAMES]
        return o, ht, grads, h0.grad

    o1, ht1, g1, dh1 = run(False)
    o2, ht2, g2, dh2 = run(True)
    assert tuple(ht2.shape) == (B, H, V, K) and tuple(dh2.shape) == (B, H, V, K)
    assert torch.equal(o1, o2)
    assert torch.equal(ht1, ht2.transpose(-1, -2))
    assert torch.equal(dh1, dh2.transpose(-1, -2))
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def _chunk_start_states(r, cu=None, C=64):
    """Oracle chunk start states [nc, H, K, V], sequence-major."""
    q, k, v, g, b, w, h0 = (r[n] for n in (*NAMES, "h0"))
    _, _, states = orc.recurrent_fwd(q, k, v, g, b, w, h0, cu_seqlens=cu, return_states=True)
    B, T = q.shape[:2]
    lens = [T] * B if cu is None else [cu[i + 1] - cu[i] for i in range(len(cu) - 1)]
    out = []
    for n, ln in enumerate(lens):
        for c in range(-(-ln // C)):
            out.append(h0[n] if c == 0 else states[n][c * C - 1])
    return np.stack(out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("transpose", [False, True])
def test_return_intermediate_states(gpu_device, dtype, transpose):
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] chunk intermediate states {dtype} transpose={transpose}", flush=True)
    B, T, H, K, V = 2, 200, 2, 64, 48
    inp = rand_inputs(B, T, H, K, V, seed=93)
    t, r = to_device(inp, gpu_device, dtype)
    h0 = t["h0"].transpose(-1, -2).contiguous() if transpose else t["h0"]
    with torch.inference_mode():
        o, ht, h = chunk_gdn2(*(t[n] for n in NAMES), initial_state=h0, output_final_state=True,
                              use_qk_l2norm_in_kernel=True, return_intermediate_states=True,
                              transpose_state_layout=transpose)
    torch.cuda.synchronize()
    nt = -(-T // 64)
    assert h.dtype == dtype
    assert tuple(h.shape) == ((B, nt, H, V, K) if transpose else (B, nt, H, K, V))
    ref = _chunk_start_states(r).reshape(B, nt, H, K, V)
    got = h.transpose(-1, -2) if transpose else h
    assert rel_l2(got, ref) <= REL_TOL[dtype]
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES), r["h0"])
    assert rel_l2(o, o_ref) <= REL_TOL[dtype]
    assert rel_l2(ht.transpose(-1, -2) if transpose else ht, s_ref) <= REL_TOL[dtype]


def test_return_intermediate_states_varlen(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] chunk intermediate states varlen", flush=True)
    cu = [0, 70, 70, 200, 264]
    T, H, K, V = cu[-1], 2, 32, 32
    inp = rand_inputs(1, T, H, K, V, seed=94, h0_std=0.0)
    inp["h0"] = np.random.default_rng(95).standard_normal((len(cu) - 1, H, K, V)) * 0.1
    t, r = to_device(inp, gpu_device, torch.float32)
    cu_t = torch.tensor(cu, dtype=torch.int64, device=gpu_device)
    with torch.inference_mode():
        _, _, h = chunk_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                             use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t, return_intermediate_states=True)
    torch.cuda.synchronize()
    ref = _chunk_start_states(r, cu)
    assert tuple(h.shape) == (1, ref.shape[0], H, K, V)
    assert rel_l2(h[0], ref) <= 1e-4


def test_return_intermediate_states_needs_inference_mode(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    inp = rand_inputs(1, 64, 1, 16, 16, seed=96)
    t, _ = to_device(inp, gpu_device, torch.float32)
    with pytest.raises(AssertionError):
        chunk_gdn2(*(t[n] for n in NAMES), return_intermediate_states=True)


@pytest.mark.parametrize("dtype,K,V,T", [(torch.float32, 64, 48, 150), (torch.bfloat16, 128, 128, 130)])
def test_chunk_sigmoid_bw_logits(gpu_device, dtype, K, V, T):
    """b and w passed to the chunk op as logits (GDN2_FLAG_SIGMOID_BW), with the in-kernel
    gate: the module's fused prefill path. The oracle gets sigmoid(b), sigmoid(w) of the
    same rounded logits in float64; the kernels activate them in fp32 without rounding."""
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] chunk sigmoid b/w {dtype} K={K} V={V} T={T}", flush=True)
    B, H = 2, 2
    inp = rand_inputs(B, T, H, K, V, seed=111)
    rng = np.random.default_rng(112)
    bl, wl = rng.standard_normal((B, T, H, K)) * 2, rng.standard_normal((B, T, H, V)) * 2
    graw = rng.standard_normal((B, T, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    g = -np.exp(A_log)[:, None] * np.logaddexp(0.0, graw + dt_bias.reshape(H, K))
    inp.update(b=bl, w=wl, g=graw)
    t, r = to_device(inp, gpu_device, dtype)
    t["g"] = torch.from_numpy(graw).to(gpu_device, torch.float32)
    with torch.no_grad():
        o, ht = chunk_gdn2(
            *(t[n] for n in NAMES), initial_state=t["h0"].float(), output_final_state=True,
            use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
            A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
            dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device), bw_logits=True,
        )
    torch.cuda.synchronize()
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))  # noqa: E731
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, sig(r["b"]), sig(r["w"]), r["h0"])
    assert rel_l2(o, o_ref) <= REL_TOL[dtype]
    assert rel_l2(ht, s_ref) <= REL_TOL[dtype]


def test_chunk_sigmoid_bw_logits_rejected_with_training_workspace(gpu_device):
    """The logits option is forward-only: the C ABI refuses it together with the saved
    training workspace, and the separate prep entry point (whose scan has no flags) refuses
    it outright."""
    from qwendopamine_amd import _native as nat
    from qwendopamine_amd.ops import chunk_gdn2_fwd

    inp = rand_inputs(1, 70, 2, 32, 32, seed=113)
    t, _ = to_device(inp, gpu_device, torch.float32)
    with pytest.raises(NotImplementedError):
        chunk_gdn2_fwd(*(t[n] for n in NAMES), 32 ** -0.5, None, False, True,
                       save_for_bwd=True, bw_logits=True)
    lib = nat.load()
    st = lib.gdn2_chunk_fwd_prep(None, None, None, None, nat.DTYPE_F32, nat.DTYPE_F32, None, None,
                                 0.0, None, None, 1, 1, 0, 2, 32, 32, 1.0, nat.FLAG_SIGMOID_BW,
                                 None, 0, None)
    assert st == nat.ERR_INVALID
