"""float32 inputs with key head dims 129..256 in the chunk op (reference
``chunk_gdn2.py:1380-1382`` accepts d_k <= 256 in any dtype).  They run the wide path
(``csrc/gdn2_chunk_wide.hip``: the recurrence token by token with chunk start states kept
for a chunk-recomputing backward), checked at the float32 bar (rel. L2 <= 1e-4) against
the float64 oracle:

* forward outputs and final states, with and without an initial state, ragged lengths,
  d_k not a multiple of 4, one and two value slices (d_v up to 256);
* all seven gradients through autograd against ``recurrent_vjp``;
* packed sequences (with an empty one) against the oracle per sequence, transposed
  states, the per-chunk intermediate states, the in-kernel gate and b / w logits;
* ``GatedDeltaNet2(head_dim=256)`` in float32: a 150-token prefill against the float64
  composition of the reference forward, and a training step whose parameter gradients
  equal those of the float64 composition (oracle recurrence with its VJP) to 1e-4.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu
NAMES = ("q", "k", "v", "g", "b", "w")
TOL = 1e-4


@pytest.mark.parametrize("K,V,T,h0", [(256, 64, 150, True), (192, 128, 130, False), (130, 200, 77, True),
                                      (256, 256, 64, True), (160, 16, 1, False)])
def test_fp32_wide_forward(gpu_device, K, V, T, h0):
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] fp32 chunk forward d_k={K} d_v={V} T={T} h0={h0}", flush=True)
    inp = rand_inputs(2, T, 2, K, V, seed=K + V + T, h0_std=0.1 if h0 else 0.0)
    t, r = to_device(inp, gpu_device, torch.float32)
    with torch.no_grad():
        o, ht = chunk_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                           use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES), r["h0"])
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert o.dtype == torch.float32 and eo <= TOL and es <= TOL


@pytest.mark.parametrize("K,V,T,decay,l2", [(256, 128, 150, "paper", True), (192, 64, 100, "paper", True),
                                             (130, 200, 70, "unit", True), (256, 64, 128, "extreme", True),
                                             (160, 32, 90, "paper", False)])
def test_fp32_wide_backward(gpu_device, K, V, T, decay, l2):
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] fp32 chunk backward d_k={K} d_v={V} T={T} {decay} l2={l2}", flush=True)
    inp = rand_inputs(2, T, 2, K, V, seed=K + 7, decay=decay)
    if not l2:  # keep the products O(1) without the in-kernel norm
        inp["q"] = inp["q"] / np.sqrt(K)
        inp["k"] = inp["k"] / np.sqrt(K)
    rng = np.random.default_rng(K + V)
    inp["do"] = rng.standard_normal((2, T, 2, V))
    inp["dht"] = rng.standard_normal((2, 2, K, V))
    t, r = to_device(inp, gpu_device, torch.float32)
    leaves = [t[n].detach().clone().requires_grad_(True) for n in NAMES]
    h0 = t["h0"].detach().clone().requires_grad_(True)
    o, ht = chunk_gdn2(*leaves, initial_state=h0, output_final_state=True, use_qk_l2norm_in_kernel=l2)
    ((o * t["do"]).sum() + (ht * t["dht"]).sum()).backward()
    torch.cuda.synchronize()
    ref = orc.recurrent_vjp(*(r[n] for n in NAMES), r["do"], r["dht"], r["h0"], use_qk_l2norm_in_kernel=l2)
    errs = {f"d{n}": rel_l2(x.grad, g) for n, x, g in zip((*NAMES, "h0"), (*leaves, h0), ref)}
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e <= TOL, (k, e)


@pytest.mark.parametrize("transpose", [False, True])
def test_fp32_wide_varlen_forward_backward(gpu_device, transpose):
    """Packed sequences, one of them empty: every sequence equals the oracle run on its own
    slice, forward and backward; with ``transpose_state_layout`` every state is [V, K]."""
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] fp32 d_k=192 varlen forward + backward transpose={transpose}", flush=True)
    cu = [0, 70, 70, 71, 200]
    K, V, N = 192, 48, len(cu) - 1
    inp = rand_inputs(1, cu[-1], 2, K, V, seed=11, h0_std=0.0)
    rng = np.random.default_rng(5)
    h0 = rng.standard_normal((N, 2, K, V)) * 0.1
    do = rng.standard_normal((1, cu[-1], 2, V))
    dht = rng.standard_normal((N, 2, K, V))
    t, r = to_device(inp, gpu_device, torch.float32)
    tr = (lambda a: np.ascontiguousarray(np.swapaxes(a, -1, -2))) if transpose else (lambda a: a)
    h0_t = torch.from_numpy(tr(h0)).float().to(gpu_device).requires_grad_(True)
    do_t = torch.from_numpy(do).float().to(gpu_device)
    dht_t = torch.from_numpy(tr(dht)).float().to(gpu_device)
    leaves = [t[n].detach().clone().requires_grad_(True) for n in NAMES]
    cu_t = torch.tensor(cu, dtype=torch.int64, device=gpu_device)
    o, ht = chunk_gdn2(*leaves, initial_state=h0_t, output_final_state=True, use_qk_l2norm_in_kernel=True,
                       cu_seqlens=cu_t, transpose_state_layout=transpose)
    ((o * do_t).sum() + (ht * dht_t).sum()).backward()
    torch.cuda.synchronize()
    for s in range(N):
        a, e = cu[s], cu[s + 1]
        sl = [r[n][:, a:e] for n in NAMES]
        o_ref, s_ref = orc.recurrent_fwd(*sl, h0[s:s + 1])
        if e > a:
            assert rel_l2(o[:, a:e], o_ref) <= TOL, s
        assert rel_l2(ht[s], tr(s_ref[0])) <= TOL, s
        grads = orc.recurrent_vjp(*sl, do[:, a:e], dht[s:s + 1], h0[s:s + 1])
        for n, x, gr in zip(NAMES, leaves, grads):
            if e > a:
                assert rel_l2(x.grad[:, a:e], gr) <= TOL, (s, n)
        assert rel_l2(h0_t.grad[s], tr(grads[6][0])) <= TOL, s


def test_fp32_wide_intermediate_states(gpu_device):
    """``return_intermediate_states`` gives each chunk's start state [B, NT, H, K, V]."""
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] fp32 d_k=256 intermediate states", flush=True)
    K, V, T = 256, 32, 150
    inp = rand_inputs(2, T, 2, K, V, seed=21)
    t, r = to_device(inp, gpu_device, torch.float32)
    with torch.inference_mode():
        o, ht, h = chunk_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                              use_qk_l2norm_in_kernel=True, return_intermediate_states=True)
    torch.cuda.synchronize()
    _, _, states = orc.recurrent_fwd(*(r[n] for n in NAMES), r["h0"], return_states=True)
    assert tuple(h.shape) == (2, 3, 2, K, V) and h.dtype == torch.float32
    for bi in range(2):
        for j in range(3):
            ref = r["h0"][bi] if j == 0 else states[bi][64 * j - 1]
            assert rel_l2(h[bi, j], ref) <= TOL, (bi, j)


def test_fp32_wide_in_kernel_gate_and_logits(gpu_device):
    """The in-kernel gate ``-exp(A_log) softplus(g + dt_bias)`` and b / w given as logits."""
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] fp32 d_k=256 in-kernel gate and b / w logits", flush=True)
    K, V, T, H = 256, 64, 100, 2
    rng = np.random.default_rng(31)
    inp = rand_inputs(2, T, H, K, V, seed=31)
    inp["g"] = rng.standard_normal((2, T, H, K))
    inp["b"] = rng.standard_normal((2, T, H, K))
    inp["w"] = rng.standard_normal((2, T, H, V))
    A_log = np.log(rng.random(H) * 15 + 1)
    dt_bias = rng.standard_normal(H * K) * 0.5
    t, r = to_device(inp, gpu_device, torch.float32)
    with torch.no_grad():
        o, ht = chunk_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                           use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True,
                           A_log=torch.from_numpy(A_log).float().to(gpu_device),
                           dt_bias=torch.from_numpy(dt_bias).float().to(gpu_device), bw_logits=True)
    torch.cuda.synchronize()
    a32 = torch.from_numpy(A_log).float().double().numpy()
    d32 = torch.from_numpy(dt_bias).float().double().numpy().reshape(H, K)
    g = -np.exp(a32)[None, None, :, None] * np.logaddexp(0.0, r["g"] + d32[None, None])
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))  # noqa: E731
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, sig(r["b"]), sig(r["w"]), r["h0"])
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= TOL and es <= TOL


class _OracleRecurrence(torch.autograd.Function):
    """The float64 oracle recurrence (``gdn2.py:100-184``) with ``recurrent_vjp`` as its backward."""

    @staticmethod
    def forward(ctx, q, k, v, g, b, w):
        ctx.arrs = [x.detach().numpy() for x in (q, k, v, g, b, w)]
        o, _ = orc.recurrent_fwd(*ctx.arrs)
        return torch.from_numpy(o)

    @staticmethod
    def backward(ctx, do):
        grads = orc.recurrent_vjp(*ctx.arrs, do.numpy())
        return tuple(torch.from_numpy(np.ascontiguousarray(x)) for x in grads[:6])


def _module_ref(P, x, H, D, eps):
    """Float64 composition of ``GatedDeltaNet2.forward`` without a cache (reference
    ``gdn2.py:815-999``) on CPU tensors ``P`` (name -> parameter), differentiable."""
    B, T, _ = x.shape

    def lin(t, n):
        y = t @ P[n + ".weight"].T
        return y + P[n + ".bias"] if n + ".bias" in P else y

    def conv(t, n):
        y = F.conv1d(t.transpose(1, 2), P[n + ".conv1d.weight"], padding=3, groups=t.shape[-1])[..., :T]
        return F.silu(y).transpose(1, 2)

    heads = lambda t: t.reshape(B, T, H, D)  # noqa: E731
    q, k, v = conv(lin(x, "q_proj"), "q_conv1d"), conv(lin(x, "k_proj"), "k_conv1d"), conv(lin(x, "v_proj"), "v_conv1d")
    g = -P["A_log"].exp().repeat_interleave(D) * F.softplus(lin(lin(x, "f_proj.0"), "f_proj.1") + P["dt_bias"])
    b, w = lin(x, "b_proj").sigmoid(), lin(x, "w_proj").sigmoid()
    o = _OracleRecurrence.apply(heads(q), heads(k), heads(v), heads(g), heads(b), heads(w))
    z = heads(lin(lin(x, "g_proj.0"), "g_proj.1"))
    on = o * torch.rsqrt(o.square().mean(-1, keepdim=True) + eps) * P["o_norm.weight"] * F.silu(z)
    return lin(on.reshape(B, T, -1), "o_proj")


def test_fp32_module_head_dim_256_prefill_and_training(gpu_device):
    from qwendopamine_amd import GatedDeltaNet2

    print("[case] fp32 module head_dim=256: prefill T=150 + training step vs float64", flush=True)
    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=256, num_heads=2, head_dim=256).to(gpu_device)
    x = torch.randn(2, 150, 256, device=gpu_device)
    R = torch.randn(2, 150, 256, device=gpu_device)
    P = {n: p.detach().double().cpu().requires_grad_(True) for n, p in m.named_parameters()}
    ref = _module_ref(P, x.double().cpu(), 2, 256, m.o_norm.eps)
    (ref * R.double().cpu()).sum().backward()
    m.eval()
    with torch.no_grad():
        out, _, _ = m(x)
    torch.cuda.synchronize()
    e = rel_l2(out, ref.detach())
    print(f"  prefill rel_l2={e:.2e}", flush=True)
    assert e <= TOL
    m.train()
    out, _, _ = m(x)
    (out * R).sum().backward()
    torch.cuda.synchronize()
    assert rel_l2(out, ref.detach()) <= TOL
    errs = {n: rel_l2(p.grad, P[n].grad) for n, p in m.named_parameters()}
    worst = max(errs, key=errs.get)
    print(f"  training: worst parameter gradient {worst} rel_l2={errs[worst]:.2e}", flush=True)
    for n, err in errs.items():
        assert err <= TOL, (n, err)
